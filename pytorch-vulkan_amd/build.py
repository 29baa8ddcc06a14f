"""Builds the gfx950 libraries in-tree.

    python pytorch-vulkan_amd/build.py [--only mx|ext] [--incremental] [-j N]

Outputs (next to the Python package so they travel with the source tree):
  torch_vulkan/libmx.so  C-ABI library (include/mx.h): HIP runtime layer and
                         every gfx950 kernel, built with hipcc.
  torch_vulkan/_C.so     PrivateUse1 "vulkan" operator surface (C++ against
                         the installed torch headers), linked to libmx.so.
  ../libmxprobe.so            HBM stream probes used by bench.py, built beside it (not part of
                         the C ABI).

libmx.so links the HIP runtime that ships inside the installed torch wheel
(torch/lib/libamdhip64.so) so that a process which imports torch never loads
a second HIP runtime; with a wheel that has none (a CPU-only torch, which the
drop-in surface supports) it links ROCm's own runtime (ROCM_PATH/lib).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
OUT = PKG / "torch_vulkan"
INCLUDE = REPO / "include"

ARCH = os.environ.get("MX_OFFLOAD_ARCH", "gfx950")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
    # Packed FP32 instructions stay off (the compiler would otherwise form
    # v_pk_{add,mul,fma}_f32 from scalar code).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]
MX_SOURCES = ["mx_runtime.hip", "mx_gemm.hip", "mx_conv.hip", "mx_conv_fwd.hip", "mx_conv_dx.hip", "mx_conv_dw.hip",
              "mx_winograd.hip", "mx_adamw.hip", "mx_util.hip", "mx_nn.hip", "mx_foreach.hip"]
EXT_SOURCES = ["backend.cpp", "ops_conv.cpp", "ops_gemm.cpp", "ops_adamw.cpp", "ops_plumbing.cpp", "ops_nn.cpp", "ops_foreach.cpp"]


def torch_paths():
    import torch.utils.cpp_extension as ce  # noqa: WPS433 (build-time only)
    import torch
    return ce.include_paths(), str(Path(torch.__file__).parent / "lib")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the gfx950 build needs ROCm's hipcc")


def run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def compile_hip(cmd: list[str]) -> None:
    """hipcc -c with the per-kernel resource remarks; a kernel that needs
    scratch (private) memory fails the build: every kernel here keeps its
    state in registers and LDS."""
    res = subprocess.run(cmd + ["-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics"], stdout=subprocess.PIPE,
                         stderr=subprocess.STDOUT, text=True)
    keep, scratch, fn = [], [], None
    for line in res.stdout.splitlines():
        if "packed-fp32-ops" in line:
            continue
        if "kernel-resource-usage" in line:
            if "Function Name:" in line:
                fn = line.split("Function Name:")[1].split("[")[0].strip()
            elif "ScratchSize [bytes/lane]:" in line:
                n = int(line.split("ScratchSize [bytes/lane]:")[1].split()[0])
                if n:
                    scratch.append(f"{fn} ({n} B/lane)")
            continue
        keep.append(line)
    out = "\n".join(keep)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)
    if scratch:
        # Drop the object so an incremental build compiles (and checks) it again.
        obj = Path(cmd[cmd.index("-o") + 1])
        obj.unlink(missing_ok=True)
        raise RuntimeError(f"{obj.name}: kernels using scratch memory:\n  " + "\n  ".join(scratch))


def wait_all(futures) -> None:
    """Waits for every job and raises the first failure after all have ended
    (a failing compile must not hide another job's result)."""
    errors = []
    for f in futures:
        try:
            f.result()
        except Exception as e:  # noqa: BLE001 (reported below)
            errors.append(e)
    if errors:
        raise RuntimeError("\n\n".join(str(e) for e in errors))


def stale(target: Path, deps: list[Path]) -> bool:
    if not target.exists():
        return True
    t = target.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def hip_runtime_dir(torch_lib: str) -> str:
    """Directory of the HIP runtime libmx.so links and finds at run time: the
    torch wheel's own copy when it ships one, else ROCm's."""
    if any(Path(torch_lib).glob("libamdhip64.so*")):
        return torch_lib
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib"
    if any(rocm.glob("libamdhip64.so*")):
        return str(rocm)
    raise RuntimeError(f"no libamdhip64.so in {torch_lib} or {rocm}: the HIP runtime is needed to link libmx.so")


def link_mx(objs, out: Path, runtime_dir: str) -> None:
    """Plain host link (non-relocatable device code needs no device link
    step); hipcc would add -lamdhip64 from /opt/rocm even where torch ships
    its own runtime."""
    tmp = out.with_name(out.name + ".tmp")
    cxx = os.environ.get("CXX", "g++")
    run([cxx, "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
         f"-L{runtime_dir}", f"-Wl,-rpath,{runtime_dir}", "-lamdhip64", "-Wl,--no-undefined"])
    tmp.replace(out)


def build_mx(jobs: int, incremental: bool) -> Path:
    BUILD.mkdir(exist_ok=True)
    OUT.mkdir(exist_ok=True)
    headers = list(CSRC.glob("*.hpp")) + [INCLUDE / "mx.h"]
    _, torch_lib = torch_paths()
    cc = hipcc()
    objs, todo = [], []
    for src in MX_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        if not incremental or stale(obj, [CSRC / src] + headers):
            todo.append([cc, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        wait_all([ex.submit(compile_hip, c) for c in todo])
    lib = OUT / "libmx.so"
    if not incremental or stale(lib, objs):
        link_mx(objs, lib, hip_runtime_dir(torch_lib))
    return lib


def build_probe(incremental: bool) -> Path:
    """libmxprobe.so at the repository root, beside bench.py: its HBM stream
    probes (csrc/bench/mx_stream_probe.hip), outside the torch_vulkan package
    and apart from the C ABI library."""
    BUILD.mkdir(exist_ok=True)
    _, torch_lib = torch_paths()
    src = CSRC / "bench" / "mx_stream_probe.hip"
    obj = BUILD / "mx_stream_probe.o"
    if not incremental or stale(obj, [src]):
        compile_hip([hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
    lib = Path(__file__).resolve().parent.parent / "libmxprobe.so"
    if not incremental or stale(lib, [obj]):
        link_mx([obj], lib, hip_runtime_dir(torch_lib))
    return lib


def build_ext(jobs: int, incremental: bool) -> Path:
    BUILD.mkdir(exist_ok=True)
    incs, torch_lib = torch_paths()
    py_inc = sysconfig.get_paths()["include"]
    cxx = os.environ.get("CXX", "g++")
    flags = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-parameter", "-D_GLIBCXX_USE_CXX11_ABI=1",
             "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
             f"-I{INCLUDE}", f"-I{PKG / 'csrc' / 'torch'}", f"-I{py_inc}", *[f"-I{i}" for i in incs]]
    try:
        import torch
        abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
        flags = [f for f in flags if not f.startswith("-D_GLIBCXX_USE_CXX11_ABI")] + [f"-D_GLIBCXX_USE_CXX11_ABI={abi}"]
    except Exception:  # pragma: no cover - torch import failure surfaces below
        pass
    headers = list((PKG / "csrc" / "torch").glob("*.h")) + [INCLUDE / "mx.h"]
    objs, todo = [], []
    for src in EXT_SOURCES:
        path = PKG / "csrc" / "torch" / src
        obj = BUILD / ("ext_" + Path(src).stem + ".o")
        objs.append(obj)
        if not incremental or stale(obj, [path] + headers):
            todo.append([cxx, *flags, "-c", str(path), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        wait_all([ex.submit(run, c) for c in todo])
    so = OUT / "_C.so"
    if not incremental or stale(so, objs + [OUT / "libmx.so"]):
        tmp = OUT / "_C.so.tmp"
        run([cxx, "-shared", "-o", str(tmp), *map(str, objs), f"-L{OUT}", "-lmx", "-Wl,-rpath,$ORIGIN",
             f"-L{torch_lib}", f"-Wl,-rpath,{torch_lib}", "-lc10", "-ltorch_cpu", "-ltorch", "-ltorch_python"])
        tmp.replace(so)
    return so


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--only", choices=["mx", "ext"], default=None)
    ap.add_argument("--incremental", action="store_true")
    ap.add_argument("-j", type=int, default=min(8, os.cpu_count() or 4))
    args = ap.parse_args(argv)
    if args.only in (None, "mx"):
        print("built", build_mx(args.j, args.incremental))
        print("built", build_probe(args.incremental))
    if args.only in (None, "ext"):
        print("built", build_ext(args.j, args.incremental))
    return 0


if __name__ == "__main__":
    sys.exit(main())
