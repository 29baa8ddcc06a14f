"""AddressSanitizer + UndefinedBehaviorSanitizer build of the C-ABI layer's
host code, run on the CPU only.

    python pytorch-vulkan_amd/sanitize.py [--build-only]

Builds _build_san/libmx.so from the same sources as build.py with the host
pass instrumented (-Xarch_host -fsanitize=address / undefined; the gfx950
device code is compiled exactly as in the product build and never runs
here), links it with clang's shared sanitizer runtimes, and runs the host
tests that drive the library's planners, descriptor checks and error paths
(tests/test_abi_host.py, tests/test_plan_coverage.py) against it in a child
Python with the ASan runtime preloaded.  A sanitizer report fails the run
(halt_on_error, UBSan reports made fatal).  Leak checking is off: the Python
interpreter and torch are not instrumented and keep their allocations to the
end of the process.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys
from pathlib import Path

import build as B

SAN_BUILD = B.PKG / "_build_san"
SAN_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
            "-Xarch_host", "-g"]
TESTS = ["tests/test_abi_host.py", "tests/test_plan_coverage.py"]


def llvm_bin(name: str) -> str:
    return str(Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "llvm" / "bin" / name)


def asan_runtime() -> str:
    libs = sorted(glob.glob(str(Path(llvm_bin("clang")).parent.parent / "lib" / "clang" / "*" / "lib" / "linux" /
                                "libclang_rt.asan-x86_64.so")))
    if not libs:
        raise RuntimeError("clang's shared ASan runtime (libclang_rt.asan-x86_64.so) was not found")
    return libs[-1]


def build(jobs: int) -> Path:
    SAN_BUILD.mkdir(exist_ok=True)
    _, torch_lib = B.torch_paths()
    objs, todo = [], []
    for src in B.MX_SOURCES:
        obj = SAN_BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        todo.append([B.hipcc(), *B.HIP_FLAGS, *SAN_HOST, "-c", str(B.CSRC / src), "-o", str(obj)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        B.wait_all([ex.submit(B.run, c) for c in todo])
    lib = SAN_BUILD / "libmx.so"
    rt = B.hip_runtime_dir(torch_lib)
    # Host-object link with clang++ so the instrumented objects get clang's
    # own (shared) sanitizer runtimes; no device code is linked here.
    B.run([llvm_bin("clang++"), "-shared", "-fPIC", "-shared-libsan", "-fsanitize=address,undefined", "-o",
           str(lib), *map(str, objs), f"-L{rt}", f"-Wl,-rpath,{rt}", "-lamdhip64"])
    return lib


def run_tests(lib: Path) -> int:
    env = dict(os.environ)
    env["MX_LIBRARY"] = str(lib)
    env["LD_PRELOAD"] = asan_runtime()
    env["ASAN_OPTIONS"] = "detect_leaks=0:halt_on_error=1:abort_on_error=0:protect_shadow_gap=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    cmd = [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", "-m", "not gpu", *TESTS]
    print("running", " ".join(cmd), "with", lib, flush=True)
    return subprocess.run(cmd, cwd=B.REPO, env=env).returncode


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--build-only", action="store_true")
    ap.add_argument("-j", type=int, default=min(8, os.cpu_count() or 1))
    args = ap.parse_args()
    lib = build(args.j)
    print("built", lib, flush=True)
    return 0 if args.build_only else run_tests(lib)


if __name__ == "__main__":
    sys.exit(main())
