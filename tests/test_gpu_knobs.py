"""The reference's dispatch knobs and Python API on the "vulkan" device.

* TORCH_VULKAN_CONV_TILE (csrc/ops/convolution.cpp:411-414): each name forces
  its tile of this build's menu (the plan's tile index changes), selections are
  counted as selected_<phase>_tiled_<name>, a fixed-3x3 name on another filter
  raises when the tiled algorithm is forced, and an unknown name raises with
  the reference's message (tests/test_conv_dispatch.py:73-110, :399-411).
* TORCH_VULKAN_CONV_AUTOTUNE (:415-418, :523-639): plan-cache hits, misses,
  tunes and entries, reuse for a new tensor of the same descriptor, a new
  descriptor tuned afresh, only the requested gradients tuned, forced
  algorithms bypass the cache, the workspace budget is part of the key
  (tests/test_conv_dispatch.py:113-255).
* TORCH_VULKAN_MM_KERNEL and TORCH_VULKAN_FUSE_ADDMM (csrc/ops/mm.cpp:299-307,
  :851-854, :900-916).
* is_hardware_accelerated, runtime_hotpath_stats, cache_stats,
  clear_algorithm_cache, get_rng_state / set_rng_state
  (torch_vulkan/__init__.py:61-199).

Every result is checked against float64 CPU torch at rel 1e-4 / abs 1e-5
(magnitude model of tests/helpers.py); a knob changes the kernel, never the
bar.
"""
import os
import subprocess
import sys

import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close_mag, conv_refs, gemm_mag

pytestmark = pytest.mark.gpu

KNOBS = ("TORCH_VULKAN_CONV_ALGO", "TORCH_VULKAN_CONV_BACKWARD_ALGO", "TORCH_VULKAN_CONV_TILE",
         "TORCH_VULKAN_CONV_AUTOTUNE", "TORCH_VULKAN_CONV_WORKSPACE_MB", "TORCH_VULKAN_MM_KERNEL",
         "TORCH_VULKAN_FUSE_ADDMM")


@pytest.fixture(scope="module", autouse=True)
def vk():
    import torch_vulkan
    assert torch_vulkan.is_available(), "no gfx950 device visible"
    return torch_vulkan


@pytest.fixture(autouse=True)
def clean_env(monkeypatch):
    for k in KNOBS:
        monkeypatch.delenv(k, raising=False)
    monkeypatch.setenv("TORCH_VULKAN_FORBID_CPU_FALLBACK", "1")


def child_env(**extra):
    """Environment of a fresh Python process that imports torch_vulkan the way
    this one did (same sys.path), with no knob set but `extra`."""
    env = {k: v for k, v in os.environ.items() if k not in KNOBS}
    env["PYTHONPATH"] = os.pathsep.join(p for p in sys.path if p)
    env.update(extra)
    return env


def check_case(xshape, cout, kernel, stride, padding, dilation, groups, seed=225, mask=(True, True, True)):
    """Forward and the requested gradients on the device against float64."""
    g = torch.Generator().manual_seed(seed)
    cin_g = xshape[1] // groups
    x = torch.randn(xshape, generator=g) * 0.2
    w = torch.randn((cout, cin_g) + tuple(kernel), generator=g) * 0.2
    b = torch.randn(cout, generator=g) * 0.2
    args = (stride, padding, dilation, groups)
    y_ref = F.conv2d(x, w, b, *args)
    dy = torch.randn(y_ref.shape, generator=g) * 0.3
    refs = conv_refs(x, w, b, dy, *args)
    xv, wv, bv = (t.to("vulkan").requires_grad_(r) for t, r in zip((x, w, b), mask))
    yv = F.conv2d(xv, wv, bv, *args)
    assert_close_mag(yv, *refs["y"], what="y")
    need = [t for t, r in zip((xv, wv, bv), mask) if r]
    grads = iter(torch.autograd.grad(yv, need, dy.to("vulkan")))
    for name, r in zip(("dx", "dw", "db"), mask):
        if r:
            assert_close_mag(next(grads), *refs[name], what=name)


TILE_NAMES = ["base", "wide", "tall", "register"]
TILE_CASES = [
    ((2, 18, 19, 23), 34, (3, 5), (2, 1), (2, 3), (2, 1), 2),
    ((2, 32, 19, 21), 32, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((1, 9, 13, 15), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1),
]


@pytest.mark.parametrize("tile", TILE_NAMES)
@pytest.mark.parametrize("case", TILE_CASES, ids=["grouped_strided", "dense3x3", "pointwise"])
def test_forced_tile_forward_and_gradients(tile, case, vk, monkeypatch):
    """tests/test_conv_dispatch.py:73-86: the tiled algorithm with a forced
    tile, every phase within the bar and counted under the tile's name."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_ALGO", "tiled")
    monkeypatch.setenv("TORCH_VULKAN_CONV_BACKWARD_ALGO", "optimized")
    monkeypatch.setenv("TORCH_VULKAN_CONV_TILE", tile)
    before = vk.conv_dispatch_stats()
    check_case(*case)
    after = vk.conv_dispatch_stats()
    for phase in ("forward", "dinput", "dweight"):
        key = f"selected_{phase}_tiled_{tile}"
        assert after.get(key, 0) > before.get(key, 0), (phase, tile, after)


def test_fixed_3x3_tile_rejects_other_filters(vk, monkeypatch):
    """tests/test_conv_dispatch.py:405-411."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_ALGO", "tiled")
    monkeypatch.setenv("TORCH_VULKAN_CONV_TILE", "register3")
    x = torch.zeros((1, 32, 9, 13), device="vulkan")
    w = torch.zeros((32, 32, 3, 5), device="vulkan")
    with pytest.raises(RuntimeError, match="incompatible|exceeds"):
        F.conv2d(x, w)


@pytest.mark.parametrize("tile", ["register3", "register3_hoist"])
def test_fixed_3x3_tiles_on_3x3_layers(tile, vk, monkeypatch):
    """tests/test_conv_dispatch.py:392-402 and :414-431."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_ALGO", "tiled")
    monkeypatch.setenv("TORCH_VULKAN_CONV_BACKWARD_ALGO", "optimized")
    monkeypatch.setenv("TORCH_VULKAN_CONV_TILE", tile)
    before = vk.conv_dispatch_stats()
    check_case((2, 32, 31, 35), 64, (3, 3), (2, 1), (2, 1), (2, 1), 2)
    check_case((1, 9, 13, 15), 17, (3, 3), (1, 2), (0, 2), (1, 2), 1)
    after = vk.conv_dispatch_stats()
    assert after.get(f"selected_forward_tiled_{tile}", 0) >= before.get(f"selected_forward_tiled_{tile}", 0) + 2


def test_invalid_knob_values_raise(vk, monkeypatch):
    x = torch.zeros((1, 4, 6, 6), device="vulkan")
    w = torch.zeros((4, 4, 3, 3), device="vulkan")
    monkeypatch.setenv("TORCH_VULKAN_CONV_TILE", "huge")
    with pytest.raises(RuntimeError, match="TORCH_VULKAN_CONV_TILE must be auto/base/wide/tall/register"):
        F.conv2d(x, w)
    monkeypatch.delenv("TORCH_VULKAN_CONV_TILE")
    monkeypatch.setenv("TORCH_VULKAN_CONV_AUTOTUNE", "2")
    with pytest.raises(RuntimeError, match="TORCH_VULKAN_CONV_AUTOTUNE must be 0 or 1"):
        F.conv2d(x, w)


AUTOTUNE_SCRIPT = r'''
import json, sys
sys.path.insert(0, "tests")
from test_gpu_knobs import check_case
import torch_vulkan
torch_vulkan.clear_conv_dispatch_cache()
args = ((1, 9, 11, 13), 17, (3, 5), (1, 1), (1, 2), (1, 1), 1)
check_case(*args)
first = torch_vulkan.conv_dispatch_stats()
assert first["tunes"] >= 3 and first["entries"] >= 3 and first["candidates_timed"] >= 3, first
for phase in ("forward", "dinput", "dweight"):
    assert first.get(f"candidates_timed_{phase}_implicit_gemm", 0) > 0, first
    assert first.get(f"candidates_timed_{phase}_direct", 0) > 0, first
check_case(*args, seed=7)   # same descriptor, new tensors: the plans are reused
second = torch_vulkan.conv_dispatch_stats()
assert second["tunes"] == first["tunes"] and second["hits"] >= first["hits"] + 3, (first, second)
check_case((1, 9, 11, 14), *args[1:])   # a new descriptor is tuned afresh
third = torch_vulkan.conv_dispatch_stats()
assert third["tunes"] > second["tunes"] and third["entries"] > second["entries"], (second, third)
assert third["entries"] <= 256
print("AUTOTUNE_REPORT=" + json.dumps({"first": first, "third": third}))
'''


def test_autotune_reuses_plans_and_keeps_results(vk):
    """tests/test_conv_dispatch.py:113-160, in a fresh process."""
    env = child_env(TORCH_VULKAN_CONV_AUTOTUNE="1", TORCH_VULKAN_FORBID_CPU_FALLBACK="1")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    run = subprocess.run([sys.executable, "-c", AUTOTUNE_SCRIPT], cwd=root, env=env, text=True,
                         capture_output=True, timeout=110)
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-3000:]
    assert any(line.startswith("AUTOTUNE_REPORT=") for line in run.stdout.splitlines()), run.stdout


@pytest.mark.parametrize("mask", [(True, False, False), (False, True, False), (False, False, True)])
def test_autotune_only_requested_gradient(mask, vk, monkeypatch):
    """tests/test_conv_dispatch.py:184-208."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_AUTOTUNE", "1")
    g = torch.Generator().manual_seed(479)
    x = torch.randn((1, 9, 7, 11), generator=g) * 0.2
    w = torch.randn((17, 9, 3, 5), generator=g) * 0.2
    go = torch.randn((1, 17, 7, 11), generator=g) * 0.3
    backward = torch.ops.aten.convolution_backward.default
    params = ([17], [1, 1], [1, 2], [1, 1], False, [0, 0], 1, list(mask))
    expected = backward(go.double(), x.double(), w.double(), *params)
    vk.clear_conv_dispatch_cache()
    result = backward(go.to("vulkan"), x.to("vulkan"), w.to("vulkan"), *params)
    for enabled, actual, ref in zip(mask, result, expected):
        if enabled:
            torch.testing.assert_close(actual.cpu().double(), ref, rtol=1e-4, atol=1e-5)
        else:
            assert actual is None
    stats = vk.conv_dispatch_stats()
    for enabled, phase in zip(mask, ("dinput", "dweight", "dbias")):
        count = sum(v for k, v in stats.items() if k.startswith(f"selected_{phase}_"))
        assert (count > 0) if enabled else (count == 0), (mask, phase, stats)
        if phase != "dbias":
            timed = stats.get(f"candidates_timed_{phase}_implicit_gemm", 0)
            assert (timed > 0) if enabled else (timed == 0), (mask, phase, stats)


def test_forced_algorithms_bypass_autotuning(vk, monkeypatch):
    """tests/test_conv_dispatch.py:211-225."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_AUTOTUNE", "1")
    vk.clear_conv_dispatch_cache()
    args = ((1, 9, 7, 11), 17, (3, 5), (1, 1), (1, 2), (1, 1), 1)
    check_case(*args)
    before = vk.conv_dispatch_stats()
    monkeypatch.setenv("TORCH_VULKAN_CONV_ALGO", "direct")
    monkeypatch.setenv("TORCH_VULKAN_CONV_BACKWARD_ALGO", "direct")
    check_case(*args)
    after = vk.conv_dispatch_stats()
    for key in ("hits", "misses", "tunes", "entries", "candidates_timed"):
        assert after[key] == before[key], (key, before, after)
    for phase in ("forward", "dinput", "dweight"):
        assert after.get(f"selected_{phase}_direct", 0) == before.get(f"selected_{phase}_direct", 0) + 1


def test_autotune_workspace_budget_is_part_of_the_key(vk, monkeypatch):
    """tests/test_conv_dispatch.py:228-255."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_AUTOTUNE", "1")
    monkeypatch.setenv("TORCH_VULKAN_CONV_WORKSPACE_MB", "64")
    vk.clear_conv_dispatch_cache()
    args = ((1, 9, 1, 257), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1)
    check_case(*args)
    first = vk.conv_dispatch_stats()
    monkeypatch.setenv("TORCH_VULKAN_CONV_WORKSPACE_MB", "0")
    check_case(*args)
    second = vk.conv_dispatch_stats()
    assert second["tunes"] > first["tunes"] and second["entries"] > first["entries"], (first, second)
    check_case(*args)
    third = vk.conv_dispatch_stats()
    assert third["tunes"] == second["tunes"] and third["hits"] >= second["hits"] + 3, (second, third)


def test_autotune_picks_a_measured_faster_algorithm(vk, monkeypatch):
    """C1's layer: AUTO's heuristic takes the implicit GEMM; autotuning times
    the Winograd candidates too and keeps whichever is 5% faster, and the
    results stay within the bar of the algorithm it picked."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_AUTOTUNE", "1")
    vk.clear_conv_dispatch_cache()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8, 64, 56, 56, generator=g)
    w = torch.randn(64, 64, 3, 3, generator=g) / 24
    xv = x.to("vulkan").requires_grad_()
    wv = w.to("vulkan").requires_grad_()
    yv = F.conv2d(xv, wv, None, 1, 1)
    yv.sum().backward()
    stats = vk.conv_dispatch_stats()
    for phase in ("forward", "dinput", "dweight"):
        assert stats.get(f"candidates_timed_{phase}_winograd_f2", 0) == 1, stats
        assert stats.get(f"candidates_timed_{phase}_implicit_gemm", 0) == 1, stats
    ref, mag = conv_refs(x, w, None, torch.ones_like(x[:, :64]), (1, 1), (1, 1), (1, 1), 1)["y"]
    wino = stats.get("selected_forward_winograd_f2", 0) > 0
    assert_close_mag(yv, ref, mag, rtol=1e-3 if wino else 1e-4, what="y")
    print(f"[knobs] C1 autotuned: forward {'winograd' if wino else 'implicit_gemm'}; "
          + ", ".join(k for k in stats if k.startswith("selected_")))


@pytest.mark.parametrize("kernel", ["register", "tiled", "auto"])
@pytest.mark.parametrize("fuse", ["1", "0"])
def test_mm_kernel_and_fuse_addmm_knobs(kernel, fuse, vk, monkeypatch):
    """csrc/ops/mm.cpp:299-307, :851-854, :900-916: both kernels and the
    unfused addmm give the same results within the bar, NaN bias ignored at
    beta = 0.  (That the kernel class reaches the tile choice is a host test,
    tests/test_abi_host.py.)"""
    monkeypatch.setenv("TORCH_VULKAN_MM_KERNEL", kernel)
    monkeypatch.setenv("TORCH_VULKAN_FUSE_ADDMM", fuse)
    g = torch.Generator().manual_seed(31)
    a = torch.randn(300, 257, generator=g)
    b = torch.randn(257, 290, generator=g)
    bias = torch.randn(290, generator=g)
    ref = torch.addmm(bias.double(), a.double(), b.double(), beta=0.5, alpha=1.5)
    out = torch.addmm(bias.to("vulkan"), a.to("vulkan"), b.to("vulkan"), beta=0.5, alpha=1.5)
    assert_close_mag(out, ref, gemm_mag(a, b, 1.5, 0.5, bias), what=f"addmm {kernel} fuse={fuse}")
    nan_bias = torch.full((290,), float("nan"))
    out0 = torch.addmm(nan_bias.to("vulkan"), a.to("vulkan"), b.to("vulkan"), beta=0.0)
    assert torch.isfinite(out0.cpu()).all()
    assert_close_mag(out0, a.double() @ b.double(), gemm_mag(a, b), what="beta 0")
    mm = torch.mm(a.to("vulkan"), b.to("vulkan"))
    assert_close_mag(mm, a.double() @ b.double(), gemm_mag(a, b), what="mm")


def test_python_api_of_the_reference(vk):
    """is_hardware_accelerated, runtime_hotpath_stats, cache_stats,
    clear_algorithm_cache and the RNG state round trip exist with the
    reference's keys."""
    assert vk.is_hardware_accelerated() is True
    hot = vk.runtime_hotpath_stats()
    for k in ("algo_hit_ns", "algo_miss_ns", "enqueue_ns", "enqueue_count", "allocator_ns", "allocator_calls",
              "allocator_fresh_calls", "allocator_reused_calls"):
        assert k in hot and hot[k] >= 0
    cs = vk.cache_stats()
    for k in ("algo_hits", "algo_misses", "seq_reuses", "seq_creates", "algo_evictions", "bound_algorithms",
              "pipeline_hits", "pipeline_misses", "pipeline_entries"):
        assert k in cs
    vk.clear_algorithm_cache()
    assert vk.conv_dispatch_stats()["entries"] == 0
    vk.manual_seed(1234)
    state = vk.get_rng_state()
    assert state.dtype == torch.uint8 and state.numel() == 16
    vk.manual_seed(99)
    assert vk.initial_seed() == 99
    vk.set_rng_state(state)
    assert vk.initial_seed() == 1234
    assert torch.equal(vk.get_rng_state(), state)


HOTPATH_SCRIPT = r'''
import torch, torch_vulkan
x = torch.randn(2, 8, 9, 9).to("vulkan")
w = torch.randn(8, 8, 3, 3).to("vulkan")
y = torch.nn.functional.conv2d(x, w, padding=1)
torch_vulkan.synchronize()
s = torch_vulkan.runtime_hotpath_stats()
assert s["enqueue_count"] >= 1 and s["enqueue_ns"] > 0, s
assert s["allocator_calls"] >= 3 and s["allocator_fresh_calls"] + s["allocator_reused_calls"] == s["allocator_calls"], s
print("HOTPATH_OK", s["enqueue_count"], s["allocator_calls"])
'''


def test_runtime_hotpath_stats_record_when_enabled(vk):
    env = child_env(TORCH_VULKAN_PROFILE_HOST_HOTPATH="1")
    run = subprocess.run([sys.executable, "-c", HOTPATH_SCRIPT], env=env, text=True, capture_output=True,
                         timeout=110)
    assert run.returncode == 0 and "HOTPATH_OK" in run.stdout, run.stdout[-2000:] + run.stderr[-2000:]
