"""mx_conv2d_backward_weight_noalloc (include/mx.h): the allocation-free
dWeight / dBias entry point, against the allocating mx_conv2d_backward_weight
on the same inputs, through the C ABI.

Both run the same kernels; their plans differ only where the allocating
call's split-K workspace would exceed the no-alloc scratch
(MX_NOALLOC_SCRATCH_BYTES), so results are compared bit for bit when the plans
agree and otherwise to the parity bar (rel 1e-4 / abs 1e-5 with the magnitude
model of tests/helpers.py; rel 1e-3 for Winograd) against float64.  Calls come
in pairs, the second on a smaller input, and the library's allocator counters
must not move across no-alloc calls.
"""
from __future__ import annotations

import math

import pytest
import torch

import plan_cases as P
from helpers import ATOL, RTOL, WINOGRAD_RTOL, assert_close_mag, conv_refs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mx():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from torch_vulkan import mx as m
    m.lib()
    return m


def stream():
    return torch.cuda.current_stream().cuda_stream


def alloc_counters(mx):
    st = mx.MemoryStats()
    mx.check(mx.lib().mx_memory_stats_get(mx.C.byref(st)))
    return st.device_mallocs, st.cache_hits, st.allocated_bytes


class Case:
    def __init__(self, mx, xs, cout, k, stride, pad, seed):
        self.d = mx.conv_desc(xs, (cout, xs[1], k, k), (stride, stride), (pad, pad))
        g = torch.Generator().manual_seed(seed)
        self.x = torch.randn(xs, generator=g)
        self.w = torch.randn(cout, xs[1], k, k, generator=g) / math.sqrt(xs[1] * k * k)
        self.b = torch.randn(cout, generator=g) * 0.1
        self.dy = torch.randn(xs[0], cout, self.d.oh, self.d.ow, generator=g)
        self.refs = conv_refs(self.x, self.w, self.b, self.dy, (stride, stride), (pad, pad), (1, 1), 1)
        self.X, self.DY = self.x.cuda(), self.dy.cuda()
        self.dw = {k_: torch.full(self.w.shape, float("nan"), device="cuda") for k_ in ("alloc", "noalloc")}
        self.db = {k_: torch.full((cout,), float("nan"), device="cuda") for k_ in ("alloc", "noalloc")}


CASES = [  # (first, smaller second) per pair
    (((8, 64, 56, 56), 64, 3, 1, 1), ((2, 32, 14, 14), 48, 3, 1, 1)),    # C1 layer, split-K within the scratch
    (((64, 64, 56, 56), 64, 3, 1, 1), ((4, 64, 28, 28), 64, 3, 1, 1)),   # plan shrinks to fit 16 MiB
    (((16, 256, 28, 28), 512, 1, 2, 0), ((3, 64, 15, 15), 96, 1, 2, 0)),  # 1x1 stride 2, 128x128 tile
]


@pytest.mark.parametrize("algo", ["implicit_gemm", "winograd"])
@pytest.mark.parametrize("pair", CASES, ids=["c1", "shrink", "strided"])
def test_noalloc_matches_allocating_entry_point(mx, pair, algo):
    A = mx.ALGO_IMPLICIT_GEMM if algo == "implicit_gemm" else mx.ALGO_WINOGRAD
    for spec in pair:
        xs, cout, k, stride, pad = spec
        if A == mx.ALGO_WINOGRAD and (k != 3 or stride != 1):
            continue
        c = Case(mx, xs, cout, k, stride, pad, seed=sum(xs) + cout)
        mx.conv2d_backward_weight(c.d, c.X, c.DY, c.dw["alloc"], c.db["alloc"], A, stream())
        torch.cuda.synchronize()
        before = alloc_counters(mx)
        mx.conv2d_backward_weight_noalloc(c.d, c.X, c.DY, c.dw["noalloc"], c.db["noalloc"], A, stream())
        torch.cuda.synchronize()
        assert alloc_counters(mx)[:2] == before[:2], "the no-alloc entry point allocated device memory"
        plan = mx.conv2d_plan(c.d, mx.MX_CONV_DWEIGHT, A, True)
        with P.env({"TORCH_VULKAN_CONV_WORKSPACE_MB": mx.NOALLOC_SCRATCH_BYTES >> 20}):
            fitted = mx.conv2d_plan(c.d, mx.MX_CONV_DWEIGHT, A, True)
        assert fitted["workspace_bytes"] <= mx.NOALLOC_SCRATCH_BYTES
        rtol = WINOGRAD_RTOL if A == mx.ALGO_WINOGRAD else RTOL
        for name, got in (("dw", c.dw), ("db", c.db)):
            ref, mag = c.refs[name]
            assert_close_mag(got["noalloc"], ref, mag, rtol=rtol, atol=ATOL, what=f"{spec} no-alloc {name}")
            assert_close_mag(got["noalloc"], got["alloc"].double(), mag, rtol=rtol, atol=ATOL,
                             what=f"{spec} no-alloc vs allocating {name}")
            if plan == fitted:
                assert torch.equal(got["noalloc"], got["alloc"]), f"{spec} {name}: same plan, different bits"


def test_noalloc_rejects_what_cannot_fit(mx, monkeypatch):
    """A batch run in chunks (made small by MX_CONV_BUFFER_LIMIT) whose partial
    gradient is larger than the scratch fails with MX_ERR_WORKSPACE before any
    launch, while the allocating entry point runs it; a forced many-way split
    shrinks to fit the scratch."""
    d = mx.conv_desc((2, 2048, 2, 2), (2049, 2048, 1, 1))
    x = torch.randn(2, 2048, 2, 2, device="cuda")
    dy = torch.randn(2, 2049, 2, 2, device="cuda")
    dw = torch.empty(2049, 2048, 1, 1, device="cuda")
    assert dw.numel() * 4 > mx.NOALLOC_SCRATCH_BYTES
    monkeypatch.setenv("MX_CONV_BUFFER_LIMIT", str(2049 * 4 * 4))  # one image per launch
    with pytest.raises(mx.MXError, match="workspace") as e:
        mx.conv2d_backward_weight_noalloc(d, x, dy, dw, None, mx.ALGO_IMPLICIT_GEMM, stream())
    assert e.value.status == mx.MX_ERR_WORKSPACE
    mx.conv2d_backward_weight(d, x, dy, dw, None, mx.ALGO_IMPLICIT_GEMM, stream())
    ref = torch.einsum("nchw,nkhw->kc", x.double(), dy.double())
    assert torch.allclose(dw.double().view(2049, 2048), ref, rtol=1e-4, atol=1e-4)
    monkeypatch.delenv("MX_CONV_BUFFER_LIMIT")
    d2 = mx.conv_desc((64, 64, 56, 56), (64, 64, 3, 3), (1, 1), (1, 1))
    monkeypatch.setenv("MX_CONV_PLAN", "5,512")
    monkeypatch.setenv("TORCH_VULKAN_CONV_WORKSPACE_MB", "4096")
    plan = mx.conv2d_plan(d2, mx.MX_CONV_DWEIGHT, mx.ALGO_IMPLICIT_GEMM, True)
    assert plan["workspace_bytes"] > mx.NOALLOC_SCRATCH_BYTES  # the allocating call would use more
    x2 = torch.randn(64, 64, 56, 56, device="cuda")
    dy2 = torch.randn(64, 64, 56, 56, device="cuda")
    dw2 = torch.empty(64, 64, 3, 3, device="cuda")
    db2 = torch.empty(64, device="cuda")
    mx.conv2d_backward_weight_noalloc(d2, x2, dy2, dw2, db2, mx.ALGO_IMPLICIT_GEMM, stream())  # shrinks to fit
    torch.cuda.synchronize()
    assert torch.isfinite(dw2).all()


def test_noalloc_chunked_batch(mx, monkeypatch):
    """A batch run one image per launch (MX_CONV_BUFFER_LIMIT) with dBias: the
    chunk sums live in the scratch's tail, the chunks' split partials in the
    rest; same result as the allocating entry point, no allocation."""
    c = Case(mx, (4, 64, 16, 16), 64, 3, 1, 1, seed=5)
    monkeypatch.setenv("MX_CONV_BUFFER_LIMIT", str(64 * 16 * 16 * 4))
    mx.conv2d_backward_weight(c.d, c.X, c.DY, c.dw["alloc"], c.db["alloc"], mx.ALGO_IMPLICIT_GEMM, stream())
    torch.cuda.synchronize()
    before = alloc_counters(mx)
    mx.conv2d_backward_weight_noalloc(c.d, c.X, c.DY, c.dw["noalloc"], c.db["noalloc"], mx.ALGO_IMPLICIT_GEMM,
                                      stream())
    torch.cuda.synchronize()
    assert alloc_counters(mx)[:2] == before[:2]
    for name, got in (("dw", c.dw), ("db", c.db)):
        ref, mag = c.refs[name]
        assert_close_mag(got["noalloc"], ref, mag, what=f"chunked no-alloc {name}")
        assert_close_mag(got["noalloc"], got["alloc"].double(), mag, what=f"chunked no-alloc vs allocating {name}")
