"""Seeded random convolution geometries and GEMM shapes through the C ABI,
against float64 CPU PyTorch.

Convolutions: every phase and algorithm that applies.

The fixed cases elsewhere pin the shapes the planner and the kernels were
built around; these cover the combinations between them: odd channel counts
per group, non-square kernels from 1 to 7, strides 1-3, dilation 2, padding up
to the kernel's reach, one to three images, grouped layers.  The same
geometry goes through AUTO, the implicit GEMM, the direct kernels (where the
serial weight gradient stays small) and, for 3x3 stride-1 layers, Winograd
F(2x2,3x3), plus the one-call backward (mx_conv2d_backward).  Tolerances as
in test_gpu_abi.py: rel 1e-4 / abs 1e-5 on the magnitude of the summed terms,
rel 1e-3 where Winograd runs.

GEMM: 1-700 per dimension, 2-D and batched, transposed and offset operand
views, column and matrix bias with alpha / beta, at rel 1e-4 / abs 1e-5.
"""
import math

import numpy as np
import pytest
import torch

from helpers import ATOL, RTOL, WINOGRAD_RTOL, assert_close_mag, conv_refs, gemm_mag

pytestmark = pytest.mark.gpu


def _geometries(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        groups = int(rng.choice([1, 1, 1, 2, 3, 4]))
        if len(out) % 4 == 3:
            # 3x3 stride 1: the Winograd-eligible family, with enough channels
            # for AUTO to pick it on some phases.
            kh = kw = 3
            sh = sw = dh = dw = 1
            cin_g, cout_g = int(rng.integers(28, 72)), int(rng.integers(28, 72))
            groups = int(rng.choice([1, 1, 2]))
        else:
            kh, kw = (int(v) for v in rng.choice([1, 2, 3, 4, 5, 7], size=2))
            sh, sw = (int(v) for v in rng.integers(1, 4, size=2))
            dh, dw = (int(v) for v in rng.choice([1, 1, 2], size=2))
            cin_g, cout_g = int(rng.integers(1, 41)), int(rng.integers(1, 41))
        reach_h, reach_w = dh * (kh - 1) + 1, dw * (kw - 1) + 1
        ph = int(rng.integers(0, min(reach_h, 5)))
        pw = int(rng.integers(0, min(reach_w, 5)))
        n = int(rng.integers(1, 4))
        h = int(rng.integers(max(1, reach_h - 2 * ph), 31))
        w = int(rng.integers(max(1, reach_w - 2 * pw), 31))
        oh = (h + 2 * ph - reach_h) // sh + 1
        ow = (w + 2 * pw - reach_w) // sw + 1
        if oh < 1 or ow < 1:
            continue
        out.append(((n, cin_g * groups, h, w), cout_g * groups, (kh, kw), (sh, sw), (ph, pw), (dh, dw), groups))
    return out


CASES = _geometries(40, seed=20261202)


@pytest.fixture(scope="module")
def mx():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from torch_vulkan import mx as m
    m.lib()
    return m


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _inputs(case, seed):
    xs, cout, kernel, stride, padding, dilation, groups = case
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(xs, generator=g)
    fan_in = xs[1] // groups * kernel[0] * kernel[1]
    w = torch.randn((cout, xs[1] // groups, *kernel), generator=g) / math.sqrt(fan_in)
    b = torch.randn(cout, generator=g) * 0.1
    return x, w, b


def _algos(case):
    xs, cout, kernel, stride, padding, dilation, groups = case
    algos = ["auto", "implicit_gemm"]
    if kernel == (3, 3) and stride == (1, 1) and dilation == (1, 1):
        algos.append("winograd")
    # The direct weight gradient is a serial loop per weight: small layers only.
    if xs[0] * xs[2] * xs[3] * cout <= 60000:
        algos.append("direct")
    return algos


PARAMS = [(i, a) for i, c in enumerate(CASES) for a in _algos(c)]


@pytest.mark.parametrize("idx,algo", PARAMS, ids=[f"r{i}-{a}" for i, a in PARAMS])
def test_random_geometry_all_phases(mx, idx, algo):
    case = CASES[idx]
    xs, cout, kernel, stride, padding, dilation, groups = case
    A = {"auto": mx.ALGO_AUTO, "implicit_gemm": mx.ALGO_IMPLICIT_GEMM, "winograd": mx.ALGO_WINOGRAD,
         "direct": mx.ALGO_DIRECT}[algo]
    x, w, b = _inputs(case, seed=1000 + idx)
    d = mx.conv_desc(xs, w.shape, stride, padding, dilation, groups)
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(2000 + idx))
    refs = conv_refs(x, w, b, dy, stride, padding, dilation, groups)
    X, W, B, DY = (t.to("cuda") for t in (x, w, b, dy))
    y = torch.empty(dy.shape, device="cuda")
    dx = torch.empty(xs, device="cuda")
    dw = torch.empty(w.shape, device="cuda")
    db = torch.empty(cout, device="cuda")
    # Winograd input gradients need padding <= 2; other phases of such a
    # layer still run Winograd.
    A_dx = A
    if A == mx.ALGO_WINOGRAD and max(padding) > 2:
        A_dx = mx.ALGO_IMPLICIT_GEMM
    mx.conv2d_forward(d, X, W, B, y, A, _stream())
    mx.conv2d_backward_input(d, DY, W, dx, A_dx, _stream())
    mx.conv2d_backward_weight(d, X, DY, dw, db, A, _stream())
    used = {"y": mx.conv2d_select(d, mx.MX_CONV_FORWARD, A), "dx": mx.conv2d_select(d, mx.MX_CONV_DINPUT, A_dx),
            "dw": mx.conv2d_select(d, mx.MX_CONV_DWEIGHT, A)}
    used["db"] = used["dw"]
    for name, got in (("y", y), ("dx", dx), ("dw", dw), ("db", db)):
        ref, mag = refs[name]
        rtol = WINOGRAD_RTOL if used[name] == mx.ALGO_WINOGRAD else RTOL
        assert_close_mag(got, ref, mag, rtol=rtol, atol=ATOL, what=f"{name} ({case}, {algo} -> algo {used[name]})")


@pytest.mark.parametrize("idx", range(0, len(CASES), 2), ids=[f"r{i}" for i in range(0, len(CASES), 2)])
def test_random_geometry_one_call_backward(mx, idx):
    """mx_conv2d_backward (dx, dW and dBias in one call, with the one-launch
    Winograd backward where it applies) against the float64 gradients."""
    case = CASES[idx]
    xs, cout, kernel, stride, padding, dilation, groups = case
    x, w, b = _inputs(case, seed=3000 + idx)
    d = mx.conv_desc(xs, w.shape, stride, padding, dilation, groups)
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(4000 + idx))
    refs = conv_refs(x, w, b, dy, stride, padding, dilation, groups)
    X, W, DY = (t.to("cuda") for t in (x, w, dy))
    dx = torch.empty(xs, device="cuda")
    dw = torch.empty(w.shape, device="cuda")
    db = torch.empty(cout, device="cuda")
    mx.conv2d_backward(d, X, W, DY, dx, dw, db, mx.ALGO_AUTO, mx.ALGO_AUTO, _stream())
    used_dx = mx.conv2d_select(d, mx.MX_CONV_DINPUT, mx.ALGO_AUTO)
    used_dw = mx.conv2d_select(d, mx.MX_CONV_DWEIGHT, mx.ALGO_AUTO)
    for name, got, used in (("dx", dx, used_dx), ("dw", dw, used_dw), ("db", db, used_dw)):
        ref, mag = refs[name]
        rtol = WINOGRAD_RTOL if used == mx.ALGO_WINOGRAD else RTOL
        assert_close_mag(got, ref, mag, rtol=rtol, atol=ATOL, what=f"{name} ({case})")


# ------------------------------------------------------------------ GEMM
def _gemm_cases(count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        dims = [int(round(math.exp(rng.uniform(0.0, math.log(700))))) for _ in range(3)]
        batch = int(rng.choice([0, 0, 1, 3, 7]))
        out.append(dict(m=dims[0], n=dims[1], k=dims[2], batch=batch, ta=bool(rng.integers(2)),
                        tb=bool(rng.integers(2)), off=int(rng.integers(0, 5)),
                        bias=str(rng.choice(["none", "col", "matrix"])),
                        alpha=float(rng.choice([1.0, 0.5, -1.25])), beta=float(rng.choice([0.0, 1.0, -0.75]))))
    return out


GEMM_CASES = _gemm_cases(40, seed=12022026)


def _operand(g, batch, rows, cols, transposed, off, device="cpu", flat=None):
    """A rows x cols operand (batched when batch > 0) as a view: transposed
    storage when asked, starting `off` elements into a larger buffer.  Returns
    the view and its buffer; pass the buffer back (moved) for the same view on
    another device."""
    lead = (batch,) if batch else ()
    shape = lead + ((cols, rows) if transposed else (rows, cols))
    if flat is None:
        flat = torch.randn(int(np.prod(shape)) + off, generator=g)
    t = flat.to(device)[off:].view(shape)
    return (t.transpose(-1, -2) if transposed else t), flat


@pytest.mark.parametrize("idx", range(len(GEMM_CASES)), ids=[f"g{i}" for i in range(len(GEMM_CASES))])
def test_random_gemm(mx, idx):
    """mx_gemm_f32 on seeded random shapes (1-700 per dimension, 2-D and
    batched), operand layouts, storage offsets, bias kinds and alpha / beta,
    against float64."""
    c_ = GEMM_CASES[idx]
    g = torch.Generator().manual_seed(500 + idx)
    m, n, k, batch = c_["m"], c_["n"], c_["k"], c_["batch"]
    a, fa = _operand(g, batch, m, k, c_["ta"], c_["off"])
    b, fb = _operand(g, batch, k, n, c_["tb"], c_["off"])
    lead = (batch,) if batch else ()
    bias, kind = None, None
    if c_["bias"] == "col":
        bias, kind = torch.randn(n, generator=g), mx.BIAS_COL
    elif c_["bias"] == "matrix":
        bias, kind = torch.randn(lead + (m, n), generator=g), mx.BIAS_MATRIX
    # The same views (strides, storage offsets) over device copies of the buffers.
    A, _ = _operand(g, batch, m, k, c_["ta"], c_["off"], "cuda", fa)
    B, _ = _operand(g, batch, k, n, c_["tb"], c_["off"], "cuda", fb)
    assert A.stride() == a.stride() and A.storage_offset() == a.storage_offset()
    out = torch.empty(lead + (m, n), device="cuda")
    mx.gemm(A, B, out, bias=bias.to("cuda") if bias is not None else None, alpha=c_["alpha"], beta=c_["beta"],
            bias_kind=kind, stream=_stream())
    ref = c_["alpha"] * (a.double() @ b.double())
    if bias is not None and c_["beta"] != 0.0:
        ref = ref + c_["beta"] * bias.double().expand_as(ref)
    assert_close_mag(out, ref, gemm_mag(a, b, c_["alpha"], c_["beta"], bias), rtol=RTOL, atol=ATOL, what=str(c_))
