"""The north star's literal elementwise bound beside CPU FP32's own.

The parity tests apply "rel 1e-4 / abs 1e-5" with the magnitude model of
tests/helpers.py (the absolute term scaled by the summed |terms| of each
output), because a plain elementwise bound fails CPU FP32 itself on outputs
that cancel.  This file measures that claim: for the C1 layer, a sample of C3
layers (batch 2) and rows of the C2 GEMMs at full size, it reports the
fraction of outputs within the plain bound |got - ref64| <= 1e-4 |ref64| +
1e-5 for CPU FP32 torch and for this library's GPU kernels, both against
float64 on the same inputs, and the fraction within the magnitude model.

Asserted: every output is within the magnitude model (rel 1e-3 for
Winograd, except on C1's reported route, which is held to rel 1e-4 / abs 1e-5
and to CPU FP32's plain-bound rate).  On the convolutions the GPU misses the plain bound no more often
than twice as often as CPU FP32 does, plus 0.1% of the outputs (measured:
at most as often).  The C2 GEMMs accumulate each output sequentially over K
in the MFMA accumulators, where CPU torch sums in blocks: at K = 8192 (dW)
the GPU misses the plain bound on about 0.5% of the outputs against CPU
FP32's 0.1%, so there the check is that at least 99% meet it.  The rates are
written to gpurun_out/tolerance_report.json when that folder exists.
"""
from __future__ import annotations

import json
import os

import pytest
import torch
import torch.nn.functional as F

from helpers import ATOL, RTOL, WINOGRAD_RTOL

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REPORT = {}


@pytest.fixture(scope="module")
def mx():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from torch_vulkan import mx as m
    m.lib()
    return m


def rates(got, ref64, mag64, rtol):
    got, ref, mag = (t.detach().cpu().double() for t in (got, ref64, mag64))
    err = (got - ref).abs()
    plain = (err <= RTOL * ref.abs() + ATOL).double().mean().item()
    model = (err <= rtol * ref.abs() + ATOL * mag.clamp_min(1.0)).double().mean().item()
    return plain, model


def record(case, phase, rtol, gpu, cpu, ref, mag, min_plain=None):
    gp, gm = rates(gpu, ref, mag, rtol)
    cp, cm = rates(cpu, ref, mag, RTOL)
    REPORT.setdefault(case, {})[phase] = {"outputs": ref.numel(), "gpu_plain": round(gp, 6),
                                          "cpu_fp32_plain": round(cp, 6), "gpu_model": round(gm, 6),
                                          "cpu_fp32_model": round(cm, 6), "gpu_rtol": rtol}
    dump()
    assert gm == 1.0, (case, phase, REPORT[case][phase])
    if min_plain is not None:
        assert gp >= min_plain, (case, phase, REPORT[case][phase])
    elif rtol == RTOL:
        assert 1 - gp <= 2 * (1 - cp) + 1e-3, (case, phase, REPORT[case][phase])


CONV_CASES = [
    # name, x shape, cout, k, stride, pad
    ("C1 8x64x56x56 3x3", (8, 64, 56, 56), 64, 3, 1, 1),
    ("C3 stem 7x7/2 (batch 2)", (2, 3, 224, 224), 64, 7, 2, 3),
    ("C3 layer1.0.conv1 1x1 (batch 2)", (2, 64, 56, 56), 64, 1, 1, 0),
    ("C3 layer2.0.conv2 3x3/2 (batch 2)", (2, 128, 56, 56), 128, 3, 2, 1),
    ("C3 layer3.1.conv2 3x3 (batch 2)", (2, 256, 14, 14), 256, 3, 1, 1),
    ("C3 layer4.0.conv3 1x1 (batch 2)", (2, 512, 7, 7), 2048, 1, 1, 0),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_conv_plain_bound_beside_cpu(mx, case):
    name, xs, cout, k, s, p = case
    g = torch.Generator().manual_seed(sum(xs) + cout)
    x = torch.randn(xs, generator=g)
    w = torch.randn(cout, xs[1], k, k, generator=g) / (xs[1] * k * k) ** 0.5
    b = torch.randn(cout, generator=g) * 0.1
    y_cpu = F.conv2d(x, w, b, s, p)
    dy = torch.randn(y_cpu.shape, generator=g)
    # float64 references and magnitudes.
    xd, wd, bd = (t.double().requires_grad_() for t in (x, w, b))
    yd = F.conv2d(xd, wd, bd, s, p)
    gxd, gwd, gbd = torch.autograd.grad(yd, (xd, wd, bd), dy.double())
    xa, wa = x.double().abs().requires_grad_(), w.double().abs().requires_grad_()
    ya = F.conv2d(xa, wa, b.double().abs(), s, p)
    mxa, mwa = torch.autograd.grad(ya, (xa, wa), dy.double().abs())
    # CPU FP32.
    xc, wc, bc = (t.clone().requires_grad_() for t in (x, w, b))
    gxc, gwc, gbc = torch.autograd.grad(F.conv2d(xc, wc, bc, s, p), (xc, wc, bc), dy)
    # GPU through the C ABI.
    d = mx.conv_desc(xs, w.shape, (s, s), (p, p))
    X, W, B, DY = (t.cuda() for t in (x, w, b, dy))
    st = torch.cuda.current_stream().cuda_stream
    algos = [("implicit_gemm", mx.ALGO_IMPLICIT_GEMM, RTOL)]
    if k == 3 and s == 1:
        algos.append(("winograd", mx.ALGO_WINOGRAD, WINOGRAD_RTOL))
    for label, algo, rtol in algos:
        Y, DX = torch.empty(y_cpu.shape, device="cuda"), torch.empty_like(X)
        mx.conv2d_forward(d, X, W, B, Y, algo, st)
        mx.conv2d_backward_input(d, DY, W, DX, algo, st)
        torch.cuda.synchronize()
        record(name, f"forward ({label})", rtol, Y, y_cpu, yd, ya)
        record(name, f"dInput ({label})", rtol, DX, gxc, gxd, mxa)
    DW, DB = torch.empty_like(W), torch.empty_like(B)
    mx.conv2d_backward_weight(d, X, DY, DW, DB, mx.ALGO_IMPLICIT_GEMM, st)
    torch.cuda.synchronize()
    record(name, "dWeight (implicit_gemm)", RTOL, DW, gwc, gwd, mwa)
    record(name, "dBias", RTOL, DB, gbc, gbd, dy.double().abs().sum((0, 2, 3)))
    if k == 3 and s == 1:
        # The Winograd weight gradient with its fused dBias (C1's and C3's route).
        DW, DB = torch.empty_like(W), torch.empty_like(B)
        mx.conv2d_backward_weight(d, X, DY, DW, DB, mx.ALGO_WINOGRAD, st)
        torch.cuda.synchronize()
        record(name, "dWeight (winograd)", WINOGRAD_RTOL, DW, gwc, gwd, mwa)
        record(name, "dBias (winograd dWeight launch)", RTOL, DB, gbc, gbd, dy.double().abs().sum((0, 2, 3)))


def test_c1_winograd_route_meets_the_direct_bar(mx):
    """C1 as bench.py reports it, on BASELINE's seeded inputs (seed 0: x and dy
    ~ N(0,1), Kaiming-uniform(a=sqrt 5) weights, bias ~ U(-1/24, 1/24)):
    every phase on Winograd F(2x2,3x3), the backward as one mx_conv2d_backward
    call (one launch for dx, dw and db).  Asserted at C1's stated tolerance,
    rel 1e-4 / abs 1e-5, not the rel 1e-3 Winograd allowance: every output of
    the forward, dInput, dWeight and dBias within the magnitude model, and the
    plain elementwise bound met at least as often as CPU FP32 meets it (the
    reference's own convolution-gradient check, tests/test_conv_dispatch.py:
    57-70, compares against float64 the same way)."""
    g = torch.Generator().manual_seed(0)
    xs, cout = (8, 64, 56, 56), 64
    x = torch.randn(xs, generator=g)
    w = torch.empty(cout, 64, 3, 3)
    torch.nn.init.kaiming_uniform_(w, a=5 ** 0.5, generator=g)
    b = torch.empty(cout).uniform_(-1 / 24, 1 / 24, generator=g)
    dy = torch.randn(8, cout, 56, 56, generator=g)
    xd, wd, bd = (t.double().requires_grad_() for t in (x, w, b))
    yd = F.conv2d(xd, wd, bd, 1, 1)
    gxd, gwd, gbd = torch.autograd.grad(yd, (xd, wd, bd), dy.double())
    xa, wa = x.double().abs().requires_grad_(), w.double().abs().requires_grad_()
    ya = F.conv2d(xa, wa, b.double().abs(), 1, 1)
    mxa, mwa = torch.autograd.grad(ya, (xa, wa), dy.double().abs())
    xc, wc, bc = (t.clone().requires_grad_() for t in (x, w, b))
    yc = F.conv2d(xc, wc, bc, 1, 1)
    gxc, gwc, gbc = torch.autograd.grad(yc, (xc, wc, bc), dy)
    d = mx.conv_desc(xs, w.shape, (1, 1), (1, 1))
    assert mx.conv2d_backward_one_launch(d, mx.ALGO_WINOGRAD, mx.ALGO_WINOGRAD)
    X, W, B, DY = (t.cuda() for t in (x, w, b, dy))
    Y, DX, DW, DB = (torch.full(t.shape, float("nan"), device="cuda") for t in (dy, x, w, b))
    st = torch.cuda.current_stream().cuda_stream
    mx.conv2d_forward(d, X, W, B, Y, mx.ALGO_WINOGRAD, st)
    mx.conv2d_backward(d, X, W, DY, DX, DW, DB, mx.ALGO_WINOGRAD, mx.ALGO_WINOGRAD, st)
    torch.cuda.synchronize()
    name = "C1 routed (Winograd, one-launch backward) at rel 1e-4 / abs 1e-5"
    for phase, gpu, cpu, ref, mag in (("forward", Y, yc, yd, ya), ("dInput", DX, gxc, gxd, mxa),
                                      ("dWeight", DW, gwc, gwd, mwa),
                                      ("dBias", DB, gbc, gbd, dy.double().abs().sum((0, 2, 3)))):
        gp, gm = rates(gpu, ref, mag, RTOL)
        cp, _ = rates(cpu, ref, mag, RTOL)
        REPORT.setdefault(name, {})[phase] = {"outputs": ref.numel(), "gpu_plain": round(gp, 6),
                                              "cpu_fp32_plain": round(cp, 6), "gpu_model": round(gm, 6),
                                              "gpu_rtol": RTOL}
        dump()
        assert gm == 1.0, (phase, REPORT[name][phase])
        assert gp >= cp, (phase, REPORT[name][phase])


def test_c2_rows_plain_bound_beside_cpu(mx):
    """C2 at full size: Y = X W^T + b, dX = dY W, dW = dY^T X; 32 rows (of Y,
    dX) and 32 rows of dW against float64 on the host."""
    M, K, N = 8192, 4096, 4096
    g = torch.Generator().manual_seed(7)
    X = torch.randn(M, K, generator=g)
    Wt = (torch.rand(N, K, generator=g) * 2 - 1) / 64
    bias = (torch.rand(N, generator=g) * 2 - 1) / 64
    dY = torch.randn(M, N, generator=g)
    rows = torch.randperm(M, generator=g)[:32]
    wrows = torch.randperm(N, generator=g)[:32]
    Xg, Wg, bg, dYg = (t.cuda() for t in (X, Wt, bias, dY))
    Y = torch.empty(M, N, device="cuda")
    dX = torch.empty(M, K, device="cuda")
    dW = torch.empty(N, K, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    mx.gemm(Xg, Wg.t(), Y, bias=bg, beta=1.0, stream=st)
    mx.gemm(dYg, Wg, dX, stream=st)
    mx.gemm(dYg.t(), Xg, dW, stream=st)
    torch.cuda.synchronize()
    Xr, dYr = X[rows], dY[rows]
    cases = [
        ("forward X.W^T+b", Y.cpu()[rows], Xr @ Wt.t() + bias, Xr.double() @ Wt.double().t() + bias.double(),
         Xr.double().abs() @ Wt.double().abs().t() + bias.double().abs()),
        ("dX = dY.W", dX.cpu()[rows], dYr @ Wt, dYr.double() @ Wt.double(), dYr.double().abs() @ Wt.double().abs()),
        ("dW = dY^T.X", dW.cpu()[wrows], dY[:, wrows].t() @ X, dY[:, wrows].double().t() @ X.double(),
         dY[:, wrows].double().abs().t() @ X.double().abs()),
    ]
    for phase, gpu, cpu, ref, mag in cases:
        record("C2 Linear 8192x4096x4096 (32 rows)", phase, RTOL, gpu, cpu, ref, mag, min_plain=0.99)


def dump():
    out = os.path.join(REPO, "gpurun_out")
    if os.path.isdir(out):
        with open(os.path.join(out, "tolerance_report.json"), "w") as f:
            json.dump(REPORT, f, indent=1)
