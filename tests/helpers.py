"""Tolerance model shared by the parity tests.

A contraction output c = sum_k a_k b_k can cancel to a value far below its
terms, and FP32 accumulation error scales with sum_k |a_k b_k| (the
"magnitude"), not with |c|.  The north-star bound "rel 1e-4 / abs 1e-5" is
therefore applied as

    |actual - ref64| <= 1e-4 * |ref64| + 1e-5 * max(1, magnitude)

where ref64 is the float64 result on the same inputs and magnitude is the
same operation applied to the absolute values of its inputs.  The CPU FP32
implementation itself satisfies this bound (checked in test_oracle_*), a
single dropped or misplaced term violates it for every reduction length used
here (an element's error would be ~magnitude/K >> 1e-5 * magnitude for
K < 1e5), and elementwise ops (AdamW) have magnitude ~ |value| so the bound is
the plain rel/abs one.
"""
from __future__ import annotations

import torch

RTOL = 1e-4
ATOL = 1e-5
WINOGRAD_RTOL = 1e-3


def assert_close_mag(actual, ref64, mag64=None, rtol=RTOL, atol=ATOL, what=""):
    a = actual.detach().cpu().double()
    r = ref64.detach().cpu().double()
    assert a.shape == r.shape, f"{what}: shape {tuple(a.shape)} != {tuple(r.shape)}"
    if mag64 is None:
        mag = torch.ones_like(r)
    else:
        mag = mag64.detach().cpu().double().clamp_min(1.0)
    err = (a - r).abs()
    bound = rtol * r.abs() + atol * mag
    bad = ~(err <= bound)  # NaN-safe: NaN errors count as failures
    if bad.any():
        idx = int(torch.nonzero(bad.flatten())[0])
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.numel()} elements outside |err| <= {rtol}*|ref| + {atol}*mag; "
            f"first at flat index {idx}: actual={a.flatten()[idx].item():.9g} ref={r.flatten()[idx].item():.9g} "
            f"mag={mag.flatten()[idx].item():.6g}; max err/bound={float((err / bound).max()):.3g}")


def gemm_mag(a, b, alpha=1.0, beta=0.0, bias=None):
    m = abs(alpha) * (a.double().abs() @ b.double().abs())
    if bias is not None and beta != 0.0:
        m = m + abs(beta) * bias.double().abs().expand_as(m)
    return m


def conv_refs(x, w, b, dy, stride, padding, dilation, groups):
    """float64 results and magnitudes of forward, dX, dW, dB."""
    F = torch.nn.functional
    xd, wd = x.double().requires_grad_(), w.double().requires_grad_()
    bd = b.double().requires_grad_() if b is not None else None
    y = F.conv2d(xd, wd, bd, stride, padding, dilation, groups)
    grads = torch.autograd.grad(y, [t for t in (xd, wd, bd) if t is not None], dy.double())
    xa, wa = x.double().abs().requires_grad_(), w.double().abs().requires_grad_()
    ya = F.conv2d(xa, wa, b.double().abs() if b is not None else None, stride, padding, dilation, groups)
    gxa, gwa = torch.autograd.grad(ya, (xa, wa), dy.double().abs())
    out = {"y": (y.detach(), ya.detach()), "dx": (grads[0], gxa), "dw": (grads[1], gwa)}
    if b is not None:
        out["db"] = (grads[2], dy.double().abs().sum((0, 2, 3)))
    return out
