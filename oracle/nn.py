"""CPU oracle for the normalisation / activation / resampling / softmax / loss /
concatenation operators of the C3/C4 training steps -- test infrastructure only.

Plain numpy restatements in float64 of what the reference computes for each
operator (its CPU results being the parity target).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use this module,
and only as the checker.

What pins each function (tests/test_oracle_nn.py):
  group_norm_forward / _backward   torch.nn.functional.group_norm and its
                                   autograd on the CPU; per-group mean 0 and
                                   variance 1; central finite differences.
  batch_norm_forward / _backward   torch.nn.functional.batch_norm (training and
                                   evaluation) and its autograd; the running-
                                   statistics update against its closed form.
  silu / silu_backward             x * sigmoid(x) in closed form; finite
                                   differences; torch.nn.functional.silu.
  relu / threshold_backward        torch.relu / autograd, NaN propagation.
  nearest_index, upsample_nearest2d(+_backward)
                                   exact doubling equals np.repeat; every size /
                                   scale case of the reference's test against
                                   torch.nn.functional.interpolate bit for bit;
                                   backward is the adjoint (<up x, g> = <x, up* g>).
  softmax / softmax_backward       rows sum to 1, shift invariance, torch.softmax
                                   and its autograd; finite differences.
  mse_loss / mse_loss_backward     closed forms and torch.nn.functional.mse_loss.
  cat                              np.concatenate.
  lerp / addcmul / addcdiv / add_alpha / maximum / minimum (float32, the
  foreach ops)                     torch.lerp / addcmul / addcdiv / add(alpha) /
                                   maximum / minimum on the CPU, bit for bit
                                   (signed zeros and NaN included).
"""
from __future__ import annotations

import math

import numpy as np


def _rows(x: np.ndarray):
    n, c = x.shape[0], x.shape[1]
    return x.reshape(n, c, -1).astype(np.float64)


# ----------------------------------------------------------------- GroupNorm
def group_norm_forward(x, gamma, beta, groups: int, eps: float):
    """csrc/shaders/group_norm_forward.comp:16-50 (centred two-pass statistics,
    y = (x - mean) * rstd * gamma + beta); mean / rstd are [N, groups]."""
    n, c = x.shape[0], x.shape[1]
    v = _rows(x).reshape(n, groups, -1)
    mean = v.mean(axis=2)
    var = ((v - mean[:, :, None]) ** 2).mean(axis=2)
    rstd = 1.0 / np.sqrt(var + eps)
    z = ((v - mean[:, :, None]) * rstd[:, :, None]).reshape(n, c, -1)
    g = np.ones(c) if gamma is None else np.asarray(gamma, np.float64)
    b = np.zeros(c) if beta is None else np.asarray(beta, np.float64)
    y = z * g[None, :, None] + b[None, :, None]
    return y.reshape(x.shape), mean, rstd


def group_norm_backward(dy, x, mean, rstd, gamma, groups: int):
    """csrc/shaders/group_norm_backward_input.comp:17-46 (dx = rstd * (v -
    mean(v) - z * mean(v z)), v = gamma * dy, z = (x - mean) * rstd) and
    group_norm_backward_affine.comp:12-32 (dgamma = sum dy z, dbeta = sum dy)."""
    n, c = x.shape[0], x.shape[1]
    cpg = c // groups
    xr, gr = _rows(x), _rows(dy)
    mu = np.repeat(np.asarray(mean, np.float64).reshape(n, groups), cpg, axis=1)[:, :, None]
    rs = np.repeat(np.asarray(rstd, np.float64).reshape(n, groups), cpg, axis=1)[:, :, None]
    z = (xr - mu) * rs
    w = np.ones(c) if gamma is None else np.asarray(gamma, np.float64)
    v = gr * w[None, :, None]
    vg, zg = v.reshape(n, groups, -1), z.reshape(n, groups, -1)
    a = vg.mean(axis=2, keepdims=True)
    b = (vg * zg).mean(axis=2, keepdims=True)
    dx = (rs.reshape(n, groups, cpg, 1) * (vg - a - zg * b).reshape(n, groups, cpg, -1)).reshape(x.shape)
    dgamma = (gr * z).sum(axis=(0, 2))
    dbeta = gr.sum(axis=(0, 2))
    return dx, dgamma, dbeta


# ----------------------------------------------------------------- BatchNorm
def batch_norm_forward(x, gamma, beta, running_mean, running_var, training: bool, momentum: float, eps: float):
    """csrc/shaders/batch_norm_forward.comp:17-51: training normalises with the
    batch mean and biased variance over (N, spatial) per channel (invstd 0 when
    var == eps == 0) and updates the running statistics with the unbiased
    variance; evaluation uses the running statistics.  Returns
    (y, save_mean, save_invstd, new_running_mean, new_running_var)."""
    c = x.shape[1]
    xr = _rows(x)
    g = np.ones(c) if gamma is None else np.asarray(gamma, np.float64)
    b = np.zeros(c) if beta is None else np.asarray(beta, np.float64)
    rm = None if running_mean is None else np.asarray(running_mean, np.float64).copy()
    rv = None if running_var is None else np.asarray(running_var, np.float64).copy()
    if training:
        m = xr.mean(axis=(0, 2))
        cnt = xr.shape[0] * xr.shape[2]
        m2 = ((xr - m[None, :, None]) ** 2).sum(axis=(0, 2))
        var = m2 / cnt
        with np.errstate(divide="ignore"):
            inv = np.where((var == 0) & (eps == 0), 0.0, 1.0 / np.sqrt(var + eps))
        if rm is not None:
            rm = momentum * m + (1 - momentum) * rm
        if rv is not None:
            rv = momentum * (m2 / (cnt - 1)) + (1 - momentum) * rv
        save_m, save_i = m, inv
    else:
        m, inv = rm, 1.0 / np.sqrt(rv + eps)
        save_m, save_i = np.zeros(0), np.zeros(0)
    y = (xr - m[None, :, None]) * (inv * g)[None, :, None] + b[None, :, None]
    return y.reshape(x.shape), save_m, save_i, rm, rv


def batch_norm_backward(dy, x, gamma, mean, invstd_or_var, training: bool, eps: float):
    """csrc/shaders/batch_norm_backward.comp:48-78: dbeta = sum dy, dgamma =
    sum dy (x - mean) * invstd, dx = gamma * invstd * (dy - sum(dy)/M -
    (x - mean) * invstd^2 * sum(dy (x - mean))/M) in training, gamma * invstd *
    dy in evaluation (invstd from the running variance)."""
    c = x.shape[1]
    xr, gr = _rows(x), _rows(dy)
    mu = np.asarray(mean, np.float64)
    inv = np.asarray(invstd_or_var, np.float64)
    if not training:
        inv = 1.0 / np.sqrt(inv + eps)
    w = np.ones(c) if gamma is None else np.asarray(gamma, np.float64)
    xc = xr - mu[None, :, None]
    s1 = gr.sum(axis=(0, 2))
    s2 = (gr * xc).sum(axis=(0, 2))
    cnt = xr.shape[0] * xr.shape[2]
    if training:
        dx = (gr - (s1 / cnt)[None, :, None] - xc * (inv * inv * s2 / cnt)[None, :, None]) * (w * inv)[None, :, None]
    else:
        dx = gr * (w * inv)[None, :, None]
    return dx.reshape(x.shape), s2 * inv, s1


# ----------------------------------------------------------------- pointwise
def silu(x):
    """csrc/shaders/diffusion_unary.comp:25-28: x / (1 + exp(-x))."""
    v = np.asarray(x, np.float64)
    return v / (1.0 + np.exp(-v))


def silu_backward(dy, x):
    """csrc/shaders/diffusion_unary_backward.comp:27-31:
    dy * s * (1 + x (1 - s)), s = sigmoid(x)."""
    v = np.asarray(x, np.float64)
    s = 1.0 / (1.0 + np.exp(-v))
    return np.asarray(dy, np.float64) * s * (1.0 + v * (1.0 - s))


def relu(x):
    """csrc/ops/mm.cpp:475-480 (relu.comp): max(x, 0) with NaN kept, as torch."""
    v = np.asarray(x, np.float64)
    return np.where(v <= 0, 0.0, v)


def threshold_backward(dy, x, threshold: float = 0.0):
    """csrc/shaders/threshold_backward.comp:14-18: x <= threshold ? 0 : dy."""
    return np.where(np.asarray(x) <= threshold, 0.0, np.asarray(dy, np.float64))


# ------------------------------------------------------------ nearest resize
def nearest_index(out_size: int, in_size: int, scale=None) -> np.ndarray:
    """Source row / column of each output index: identity for equal sizes, o >> 1
    for exact doubling, else min(floor(float32(o) * float32(s)), in - 1) with
    s = 1/scale or in/out in float32 (csrc/ops/upsample.cpp:8-14,
    csrc/shaders/upsample_nearest2d.comp:6)."""
    o = np.arange(out_size)
    if out_size == in_size:
        return o
    if out_size == 2 * in_size:
        return o >> 1
    s = np.float32(1.0 / scale) if scale is not None and scale > 0 else np.float32(in_size) / np.float32(out_size)
    src = np.floor(o.astype(np.float32) * s).astype(np.int64)
    return np.minimum(src, in_size - 1)


def upsample_nearest2d(x, oh: int, ow: int, scale_h=None, scale_w=None):
    """csrc/shaders/upsample_nearest2d.comp:19-23 (gather)."""
    ih, iw = x.shape[2], x.shape[3]
    hi = nearest_index(oh, ih, scale_h)
    wi = nearest_index(ow, iw, scale_w)
    return np.asarray(x)[:, :, hi][:, :, :, wi]


def upsample_nearest2d_backward(dy, ih: int, iw: int, scale_h=None, scale_w=None):
    """csrc/shaders/upsample_nearest2d.comp:24-33: each input pixel sums the
    output gradients that read it (scatter-add of the gather's indices)."""
    n, c, oh, ow = dy.shape
    hi = nearest_index(oh, ih, scale_h)
    wi = nearest_index(ow, iw, scale_w)
    dx = np.zeros((n, c, ih, iw), np.float64)
    g = np.asarray(dy, np.float64)
    for a in range(oh):
        for b in range(ow):
            dx[:, :, hi[a], wi[b]] += g[:, :, a, b]
    return dx


# ------------------------------------------------------------------- softmax
def softmax(x, dim: int):
    """csrc/shaders/softmax_axis.comp:12-38: exp(x - max) / sum over the axis."""
    v = np.asarray(x, np.float64)
    if v.ndim == 0:
        v = v.reshape(1)
        e = np.exp(v - v.max())
        return (e / e.sum()).reshape(())
    e = np.exp(v - v.max(axis=dim, keepdims=True))
    return e / e.sum(axis=dim, keepdims=True)


def softmax_backward(dy, y, dim: int):
    """csrc/ops/softmax_axis_backward.cpp:11-38 (softmax_axis_backward.comp):
    dx = y * (dy - sum(dy * y))."""
    g, p = np.asarray(dy, np.float64), np.asarray(y, np.float64)
    if p.ndim == 0:
        return p * (g - g * p)
    return p * (g - (g * p).sum(axis=dim, keepdims=True))


# ------------------------------------------------------------------ MSE loss
def mse_loss(x, t, reduction: str = "mean"):
    """csrc/ops/loss_primitives.cpp:349-352: (x - t)^2, then mean / sum / none."""
    d = (np.asarray(x, np.float64) - np.asarray(t, np.float64)) ** 2
    if reduction == "none":
        return d
    if reduction == "sum":
        return d.sum()
    return d.mean() if d.size else math.nan


def mse_loss_backward(dy, x, t, reduction: str = "mean"):
    """csrc/ops/loss_primitives.cpp:353-356: (x - t) * (2/n for mean else 2) * dy."""
    d = np.asarray(x, np.float64) - np.asarray(t, np.float64)
    norm = 2.0 / d.size if reduction == "mean" else 2.0
    return d * norm * np.asarray(dy, np.float64)


# ----------------------------------------------------------------------- cat
def cat(xs, dim: int):
    """csrc/ops/cat.cpp:8-58: concatenation, 1-D empty inputs skipped."""
    keep = [np.asarray(v) for v in xs if not (np.asarray(v).ndim == 1 and np.asarray(v).size == 0)]
    return np.concatenate(keep, axis=dim)


# ------------------------------------------------------------- foreach ops
def _f32(x):
    return np.asarray(x, np.float32).astype(np.float64)


def fma32(a, b, c):
    """float32 fused multiply-add: the exact a*b + c rounded once to nearest
    even.  float64 holds the product of two float32 exactly; the float64 sum s
    is one rounding away from the exact value s + e (e recovered exactly by
    Knuth's TwoSum), and rounding s to float32 gives the correctly rounded
    result except when s lands exactly on a float32 midpoint with e != 0: then
    the neighbour on e's side is the answer."""
    p, c64 = _f32(a) * _f32(b), _f32(c)
    with np.errstate(invalid="ignore", over="ignore"):
        s = p + c64
        bv = s - p
        e = (p - (s - bv)) + (c64 - bv)
        f = s.astype(np.float32)
        g = np.where(s > f, np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf)))
        tie = np.isfinite(s) & (f.astype(np.float64) != s) & \
            ((f.astype(np.float64) + g.astype(np.float64)) * 0.5 == s) & (e != 0) & np.isfinite(e)
        up = np.maximum(f, g)
        dn = np.minimum(f, g)
        return np.where(tie, np.where(e > 0, up, dn), f).astype(np.float32)


def lerp(a, b, w):
    """torch's vectorised CPU lerp (ATen/native/Lerp.h, cpu/LerpKernel.cpp):
    |w| < 0.5 ? fma(w, b - a, a) : fma(w - 1, b - a, b), in float32.
    The reference's optimizer_pointwise op 0/1 (csrc/ops/optimizer_primitives.cpp:50-51)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    w = np.broadcast_to(np.asarray(w, np.float32), a.shape)
    d = (b - a).astype(np.float32)
    return np.where(np.abs(w) < 0.5, fma32(w, d, a), fma32((w - np.float32(1)).astype(np.float32), d, b))


def addcmul(a, t1, t2, v):
    """fma(v * t1, t2, a) in float32: torch's CPU addcmul (one fused
    multiply-add after the scalar product; csrc/ops/optimizer_primitives.cpp:52)."""
    v = np.float32(v)
    return fma32((v * np.asarray(t1, np.float32)).astype(np.float32), t2, a)


def add_alpha(a, b, alpha):
    """fma(b, alpha, a) in float32: torch's CPU add with alpha."""
    return fma32(b, np.float32(alpha), a)


def addcdiv(a, t1, t2, v):
    """a + (v * t1) / t2 in float32 (csrc/ops/optimizer_primitives.cpp:53)."""
    v = np.float32(v)
    return (np.asarray(a, np.float32) + (v * np.asarray(t1, np.float32)) / np.asarray(t2, np.float32)).astype(np.float32)


def maximum(a, b):
    """NaN-propagating maximum as torch's vectorised CPU kernel (max_ps: the
    second operand unless the first is greater, so max(-0, +0) = +0)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.where(np.isnan(a) | np.isnan(b), np.float32(np.nan), np.where(a > b, a, b))


def minimum(a, b):
    """NaN-propagating minimum (min_ps: the second operand unless the first is smaller)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.where(np.isnan(a) | np.isnan(b), np.float32(np.nan), np.where(a < b, a, b))
