"""Pins oracle/nn.py (CPU, no GPU): every restated operator against torch's
CPU implementation (the parity target of the reference's kernels for these
ops), against invariants the mathematics fixes (normalised groups have mean 0
and variance 1, softmax rows sum to 1 and ignore shifts, nearest doubling is
np.repeat, the upsample backward is the forward's adjoint) and against central
finite differences for the backward passes, so that a dropped term, a wrong
sign or a transposed index fails at least one check."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import nn as O


def t64(a):
    return torch.as_tensor(np.asarray(a, np.float64))


def fd_grad(f, x, g, h=1e-6):
    """<g, df/dx> by central differences, one coordinate at a time (tiny x)."""
    out = np.zeros_like(x)
    flat = x.reshape(-1)
    for i in range(flat.size):
        old = flat[i]
        flat[i] = old + h
        fp = np.sum(f(x) * g)
        flat[i] = old - h
        fm = np.sum(f(x) * g)
        flat[i] = old
        out.reshape(-1)[i] = (fp - fm) / (2 * h)
    return out


# ---------------------------------------------------------------- GroupNorm
@pytest.mark.parametrize("shape,groups", [((2, 8, 4, 5), 4), ((1, 8, 8, 8), 1), ((1, 12, 3, 7), 3),
                                          ((2, 16, 8), 8), ((2, 8, 2, 3, 4), 2), ((2, 4, 1, 1), 2)])
@pytest.mark.parametrize("affine", [False, True])
def test_group_norm_matches_torch(shape, groups, affine):
    rng = np.random.default_rng(sum(shape) + groups)
    x = rng.standard_normal(shape)
    c = shape[1]
    w = rng.standard_normal(c) if affine else None
    b = rng.standard_normal(c) if affine else None
    y, mean, rstd = O.group_norm_forward(x, w, b, groups, 1e-5)
    xt = t64(x).requires_grad_()
    wt = t64(w).requires_grad_() if affine else None
    bt = t64(b).requires_grad_() if affine else None
    yt = F.group_norm(xt, groups, wt, bt, 1e-5)
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=1e-12, atol=1e-12)
    _, m_t, r_t = torch.ops.aten.native_group_norm(t64(x), wt.detach() if affine else None,
                                                   bt.detach() if affine else None, shape[0], c,
                                                   int(np.prod(shape[2:])), groups, 1e-5)
    np.testing.assert_allclose(mean, m_t.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(rstd, r_t.numpy(), rtol=1e-10)
    g = rng.standard_normal(shape)
    grads = torch.autograd.grad(yt, [v for v in (xt, wt, bt) if v is not None], t64(g))
    dx, dw, db = O.group_norm_backward(g, x, mean, rstd, w, groups)
    np.testing.assert_allclose(dx, grads[0].numpy(), rtol=1e-9, atol=1e-11)
    if affine:
        np.testing.assert_allclose(dw, grads[1].numpy(), rtol=1e-9, atol=1e-11)
        np.testing.assert_allclose(db, grads[2].numpy(), rtol=1e-9, atol=1e-11)


def test_group_norm_invariants_and_finite_differences():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 6, 3, 3)) * 3 + 7
    y, _, _ = O.group_norm_forward(x, None, None, 3, 0.0)
    yg = y.reshape(2, 3, -1)
    np.testing.assert_allclose(yg.mean(axis=2), 0, atol=1e-12)
    np.testing.assert_allclose(yg.var(axis=2), 1, rtol=1e-10)
    w = rng.standard_normal(6)
    g = rng.standard_normal(x.shape)
    _, mean, rstd = O.group_norm_forward(x, w, None, 3, 1e-3)
    dx, _, _ = O.group_norm_backward(g, x, mean, rstd, w, 3)
    fd = fd_grad(lambda v: O.group_norm_forward(v, w, None, 3, 1e-3)[0], x.copy(), g)
    np.testing.assert_allclose(dx, fd, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- BatchNorm
@pytest.mark.parametrize("shape", [(4, 3, 5, 6), (8, 5), (2, 4, 3, 2, 2)])
@pytest.mark.parametrize("training", [True, False])
def test_batch_norm_matches_torch(shape, training):
    rng = np.random.default_rng(len(shape) * 10 + training)
    c = shape[1]
    x = rng.standard_normal(shape) * 2 + 0.5
    w, b = rng.standard_normal(c), rng.standard_normal(c)
    rm, rv = rng.standard_normal(c), rng.random(c) + 0.5
    y, sm, si, nrm, nrv = O.batch_norm_forward(x, w, b, rm, rv, training, 0.1, 1e-5)
    rmt, rvt = t64(rm), t64(rv)
    xt, wt, bt = t64(x).requires_grad_(), t64(w).requires_grad_(), t64(b).requires_grad_()
    yt = F.batch_norm(xt, rmt, rvt, wt, bt, training=training, momentum=0.1, eps=1e-5)
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(nrm, rmt.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(nrv, rvt.numpy(), rtol=1e-12, atol=1e-14)
    g = rng.standard_normal(shape)
    gx, gw, gb = torch.autograd.grad(yt, (xt, wt, bt), t64(g))
    mean, iv = (sm, si) if training else (rm, rv)
    dx, dw, db = O.batch_norm_backward(g, x, w, mean, iv, training, 1e-5)
    np.testing.assert_allclose(dx, gx.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dw, gw.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(db, gb.numpy(), rtol=1e-9, atol=1e-11)


def test_batch_norm_running_update_closed_form_and_zero_variance():
    x = np.full((2, 1, 2, 2), 3.0)
    y, sm, si, rm, rv = O.batch_norm_forward(x, None, None, np.array([1.0]), np.array([2.0]), True, 0.25, 0.0)
    assert si[0] == 0.0 and np.all(y == 0)  # var == eps == 0 -> invstd 0
    assert rm[0] == 0.25 * 3.0 + 0.75 * 1.0 and rv[0] == 0.75 * 2.0


# ---------------------------------------------------------------- pointwise
def test_silu_closed_form_torch_and_derivative():
    x = np.linspace(-20, 20, 101)
    np.testing.assert_allclose(O.silu(x), x * (1 / (1 + np.exp(-x))), rtol=1e-14, atol=1e-300)
    np.testing.assert_allclose(O.silu(x), F.silu(t64(x)).numpy(), rtol=1e-13, atol=1e-300)
    g = np.cos(x)
    fd = fd_grad(O.silu, x.copy(), g)
    np.testing.assert_allclose(O.silu_backward(g, x), fd, rtol=1e-6, atol=1e-8)
    xt = t64(x).requires_grad_()
    (gt,) = torch.autograd.grad(F.silu(xt), xt, t64(g))
    np.testing.assert_allclose(O.silu_backward(g, x), gt.numpy(), rtol=1e-12, atol=1e-14)


def test_relu_and_threshold_backward_keep_torch_semantics():
    x = np.array([-1.0, 0.0, 2.0, np.nan, -0.0])
    np.testing.assert_array_equal(O.relu(x), torch.relu(t64(x)).numpy())
    g = np.array([1.0, 2.0, 3.0, 4.0, 5.0])
    np.testing.assert_array_equal(O.threshold_backward(g, x, 0.0),
                                  torch.ops.aten.threshold_backward(t64(g), t64(x), 0.0).numpy())


# ----------------------------------------------------------- nearest resize
NEAREST_CASES = [((2, 3, 5, 7), (10, 14), None), ((1, 7, 3, 5), (7, 13), None), ((2, 3, 9, 11), (4, 3), None),
                 ((1, 2, 1, 7), (3, 1), None), ((1, 2, 7, 9), (7, 9), None), ((2, 3, 5, 7), None, (1.7, 2.3)),
                 ((2, 3, 13, 11), None, (.6, .7)), ((2, 3, 7, 9), None, (1.001, 1.5)), ((1, 2, 4, 4), None, (2.0, 2.0))]


@pytest.mark.parametrize("shape,size,scales", NEAREST_CASES)
def test_nearest_matches_torch_exactly(shape, size, scales):
    rng = np.random.default_rng(45)
    x = rng.standard_normal(shape).astype(np.float32)
    xt = torch.from_numpy(x).requires_grad_()
    yt = F.interpolate(xt, size=size, scale_factor=scales, mode="nearest")
    oh, ow = yt.shape[2], yt.shape[3]
    sh, sw = scales if scales else (None, None)
    y = O.upsample_nearest2d(x, oh, ow, sh, sw)
    np.testing.assert_array_equal(y, yt.detach().numpy())
    g = rng.standard_normal(yt.shape).astype(np.float32)
    (gx,) = torch.autograd.grad(yt, xt, torch.from_numpy(g))
    dx = O.upsample_nearest2d_backward(g, shape[2], shape[3], sh, sw)
    np.testing.assert_allclose(dx, gx.numpy(), rtol=1e-6, atol=1e-6)
    # adjoint identity <up x, g> == <x, up* g>
    np.testing.assert_allclose(np.sum(y.astype(np.float64) * g), np.sum(x.astype(np.float64) * dx), rtol=1e-12)


def test_nearest_doubling_is_repeat():
    x = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)
    np.testing.assert_array_equal(O.upsample_nearest2d(x, 8, 10), x.repeat(2, axis=2).repeat(2, axis=3))


# ------------------------------------------------------------------ softmax
@pytest.mark.parametrize("shape,dim", [((2, 3, 5), 0), ((2, 3, 5), 1), ((2, 3, 5), 2), ((2, 4, 3, 7), -3),
                                       ((3, 13, 2), 1), ((1, 7, 32), -1), ((1,), 0)])
def test_softmax_matches_torch(shape, dim):
    rng = np.random.default_rng(62)
    x = rng.standard_normal(shape) * 4
    y = O.softmax(x, dim)
    np.testing.assert_allclose(y.sum(axis=dim), 1.0, rtol=1e-14)
    np.testing.assert_allclose(O.softmax(x + 100.0, dim), y, rtol=1e-12)
    xt = t64(x).requires_grad_()
    yt = torch.softmax(xt, dim)
    np.testing.assert_allclose(y, yt.detach().numpy(), rtol=1e-13, atol=1e-300)
    g = rng.standard_normal(shape)
    (gx,) = torch.autograd.grad(yt, xt, t64(g))
    np.testing.assert_allclose(O.softmax_backward(g, y, dim), gx.numpy(), rtol=1e-11, atol=1e-14)


def test_softmax_backward_finite_differences():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 4))
    g = rng.standard_normal((3, 4))
    fd = fd_grad(lambda v: O.softmax(v, 1), x.copy(), g)
    np.testing.assert_allclose(O.softmax_backward(g, O.softmax(x, 1), 1), fd, rtol=1e-6, atol=1e-9)


# ----------------------------------------------------------- MSE and cat
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_mse_loss_closed_form_and_torch(reduction):
    rng = np.random.default_rng(9)
    x, t = rng.standard_normal((4, 5)), rng.standard_normal((4, 5))
    xt = t64(x).requires_grad_()
    lt = F.mse_loss(xt, t64(t), reduction=reduction)
    np.testing.assert_allclose(O.mse_loss(x, t, reduction), lt.detach().numpy(), rtol=1e-14)
    g = rng.standard_normal(lt.shape) if reduction == "none" else np.float64(1.7)
    (gx,) = torch.autograd.grad(lt, xt, t64(g))
    np.testing.assert_allclose(O.mse_loss_backward(g, x, t, reduction), gx.numpy(), rtol=1e-14)
    assert O.mse_loss(x, x, reduction).sum() == 0


def test_cat_matches_concatenate_and_skips_legacy_empty():
    a, b = np.ones((2, 3, 4)), np.zeros((2, 5, 4))
    np.testing.assert_array_equal(O.cat([a, np.zeros(0), b], 1), np.concatenate([a, b], 1))
    np.testing.assert_array_equal(O.cat([a, a], -1), torch.cat([t64(a), t64(a)], -1).numpy())


# ------------------------------------------------------------- foreach ops
def _ulp_close(a, b, ulps=0):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    diff = np.abs(a.astype(np.float64) - b.astype(np.float64))
    tol = ulps * np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float32)).astype(np.float64)
    assert np.all(both_nan | (diff <= tol)), float(np.max(np.where(both_nan, 0, diff - tol)))


@pytest.mark.parametrize("w", [0.1, 0.49, 0.5, 0.9, -0.3, 1.7])
def test_lerp_matches_torch_cpu(w):
    rng = np.random.default_rng(31)
    a, b = (rng.standard_normal(1000) * 3).astype(np.float32), rng.standard_normal(1000).astype(np.float32)
    _ulp_close(O.lerp(a, b, w), torch.lerp(torch.from_numpy(a), torch.from_numpy(b), w).numpy())
    wt = rng.uniform(-1, 2, 1000).astype(np.float32)
    _ulp_close(O.lerp(a, b, wt), torch.lerp(torch.from_numpy(a), torch.from_numpy(b), torch.from_numpy(wt)).numpy())
    assert np.array_equal(O.lerp(a, b, 0.0), a) and np.array_equal(O.lerp(a, b, 1.0), b)


def test_addcmul_addcdiv_extrema_match_torch_cpu():
    rng = np.random.default_rng(32)
    a, t1, t2 = (rng.standard_normal((3, 1000)) * 2).astype(np.float32)
    t2 = np.abs(t2) + np.float32(0.1)
    A, T1, T2 = map(torch.from_numpy, (a, t1, t2))
    _ulp_close(O.addcmul(a, t1, t2, -0.37), torch.addcmul(A, T1, T2, value=-0.37).numpy())
    _ulp_close(O.addcdiv(a, t1, t2, 1.9), torch.addcdiv(A, T1, T2, value=1.9).numpy())
    _ulp_close(O.add_alpha(a, t1, -0.71), torch.add(A, T1, alpha=-0.71).numpy())
    # 64 elements so torch takes its vectorised path throughout
    x = np.resize(np.array([1.0, np.nan, -0.0, 0.0, 3.0, -2.0, 0.5, 7.0], np.float32), 64)
    y = np.resize(np.array([2.0, 1.0, 0.0, -0.0, np.nan, -5.0, 0.5, -7.0], np.float32), 64)
    for f, t in ((O.maximum, torch.maximum), (O.minimum, torch.minimum)):
        got, want = f(x, y), t(torch.from_numpy(x), torch.from_numpy(y)).numpy()
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert np.array_equal(got[~np.isnan(got)], want[~np.isnan(want)])
        assert np.array_equal(np.signbit(got[~np.isnan(got)]), np.signbit(want[~np.isnan(want)]))


# ---------------------------------------------------------------- fma32 exactness and planted mistakes
def _round_f32_exact(v):
    """Correctly rounded float32 (nearest, ties to even) of an exact rational."""
    from fractions import Fraction
    f0 = np.float32(float(v))
    cands = [f0, np.nextafter(f0, np.float32(np.inf)), np.nextafter(f0, np.float32(-np.inf))]
    best = min(cands, key=lambda f: (abs(Fraction(float(f)) - v), int(np.float32(f).view(np.int32)) & 1))
    return np.float32(best)


def _fma_exact(a, b, c):
    from fractions import Fraction
    return np.array([_round_f32_exact(Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z)))
                     for x, y, z in zip(a, b, c)], np.float32)


# a*b lies 2^-70 below the float32 midpoint 1 + 2^-23 + 2^-24: one float64
# rounding lands on the midpoint, and ties-to-even would then round up.
TIE = (np.float32(1 + 2 ** -23), np.float32(2 ** -24 - 2 ** -47), np.float32(1 + 2 ** -23))


def test_fma32_is_correctly_rounded():
    rng = np.random.default_rng(41)
    a = (rng.standard_normal(3000) * 2).astype(np.float32)
    b = (rng.standard_normal(3000) * 2).astype(np.float32)
    c = (rng.standard_normal(3000) * 4).astype(np.float32)
    a, b, c = (np.append(x, t) for x, t in zip((a, b, c), TIE))
    assert np.array_equal(O.fma32(a, b, c), _fma_exact(a, b, c))
    assert O.fma32(*TIE) == np.float32(1 + 2 ** -23)


def test_planted_mistakes_are_caught():
    """Each planted variant of an oracle function fails a check above."""
    # fma by one float64 sum then a float32 cast (double rounding): the tie vector
    naive = lambda x, y, z: (_f64(x) * _f64(y) + _f64(z)).astype(np.float32)  # noqa: E731
    assert naive(*TIE) != _fma_exact(*[np.array([t]) for t in TIE])[0]
    rng = np.random.default_rng(43)
    a, t1, t2 = (rng.standard_normal((3, 4096)) * 2).astype(np.float32)
    A, T1, T2 = map(torch.from_numpy, (a, t1, t2))
    # addcmul as two roundings (v*t1*t2 + a)
    two = ((np.float32(-0.37) * t1 * t2).astype(np.float32) + a).astype(np.float32)
    assert not np.array_equal(two, torch.addcmul(A, T1, T2, value=-0.37).numpy())
    # lerp without the w >= 0.5 branch
    one_branch = O.fma32(np.float32(0.9), (t1 - a).astype(np.float32), a)
    assert not np.array_equal(one_branch, torch.lerp(A, T1, 0.9).numpy())
    # GroupNorm variance with the n-1 denominator: the variance-1 invariant fails
    x = rng.standard_normal((2, 6, 3, 3)) * 3 + 7
    v = x.reshape(2, 3, -1)
    z = (v - v.mean(axis=2, keepdims=True)) / np.sqrt(v.var(axis=2, ddof=1, keepdims=True))
    assert not np.allclose(z.var(axis=2), 1, rtol=1e-10)
    # GroupNorm backward without the mean(dy) term: finite differences disagree
    w = rng.standard_normal(6)
    g = rng.standard_normal(x.shape)
    _, mean, rstd = O.group_norm_forward(x, w, None, 3, 1e-3)
    dx, _, _ = O.group_norm_backward(g, x, mean, rstd, w, 3)
    vg = (g * w[None, :, None, None]).reshape(2, 3, -1)
    wrong = dx + np.repeat(rstd, 2, axis=1)[:, :, None, None] * \
        np.repeat(vg.mean(axis=2), 2, axis=1)[:, :, None, None]
    fd = fd_grad(lambda u: O.group_norm_forward(u, w, None, 3, 1e-3)[0], x.copy(), g)
    np.testing.assert_allclose(dx, fd, rtol=1e-5, atol=1e-6)
    assert not np.allclose(wrong, fd, rtol=1e-5, atol=1e-6)


def _f64(x):
    return np.asarray(x, np.float32).astype(np.float64)
