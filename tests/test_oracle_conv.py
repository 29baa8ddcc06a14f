"""Pins the convolution oracle (oracle/oracle.c) on the CPU.

Checks: CPU PyTorch golden fixtures (the reference tests' case lists and
seeds, tests/golden/make_golden.py) in float64 and float32, the reference's
closed-form known answer (tests/test_conv_dispatch.py:315-333: y = 2x + 1,
dx = 0.5), invariants (dB == sum of dY; Winograd == direct; integer inputs are
exact), the validation rules of csrc/ops/convolution.cpp:101-156, and planted
mistakes that the tolerance must reject.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import winograd as wino
from helpers import RTOL, ATOL, WINOGRAD_RTOL, assert_close_mag

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "conv.npz"))
CASES = sorted({k.split("/")[0] for k in GOLD.files if not k.startswith("meta")})


def case(name):
    g = {k.split("/", 1)[1]: GOLD[k] for k in GOLD.files if k.startswith(name + "/")}
    s = g["params"]
    return g, (tuple(s[0:2]), tuple(s[2:4]), tuple(s[4:6]), int(s[6]))


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_cpu_torch(name):
    g, (stride, padding, dilation, groups) = case(name)
    b = g.get("b")
    y, my = oracle.conv2d_forward(g["x"], g["w"], b, stride, padding, dilation, groups)
    back = oracle.conv2d_backward(g["x"], g["w"], g["dy"], stride, padding, dilation, groups)
    got = {"y": (y, my), **back}
    for key in ("y", "dx", "dw", "db"):
        if key + "64" not in g:
            continue
        val, mag = got[key]
        # float64 CPU torch: the oracle (double accumulation) must agree to ~1e-12.
        np.testing.assert_allclose(val, g[key + "64"], rtol=1e-9, atol=1e-9 * (1 + mag.max()))
        # float32 CPU torch (the reference's CPU result) is within the tolerance model.
        assert_close_mag(torch.from_numpy(g[key + "32"]), torch.from_numpy(val), torch.from_numpy(mag),
                         what=f"{name}:{key} torch fp32 vs oracle")


@pytest.mark.parametrize("name", [c for c in CASES if c.startswith("winograd")])
def test_oracle_winograd_equals_direct(name):
    g, (stride, padding, dilation, groups) = case(name)
    yw, mag = oracle.conv2d_forward(g["x"], g["w"], g["b"], stride, padding, dilation, groups, winograd=True)
    np.testing.assert_allclose(yw, g["y64"], rtol=1e-9, atol=1e-9 * (1 + mag.max()))


@pytest.mark.parametrize("name", [c for c in CASES if c.startswith("winograd")])
def test_oracle_winograd_dinput_identity(name):
    """dx of a 3x3 stride-1 layer equals the Winograd convolution of dy with
    the flipped, channel-swapped filter at padding 2 - p (the identity behind
    the device's Winograd input gradient), against CPU torch float64's dx;
    the same call with the taps left unflipped must not match."""
    g, (stride, padding, dilation, groups) = case(name)
    assert stride == (1, 1) and dilation == (1, 1) and max(padding) <= 2
    pad_t = (2 - padding[0], 2 - padding[1])
    dx, mag = oracle.conv2d_forward(g["dy"], wino.flipped_filter(g["w"], groups), None, (1, 1), pad_t, (1, 1), groups,
                                    winograd=True)
    assert dx.shape == g["dx64"].shape
    np.testing.assert_allclose(dx, g["dx64"], rtol=1e-9, atol=1e-9 * (1 + mag.max()))
    go, c = g["w"].shape[:2]
    unflipped = np.ascontiguousarray(
        g["w"].reshape(groups, go // groups, c, 3, 3).transpose(0, 2, 1, 3, 4).reshape(groups * c, go // groups, 3, 3))
    bad, _ = oracle.conv2d_forward(g["dy"], unflipped, None, (1, 1), pad_t, (1, 1), groups, winograd=True)
    assert not np.allclose(bad, g["dx64"], rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("name", [c for c in CASES if c.startswith("winograd")])
def test_oracle_winograd_dweight_adjoint(name):
    """dw of a 3x3 stride-1 layer as the adjoint of the Winograd forward
    (G^T sum_tiles (A dY A^T) * (B^T d B) G) equals CPU torch float64's dw;
    a sign flipped in A or an entry of G changed must not match."""
    g, (stride, padding, dilation, groups) = case(name)
    dw = wino.dweight_adjoint(g["x"], g["dy"], padding, groups)
    mag = wino.dweight_adjoint(np.abs(g["x"]), np.abs(g["dy"]), padding, groups)
    np.testing.assert_allclose(dw, g["dw64"], rtol=1e-9, atol=1e-9 * (1 + mag.max()))
    bad_a = wino.AT.copy()
    bad_a[1, 3] = 1.0
    bad_g = wino.G.copy()
    bad_g[2, 1] = 0.5
    for kw in ({"at": bad_a}, {"g": bad_g}):
        bad = wino.dweight_adjoint(g["x"], g["dy"], padding, groups, **kw)
        assert not np.allclose(bad, g["dw64"], rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("hw,pad", [((5, 7), (0, 0)), ((6, 5), (1, 1)), ((4, 4), (2, 2)), ((7, 6), (0, 2))])
def test_oracle_winograd_dweight_brute_force(hw, pad):
    """Odd and even output sizes (half tiles at the edges) and paddings 0..2
    against the direct restatement of conv2d_backward_weight.comp."""
    rng = np.random.default_rng(sum(hw) + pad[0])
    x = rng.standard_normal((2, 5, *hw)).astype(np.float32)
    w = rng.standard_normal((3, 5, 3, 3)).astype(np.float32)
    oh, ow = hw[0] + 2 * pad[0] - 2, hw[1] + 2 * pad[1] - 2
    dy = rng.standard_normal((2, 3, oh, ow)).astype(np.float32)
    ref, mag = oracle.conv2d_backward(x, w, dy, (1, 1), pad)["dw"]
    got = wino.dweight_adjoint(x, dy, pad, 1)
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-9 * (1 + mag.max()))


def test_winograd_rejects_ineligible():
    x = np.zeros((1, 2, 8, 8), np.float32)
    with pytest.raises(oracle.ConvError):
        oracle.conv2d_forward(x, np.zeros((2, 2, 3, 3), np.float32), stride=(2, 2), winograd=True)


def test_closed_form_1x1():
    # tests/test_conv_dispatch.py:315-333: w = 2, b = 1 -> y = 2x + 1; dy = 0.25 -> dx = 0.5.
    x = (np.arange(4099, dtype=np.float32) % 97 / 97).reshape(1, 1, 1, -1)
    y, _ = oracle.conv2d_forward(x, np.full((1, 1, 1, 1), 2, np.float32), np.ones(1, np.float32))
    np.testing.assert_array_equal(y, 2 * x.astype(np.float64) + 1)
    back = oracle.conv2d_backward(x, np.full((1, 1, 1, 1), 2, np.float32), np.full(x.shape, 0.25, np.float32))
    np.testing.assert_array_equal(back["dx"][0], np.full(x.shape, 0.5))


def test_dbias_is_sum_of_dy_and_integer_inputs_are_exact():
    rng = np.random.default_rng(3)
    x = rng.integers(-3, 4, (2, 3, 7, 6)).astype(np.float32)
    w = rng.integers(-2, 3, (5, 3, 3, 3)).astype(np.float32)
    dy = rng.integers(-2, 3, (2, 5, 7, 6)).astype(np.float32)
    y, _ = oracle.conv2d_forward(x, w, None, (1, 1), (1, 1))
    ref = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(), padding=1)
    np.testing.assert_array_equal(y, ref.numpy())
    back = oracle.conv2d_backward(x, w, dy, (1, 1), (1, 1))
    np.testing.assert_array_equal(back["db"][0], dy.astype(np.float64).sum((0, 2, 3)))
    xt, wt = torch.from_numpy(x).double().requires_grad_(), torch.from_numpy(w).double().requires_grad_()
    gx, gw = torch.autograd.grad(torch.nn.functional.conv2d(xt, wt, padding=1), (xt, wt), torch.from_numpy(dy).double())
    np.testing.assert_array_equal(back["dx"][0], gx.numpy())
    np.testing.assert_array_equal(back["dw"][0], gw.numpy())


@pytest.mark.parametrize("xs,ws,kw", [
    ((1, 2, 2, 2), (3, 2, 3, 3), dict(stride=(2, 2))),                 # kernel larger than input
    ((1, 4, 5, 5), (3, 3, 1, 1), dict(groups=2)),                      # channels not divisible
    ((1, 1, 1, 1), (1, 1, 1, 1), dict(stride=(2147483648, 1))),        # int32 coordinates
    ((1, 2, 5, 5), (2, 2, 3, 3), dict(padding=(-1, 0))),               # negative padding
])
def test_validation_rejects(xs, ws, kw):
    with pytest.raises(oracle.ConvError):
        oracle.conv2d_shape(xs, ws, kw.get("stride", (1, 1)), kw.get("padding", (0, 0)), (1, 1), kw.get("groups", 1))


def test_output_shape_formula():
    assert oracle.conv2d_shape((8, 64, 56, 56), (64, 64, 3, 3), (1, 1), (1, 1)) == (56, 56)
    assert oracle.conv2d_shape((64, 3, 224, 224), (64, 3, 7, 7), (2, 2), (3, 3)) == (112, 112)
    assert oracle.conv2d_shape((1, 1, 10, 10), (1, 1, 3, 3), (1, 1), (0, 0), (2, 2)) == (6, 6)


@pytest.mark.parametrize("mistake", ["drop_tap", "swap_kernel_axes", "sign_of_bias"])
def test_planted_mistakes_are_rejected(mistake):
    """The tolerance model must catch plausible indexing/sign errors."""
    g, (stride, padding, dilation, groups) = case("dispatch12")  # 3x5 kernel, strides (2,3)
    x, w, b = g["x"], g["w"], g["b"]
    if mistake == "drop_tap":
        w = w.copy()
        w[:, :, 1, 2] = 0
    elif mistake == "swap_kernel_axes":
        w = np.ascontiguousarray(w[:, :, ::-1, :])
    else:
        b = -b
    y, mag = oracle.conv2d_forward(x, w, b, stride, padding, dilation, groups)
    with pytest.raises(AssertionError):
        assert_close_mag(torch.from_numpy(y), torch.from_numpy(g["y64"]), torch.from_numpy(mag))
