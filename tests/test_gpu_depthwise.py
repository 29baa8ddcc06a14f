"""Depthwise forward (groups == C_in, any channel multiplier) and the
large-grid known answers.

Reference: conv2d_depthwise.comp:15-41 (one output per invocation, bias then
taps in (kh, kw) order), selected for the forward when groups == cin and
cin >= 8 (csrc/ops/convolution.cpp:462) and forced by
TORCH_VULKAN_CONV_ALGO=depthwise (:450), which raises when the layer is not
depthwise (:361, :472-473).  Its cases follow tests/test_conv_dispatch.py:37-42
("depthwise-multiplier3", "unit-stride-dilated-depthwise"); the large-grid
closed form follows tests/test_conv_dispatch.py:315-333.  References are
float64 CPU torch; bound rel 1e-4 / abs 1e-5 (tests/helpers.py).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close_mag, conv_refs

pytestmark = pytest.mark.gpu

# xshape, multiplier, kernel, stride, padding, dilation
DEPTHWISE_CASES = [
    ((1, 5, 11, 13), 3, (3, 5), (1, 2), (1, 4), (1, 2)),    # depthwise-multiplier3
    ((1, 5, 11, 13), 3, (3, 5), (1, 1), (2, 4), (2, 2)),    # unit-stride-dilated-depthwise
    ((4, 32, 56, 56), 1, (3, 3), (1, 1), (1, 1), (1, 1)),   # MobileNet-style 3x3, several 16x64 tiles per plane
    ((2, 16, 33, 70), 2, (5, 5), (2, 2), (2, 2), (1, 1)),   # ragged tiles in both directions, stride 2
    ((2, 8, 17, 130), 1, (7, 7), (2, 2), (3, 3), (1, 1)),   # 7x7 stride 2: 133-column patch
    ((1, 8, 9, 9), 4, (1, 1), (1, 1), (0, 0), (1, 1)),      # 1x1 per-channel scale
    ((1, 9, 120, 200), 1, (3, 3), (1, 1), (40, 40), (40, 40)),  # patch beyond the LDS budget: direct reads
    ((3, 12, 6, 5), 2, (3, 3), (1, 1), (0, 0), (2, 1)),     # output smaller than one tile
]


def _inputs(xs, mult, kernel, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(xs, generator=g)
    w = torch.randn((xs[1] * mult, 1, *kernel), generator=g) / math.sqrt(kernel[0] * kernel[1])
    b = torch.randn(xs[1] * mult, generator=g) * 0.1
    return x, w, b


@pytest.fixture(scope="module")
def mx():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from torch_vulkan import mx as m
    m.lib()
    return m


@pytest.mark.parametrize("case", DEPTHWISE_CASES, ids=[f"dw{i}" for i in range(len(DEPTHWISE_CASES))])
def test_depthwise_forward_c_abi(mx, case):
    xs, mult, kernel, stride, padding, dilation = case
    x, w, b = _inputs(xs, mult, kernel, seed=sum(xs) + mult)
    d = mx.conv_desc(xs, w.shape, stride, padding, dilation, xs[1])
    assert mx.conv2d_select(d, mx.MX_CONV_FORWARD, mx.ALGO_DEPTHWISE) == mx.ALGO_DEPTHWISE
    dy = torch.zeros((xs[0], w.shape[0], d.oh, d.ow))
    ref, mag = conv_refs(x, w, b, dy, stride, padding, dilation, xs[1])["y"]
    s = torch.cuda.current_stream().cuda_stream
    for bias in (b, None):
        y = torch.full(dy.shape, float("nan"), device="cuda")  # every output must be written
        mx.conv2d_forward(d, x.cuda(), w.cuda(), bias.cuda() if bias is not None else None, y, mx.ALGO_DEPTHWISE, s)
        if bias is None:
            ref, mag = conv_refs(x, w, None, dy, stride, padding, dilation, xs[1])["y"]
        assert_close_mag(y, ref, mag, what=f"depthwise y (bias={bias is not None})")


def test_depthwise_variant_names(mx):
    staged = mx.conv_desc((1, 8, 40, 40), (8, 1, 3, 3), (1, 1), (1, 1), (1, 1), 8)
    wide = mx.conv_desc((1, 9, 120, 200), (9, 1, 3, 3), (1, 1), (40, 40), (40, 40), 9)
    assert mx.conv2d_plan(staged, mx.MX_CONV_FORWARD)["variant"] == "conv_depthwise_kernel<staged>"
    assert mx.conv2d_plan(wide, mx.MX_CONV_FORWARD)["variant"] == "conv_depthwise_kernel<global>"


@pytest.mark.parametrize("forced", [False, True])
def test_depthwise_through_torch(forced, monkeypatch):
    """Auto-selected (cin >= 8) or forced depthwise forward, autograd backward
    on the input- and weight-gradient kernels, against float64 CPU torch."""
    import torch_vulkan as vk
    monkeypatch.setenv("TORCH_VULKAN_FORBID_CPU_FALLBACK", "1")
    if forced:
        monkeypatch.setenv("TORCH_VULKAN_CONV_ALGO", "depthwise")
    vk.clear_conv_dispatch_cache()
    xs, mult, kernel, stride, padding, dilation = ((2, 16, 20, 70), 2, (3, 5), (1, 2), (1, 2), (2, 1))
    x, w, b = _inputs(xs, mult, kernel, seed=77)
    args = (stride, padding, dilation, xs[1])
    y_shape = F.conv2d(x, w, b, *args).shape
    dy = torch.randn(y_shape, generator=torch.Generator().manual_seed(78))
    refs = conv_refs(x, w, b, dy, *args)
    before = vk.conv_dispatch_stats().get("selected_forward_depthwise", 0)
    xv, wv, bv = (t.to("vulkan").requires_grad_() for t in (x, w, b))
    yv = F.conv2d(xv, wv, bv, *args)
    gx, gw, gb = torch.autograd.grad(yv, (xv, wv, bv), dy.to("vulkan"))
    for name, got in (("y", yv), ("dx", gx), ("dw", gw), ("db", gb)):
        assert_close_mag(got, *refs[name], what=name)
    assert vk.conv_dispatch_stats().get("selected_forward_depthwise", 0) == before + 1


def test_forced_depthwise_rejects_dense_layer(monkeypatch):
    import torch_vulkan  # noqa: F401
    monkeypatch.setenv("TORCH_VULKAN_CONV_ALGO", "depthwise")
    x = torch.randn(1, 8, 6, 6).to("vulkan")
    w = torch.randn(8, 4, 3, 3).to("vulkan")
    with pytest.raises(RuntimeError, match="depthwise"):
        F.conv2d(x, w, None, 1, 1, 1, 2)


def test_direct_forward_and_input_gradient_cross_65535_workgroups(monkeypatch):
    """1x1 conv with w = 2, b = 1 over 65535 * 128 + 17 positions: y = 2x + 1
    and dx = 0.25 * 2 exactly (tests/test_conv_dispatch.py:315-333); only
    dInput is requested."""
    import torch_vulkan  # noqa: F401
    monkeypatch.setenv("TORCH_VULKAN_CONV_ALGO", "direct")
    monkeypatch.setenv("TORCH_VULKAN_CONV_BACKWARD_ALGO", "direct")
    count = 65535 * 128 + 17
    x = torch.arange(count, dtype=torch.float32).remainder_(97).div_(97).view(1, 1, 1, count)
    xv = x.to("vulkan")
    wv = torch.full((1, 1, 1, 1), 2.0).to("vulkan")
    bv = torch.ones(1).to("vulkan")
    actual = F.conv2d(xv, wv, bv)
    torch.testing.assert_close(actual.cpu(), x * 2 + 1, rtol=1e-6, atol=1e-6)
    gradv = torch.full(x.shape, 0.25).to("vulkan")
    dx, dw, db = torch.ops.aten.convolution_backward.default(
        gradv, xv, wv, [1], [1, 1], [0, 0], [1, 1], False, [0, 0], 1, [True, False, False])
    torch.testing.assert_close(dx.cpu(), torch.full_like(x, 0.5), rtol=0, atol=0)
    assert dw is None and db is None


def test_implicit_gemm_and_depthwise_cross_65535_workgroups():
    """The same closed form on the default kernels: 8 channels of 1x1 conv
    (implicit GEMM, > 65535 tiles along the positions) and a depthwise 1x1
    over the same positions."""
    import torch_vulkan as vk
    vk.clear_conv_dispatch_cache()
    count = 65535 * 128 + 17
    x = torch.arange(count * 8, dtype=torch.float32).remainder_(97).div_(97).view(1, 8, 1, count)
    xv = x.to("vulkan")
    w = torch.zeros(8, 8, 1, 1)
    w[torch.arange(8), torch.arange(8)] = 2.0
    y = F.conv2d(xv, w.to("vulkan"), torch.ones(8).to("vulkan"))
    torch.testing.assert_close(y.cpu(), x * 2 + 1, rtol=0, atol=0)
    del y
    yd = F.conv2d(xv, torch.full((8, 1, 1, 1), 2.0).to("vulkan"), torch.ones(8).to("vulkan"), groups=8)
    torch.testing.assert_close(yd.cpu(), x * 2 + 1, rtol=0, atol=0)
    stats = vk.conv_dispatch_stats()
    assert stats.get("selected_forward_implicit_gemm", 0) >= 1 and stats.get("selected_forward_depthwise", 0) >= 1


def test_bmm_batch_beyond_65535():
    """bmm over 70,001 batches crosses the 65,535 grid.z launch split; integer
    operands make every product exact."""
    import torch_vulkan  # noqa: F401
    batch = 70001
    g = torch.Generator().manual_seed(3)
    a = torch.randint(-4, 5, (batch, 3, 5), generator=g).float()
    b = torch.randint(-4, 5, (batch, 5, 2), generator=g).float()
    out = torch.bmm(a.to("vulkan"), b.to("vulkan")).cpu()
    torch.testing.assert_close(out, torch.bmm(a, b), rtol=0, atol=0)
