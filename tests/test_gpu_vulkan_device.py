"""The PrivateUse1 ("vulkan") operator surface on the MI355X, exercised the way
the reference's own tests do (tests/test_convolution.py, test_conv_dispatch.py,
test_fused_addmm.py, test_native_bmm.py, test_direct_mm_out.py,
test_fused_adamw.py, test_multitensor_adamw.py): tensors moved with
.to("vulkan"), ops through torch, gradients through autograd, results against
CPU PyTorch, and the hot path must not touch the CPU fallback.
"""
import math

import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close_mag, conv_refs, gemm_mag

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def vk():
    import torch_vulkan
    assert torch_vulkan.is_available(), "no gfx950 device visible"
    return torch_vulkan


@pytest.fixture
def no_fallback(vk, monkeypatch):
    monkeypatch.setenv("TORCH_VULKAN_FORBID_CPU_FALLBACK", "1")
    before = vk.execution_stats()["cpu_fallback_calls"]
    yield
    assert vk.execution_stats()["cpu_fallback_calls"] == before


def test_device_basics(vk):
    assert torch._C._get_privateuse1_backend_name() == "vulkan"
    x = torch.arange(10, dtype=torch.float32).to("vulkan")
    assert x.device.type == "vulkan"
    assert torch.equal(x.cpu(), torch.arange(10, dtype=torch.float32))
    z = torch.zeros(3, 4, device="vulkan")
    o = torch.ones(5, device="vulkan")
    assert torch.count_nonzero(z.cpu()) == 0 and torch.equal(o.cpu(), torch.ones(5))
    assert "gfx950" in vk.device_name()
    v = x.view(2, 5).t()
    assert torch.equal(v.cpu(), torch.arange(10, dtype=torch.float32).view(2, 5).t())
    assert torch.equal(v.contiguous().cpu(), v.cpu())
    assert x[3].item() == 3.0
    y = x.clone()
    y[2:5] = torch.tensor([7.0, 8.0, 9.0]).to("vulkan")
    assert y.cpu().tolist()[2:5] == [7.0, 8.0, 9.0]


def test_streams_and_events(vk):
    s = vk.Stream()
    e0, e1 = vk.Event(enable_timing=True), vk.Event(enable_timing=True)
    with vk.stream(s):
        a = torch.ones(1 << 20, device="vulkan")
        e0.record()
        b = a + a
        e1.record()
    e1.synchronize()
    assert e0.elapsed_time(e1) >= 0
    vk.synchronize()
    assert b.cpu()[0].item() == 2.0


# ---------------------------------------------------------------- convolution
BASIC = [
    ((2, 3, 9, 11), 4, 3, 1, 1, 1, 1, True),
    ((1, 2, 11, 12), 3, 3, 2, 1, 1, 1, False),
    ((2, 4, 8, 7), 6, 3, 1, 2, 2, 2, True),
    ((1, 8, 8, 8), 8, 1, 1, 0, 1, 8, True),
    ((8, 64, 56, 56), 64, 3, 1, 1, 1, 1, True),
]


@pytest.mark.parametrize("case", BASIC, ids=[f"b{i}" for i in range(len(BASIC))])
def test_conv2d_forward_backward_matches_cpu(case, no_fallback):
    shape, ch, k, s, p, d, grp, bias = case
    torch.manual_seed(72)
    x = torch.randn(*shape)
    w = torch.randn(ch, shape[1] // grp, k, k) / math.sqrt(shape[1] // grp * k * k)
    b = torch.randn(ch) if bias else None
    y_ref = F.conv2d(x, w, b, s, p, d, grp)
    dy = torch.randn_like(y_ref)
    refs = conv_refs(x, w, b, dy, (s, s), (p, p), (d, d), grp)
    xv = x.to("vulkan").requires_grad_()
    wv = w.to("vulkan").requires_grad_()
    bv = b.to("vulkan").requires_grad_() if bias else None
    yv = F.conv2d(xv, wv, bv, s, p, d, grp)
    assert yv.device.type == "vulkan"
    grads = torch.autograd.grad(yv, [t for t in (xv, wv, bv) if t is not None], dy.to("vulkan"))
    assert_close_mag(yv, *refs["y"], what="y")
    assert_close_mag(grads[0], *refs["dx"], what="dx")
    assert_close_mag(grads[1], *refs["dw"], what="dw")
    if bias:
        assert_close_mag(grads[2], *refs["db"], what="db")


@pytest.mark.parametrize("algo,bwd", [("direct", "direct"), ("tiled", "optimized"), ("auto", "auto")])
def test_forced_algorithms_are_selected(vk, monkeypatch, algo, bwd):
    monkeypatch.setenv("TORCH_VULKAN_CONV_ALGO", algo)
    monkeypatch.setenv("TORCH_VULKAN_CONV_BACKWARD_ALGO", bwd)
    vk.clear_conv_dispatch_cache()
    g = torch.Generator().manual_seed(813)
    x, w = torch.randn(2, 18, 19, 23, generator=g) * 0.2, torch.randn(34, 9, 3, 5, generator=g) * 0.2
    b = torch.randn(34, generator=g) * 0.2
    args = ((2, 1), (2, 3), (2, 1), 2)
    y_ref = F.conv2d(x, w, b, *args)
    dy = torch.randn(y_ref.shape, generator=g) * 0.3
    refs = conv_refs(x, w, b, dy, *args)
    xv, wv, bv = (t.to("vulkan").requires_grad_() for t in (x, w, b))
    yv = F.conv2d(xv, wv, bv, *args)
    gx, gw, gb = torch.autograd.grad(yv, (xv, wv, bv), dy.to("vulkan"))
    for name, got in (("y", yv), ("dx", gx), ("dw", gw), ("db", gb)):
        assert_close_mag(got, *refs[name], what=name)
    stats = vk.conv_dispatch_stats()
    want = {"direct": "direct", "tiled": "implicit_gemm", "auto": "implicit_gemm"}[algo]
    assert stats.get(f"selected_forward_{want}", 0) >= 1, stats


def test_forced_winograd(vk, monkeypatch):
    monkeypatch.setenv("TORCH_VULKAN_CONV_ALGO", "winograd")
    vk.clear_conv_dispatch_cache()
    g = torch.Generator().manual_seed(4)
    x, w = torch.randn(2, 16, 12, 12, generator=g), torch.randn(24, 16, 3, 3, generator=g) / 12
    ref, mag = conv_refs(x, w, None, torch.zeros(2, 24, 12, 12), (1, 1), (1, 1), (1, 1), 1)["y"]
    y = F.conv2d(x.to("vulkan"), w.to("vulkan"), None, 1, 1)
    assert_close_mag(y, ref, mag, rtol=1e-3, what="winograd")
    assert vk.conv_dispatch_stats().get("selected_forward_winograd_f2", 0) >= 1
    with pytest.raises(RuntimeError):
        F.conv2d(x.to("vulkan"), w.to("vulkan"), None, 2, 1)  # stride 2 is not Winograd-eligible


def test_backward_winograd_knob(vk, monkeypatch):
    """TORCH_VULKAN_CONV_BACKWARD_ALGO=winograd: Winograd input and weight
    gradients for 3x3 stride-1 layers, the implicit GEMM for the rest
    (stride 2 here)."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_BACKWARD_ALGO", "winograd")
    vk.clear_conv_dispatch_cache()
    g = torch.Generator().manual_seed(15)
    x, w = torch.randn(2, 16, 12, 12, generator=g), torch.randn(24, 16, 3, 3, generator=g) / 12
    for stride, algo in ((1, "winograd_f2"), (2, "implicit_gemm")):
        args = ((stride, stride), (1, 1), (1, 1), 1)
        y_shape = (2, 24, 12 // stride, 12 // stride)
        dy = torch.randn(y_shape, generator=g)
        refs = conv_refs(x, w, None, dy, *args)
        xv, wv = x.to("vulkan").requires_grad_(), w.to("vulkan").requires_grad_()
        yv = F.conv2d(xv, wv, None, stride, 1)
        gx, gw = torch.autograd.grad(yv, (xv, wv), dy.to("vulkan"))
        assert_close_mag(gx, *refs["dx"], rtol=1e-3, what=f"dx stride {stride}")
        assert_close_mag(gw, *refs["dw"], rtol=1e-3, what=f"dw stride {stride}")
        stats = vk.conv_dispatch_stats()
        assert stats.get(f"selected_dinput_{algo}", 0) >= 1, stats
        assert stats.get(f"selected_dweight_{algo}", 0) >= 1, stats


def test_conv_views_and_output_mask(no_fallback):
    torch.manual_seed(9)
    base = torch.randn(2, 4, 10, 20)
    wb = torch.randn(10, 2, 3, 5)
    bb = torch.randn(20)
    x, xv = base[..., ::2], base.to("vulkan")[..., ::2]
    w, wv = wb.transpose(2, 3), wb.to("vulkan").transpose(2, 3)
    b, bv = bb[1::2], bb.to("vulkan")[1::2]
    args = ([1, 2], [2, 1], [1, 1], 2)
    ref = F.conv2d(x, w, b, *args)
    out = F.conv2d(xv, wv, bv, *args)
    torch.testing.assert_close(out.cpu(), ref, atol=4e-4, rtol=3e-4)
    gb = torch.randn(*ref.shape[:-1], ref.shape[-1] * 2)
    grad, gradv = gb[..., 1::2], gb.to("vulkan")[..., 1::2]

    def backward(go, inp, wt, mask):
        return torch.ops.aten.convolution_backward.default(go, inp, wt, [10], args[0], args[1], args[2], False,
                                                           [0, 0], 2, mask)

    for mask in ([True, True, True], [True, False, False], [False, True, False], [False, False, True]):
        expected = backward(grad, x, w, mask)
        actual = backward(gradv, xv, wv, mask)
        for enabled, a, e in zip(mask, actual, expected):
            if enabled:
                torch.testing.assert_close(a.cpu(), e, atol=5e-4, rtol=4e-4)
            else:
                assert a is None


def test_conv_rejects_kernel_larger_than_input():
    with pytest.raises(RuntimeError):
        F.conv2d(torch.randn(1, 2, 2, 2).to("vulkan"), torch.randn(3, 2, 3, 3).to("vulkan"), stride=2)


def test_conv_layer_sgd_decreases_loss():
    torch.manual_seed(7)
    m = torch.nn.Conv2d(1, 2, 3, padding=1).to("vulkan")
    opt = torch.optim.SGD(m.parameters(), lr=0.1)
    x = torch.randn(4, 1, 8, 8).to("vulkan")
    target = torch.randn(4, 2, 8, 8).to("vulkan")
    losses = []
    for _ in range(3):
        opt.zero_grad()
        loss = ((m(x) - target) ** 2).mean()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert losses[2] < losses[0]


# ---------------------------------------------------------------------- GEMM
def test_mm_known_answer_and_random(no_fallback):
    a = torch.tensor([[1.0, 2.0], [3.0, 4.0]]).to("vulkan")
    b = torch.tensor([[5.0, 6.0], [7.0, 8.0]]).to("vulkan")
    assert torch.mm(a, b).cpu().tolist() == [[19.0, 22.0], [43.0, 50.0]]
    x, y = torch.randn(64, 64), torch.randn(64, 64)
    assert_close_mag(torch.mm(x.to("vulkan"), y.to("vulkan")), x.double() @ y.double(), gemm_mag(x, y))


@pytest.mark.parametrize("shape", [(5, 7, 11), (32, 64, 19), (128, 256, 128), (256, 512, 512)])
@pytest.mark.parametrize("coefficients", [(1.0, 1.0), (0.25, 0.8), (-0.5, 1.5)])
def test_addmm_forward_backward(shape, coefficients, no_fallback):
    m, k, n = shape
    beta, alpha = coefficients
    torch.manual_seed(1234 + m + k + n)
    lhs, rhs, bias = torch.randn(m, k), torch.randn(k, n), torch.randn(n)
    lv, rv, bv = (t.to("vulkan").requires_grad_() for t in (lhs, rhs, bias))
    got = torch.addmm(bv, lv, rv, beta=beta, alpha=alpha)
    assert got.device.type == "vulkan"
    ref = beta * bias.double() + alpha * (lhs.double() @ rhs.double())
    assert_close_mag(got, ref, gemm_mag(lhs, rhs, alpha, beta, bias), what="addmm")
    grad = torch.randn(m, n)
    gl, gr, gb = torch.autograd.grad(got, (lv, rv, bv), grad.to("vulkan"))
    assert_close_mag(gl, alpha * grad.double() @ rhs.double().t(), gemm_mag(grad, rhs.t(), alpha), what="dlhs")
    assert_close_mag(gr, alpha * lhs.double().t() @ grad.double(), gemm_mag(lhs.t(), grad, alpha), what="drhs")
    assert_close_mag(gb, beta * grad.double().sum(0), abs(beta) * grad.double().abs().sum(0), what="dbias")


def test_linear_training_closed_form(no_fallback):
    lin = torch.nn.Linear(4, 2).to("vulkan")
    x = (torch.arange(12, dtype=torch.float32).reshape(3, 4) / 7).to("vulkan")
    out = lin(x)
    g = ((torch.arange(6, dtype=torch.float32).reshape(3, 2) - 2) / 3)
    out.backward(g.to("vulkan"))
    torch.testing.assert_close(lin.weight.grad.cpu(), g.t() @ x.cpu(), rtol=6e-5, atol=1e-4)
    torch.testing.assert_close(lin.bias.grad.cpu(), g.sum(0), rtol=6e-5, atol=1e-4)


def test_mm_out_semantics():
    a, b = torch.randn(7, 5), torch.randn(5, 3)
    out = torch.empty(7, 3).to("vulkan")
    r = torch.mm(a.to("vulkan"), b.to("vulkan"), out=out)
    assert r.data_ptr() == out.data_ptr()
    torch.testing.assert_close(out.cpu(), a @ b, rtol=1e-4, atol=1e-5)
    wrong = torch.empty(2, 2).to("vulkan")
    torch.mm(a.to("vulkan"), b.to("vulkan"), out=wrong)  # resized like ATen's out= contract
    assert wrong.shape == (7, 3)
    torch.testing.assert_close(wrong.cpu(), a @ b, rtol=1e-4, atol=1e-5)
    empty = torch.mm(torch.empty(0, 5).to("vulkan"), b.to("vulkan"))
    assert empty.shape == (0, 3)
    with pytest.raises(RuntimeError):
        torch.mm(a.to("vulkan"), b.double().to("vulkan"))


@pytest.mark.parametrize("shape", [(1, 2, 3, 7), (2, 8, 16, 11), (4, 16, 8, 32), (8, 32, 32, 32), (2, 2, 128, 4)])
@pytest.mark.parametrize("style", ["contiguous", "left_transpose", "right_transpose", "both", "offset",
                                   "batch_broadcast"])
def test_bmm_layouts_and_autograd(shape, style, no_fallback):
    torch.manual_seed(82 + sum(shape))
    bsz, m, k, n = shape
    xb, yb = torch.randn(bsz, m, k), torch.randn(bsz, k, n)
    if style == "left_transpose":
        xb = torch.randn(bsz, k, m)
    if style in ("right_transpose", "both"):
        yb = torch.randn(bsz, n, k)
    if style == "both":
        xb = torch.randn(bsz, k, m)
    if style == "offset":
        xb, yb = torch.randn(bsz, m + 1, k + 1), torch.randn(bsz, k + 1, n + 1)

    def views(xx, yy):
        if style == "left_transpose":
            return xx.transpose(1, 2), yy
        if style == "right_transpose":
            return xx, yy.transpose(1, 2)
        if style == "both":
            return xx.transpose(1, 2), yy.transpose(1, 2)
        if style == "offset":
            return xx[:, :m, :k], yy[:, :k, :n]
        if style == "batch_broadcast":
            return xx[:1].expand(bsz, -1, -1), yy[:1].expand(bsz, -1, -1)
        return xx, yy

    x, y = views(xb, yb)
    xv, yv = views(xb.to("vulkan"), yb.to("vulkan"))
    got = torch.bmm(xv, yv)
    assert_close_mag(got, x.double() @ y.double(), gemm_mag(x, y), what="bmm")
    xr, yr = xv.detach().requires_grad_(), yv.detach().requires_grad_()
    out = torch.bmm(xr, yr)
    grad = torch.randn(out.shape)
    gx, gy = torch.autograd.grad(out, (xr, yr), grad.to("vulkan"))
    assert_close_mag(gx, grad.double() @ y.double().transpose(1, 2), gemm_mag(grad, y.transpose(1, 2)), what="dx")
    assert_close_mag(gy, x.double().transpose(1, 2) @ grad.double(), gemm_mag(x.transpose(1, 2), grad), what="dy")


def test_sdpa_style_attention_through_bmm(no_fallback):
    torch.manual_seed(3)
    q, kk, v = (torch.randn(64, 256, 64) for _ in range(3))
    s = torch.bmm(q.to("vulkan"), kk.to("vulkan").transpose(1, 2))
    ref = q.double() @ kk.double().transpose(1, 2)
    assert_close_mag(s, ref, gemm_mag(q, kk.transpose(1, 2)), what="qk")
    o = torch.bmm(s, v.to("vulkan"))
    assert_close_mag(o, ref @ v.double(), ref.abs() @ v.double().abs(), rtol=2e-4, what="av")


# ------------------------------------------------------- baddbmm / addbmm
def test_baddbmm_beta_zero_ignores_nan_bias(no_fallback):
    # tests/test_opinfo_regressions.py:808-811 of the reference
    m, n = torch.randn(2, 3, 4), torch.randn(2, 4, 5)
    bias = torch.full((5,), float("nan"))
    got = torch.baddbmm(bias.to("vulkan"), m.to("vulkan"), n.to("vulkan"), beta=0, alpha=.5)
    torch.testing.assert_close(got.cpu(), torch.baddbmm(bias, m, n, beta=0, alpha=.5))


@pytest.mark.parametrize("bias_shape", [(7, 5, 9), (5, 9), (1, 9), (9,), (7, 1, 1)])
@pytest.mark.parametrize("coefficients", [(1.0, 1.0), (0.25, -1.5)])
def test_baddbmm_broadcast_bias_and_autograd(bias_shape, coefficients, no_fallback):
    g = torch.Generator().manual_seed(sum(bias_shape))
    beta, alpha = coefficients
    a, b = torch.randn(7, 5, 33, generator=g), torch.randn(7, 9, 33, generator=g).transpose(1, 2)
    bias = torch.randn(bias_shape, generator=g)
    av, bv, cv = (t.to("vulkan").requires_grad_() for t in (a, b, bias))
    out = torch.baddbmm(cv, av, bv, beta=beta, alpha=alpha)
    ref = beta * bias.double() + alpha * (a.double() @ b.double())
    mag = abs(beta) * bias.double().abs().expand(7, 5, 9) + abs(alpha) * (a.double().abs() @ b.double().abs())
    assert_close_mag(out, ref, mag, what="baddbmm")
    grad = torch.randn(7, 5, 9, generator=g)
    ga, gb, gc = torch.autograd.grad(out, (av, bv, cv), grad.to("vulkan"))
    assert_close_mag(ga, alpha * (grad.double() @ b.double().transpose(1, 2)),
                     abs(alpha) * (grad.double().abs() @ b.double().abs().transpose(1, 2)), what="d batch1")
    assert_close_mag(gb, alpha * (a.double().transpose(1, 2) @ grad.double()),
                     abs(alpha) * (a.double().abs().transpose(1, 2) @ grad.double().abs()), what="d batch2")
    gc_ref = (beta * grad.double()).sum_to_size(bias_shape)
    assert_close_mag(gc, gc_ref, (abs(beta) * grad.double().abs()).sum_to_size(bias_shape), what="d self")


@pytest.mark.parametrize("bias_shape", [(6, 10), (10,), (1, 1)])
@pytest.mark.parametrize("coefficients", [(1.0, 1.0), (0.0, 0.75), (-0.5, 2.0)])
def test_addbmm_sums_batches_in_order(bias_shape, coefficients, no_fallback):
    g = torch.Generator().manual_seed(len(bias_shape))
    beta, alpha = coefficients
    a, b = torch.randn(4, 6, 17, generator=g), torch.randn(4, 17, 10, generator=g)
    bias = torch.randn(bias_shape, generator=g)
    if beta == 0:
        bias = torch.full(bias_shape, float("nan"))
    out = torch.addbmm(bias.to("vulkan"), a.to("vulkan"), b.to("vulkan"), beta=beta, alpha=alpha)
    prod = (a.double() @ b.double()).sum(0)
    ref = alpha * prod + (beta * bias.double() if beta != 0 else 0)
    mag = abs(alpha) * (a.double().abs() @ b.double().abs()).sum(0) + (abs(beta) * bias.double().abs() if beta else 0)
    assert_close_mag(out, ref, torch.as_tensor(mag).expand(6, 10), what="addbmm")


def test_baddbmm_addbmm_out_and_in_place(no_fallback):
    g = torch.Generator().manual_seed(9)
    a, b = torch.randn(3, 4, 8, generator=g), torch.randn(3, 8, 5, generator=g)
    c3, c2 = torch.randn(3, 4, 5, generator=g), torch.randn(4, 5, generator=g)
    av, bv = a.to("vulkan"), b.to("vulkan")
    out3 = torch.empty(0, device="vulkan")
    torch.baddbmm(c3.to("vulkan"), av, bv, beta=0.5, alpha=2.0, out=out3)
    torch.testing.assert_close(out3.cpu(), torch.baddbmm(c3, a, b, beta=0.5, alpha=2.0), rtol=1e-4, atol=1e-5)
    inp = c3.to("vulkan")
    inp.baddbmm_(av, bv, alpha=-1.0)
    torch.testing.assert_close(inp.cpu(), c3.baddbmm(a, b, alpha=-1.0), rtol=1e-4, atol=1e-5)
    out2 = torch.empty(4, 5, device="vulkan")
    torch.addbmm(c2.to("vulkan"), av, bv, out=out2)
    torch.testing.assert_close(out2.cpu(), torch.addbmm(c2, a, b), rtol=1e-4, atol=1e-5)
    inp2 = c2.to("vulkan")
    inp2.addbmm_(av, bv, beta=3.0)
    torch.testing.assert_close(inp2.cpu(), c2.addbmm(a, b, beta=3.0), rtol=1e-4, atol=1e-5)
    empty = torch.addbmm(c2.to("vulkan"), torch.empty(0, 4, 8, device="vulkan"), torch.empty(0, 8, 5, device="vulkan"),
                         beta=0.5)
    torch.testing.assert_close(empty.cpu(), 0.5 * c2)


# --------------------------------------------------------------------- AdamW
@pytest.mark.parametrize("shape", [(3,), (4, 5), (137, 351), (256, 1024)])
def test_fused_adamw_matches_pytorch_cpu(shape, vk, no_fallback):
    from torch_vulkan.optim import AdamW as VkAdamW
    torch.manual_seed(2026)
    pc = torch.nn.Parameter(torch.randn(*shape))
    pv = torch.nn.Parameter(pc.detach().to("vulkan"))
    oc = torch.optim.AdamW([pc], lr=0.005, betas=(0.8, 0.91), eps=1e-6, weight_decay=0.031, foreach=False)
    ov = VkAdamW([pv], lr=0.005, betas=(0.8, 0.91), eps=1e-6, weight_decay=0.031)
    for i in range(8):
        grad = torch.randn(*shape) * (0.1 + i)
        pc.grad = grad.clone()
        pv.grad = grad.to("vulkan")
        oc.step()
        ov.step()
        torch.testing.assert_close(pv.detach().cpu(), pc.detach(), atol=1e-5, rtol=1e-4)
        for key in ("exp_avg", "exp_avg_sq"):
            torch.testing.assert_close(ov.state[pv][key].cpu(), oc.state[pc][key], atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("amsgrad", [False, True])
@pytest.mark.parametrize("count", [2, 11, 53])
def test_multitensor_state_parity_one_launch(amsgrad, count, vk):
    from torch_vulkan.optim import AdamW as VkAdamW
    gen = torch.Generator().manual_seed(7521)
    lengths = [1, 257, 513, 5, 2049, 2, 65, 0, 117, 4056, 16]
    original = [torch.randn((lengths[i % len(lengths)],), generator=gen) for i in range(count)]
    cpu = [torch.nn.Parameter(x.clone()) for x in original]
    gpu = [torch.nn.Parameter(x.to("vulkan")) for x in original]
    opts = {"lr": .0017, "betas": (.79, .933), "eps": 1e-7, "weight_decay": .014, "amsgrad": amsgrad}
    ref = torch.optim.AdamW(cpu, foreach=False, **opts)
    grouped = VkAdamW(gpu, batched=True, **opts)
    for it in range(9):
        for i, (c, v) in enumerate(zip(cpu, gpu)):
            if (i + it) % 13 == 0:
                c.grad = v.grad = None
            else:
                g = torch.randn(c.shape, generator=gen) * .03
                c.grad, v.grad = g, g.to("vulkan")
        ref.step()
        before = vk.execution_stats()["adamw_launches"]
        grouped.step()
        assert vk.execution_stats()["adamw_launches"] - before == 1
    vk.synchronize()
    for c, v in zip(cpu, gpu):
        torch.testing.assert_close(v.detach().cpu(), c.detach(), rtol=1e-4, atol=1e-5)
        if c in ref.state:
            for k in ("exp_avg", "exp_avg_sq") + (("max_exp_avg_sq",) if amsgrad else ()):
                torch.testing.assert_close(grouped.state[v][k].cpu(), ref.state[c][k], rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("amsgrad", [False, True])
def test_shared_update_buffer_keeps_sequential_semantics(amsgrad, vk):
    reference = torch.nn.Parameter(torch.linspace(.2, .9, 257))
    optimizer = torch.optim.AdamW([reference], amsgrad=amsgrad, lr=.003, betas=(.8, .93), eps=1e-7,
                                  weight_decay=.02, foreach=False)
    g1, g2 = torch.full_like(reference, .025), torch.full_like(reference, -.04)
    for g in (g1, g2):
        reference.grad = g
        optimizer.step()
    param = torch.linspace(.2, .9, 257).to("vulkan")
    avg, sq, maximum = torch.zeros_like(param), torch.zeros_like(param), torch.zeros_like(param)
    inputs = ([param, param], [g1.to("vulkan"), g2.to("vulkan")], [avg, avg], [sq, sq])
    options = (.003, .8, .93, 1e-7, .02, [1, 2])
    before = vk.execution_stats()["adamw_launches"]
    if amsgrad:
        torch.ops.torch_vulkan.adamw_amsgrad_step_batch_(*inputs, [maximum, maximum], *options)
    else:
        torch.ops.torch_vulkan.adamw_step_batch_(*inputs, *options)
    assert vk.execution_stats()["adamw_launches"] - before == 2
    torch.testing.assert_close(param.cpu(), reference.detach(), atol=4e-5, rtol=4e-5)
    state = optimizer.state[reference]
    torch.testing.assert_close(avg.cpu(), state["exp_avg"], atol=4e-5, rtol=4e-5)
    torch.testing.assert_close(sq.cpu(), state["exp_avg_sq"], atol=4e-5, rtol=4e-5)


@pytest.mark.parametrize("amsgrad", [False, True])
def test_torch_optim_adamw_fused_runs_on_device(amsgrad, vk):
    """torch.optim.AdamW(fused=True) dispatches aten::_fused_adamw_ (and
    _foreach_add_ on the device step tensors) to this backend."""
    torch.manual_seed(11)
    shapes = [(33, 7), (1000,), (4, 4, 3, 3), (5,)]
    cpu = [torch.nn.Parameter(torch.randn(s)) for s in shapes]
    gpu = [torch.nn.Parameter(p.detach().to("vulkan")) for p in cpu]
    oc = torch.optim.AdamW(cpu, lr=2e-3, weight_decay=0.05, amsgrad=amsgrad, foreach=False)
    ov = torch.optim.AdamW(gpu, lr=2e-3, weight_decay=0.05, amsgrad=amsgrad, fused=True)
    fb = vk.execution_stats()["cpu_fallback_calls"]
    for _ in range(5):
        for c, v in zip(cpu, gpu):
            g = torch.randn(c.shape) * 0.1
            c.grad, v.grad = g, g.to("vulkan")
        oc.step()
        ov.step()
    for c, v in zip(cpu, gpu):
        torch.testing.assert_close(v.detach().cpu(), c.detach(), rtol=1e-4, atol=1e-5)
    assert ov.state[gpu[0]]["step"].device.type == "vulkan"
    assert vk.execution_stats()["cpu_fallback_calls"] == fb


@pytest.mark.parametrize("maximize", [False, True])
@pytest.mark.parametrize("amsgrad", [False, True])
def test_fused_adamw_grad_scale_and_found_inf(no_fallback, amsgrad, maximize):
    """aten::_fused_adamw_ under a GradScaler: with found_inf == 0 the
    gradients are divided by grad_scale, the unscaled gradients are written
    back (before maximize negates them) and the step runs; with found_inf == 1
    nothing changes.  Compared with CPU torch._fused_adamw_ bit for bit on the
    gradients and within rel 1e-4 / abs 1e-5 on parameters and moments."""
    torch.manual_seed(21)
    shapes = [(37, 5), (4099,), (3,)]
    kw = dict(lr=3e-3, beta1=0.85, beta2=0.995, weight_decay=0.02, eps=1e-7, amsgrad=amsgrad, maximize=maximize)
    for found in (0.0, 1.0):
        cpu = {k: [torch.randn(sh) * (4.0 if k == "g" else 1.0) for sh in shapes] for k in ("p", "g")}
        cpu["m"] = [torch.randn(sh) * 0.1 for sh in shapes]
        cpu["v"] = [torch.rand(sh) * 0.01 for sh in shapes]
        cpu["x"] = [v.clone() * 1.5 for v in cpu["v"]] if amsgrad else []
        steps_c = [torch.tensor(3.0) for _ in shapes]
        dev = {k: [t.to("vulkan") for t in ts] for k, ts in cpu.items()}
        steps_d = [t.to("vulkan") for t in steps_c]
        scale, inf = torch.tensor(8.0), torch.tensor(found)
        torch._fused_adamw_(cpu["p"], cpu["g"], cpu["m"], cpu["v"], cpu["x"], steps_c, grad_scale=scale,
                            found_inf=inf, **kw)
        torch._fused_adamw_(dev["p"], dev["g"], dev["m"], dev["v"], dev["x"], steps_d,
                            grad_scale=scale.to("vulkan"), found_inf=inf.to("vulkan"), **kw)
        for k in ("g", "p", "m", "v", "x"):
            for c, d in zip(cpu[k], dev[k]):
                if k == "g":
                    assert torch.equal(d.cpu(), c), f"found_inf={found}: gradient not unscaled as torch does"
                else:
                    torch.testing.assert_close(d.cpu(), c, rtol=1e-4, atol=1e-5)


def test_fallback_is_counted_and_forbiddable(vk, monkeypatch):
    x = torch.randn(5).to("vulkan")
    before = vk.execution_stats()["cpu_fallback_calls"]
    torch.exp(x)  # not on this backend's path
    assert vk.execution_stats()["cpu_fallback_calls"] > before
    monkeypatch.setenv("TORCH_VULKAN_FORBID_CPU_FALLBACK", "1")
    with pytest.raises(RuntimeError, match="forbidden"):
        torch.exp(x)


def test_gpu_timing_stats(vk, monkeypatch):
    """gpu_timing_stats() (the reference's torch_vulkan.gpu_timing_stats,
    opt-in through TORCH_VULKAN_PROFILE_TIMESTAMPS=1) reports the kernels of
    timed conv / GEMM / AdamW ops with their GPU time, and nothing while off."""
    vk.reset_gpu_timing_stats()
    x = torch.randn(2, 16, 12, 12).to("vulkan").requires_grad_()
    w = torch.randn(16, 16, 3, 3).to("vulkan").requires_grad_()
    F.conv2d(x, w, padding=1)
    assert vk.gpu_timing_stats() == {}
    monkeypatch.setenv("TORCH_VULKAN_PROFILE_TIMESTAMPS", "1")
    y = F.conv2d(x, w, padding=1)
    y.backward(torch.ones_like(y))
    a = torch.randn(300, 200).to("vulkan")
    a @ a.t()
    p = torch.nn.Parameter(torch.randn(1000).to("vulkan"))
    p.grad = torch.randn(1000).to("vulkan")
    from torch_vulkan.optim import AdamW as VkAdamW
    VkAdamW([p]).step()
    stats = vk.gpu_timing_stats()
    names = " ".join(stats)
    for kind in ("conv_fwd_kernel", "conv_dx_kernel", "conv_dw_kernel", "gemm_kernel", "adamw_kernel"):
        assert kind in names, (kind, stats)
    for name, v in stats.items():
        assert v["samples"] >= 1 and v["shader_ms"] > 0 and v["host_eval_ms"] >= 0, (name, v)
        assert v["upload_ms"] == 0 and v["download_ms"] == 0
    monkeypatch.delenv("TORCH_VULKAN_PROFILE_TIMESTAMPS")
    before = {k: v["samples"] for k, v in vk.gpu_timing_stats().items()}
    a @ a.t()
    assert {k: v["samples"] for k, v in vk.gpu_timing_stats().items()} == before
    vk.reset_gpu_timing_stats()
    assert vk.gpu_timing_stats() == {}


@pytest.mark.parametrize("budget_mb", ["1", "64"])
def test_weight_split_scales_to_workspace_through_torch(vk, monkeypatch, budget_mb):
    """/root/reference/tests/test_conv_dispatch.py:255-297 through the vulkan
    device: a many-way dWeight split forced around the weight-gradient call
    shrinks to the TORCH_VULKAN_CONV_WORKSPACE_MB budget (the dispatch
    counters record splits, span and workspace), and dW / dB match float64."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_BACKWARD_ALGO", "optimized")
    monkeypatch.setenv("TORCH_VULKAN_CONV_WORKSPACE_MB", budget_mb)
    g = torch.Generator().manual_seed(31)
    x, w, b = torch.randn(1, 48, 64, 64, generator=g), torch.randn(96, 48, 3, 3, generator=g) * 0.05, torch.randn(96)
    gy = torch.randn(1, 96, 64, 64, generator=g)
    prior = vk.conv_dispatch_stats()
    monkeypatch.setenv("MX_CONV_PLAN", "5,512")
    _, dw, db = torch.ops.aten.convolution_backward.default(
        gy.to("vulkan"), x.to("vulkan"), w.to("vulkan"), [96], [1, 1], [1, 1], [1, 1], False, [0, 0], 1,
        [False, True, True])
    monkeypatch.delenv("MX_CONV_PLAN")
    stats = vk.conv_dispatch_stats()
    delta = {k: stats.get(k, 0) - prior.get(k, 0) for k in stats}
    parts, span = delta["dweight_tiled_split_count_total"], delta["dweight_tiled_split_span_total"]
    assert delta["dweight_tiled_dispatches"] == 1 and parts >= 2
    assert (parts - 1) * span < 64 * 64 <= parts * span
    assert delta["dweight_tiled_workspace_bytes_total"] <= int(budget_mb) << 20
    refs = conv_refs(x, w, b, gy, (1, 1), (1, 1), (1, 1), 1)
    assert_close_mag(dw, *refs["dw"], what="dw")
    assert_close_mag(db, *refs["db"], what="db")


def test_forced_split_rejects_zero_workspace_through_torch(vk, monkeypatch):
    """/root/reference/tests/test_conv_dispatch.py:302-313."""
    monkeypatch.setenv("TORCH_VULKAN_CONV_BACKWARD_ALGO", "optimized")
    monkeypatch.setenv("TORCH_VULKAN_CONV_WORKSPACE_MB", "0")
    monkeypatch.setenv("MX_CONV_PLAN", "5,2")
    x = torch.zeros((1, 9, 1, 257), device="vulkan")
    w = torch.zeros((17, 9, 1, 1), device="vulkan")
    go = torch.zeros((1, 17, 1, 257), device="vulkan")
    with pytest.raises(RuntimeError, match="[Ww]orkspace"):
        torch.ops.aten.convolution_backward.default(go, x, w, [17], [1, 1], [0, 0], [1, 1], False, [0, 0], 1,
                                                    [False, True, False])
