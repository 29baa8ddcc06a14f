"""GPU parity of the multi-tensor pointwise path (csrc/mx_foreach.hip and
csrc/torch/ops_foreach.cpp): torch.optim's foreach ops and the per-tensor
lerp / addcmul / addcdiv / maximum / minimum, modelled on the reference's
tests/test_optimizer_primitives.py cases.

Each op is one IEEE operation or one fused multiply-add per element in the
same form as torch's CPU kernel (pinned bit for bit in test_oracle_nn.py), so
the device results are compared with torch's CPU results EXACTLY (NaN and
signed zeros included), except sqrt: neither torch's CPU sqrt nor the GPU's is
correctly rounded, so it is held to one float32 ulp.  The optimizer runs,
whose steps compose these ops, use a tolerance (rel 1e-5 / abs 1e-7 after 5
steps).
"""
import copy

import numpy as np
import pytest
import torch

from oracle import nn as O

pytestmark = pytest.mark.gpu

# Sizes: below, at and past a 4096-element chunk, unaligned tails, empty.
SIZES = [(5, 3), (4096,), (4099,), (7, 611), (1,), (0,), (64, 64, 3), (33,)]


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


def lists(seed, k=1, positive=False):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(k):
        ts = [torch.randn(s, generator=g) * 3 for s in SIZES]
        if positive:
            ts = [t.abs() + 0.1 for t in ts]
        out.append(ts)
    return out


def dev(ts):
    return [t.to("vulkan") for t in ts]


def same(got, want, ulps=0):
    for g, w in zip(got, want):
        g = g.cpu()
        assert g.shape == w.shape
        assert torch.equal(torch.isnan(g), torch.isnan(w))
        m = ~torch.isnan(w)
        d = (g[m].view(torch.int32).long() - w[m].view(torch.int32).long()).abs()
        assert d.numel() == 0 or int(d.max()) <= ulps, f"{int(d.max())} ulp, max abs {(g[m] - w[m]).abs().max()}"


@pytest.mark.parametrize("op", ["mul_", "div_", "add_"])
def test_foreach_scalar_and_scalarlist(no_fallback, op):
    (a,) = lists(1)
    scalars = [0.5 + 0.25 * i for i in range(len(a))]
    for arg in (1.7, scalars):
        cpu = [t.clone() for t in a]
        d = dev(a)
        getattr(torch, f"_foreach_{op}")(cpu, arg)
        getattr(torch, f"_foreach_{op}")(d, arg)
        same(d, cpu)


def test_foreach_lerp_addcmul_addcdiv(no_fallback, vk):
    a, b, c = lists(2, 3)
    (pos,) = lists(3, positive=True)
    for weight in (0.1, 0.9):
        cpu, d = [t.clone() for t in a], dev(a)
        torch._foreach_lerp_(cpu, b, weight)
        torch._foreach_lerp_(d, dev(b), weight)
        same(d, cpu)
    w = [torch.rand_like(t) * 2 - 0.5 for t in a]
    cpu, d = [t.clone() for t in a], dev(a)
    torch._foreach_lerp_(cpu, b, w)
    torch._foreach_lerp_(d, dev(b), dev(w))
    same(d, cpu)
    for value in (0.37, [0.1 * (i + 1) for i in range(len(a))]):
        cpu, d = [t.clone() for t in a], dev(a)
        torch._foreach_addcmul_(cpu, b, c, value)
        torch._foreach_addcmul_(d, dev(b), dev(c), value)
        same(d, cpu)
        cpu, d = [t.clone() for t in a], dev(a)
        torch._foreach_addcdiv_(cpu, b, pos, value)
        torch._foreach_addcdiv_(d, dev(b), dev(pos), value)
        same(d, cpu)
    before = vk.execution_stats()["kernel_launches"]
    torch._foreach_addcdiv_(dev(a), dev(b), dev(pos), 0.5)
    assert vk.execution_stats()["kernel_launches"] - before == 1  # the whole list in one launch


def test_foreach_maximum_sqrt_add_list(no_fallback):
    a, b = lists(4, 2)
    a[0][0, 0] = float("nan")
    b[1][5] = float("nan")
    a[2][3], b[2][3] = -0.0, 0.0
    cpu, d = [t.clone() for t in a], dev(a)
    torch._foreach_maximum_(cpu, b)
    torch._foreach_maximum_(d, dev(b))
    same(d, cpu)
    cpu, d = [t.clone() for t in a], dev(a)
    torch._foreach_minimum_(cpu, b)
    torch._foreach_minimum_(d, dev(b))
    same(d, cpu)
    (pos,) = lists(5, positive=True)
    same(torch._foreach_sqrt(dev(pos)), torch._foreach_sqrt(pos), ulps=1)
    d = dev(pos)
    torch._foreach_sqrt_(d)
    same(d, torch._foreach_sqrt(pos), ulps=1)
    same(torch._foreach_add(dev(a), dev(b), alpha=-0.3), torch._foreach_add(a, b, alpha=-0.3))
    cpu, d = [t.clone() for t in a], dev(a)
    torch._foreach_add_(cpu, b, alpha=2.5)
    torch._foreach_add_(d, dev(b), alpha=2.5)
    same(d, cpu)
    same(torch._foreach_mul(dev(a), 0.3), torch._foreach_mul(a, 0.3))


def test_foreach_repeated_tensor_updates_in_order(no_fallback, vk):
    t = torch.randn(1000)
    d = t.to("vulkan")
    before = vk.execution_stats()["kernel_launches"]
    torch._foreach_mul_([d, d, d], 2.0)
    assert vk.execution_stats()["kernel_launches"] - before == 3  # each write starts a new launch
    assert torch.equal(d.cpu(), t * 8)
    x, y = torch.randn(777), torch.randn(777)
    dx, dy = x.to("vulkan"), y.to("vulkan")
    torch._foreach_add_([dx, dy], [dy, dx])  # the second entry reads the first's output
    assert torch.equal(dx.cpu(), x + y) and torch.equal(dy.cpu(), y + (x + y))


def test_foreach_strided_tensors(no_fallback):
    base = torch.randn(40, 30)
    ref = base.t().clone()
    d = base.to("vulkan").t()  # non-contiguous view, written back in place
    other = torch.randn(30, 40)
    torch._foreach_lerp_([d], [other.to("vulkan")], 0.3)
    torch._foreach_lerp_([ref], [other], 0.3)
    same([d], [ref])


@pytest.mark.parametrize("op", ["lerp", "addcmul", "addcdiv", "maximum", "minimum"])
def test_pointwise_per_tensor_broadcast_out_and_inplace(no_fallback, op):
    g = torch.Generator().manual_seed(9)
    a, b = torch.randn(4, 5, 6, generator=g), torch.randn(5, 1, generator=g)
    c = torch.rand(1, 6, generator=g) + 0.5
    fn = {"lerp": lambda x, y, z: torch.lerp(x, y, 0.7), "addcmul": lambda x, y, z: torch.addcmul(x, y, z, value=-1.3),
          "addcdiv": lambda x, y, z: torch.addcdiv(x, y, z, value=0.4), "maximum": lambda x, y, z: torch.maximum(x, y),
          "minimum": lambda x, y, z: torch.minimum(x, y)}[op]
    want = fn(a, b, c)
    got = fn(a.to("vulkan"), b.to("vulkan"), c.to("vulkan"))
    same([got], [want])
    if op == "lerp":
        w = torch.rand(4, 5, 6, generator=g)
        same([torch.lerp(a.to("vulkan"), b.to("vulkan"), w.to("vulkan"))], [torch.lerp(a, b, w)])
        d = a.to("vulkan")
        d.lerp_(b.to("vulkan"), 0.2)
        same([d], [a.clone().lerp_(b, 0.2)])
    if op in ("addcmul", "addcdiv"):
        d = a.to("vulkan")
        getattr(d, op + "_")(b.to("vulkan"), c.to("vulkan"), value=0.9)
        same([d], [getattr(a.clone(), op + "_")(b, c, value=0.9)])
        out = torch.empty(1, device="vulkan")
        getattr(torch, op)(a.to("vulkan"), b.to("vulkan"), c.to("vulkan"), value=0.9, out=out)
        same([out], [getattr(torch, op)(a, b, c, value=0.9)])


def test_oracle_agrees_with_device_kernels(no_fallback):
    """The C ABI on a list against oracle/nn.py's float32 restatements."""
    from torch_vulkan import mx
    import torch_vulkan
    a, b, c = lists(7, 3)
    c = [t.abs() + 0.2 for t in c]
    outs = dev([torch.empty_like(t) for t in a])
    da, db, dc = dev(a), dev(b), dev(c)
    st = torch_vulkan._C._current_stream_ptr()
    mx.foreach(mx.FE_ADDCDIV, outs, da, db, dc, scalars=[0.3] * len(a), stream=st)
    for o, x, y, z in zip(outs, a, b, c):
        assert np.array_equal(o.cpu().numpy(), O.addcdiv(x.numpy(), y.numpy(), z.numpy(), 0.3))
    mx.foreach(mx.FE_LERP_SCALAR, outs, da, db, scalars=0.62, stream=st)
    for o, x, y in zip(outs, a, b):
        assert np.array_equal(o.cpu().numpy(), O.lerp(x.numpy(), y.numpy(), 0.62))


@pytest.mark.parametrize("name,make", [
    ("adamw", lambda p: torch.optim.AdamW(p, lr=1e-3, weight_decay=0.01, foreach=True)),
    ("adamw_amsgrad", lambda p: torch.optim.AdamW(p, lr=1e-3, weight_decay=0.01, amsgrad=True, foreach=True)),
    ("adam", lambda p: torch.optim.Adam(p, lr=2e-3, foreach=True)),
    ("sgd_momentum", lambda p: torch.optim.SGD(p, lr=1e-2, momentum=0.9, weight_decay=1e-4, nesterov=True,
                                               foreach=True)),
])
def test_torch_optim_foreach_on_device(no_fallback, vk, name, make):
    g = torch.Generator().manual_seed(11)
    shapes = [(64, 32), (32,), (7, 5, 3), (4099,), (1,)]
    ref = [torch.nn.Parameter(torch.randn(s, generator=g) * 0.02) for s in shapes]
    devp = [torch.nn.Parameter(p.detach().to("vulkan")) for p in ref]
    o_ref, o_dev = make(ref), make(devp)
    for step in range(5):
        grads = [torch.randn(s, generator=g) * 1e-3 for s in shapes]
        for p, q, gr in zip(ref, devp, grads):
            p.grad = gr.clone()
            q.grad = gr.to("vulkan")
        o_ref.step()
        o_dev.step()
    for p, q in zip(ref, devp):
        torch.testing.assert_close(q.detach().cpu(), p.detach(), rtol=1e-5, atol=1e-7)
