"""torch_vulkan.optim.AdamW across parameter groups, checkpoints and missing
gradients, as the reference's tests/test_fused_amsgrad.py:10-142 exercises its
optimizer: per-group ``lr`` / ``betas`` against CPU ``torch.optim.AdamW``
(foreach=False), a ``state_dict()`` / ``load_state_dict()`` round trip that
continues bit for bit, import of a standard torch AdamW checkpoint whose
``step`` is a tensor, queued steps through autograd, and NaN propagation in
the AMSGrad maximum.  Parity bar: rel 1e-4 / abs 1e-5 against CPU torch (the
reference's own tests use rel 6e-5 / abs 3e-5); the restored optimizer runs
the same launches on the same state, so it must match to the bit.
"""
import copy

import pytest
import torch

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


def _close(got, ref, **kw):
    torch.testing.assert_close(got.detach().cpu(), ref.detach(), rtol=1e-4, atol=1e-5, **kw)


def _bits_equal(a, b):
    a, b = a.detach().cpu(), b.detach().cpu()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32)), f"{int((a != b).sum())} elements differ"


@pytest.mark.parametrize("batched", [True, False])
@pytest.mark.parametrize("shapes", [[(37,)], [(3, 7), (8,), (2, 3, 5)], [(8193,), (0,), (1, 16)],
                                    [(9, 12, 7), (7, 4)]])
def test_amsgrad_state_with_missing_gradients_matches_cpu(batched, shapes, no_fallback):
    """Reference tests/test_fused_amsgrad.py:10-44: gradients go missing after
    the state exists; parameters, all three moments and the step count follow
    CPU torch."""
    from torch_vulkan.optim import AdamW as VkAdamW
    g = torch.Generator().manual_seed(88219)
    initial = [torch.randn(s, generator=g) for s in shapes]
    cpu = [torch.nn.Parameter(p.clone()) for p in initial]
    dev = [torch.nn.Parameter(p.to("vulkan")) for p in initial]
    opts = dict(lr=.005, betas=(.8, .91), eps=1e-6, weight_decay=.031, amsgrad=True)
    ref = torch.optim.AdamW(cpu, foreach=False, **opts)
    opt = VkAdamW(dev, batched=batched, **opts)
    for step in range(1, 12):
        for i, (c, v) in enumerate(zip(cpu, dev)):
            if (step + i) % 5 == 0:
                c.grad = v.grad = None
            else:
                grad = torch.randn(c.shape, generator=g) * (0.1 + .01 * step)
                c.grad, v.grad = grad, grad.to("vulkan")
        ref.step()
        opt.step()
        for c, v in zip(cpu, dev):
            _close(v, c)
            if c in ref.state:
                for key in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"):
                    _close(opt.state[v][key], ref.state[c][key])
                assert opt.state[v]["step"] == int(ref.state[c]["step"].item())


@pytest.mark.parametrize("amsgrad", [False, True])
def test_parameter_groups_and_checkpoint_round_trip(amsgrad, no_fallback):
    """Reference tests/test_fused_amsgrad.py:47-89: two groups with their own
    lr and betas against CPU torch, then state_dict() -> a fresh optimizer ->
    load_state_dict(); both continue three more steps identically."""
    from torch_vulkan.optim import AdamW as VkAdamW
    torch.manual_seed(405)
    layers = [torch.nn.Parameter(torch.randn(7, 11)), torch.nn.Parameter(torch.randn(4, 3))]
    dev = [torch.nn.Parameter(p.detach().to("vulkan")) for p in layers]
    hyper = [{"lr": .001, "betas": (.75, .88)}, {"lr": .005, "betas": (.91, .975)}]
    ref = torch.optim.AdamW([dict(h, params=[p]) for h, p in zip(hyper, layers)], amsgrad=amsgrad, foreach=False)
    opt = VkAdamW([dict(h, params=[p]) for h, p in zip(hyper, dev)], amsgrad=amsgrad, batched=True)
    for step in range(9):
        for c, v in zip(layers, dev):
            grad = torch.randn_like(c) * (.001 + step * .003)
            c.grad, v.grad = grad, grad.to("vulkan")
        ref.step()
        opt.step()
    keys = ("exp_avg", "exp_avg_sq") + (("max_exp_avg_sq",) if amsgrad else ())
    # The groups kept their own hyperparameters (no mixing of lr / betas).
    for c, v in zip(layers, dev):
        _close(v, c)
        for key in keys:
            _close(opt.state[v][key], ref.state[c][key])

    checkpoint = copy.deepcopy(opt.state_dict())
    assert [g["lr"] for g in checkpoint["param_groups"]] == [.001, .005]
    assert [tuple(g["betas"]) for g in checkpoint["param_groups"]] == [(.75, .88), (.91, .975)]
    restored_params = [torch.nn.Parameter(p.detach().clone()) for p in dev]
    restored = VkAdamW([dict(h, params=[p]) for h, p in zip(hyper, restored_params)], amsgrad=amsgrad,
                       batched=True)
    restored.load_state_dict(checkpoint)
    for v, r in zip(dev, restored_params):
        _bits_equal(v, r)
        for key in keys:
            assert restored.state[r][key].device.type == "vulkan"
            _bits_equal(opt.state[v][key], restored.state[r][key])
        assert opt.state[v]["step"] == restored.state[r]["step"] == 9
    for _ in range(3):
        for v, r in zip(dev, restored_params):
            grad = torch.randn(v.shape)
            v.grad, r.grad = grad.to("vulkan"), grad.to("vulkan")
        opt.step()
        restored.step()
    for v, r in zip(dev, restored_params):
        _bits_equal(v, r)
        for key in keys:
            _bits_equal(opt.state[v][key], restored.state[r][key])
        assert restored.state[r]["step"] == 12


@pytest.mark.parametrize("amsgrad", [False, True])
def test_queued_steps_through_autograd(amsgrad, no_fallback):
    """Reference tests/test_fused_amsgrad.py:92-106: eight steps of
    zero_grad / backward / step with no host read in between (the loss is
    sum(p * p), the reference's square().sum() through ops this backend
    registers)."""
    from torch_vulkan.optim import AdamW as VkAdamW
    cpu = torch.nn.Parameter(torch.linspace(-.5, .6, 97))
    dev = torch.nn.Parameter(cpu.detach().to("vulkan"))
    ref = torch.optim.AdamW([cpu], amsgrad=amsgrad, foreach=False)
    opt = VkAdamW([dev], amsgrad=amsgrad)
    for _ in range(8):
        ref.zero_grad(set_to_none=True)
        opt.zero_grad(set_to_none=True)
        (cpu * cpu).sum().backward()
        (dev * dev).sum().backward()
        ref.step()
        opt.step()
    _close(dev, cpu)
    for key in ("exp_avg", "exp_avg_sq") + (("max_exp_avg_sq",) if amsgrad else ()):
        _close(opt.state[dev][key], ref.state[cpu][key])


@pytest.mark.parametrize("amsgrad", [False, True])
def test_imports_standard_torch_checkpoint_with_tensor_step(amsgrad, no_fallback):
    """Reference tests/test_fused_amsgrad.py:109-125: a CPU torch.optim.AdamW
    checkpoint (its 'step' a scalar tensor) loads into the device optimizer,
    which then steps exactly as the CPU optimizer continues."""
    from torch_vulkan.optim import AdamW as VkAdamW
    original = torch.nn.Parameter(torch.linspace(-1, 1, 17))
    ref = torch.optim.AdamW([original], lr=.002, amsgrad=amsgrad, foreach=False)
    for _ in range(4):
        original.grad = torch.full_like(original, .04)
        ref.step()
    state = copy.deepcopy(ref.state_dict())
    dev = torch.nn.Parameter(original.detach().to("vulkan"))
    opt = VkAdamW([dev], lr=.002, amsgrad=amsgrad)
    opt.load_state_dict(state)
    assert isinstance(opt.state[dev]["step"], torch.Tensor)
    for key in ("exp_avg", "exp_avg_sq"):
        assert opt.state[dev][key].device.type == "vulkan"  # moved to the parameter's device
    original.grad = torch.full_like(original, .05)
    dev.grad = original.grad.to("vulkan")
    ref.step()
    opt.step()
    assert opt.state[dev]["step"] == 5
    _close(dev, original)
    for key in ("exp_avg", "exp_avg_sq") + (("max_exp_avg_sq",) if amsgrad else ()):
        _close(opt.state[dev][key], ref.state[original][key])


def test_checkpoint_moves_back_to_standard_torch(no_fallback):
    """The other direction: the device optimizer's state_dict, moved to the
    CPU, resumes a standard torch.optim.AdamW (integer step accepted)."""
    from torch_vulkan.optim import AdamW as VkAdamW
    torch.manual_seed(11)
    init = torch.randn(5, 6)
    dev = torch.nn.Parameter(init.to("vulkan"))
    twin = torch.nn.Parameter(init.clone())
    opt = VkAdamW([dev], lr=.003, betas=(.85, .95), weight_decay=.02)
    ref = torch.optim.AdamW([twin], lr=.003, betas=(.85, .95), weight_decay=.02, foreach=False)
    grads = [torch.randn(5, 6) * .1 for _ in range(6)]
    for g in grads[:3]:
        dev.grad, twin.grad = g.to("vulkan"), g.clone()
        opt.step()
        ref.step()
    sd = opt.state_dict()
    cpu_sd = {"param_groups": sd["param_groups"],
              "state": {k: {n: (v.cpu() if isinstance(v, torch.Tensor) else torch.tensor(float(v)))
                            for n, v in st.items()} for k, st in sd["state"].items()}}
    resumed_param = torch.nn.Parameter(dev.detach().cpu())
    resumed = torch.optim.AdamW([resumed_param], lr=.003, betas=(.85, .95), weight_decay=.02, foreach=False)
    resumed.load_state_dict(cpu_sd)
    for g in grads[3:]:
        resumed_param.grad, twin.grad = g.clone(), g.clone()
        resumed.step()
        ref.step()
    torch.testing.assert_close(resumed_param.detach(), twin.detach(), rtol=1e-4, atol=1e-5)


def test_amsgrad_propagates_nan_in_maximum_moment(no_fallback):
    """Reference tests/test_fused_amsgrad.py:127-142 (torch.maximum semantics:
    a NaN second moment wins over a finite maximum)."""
    from torch_vulkan.optim import AdamW as VkAdamW
    cpu = torch.nn.Parameter(torch.tensor([.25, .5, .75]))
    dev = torch.nn.Parameter(cpu.detach().to("vulkan"))
    a = torch.optim.AdamW([cpu], amsgrad=True, foreach=False)
    b = VkAdamW([dev], amsgrad=True, batched=True)
    for grad in (torch.tensor([.1, .2, .3]), torch.tensor([float("nan"), .1, .15])):
        cpu.grad, dev.grad = grad, grad.to("vulkan")
        a.step()
        b.step()
    for key in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"):
        torch.testing.assert_close(b.state[dev][key].cpu(), a.state[cpu][key], equal_nan=True)
    torch.testing.assert_close(dev.detach().cpu(), cpu.detach(), equal_nan=True)
    assert torch.isnan(b.state[dev]["max_exp_avg_sq"].cpu()[0])
