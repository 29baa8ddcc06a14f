"""Opt-in fused AdamW for ``"vulkan"`` parameters.

Interface of the reference's ``torch_vulkan.optim.AdamW``
(torch_vulkan/optim.py:13-75 there): the constructor keywords ``lr``,
``betas``, ``eps``, ``weight_decay``, ``batched`` and ``amsgrad``, and per
parameter the state keys of ``torch.optim.AdamW`` (``step``, ``exp_avg``,
``exp_avg_sq``, ``max_exp_avg_sq``), so checkpoints move between this
optimizer and torch's.

How it runs here: each parameter group becomes one ``_GroupStep`` -- the
parameters that have gradients, their moment buffers and their host step
counts -- which is handed to the backend's custom ops
(``torch.ops.torch_vulkan.adamw_step_batch_`` / ``adamw_amsgrad_step_batch_``,
schemas of csrc/ops/adamw.cpp:307-317).  The backend turns one batch call into
one multi-tensor launch over every tensor of the group (a new launch only where
two entries alias).  ``batched=False`` issues one call per parameter instead
(``adamw_step_`` for plain AdamW; the AMSGrad variant has no single-tensor op,
so it gets a one-entry batch).  ``torch.optim.AdamW(fused=True)`` also runs on
the device, through ``aten::_fused_adamw_``.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

_ops = None


def _backend_ops():
    global _ops
    if _ops is None:
        _ops = torch.ops.torch_vulkan
    return _ops


def _check_hyperparameters(lr, betas, eps, weight_decay):
    beta1, beta2 = betas
    problems = [name for name, ok in (("lr", lr >= 0), ("eps", eps >= 0), ("weight_decay", weight_decay >= 0),
                                      ("beta1", 0 <= beta1 < 1), ("beta2", 0 <= beta2 < 1)) if not ok]
    if problems:
        raise ValueError(f"AdamW: out-of-range hyperparameter(s) {', '.join(problems)} "
                         f"(lr={lr}, betas={betas}, eps={eps}, weight_decay={weight_decay})")


def _host_step(value) -> int:
    """A step count as a Python int (torch.optim checkpoints store a tensor)."""
    return int(value.item()) if isinstance(value, torch.Tensor) else int(value)


@dataclass
class _GroupStep:
    """The tensors of one parameter group that take part in this step."""
    amsgrad: bool
    params: list = field(default_factory=list)
    grads: list = field(default_factory=list)
    exp_avgs: list = field(default_factory=list)
    exp_avg_sqs: list = field(default_factory=list)
    max_exp_avg_sqs: list = field(default_factory=list)
    steps: list = field(default_factory=list)

    def add(self, p, state):
        self.params.append(p)
        self.grads.append(p.grad)
        self.exp_avgs.append(state["exp_avg"])
        self.exp_avg_sqs.append(state["exp_avg_sq"])
        if self.amsgrad:
            self.max_exp_avg_sqs.append(state["max_exp_avg_sq"])
        self.steps.append(state["step"])

    def lists(self, sl=slice(None)):
        out = [self.params[sl], self.grads[sl], self.exp_avgs[sl], self.exp_avg_sqs[sl]]
        if self.amsgrad:
            out.append(self.max_exp_avg_sqs[sl])
        return out

    def launch(self, hyper, batched):
        ops = _backend_ops()
        batch_op = ops.adamw_amsgrad_step_batch_ if self.amsgrad else ops.adamw_step_batch_
        if batched:
            batch_op(*self.lists(), *hyper, self.steps)
            return
        for i in range(len(self.params)):
            if self.amsgrad:
                batch_op(*self.lists(slice(i, i + 1)), *hyper, self.steps[i:i + 1])
            else:
                ops.adamw_step_(*(lst[i] for lst in self.lists()), *hyper, self.steps[i])


class AdamW(torch.optim.Optimizer):
    """Decoupled-weight-decay Adam whose update runs as multi-tensor gfx950
    launches (see the module docstring)."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, batched=True,
                 amsgrad=False):
        _check_hyperparameters(lr, betas, eps, weight_decay)
        defaults = {"lr": lr, "betas": betas, "eps": eps, "weight_decay": weight_decay, "batched": batched,
                    "amsgrad": amsgrad}
        super().__init__(params, defaults)

    def _state_of(self, p, amsgrad):
        """The parameter's state, created on first use; the step advanced by one."""
        state = self.state[p]
        state.setdefault("step", 0)
        # Missing buffers start at zero (a fresh parameter, or a checkpoint
        # written without AMSGrad that is resumed with it).
        for key in ("exp_avg", "exp_avg_sq") + (("max_exp_avg_sq",) if amsgrad else ()):
            if key not in state:
                state[key] = torch.zeros_like(p, memory_format=torch.preserve_format)
        state["step"] = _host_step(state["step"]) + 1
        return state

    def _collect(self, group) -> _GroupStep:
        batch = _GroupStep(amsgrad=bool(group["amsgrad"]))
        for p in group["params"]:
            g = p.grad
            if g is None:
                continue
            if g.is_sparse:
                raise RuntimeError("torch_vulkan AdamW: sparse gradients are not supported")
            if p.device.type != "vulkan":
                raise RuntimeError(f"torch_vulkan AdamW: parameter on {p.device}, expected a vulkan tensor")
            batch.add(p, self._state_of(p, batch.amsgrad))
        return batch

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            batch = self._collect(group)
            if not batch.params:
                continue
            beta1, beta2 = group["betas"]
            hyper = (group["lr"], beta1, beta2, group["eps"], group["weight_decay"])
            batch.launch(hyper, group.get("batched", True))
        return loss
