"""Opt-in fused AdamW for ``"vulkan"`` parameters.

Same API, state keys and checkpoint behaviour as the reference's
torch_vulkan/optim.py:13-75: state is created lazily with ``zeros_like``, the
step is a host int (a tensor step restored from a ``torch.optim.AdamW``
checkpoint is converted), and every parameter group is updated by one call of
``torch.ops.torch_vulkan.adamw_step_batch_`` (or the AMSGrad variant), which
the backend runs as a single multi-tensor launch.  ``torch.optim.AdamW(fused=True)``
also runs on the device (``aten::_fused_adamw_``).
"""
from __future__ import annotations

import torch


class AdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2, batched=True,
                 amsgrad=False):
        if lr < 0 or eps < 0 or weight_decay < 0 or not all(0 <= b < 1 for b in betas):
            raise ValueError("Invalid AdamW hyperparameters")
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay, batched=batched,
                                      amsgrad=amsgrad))

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            beta1, beta2 = group["betas"]
            params, grads, m1, m2, mx, steps = [], [], [], [], [], []
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("Vulkan AdamW does not support sparse gradients")
                if p.device.type != "vulkan":
                    raise RuntimeError("Vulkan AdamW only supports Vulkan parameters")
                state = self.state[p]
                if not state:
                    state["step"] = 0
                    state["exp_avg"] = torch.zeros_like(p)
                    state["exp_avg_sq"] = torch.zeros_like(p)
                    if group["amsgrad"]:
                        state["max_exp_avg_sq"] = torch.zeros_like(p)
                if isinstance(state["step"], torch.Tensor):
                    state["step"] = int(state["step"].item())
                state["step"] += 1
                params.append(p)
                grads.append(p.grad)
                m1.append(state["exp_avg"])
                m2.append(state["exp_avg_sq"])
                if group["amsgrad"]:
                    mx.append(state["max_exp_avg_sq"])
                steps.append(state["step"])
            if not params:
                continue
            hp = (group["lr"], beta1, beta2, group["eps"], group["weight_decay"])
            if group["amsgrad"]:
                if group.get("batched", True):
                    torch.ops.torch_vulkan.adamw_amsgrad_step_batch_(params, grads, m1, m2, mx, *hp, steps)
                else:
                    for args in zip(params, grads, m1, m2, mx, steps):
                        torch.ops.torch_vulkan.adamw_amsgrad_step_batch_(*[[a] for a in args[:5]], *hp, [args[5]])
            elif group.get("batched", True):
                torch.ops.torch_vulkan.adamw_step_batch_(params, grads, m1, m2, *hp, steps)
            else:
                for p, g, a, b, s in zip(params, grads, m1, m2, steps):
                    torch.ops.torch_vulkan.adamw_step_(p, g, a, b, *hp, s)
        return loss
