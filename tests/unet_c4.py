"""The C4 workload: a diffusion-style U-Net training step (FP32).

Batch 16 of 3x64x64 N(0,1) inputs; base width 128 with channel multipliers
(1, 2, 2, 4), so levels run at 64, 32, 16 and 8 pixels with 128, 256, 256 and
512 channels; two ResBlocks per level (GroupNorm with 32 groups, SiLU, 3x3
convolution, a 1x1 projection when the width changes); a stride-2 3x3
convolution to go down a level and a 2x nearest upsample plus 3x3 convolution
to come back up, with the level's output concatenated as the skip; bmm
self-attention with 4 heads at 16x16; MSE loss against N(0,1) targets; Kaiming
initialisation (torch's default for Conv2d).

The reference's own diffusion probe (benchmarks/probe_diffusion_train.py:27-85)
is a smaller model of the same family (GroupNorm/SiLU ResBlocks, conv
down/upsampling, concatenated skips, self-attention); this one is sized to the
C4 configuration. It uses only stock torch.nn modules, so the same module runs
on the CPU and on the "vulkan" device, and every operator it dispatches is one
of the backend's registrations (or a view).
"""
from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional as F


class ResBlock(nn.Module):
    def __init__(self, cin: int, cout: int, groups: int = 32):
        super().__init__()
        self.norm1 = nn.GroupNorm(groups, cin)
        self.conv1 = nn.Conv2d(cin, cout, 3, padding=1)
        self.norm2 = nn.GroupNorm(groups, cout)
        self.conv2 = nn.Conv2d(cout, cout, 3, padding=1)
        self.skip = nn.Conv2d(cin, cout, 1) if cin != cout else None

    def forward(self, x):
        h = self.conv1(F.silu(self.norm1(x)))
        h = self.conv2(F.silu(self.norm2(h)))
        return h + (self.skip(x) if self.skip is not None else x)


class Attention(nn.Module):
    """Multi-head self-attention over the pixels of a feature map, as bmm."""

    def __init__(self, channels: int, heads: int = 4, groups: int = 32):
        super().__init__()
        self.heads = heads
        self.norm = nn.GroupNorm(groups, channels)
        self.qkv = nn.Conv2d(channels, 3 * channels, 1)
        self.proj = nn.Conv2d(channels, channels, 1)

    def forward(self, x):
        b, c, h, w = x.shape
        d = c // self.heads
        qkv = self.qkv(self.norm(x)).reshape(b, 3, self.heads, d, h * w)
        q = qkv[:, 0].reshape(b * self.heads, d, h * w)
        k = qkv[:, 1].reshape(b * self.heads, d, h * w)
        v = qkv[:, 2].reshape(b * self.heads, d, h * w)
        # [B*heads, HW, HW] scores; bmm on a transposed view of q.
        scores = torch.bmm(q.transpose(1, 2), k) * (d ** -0.5)
        attn = torch.softmax(scores, dim=-1)
        out = torch.bmm(v, attn.transpose(1, 2))  # [B*heads, d, HW]
        return x + self.proj(out.reshape(b, c, h, w))


class UNetC4(nn.Module):
    def __init__(self, base: int = 128, mults=(1, 2, 2, 4), blocks: int = 2, attn_res: int = 16,
                 image: int = 64, in_ch: int = 3, heads: int = 4, groups: int = 32):
        super().__init__()
        self.conv_in = nn.Conv2d(in_ch, base, 3, padding=1)
        chans = [base * m for m in mults]
        self.down = nn.ModuleList()
        self.downsample = nn.ModuleList()
        res, cin = image, base
        for i, c in enumerate(chans):
            level = nn.ModuleList()
            for _ in range(blocks):
                level.append(ResBlock(cin, c, groups))
                if res == attn_res:
                    level.append(Attention(c, heads, groups))
                cin = c
            self.down.append(level)
            if i + 1 < len(chans):
                self.downsample.append(nn.Conv2d(c, c, 3, stride=2, padding=1))
                res //= 2
        self.mid = nn.ModuleList([ResBlock(cin, cin, groups), ResBlock(cin, cin, groups)])
        self.up = nn.ModuleList()
        self.upsample = nn.ModuleList()
        for i in reversed(range(len(chans))):
            c = chans[i]
            level = nn.ModuleList()
            cat_in = cin + c
            for j in range(blocks):
                level.append(ResBlock(cat_in if j == 0 else c, c, groups))
                if res == attn_res:
                    level.append(Attention(c, heads, groups))
            self.up.append(level)
            cin = c
            if i > 0:
                self.upsample.append(nn.Conv2d(c, c, 3, padding=1))
                res *= 2
        self.norm_out = nn.GroupNorm(groups, cin)
        self.conv_out = nn.Conv2d(cin, in_ch, 3, padding=1)

    def forward(self, x):
        h = self.conv_in(x)
        skips = []
        for i, level in enumerate(self.down):
            for m in level:
                h = m(h)
            skips.append(h)
            if i < len(self.downsample):
                h = self.downsample[i](h)
        for m in self.mid:
            h = m(h)
        for j, level in enumerate(self.up):
            h = torch.cat([h, skips[len(skips) - 1 - j]], dim=1)
            for m in level:
                h = m(h)
            if j < len(self.upsample):
                h = self.upsample[j](F.interpolate(h, scale_factor=2.0, mode="nearest"))
        return self.conv_out(F.silu(self.norm_out(h)))


def make_inputs(batch: int = 16, image: int = 64, seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, 3, image, image, generator=g)
    target = torch.randn(batch, 3, image, image, generator=g)
    return x, target


def make_model(seed: int = 0, **kw) -> UNetC4:
    torch.manual_seed(seed)
    return UNetC4(**kw)


def train_step_loss(model, x, target):
    """Forward, MSE loss and backward of one step; returns the loss tensor."""
    model.zero_grad(set_to_none=True)
    loss = F.mse_loss(model(x), target)
    loss.backward()
    return loss


def step_flops(model, x) -> float:
    """GEMM FLOPs of one training step on input x (2 per multiply-add):
    every convolution three times (forward, dInput, dWeight) except conv_in,
    whose input needs no gradient (two), and every attention bmm three times
    (forward and the two operand gradients).  Shapes are read by forward hooks
    in one no-grad forward pass, so this runs wherever the model lives."""
    total = [0.0]
    hooks = []

    def conv_hook(mod, inp, out):
        k = mod.weight.shape[1] * mod.weight.shape[2] * mod.weight.shape[3]
        total[0] += (2 if mod is model.conv_in else 3) * 2.0 * out.numel() * k

    def attn_hook(mod, inp, out):
        b, c, h, w = inp[0].shape
        n = h * w
        # scores = q^T k and out = v attn^T, each 2*(b*heads)*n*n*d FLOPs
        total[0] += 3 * 2 * (2.0 * b * mod.heads * n * n * (c // mod.heads))

    for m in model.modules():
        if isinstance(m, nn.Conv2d):
            hooks.append(m.register_forward_hook(conv_hook))
        elif isinstance(m, Attention):
            hooks.append(m.register_forward_hook(attn_hook))
    with torch.no_grad():
        model(x)
    for h in hooks:
        h.remove()
    return total[0]
