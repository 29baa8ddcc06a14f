"""Writes the golden fixtures under tests/golden/ from CPU PyTorch.

    python tests/golden/make_golden.py

CPU PyTorch is the reference's CPU implementation of every op on this path
(mistrjirka/Pytorch-vulkan tests compare against it live), so these fixtures
freeze its outputs for the reference tests' own case lists and seeds:

  conv.npz   tests/test_conv_dispatch.py:20-47 (17 geometries incl. the
             255/256/257 split boundaries, `_check_case` seeds and scales),
             tests/test_convolution.py:8-13 (4 geometries, seed 72), plus
             small Winograd-eligible 3x3/s1 cases; float64 and float32 results
             for forward, dX, dW, dB.
  gemm.npz   tests/test_mm.py:29-35 known answer, tests/test_fused_addmm.py
             shapes x (beta, alpha), tests/test_native_bmm.py shapes.
  adamw.npz  tests/test_fused_adamw.py trajectories (8 steps) and the
             tests/test_multitensor_adamw.py lengths list (9 iterations with
             missing gradients, plain and AMSGrad).

Every file records the torch version and seeds.  Inputs are float32; results
are what CPU torch computes on exactly those inputs.
"""
from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

DISPATCH_CASES = [
    ((1, 7, 1, 15), 7, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 1, 17), 9, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 15, 1, 31), 15, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 17, 1, 33), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 31, 1, 63), 31, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 33, 1, 65), 33, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    *[((1, 9, k + 3, k + 5), 17, (k, k), (1, 1), (0, 0), (1, 1), 1) for k in (9, 10, 11, 12)],
    ((2, 18, 19, 23), 34, (3, 5), (2, 1), (2, 3), (2, 1), 2),
    ((1, 5, 11, 13), 15, (3, 5), (1, 2), (1, 4), (1, 2), 5),
    ((2, 6, 15, 19), 9, (3, 5), (1, 1), (3, 4), (2, 3), 3),
    ((1, 5, 11, 13), 15, (3, 5), (1, 1), (2, 4), (2, 2), 5),
    ((1, 9, 17, 23), 17, (3, 5), (2, 3), (3, 2), (2, 1), 1),
    *[((1, 9, 1, p), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1) for p in (255, 256, 257)],
]

BASIC_CASES = [  # (shape, channels, kernel, stride, padding, dilation, groups, bias)
    ((2, 3, 9, 11), 4, 3, 1, 1, 1, 1, True),
    ((1, 2, 11, 12), 3, 3, 2, 1, 1, 1, False),
    ((2, 4, 8, 7), 6, 3, 1, 2, 2, 2, True),
    ((1, 8, 8, 8), 8, 1, 1, 0, 1, 8, True),
]

WINOGRAD_CASES = [  # 3x3, stride 1, dilation 1
    ((2, 8, 12, 12), 8, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((1, 16, 9, 11), 24, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((2, 32, 8, 8), 32, (3, 3), (1, 1), (0, 0), (1, 1), 4),
]


def conv_case(out, name, x, w, b, dy, stride, padding, dilation, groups):
    rec = {"x": x, "w": w, "dy": dy, "params": np.array([*stride, *padding, *dilation, groups], dtype=np.int64)}
    if b is not None:
        rec["b"] = b
    for dt, tag in ((torch.float64, "64"), (torch.float32, "32")):
        ts = [t.to(dt).requires_grad_() for t in (x, w) + ((b,) if b is not None else ())]
        y = F.conv2d(ts[0], ts[1], ts[2] if b is not None else None, stride, padding, dilation, groups)
        grads = torch.autograd.grad(y, ts, dy.to(dt))
        rec["y" + tag] = y.detach()
        rec["dx" + tag], rec["dw" + tag] = grads[0], grads[1]
        if b is not None:
            rec["db" + tag] = grads[2]
    for k, v in rec.items():
        out[f"{name}/{k}"] = v.detach().numpy() if isinstance(v, torch.Tensor) else v


def make_conv():
    out = {}
    for i, (xs, cout, kernel, stride, padding, dilation, groups) in enumerate(DISPATCH_CASES):
        g = torch.Generator().manual_seed(813 + sum(xs) + sum(kernel))  # tests/test_conv_dispatch.py:51
        x = torch.randn(xs, generator=g) * 0.2
        w = torch.randn((cout, xs[1] // groups, *kernel), generator=g) * 0.2
        b = torch.randn((cout,), generator=g) * 0.2
        oh = (xs[2] + 2 * padding[0] - dilation[0] * (kernel[0] - 1) - 1) // stride[0] + 1
        ow = (xs[3] + 2 * padding[1] - dilation[1] * (kernel[1] - 1) - 1) // stride[1] + 1
        dy = torch.randn((xs[0], cout, oh, ow), generator=g) * 0.3
        conv_case(out, f"dispatch{i:02d}", x, w, b, dy, stride, padding, dilation, groups)
    for i, (shape, ch, k, s, p, d, grp, bias) in enumerate(BASIC_CASES):
        torch.manual_seed(72)  # tests/test_convolution.py:23
        x = torch.randn(*shape)
        w = torch.randn(ch, shape[1] // grp, k, k)
        b = torch.randn(ch) if bias else None
        y = F.conv2d(x, w, b, s, p, d, grp)
        dy = torch.randn_like(y)
        conv_case(out, f"basic{i}", x, w, b, dy, (s, s), (p, p), (d, d), grp)
    for i, (xs, cout, kernel, stride, padding, dilation, groups) in enumerate(WINOGRAD_CASES):
        g = torch.Generator().manual_seed(4242 + i)
        x = torch.randn(xs, generator=g)
        w = torch.randn((cout, xs[1] // groups, *kernel), generator=g) / 3.0
        b = torch.randn((cout,), generator=g) * 0.1
        oh = xs[2] + 2 * padding[0] - 2
        ow = xs[3] + 2 * padding[1] - 2
        dy = torch.randn((xs[0], cout, oh, ow), generator=g)
        conv_case(out, f"winograd{i}", x, w, b, dy, stride, padding, dilation, groups)
    out["meta/torch"] = np.array(torch.__version__)
    np.savez_compressed(os.path.join(HERE, "conv.npz"), **out)


def make_gemm():
    out = {"known/a": np.array([[1, 2], [3, 4]], np.float32), "known/b": np.array([[5, 6], [7, 8]], np.float32)}
    out["known/c"] = (torch.from_numpy(out["known/a"]) @ torch.from_numpy(out["known/b"])).numpy()
    for m, k, n in [(5, 7, 11), (32, 64, 19), (128, 256, 128)]:  # tests/test_fused_addmm.py:8-12
        torch.manual_seed(1234 + m + k + n)
        lhs, rhs, bias = torch.randn(m, k), torch.randn(k, n), torch.randn(n)
        key = f"addmm_{m}_{k}_{n}"
        out[f"{key}/lhs"], out[f"{key}/rhs"], out[f"{key}/bias"] = lhs.numpy(), rhs.numpy(), bias.numpy()
        for j, (beta, alpha) in enumerate([(1.0, 1.0), (0.25, 0.8), (-0.5, 1.5)]):
            out[f"{key}/coef{j}"] = np.array([beta, alpha])
            out[f"{key}/out32_{j}"] = torch.addmm(bias, lhs, rhs, beta=beta, alpha=alpha).numpy()
            out[f"{key}/out64_{j}"] = torch.addmm(bias.double(), lhs.double(), rhs.double(), beta=beta,
                                                  alpha=alpha).numpy()
    for shape in [(1, 2, 3, 7), (2, 8, 16, 11), (4, 16, 8, 32), (8, 32, 32, 32), (2, 2, 128, 4)]:
        torch.manual_seed(82 + sum(shape))  # tests/test_native_bmm.py:13
        bt, m, k, n = shape
        x, y = torch.randn(bt, m, k), torch.randn(bt, k, n)
        key = "bmm_" + "_".join(map(str, shape))
        out[f"{key}/a"], out[f"{key}/b"] = x.numpy(), y.numpy()
        out[f"{key}/out32"] = torch.bmm(x, y).numpy()
        out[f"{key}/out64"] = torch.bmm(x.double(), y.double()).numpy()
    out["meta/torch"] = np.array(torch.__version__)
    np.savez_compressed(os.path.join(HERE, "gemm.npz"), **out)


def make_adamw():
    out = {}
    for shape in [(3,), (4, 5), (64, 65)]:  # tests/test_fused_adamw.py:9 (largest shape reduced)
        torch.manual_seed(2026)
        p = torch.nn.Parameter(torch.randn(*shape))
        key = "traj_" + "_".join(map(str, shape))
        out[f"{key}/p0"] = p.detach().clone().numpy()
        opt = torch.optim.AdamW([p], lr=0.005, betas=(0.8, 0.91), eps=1e-6, weight_decay=0.031, foreach=False)
        for i in range(8):
            grad = torch.randn(*shape) * (0.1 + i)
            p.grad = grad.clone()
            opt.step()
            out[f"{key}/g{i}"] = grad.numpy()
            out[f"{key}/p{i + 1}"] = p.detach().clone().numpy()
            out[f"{key}/m{i + 1}"] = opt.state[p]["exp_avg"].clone().numpy()
            out[f"{key}/v{i + 1}"] = opt.state[p]["exp_avg_sq"].clone().numpy()
    lengths = [1, 257, 513, 5, 2049, 2, 65, 0, 117, 4056, 16]  # tests/test_multitensor_adamw.py:13
    for amsgrad in (False, True):
        generator = torch.Generator().manual_seed(7521)
        count = 11
        shapes = [(lengths[i % len(lengths)],) for i in range(count)]
        original = [torch.randn(s, generator=generator) for s in shapes]
        cpu = [torch.nn.Parameter(x.clone()) for x in original]
        opts = {"lr": .0017, "betas": (.79, .933), "eps": 1e-7, "weight_decay": .014, "amsgrad": amsgrad}
        ref = torch.optim.AdamW(cpu, foreach=False, **opts)
        key = f"multi_ams{int(amsgrad)}"
        for i, x in enumerate(original):
            out[f"{key}/p0_{i}"] = x.numpy()
        for it in range(9):
            for i, c in enumerate(cpu):
                if (i + it) % 13 == 0:
                    c.grad = None
                    out[f"{key}/g{it}_{i}"] = np.zeros(0, np.float32)
                else:
                    g = torch.randn(c.shape, generator=generator) * .03
                    c.grad = g
                    out[f"{key}/g{it}_{i}"] = g.numpy()
            ref.step()
        for i, c in enumerate(cpu):
            out[f"{key}/p_{i}"] = c.detach().numpy()
            st = ref.state.get(c, {})
            for k in ("exp_avg", "exp_avg_sq", "max_exp_avg_sq"):
                if k in st:
                    out[f"{key}/{k}_{i}"] = st[k].numpy()
            out[f"{key}/step_{i}"] = np.array(float(st["step"]) if "step" in st else 0.0)
    out["meta/torch"] = np.array(torch.__version__)
    np.savez_compressed(os.path.join(HERE, "adamw.npz"), **out)


if __name__ == "__main__":
    torch.set_num_threads(1)
    make_conv()
    make_gemm()
    make_adamw()
    for f in ("conv.npz", "gemm.npz", "adamw.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
