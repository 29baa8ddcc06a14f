"""Parity at BASELINE.json's full configuration sizes (C2, C3, C4, C5).

Full-size outputs are too large for a float64 CPU reference of every element
in a test's time budget, so each configuration is checked by a property that
does not depend on size:

* C2 (Linear 8192 x 4096 x 4096): the forward addmm, dX, dW and both
  transposed-input products at their real shapes, 1024 sampled outputs each
  against float64 dot products of the same rows and columns on the host;
* C3 (ResNet-50 conv stack at batch 64): all 53 layers, forward / dInput /
  dWeight routed as bench.py routes them (3x3 stride-1 layers on Winograd),
  ~400 sampled outputs per phase against float64 on the host;
* C4 (the U-Net at base width 128, 64 x 64 images, batch 16): one training
  step on the "vulkan" device against the same step in float64 on the CPU,
  each gradient within a small multiple of CPU FP32's own error;
* C5 (AdamW over 250 tensors, 125M elements): one step from a state warmed for
  10 steps, bit-identical to the oracle's restatement.

Tolerance: rel 1e-4 / abs 1e-5 with the magnitude model of tests/helpers.py
(rel 1e-3 for Winograd), as everywhere else.
"""
from __future__ import annotations

import copy
import math

import numpy as np
import pytest
import torch

from helpers import ATOL, RTOL, WINOGRAD_RTOL

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mx():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from torch_vulkan import mx as m
    m.lib()
    return m


def stream():
    return torch.cuda.current_stream().cuda_stream


def check_samples(got, ref, mag, rtol, what):
    got, ref, mag = (np.asarray(a, dtype=np.float64) for a in (got, ref, mag))
    err = np.abs(got - ref)
    bound = rtol * np.abs(ref) + ATOL * np.maximum(mag, 1.0)
    bad = ~(err <= bound)
    assert not bad.any(), (f"{what}: {int(bad.sum())}/{bad.size} samples out of bound; worst err/bound "
                           f"{float(np.max(err / bound)):.3g}; first {np.argmax(bad)}: got {got[np.argmax(bad)]} "
                           f"ref {ref[np.argmax(bad)]}")
    return float(np.max(err / bound))


# ------------------------------------------------------------------ C2
def test_c2_linear_full_size(mx):
    M, K, N = 8192, 4096, 4096
    g = torch.Generator().manual_seed(0)
    X = torch.randn(M, K, generator=g)
    W = torch.empty(N, K)
    torch.nn.init.kaiming_uniform_(W, a=math.sqrt(5), generator=g)
    b = torch.empty(N).uniform_(-1 / 64, 1 / 64, generator=g)
    dY = torch.randn(M, N, generator=g)
    Xd, Wd, bd, dYd = X.cuda(), W.cuda(), b.cuda(), dY.cuda()
    # (label, device A, device B, bias, host A rows getter, host B columns getter)
    cases = [
        ("addmm X.W^T+b", Xd, Wd.t(), bd, X, W.t()),
        ("dX=dY.W", dYd, Wd, None, dY, W),
        ("dW=dY^T.X", dYd.t(), Xd, None, dY.t(), X),
        ("X^T.G", Xd.t(), dYd, None, X.t(), dY),
        ("X.W^T", Xd, Wd.t(), None, X, W.t()),
    ]
    rng = np.random.default_rng(1)
    for label, A, B, bias, Ah, Bh in cases:
        c = torch.empty(A.shape[0], B.shape[1], device="cuda")
        mx.gemm(A, B, c, bias=bias, beta=1.0 if bias is not None else 0.0, stream=stream())
        rows = rng.integers(0, A.shape[0], 1024)
        cols = rng.integers(0, B.shape[1], 1024)
        got = c[torch.from_numpy(rows).cuda(), torch.from_numpy(cols).cuda()].cpu().numpy()
        a = Ah[torch.from_numpy(rows)].double().numpy()          # [1024, K]
        bt = Bh[:, torch.from_numpy(cols)].t().double().numpy()  # [1024, K]
        ref = np.einsum("ik,ik->i", a, bt)
        mag = np.einsum("ik,ik->i", np.abs(a), np.abs(bt))
        if bias is not None:
            ref = ref + b.double().numpy()[cols]
            mag = mag + np.abs(b.double().numpy()[cols])
        worst = check_samples(got, ref, mag, RTOL, f"C2 {label}")
        print(f"[fullsize] C2 {label}: worst err/bound {worst:.3f}", flush=True)
        del c


# ------------------------------------------------------------------ C3
def resnet50_layers(batch):
    import plan_cases
    return plan_cases.resnet50_layers(batch)


def sample_forward(x, w, y, s, p, rng, per_image=128):
    """Sampled forward outputs of two images vs float64."""
    n, cin, H, W = x.shape
    cout, _, k, _ = w.shape
    _, _, OH, OW = y.shape
    wh = w.double().cpu().numpy()
    got, ref, mag = [], [], []
    for img in rng.choice(n, 2, replace=False):
        xp = np.pad(x[img].double().cpu().numpy(), ((0, 0), (p, p), (p, p)))
        co = rng.integers(0, cout, per_image)
        oh = rng.integers(0, OH, per_image)
        ow = rng.integers(0, OW, per_image)
        got.append(y[int(img)][torch.from_numpy(co).cuda(), torch.from_numpy(oh).cuda(),
                               torch.from_numpy(ow).cuda()].cpu().numpy())
        for c_, h_, w_ in zip(co, oh, ow):
            patch = xp[:, h_ * s:h_ * s + k, w_ * s:w_ * s + k]
            ref.append(float((patch * wh[c_]).sum()))
            mag.append(float((np.abs(patch) * np.abs(wh[c_])).sum()))
    return np.concatenate(got), np.array(ref), np.array(mag)


def sample_dinput(dy, w, dx, s, p, rng, per_image=128):
    n, cout, OH, OW = dy.shape
    _, cin, H, W = dx.shape
    k = w.shape[2]
    wh = w.double().cpu().numpy()
    got, ref, mag = [], [], []
    for img in rng.choice(n, 2, replace=False):
        dyh = dy[img].double().cpu().numpy()
        ci = rng.integers(0, cin, per_image)
        ih = rng.integers(0, H, per_image)
        iw = rng.integers(0, W, per_image)
        got.append(dx[int(img)][torch.from_numpy(ci).cuda(), torch.from_numpy(ih).cuda(),
                                torch.from_numpy(iw).cuda()].cpu().numpy())
        for c_, h_, w_ in zip(ci, ih, iw):
            r = m = 0.0
            for kh in range(k):
                th = h_ + p - kh
                if th < 0 or th % s or th // s >= OH:
                    continue
                for kw in range(k):
                    tw = w_ + p - kw
                    if tw < 0 or tw % s or tw // s >= OW:
                        continue
                    a, bb = dyh[:, th // s, tw // s], wh[:, c_, kh, kw]
                    r += float(a @ bb)
                    m += float(np.abs(a) @ np.abs(bb))
            ref.append(r)
            mag.append(m)
    return np.concatenate(got), np.array(ref), np.array(mag)


def sample_dweight(x, dy, dw, s, p, rng, nc=4):
    n, cin, H, W = x.shape
    _, cout, OH, OW = dy.shape
    k = dw.shape[2]
    cos = rng.choice(cout, min(nc, cout), replace=False)
    cis = rng.choice(cin, min(nc, cin), replace=False)
    xs = np.pad(x[:, torch.from_numpy(cis).cuda()].double().cpu().numpy(), ((0, 0), (0, 0), (p, p), (p, p)))
    dys = dy[:, torch.from_numpy(cos).cuda()].double().cpu().numpy()
    dwh = dw.cpu().numpy()
    got, ref, mag = [], [], []
    for a, co in enumerate(cos):
        for b_, ci in enumerate(cis):
            for kh in range(k):
                for kw in range(k):
                    xv = xs[:, b_, kh:kh + s * (OH - 1) + 1:s, kw:kw + s * (OW - 1) + 1:s]
                    dv = dys[:, a]
                    got.append(dwh[co, ci, kh, kw])
                    ref.append(float((xv * dv).sum()))
                    mag.append(float((np.abs(xv) * np.abs(dv)).sum()))
    return np.array(got), np.array(ref), np.array(mag)


def test_c3_conv_stack_full_size(mx):
    """All 53 ResNet-50 convolutions at batch 64, every phase bench.py times."""
    gen = torch.Generator(device="cuda").manual_seed(0)
    rng = np.random.default_rng(3)
    worst = {}
    for name, xs, cout, k, s, p in resnet50_layers(64):
        d = mx.conv_desc(xs, (cout, xs[1], k, k), (s, s), (p, p))
        x = torch.randn(xs, device="cuda", generator=gen)
        w = torch.randn((cout, xs[1], k, k), device="cuda", generator=gen) * math.sqrt(2.0 / (cout * k * k))
        dy = torch.randn((xs[0], cout, d.oh, d.ow), device="cuda", generator=gen)
        wino = k == 3 and s == 1
        algo = mx.ALGO_WINOGRAD if wino else mx.ALGO_IMPLICIT_GEMM
        rtol = WINOGRAD_RTOL if wino else RTOL
        y, dw = torch.empty_like(dy), torch.empty_like(w)
        mx.conv2d_forward(d, x, w, None, y, algo, stream())
        mx.conv2d_backward_weight(d, x, dy, dw, None, algo, stream())
        res = {"fwd": sample_forward(x, w, y, s, p, rng), "dw": sample_dweight(x, dy, dw, s, p, rng)}
        if name != "stem":
            dx = torch.empty_like(x)
            mx.conv2d_backward_input(d, dy, w, dx, algo, stream())
            res["dx"] = sample_dinput(dy, w, dx, s, p, rng)
        for phase, (got, ref, mag) in res.items():
            worst[f"{name}.{phase}"] = check_samples(got, ref, mag, rtol, f"C3 {name} {phase}")
        print(f"[fullsize] C3 {name}: " + " ".join(f"{ph} {worst[f'{name}.{ph}']:.3f}" for ph in res), flush=True)
        del x, w, dy, y, dw
        torch.cuda.empty_cache()
    assert len(worst) == 53 * 3 - 1


# ------------------------------------------------------------------ C4
def test_c4_unet_full_width_step(mx):
    """The C4 U-Net at its real configuration (base 128, 64 x 64, batch 16,
    the step bench.py times), on the "vulkan" device: loss and every gradient
    against float64 CPU, each within four times CPU FP32's own error plus 1e-6
    of the tensor's largest gradient."""
    import os

    import torch_vulkan  # noqa: F401
    import unet_c4 as U

    os.environ["TORCH_VULKAN_FORBID_CPU_FALLBACK"] = "1"
    try:
        torch.manual_seed(0)
        model = U.make_model()
        x, t = U.make_inputs(batch=16)
        ref = copy.deepcopy(model).double()
        loss_ref = U.train_step_loss(ref, x.double(), t.double())
        cpu32 = copy.deepcopy(model)
        loss32 = U.train_step_loss(cpu32, x, t)
        devm = copy.deepcopy(model).to("vulkan")
        loss = U.train_step_loss(devm, x.to("vulkan"), t.to("vulkan"))
        lr = loss_ref.item()
        assert abs(loss.item() - lr) <= 1e-4 * abs(lr), (loss.item(), lr)
        worst = 0.0
        for (name, p_ref), (_, p32), (_, p) in zip(ref.named_parameters(), cpu32.named_parameters(),
                                                   devm.named_parameters()):
            g_ref = p_ref.grad.double()
            scale = g_ref.abs().max().item()
            e32 = (p32.grad.double() - g_ref).abs().max().item()
            err = (p.grad.cpu().double() - g_ref).abs().max().item()
            bound = 4.0 * e32 + 1e-6 * scale
            worst = max(worst, err / bound if bound else 0.0)
            assert err <= bound, f"{name}: vulkan err {err:.3g}, CPU FP32 err {e32:.3g}, max |grad| {scale:.3g}"
        print(f"[fullsize] C4 loss {loss.item():.6f} (float64 {lr:.6f}, CPU FP32 {loss32.item():.6f}); "
              f"worst gradient error {worst:.3f} of bound", flush=True)
    finally:
        os.environ.pop("TORCH_VULKAN_FORBID_CPU_FALLBACK", None)


# ------------------------------------------------------------------ C5
def test_c5_adamw_full_size_bit_exact(mx):
    """250 tensors (125M elements, sizes log-uniform in [64, 4M] as bench.py
    draws them), 10 warm-up steps, then step 11 on the device and in the
    oracle from the same state: identical bits."""
    import oracle

    rng = np.random.default_rng(0)
    sizes = np.exp(rng.uniform(math.log(64), math.log(4194304), 250)).astype(np.int64)
    hp = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01)
    gen = torch.Generator(device="cuda").manual_seed(0)
    P = [torch.randn(int(n), device="cuda", generator=gen) * 0.02 for n in sizes]
    G = [torch.randn(int(n), device="cuda", generator=gen) * 1e-3 for n in sizes]
    M = [torch.zeros(int(n), device="cuda") for n in sizes]
    V = [torch.zeros(int(n), device="cuda") for n in sizes]
    for step in range(1, 11):
        mx.adamw_step(P, G, M, V, steps=[step] * 250, stream=stream(), **hp)
    host = [(p.cpu().numpy(), g.cpu().numpy(), m.cpu().numpy(), v.cpu().numpy()) for p, g, m, v in zip(P, G, M, V)]
    mx.adamw_step(P, G, M, V, steps=[11] * 250, stream=stream(), **hp)
    torch.cuda.synchronize()
    total = 0
    for i, (p, g, m, v) in enumerate(host):
        oracle.adamw_step(p, g, m, v, step=11, **hp)
        for name, dev, ref in (("param", P[i], p), ("exp_avg", M[i], m), ("exp_avg_sq", V[i], v)):
            got = dev.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
                f"tensor {i} ({ref.size} elements) {name}: {int((got != ref).sum())} elements differ"
        total += p.size
    assert total == int(sizes.sum())
    print(f"[fullsize] C5: {total} elements over 250 tensors bit-identical to the oracle", flush=True)
