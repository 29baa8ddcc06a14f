#!/usr/bin/env python
"""Benchmark of the MI355X FP32 conv / GEMM / fused-AdamW path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c3|c1|c4|c4ops|c5|copy] [--no-cpu-baseline]
    python bench.py --pmc-summary FETCH_DIR WRITE_DIR COPY_FETCH_DIR COPY_WRITE_DIR
    python bench.py --trace-summary KERNEL_TRACE_CSV BENCH_LOG
    python bench.py --stats-table KERNEL_STATS_OR_TRACE_CSV STEPS_RUN

Prints ONE JSON line.  The headline (`value`) is BASELINE.json's Conv2D
fwd+bwd FP32 TFLOP/s on its largest single-GPU Conv2D configuration, C3: the
53 convolutions of ResNet-50 v1.5 at batch 64, 224x224, each run forward +
dInput + dWeight (the stem needs no dInput), 3x3 stride-1 layers routed to
Winograd F(2x2,3x3) as the configuration states: their forwards, their
input gradients, which are 3x3 stride-1 convolutions of dy with the flipped
filter, and their weight gradients, the adjoint of the transform.  A "step" is one pass of
every layer; inputs are resident in HBM before timing.  `components` holds
C1 (single conv layer fwd+dX+dW+dB, every phase on Winograd; c1_implicit
the same on the implicit GEMM only), C2 (Linear addmm fwd+bwd, 8192x4096x4096),
C5 (multi-tensor AdamW, 250 tensors, GB/s), C4 (the diffusion U-Net training
step on the "vulkan" device, TFLOP/s of its convolutions and bmm over the
whole step), c4_ops (its normalisation / activation kernels, GB/s) and
streams (copy / compute overlap across HIP streams on the "vulkan" device).

Every kernel runs through the C ABI (libmx.so, include/mx.h); torch ROCm
tensors only provide device memory and the stream.  `roofline` is measured
live with HIP events around every launch of the timed steps, on the stream the
kernels run on; `cpu_baseline` (and each component's) is CPU PyTorch (the
reference's CPU implementation of these ops) on a bounded sample of the same
workload, with torch's threads set to every core in the process's affinity
mask and the CPU model recorded.

`roofline.traffic` (HBM bytes per launch of the dominant kernel) comes from
two rocprofv3 PMC passes over this script (FETCH_SIZE, then WRITE_SIZE, KiB
per dispatch), each scaled by what the same counter reads for a plain copy of
known size (`--workload copy`); `--pmc-summary` turns the four passes into
profiles/traffic_c3.json, which the headline run reads.  Without that file
traffic is null.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from collections import defaultdict

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "pytorch-vulkan_amd"))

PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(REPO, "profiles", "traffic_c3.json")
TRAFFIC_C5_FILE = os.path.join(REPO, "profiles", "traffic_c5.json")
COPY_FLOATS = 256 * 1024 * 1024  # calibration copy: 1 GiB read, 1 GiB written
METRIC = "Conv2D fwd+bwd FP32 TFLOP/s & % MFMA peak; fused AdamW GB/s; 1 MI355X"


# ------------------------------------------------------------------ workloads
def resnet50_convs(batch: int):
    """(name, x_shape, cout, k, stride, pad) for the 53 ResNet-50 v1.5 convolutions."""
    layers = [("stem", (batch, 3, 224, 224), 64, 7, 2, 3)]
    cin, size = 64, 56
    for stage, (width, blocks) in enumerate([(64, 3), (128, 4), (256, 6), (512, 3)]):
        out = width * 4
        for b in range(blocks):
            s = 2 if (b == 0 and stage > 0) else 1
            pre = f"layer{stage + 1}.{b}"
            layers.append((f"{pre}.conv1", (batch, cin, size, size), width, 1, 1, 0))
            layers.append((f"{pre}.conv2", (batch, width, size, size), width, 3, s, 1))
            osz = size // s
            layers.append((f"{pre}.conv3", (batch, width, osz, osz), out, 1, 1, 0))
            if b == 0:
                layers.append((f"{pre}.downsample", (batch, cin, size, size), out, 1, s, 0))
            cin, size = out, osz
    return layers


def conv_flops(xs, cout, k, stride, pad):
    oh = (xs[2] + 2 * pad - k) // stride + 1
    ow = (xs[3] + 2 * pad - k) // stride + 1
    return 2.0 * xs[0] * cout * oh * ow * xs[1] * k * k, (oh, ow)


def winograd_flops(xs, cout):
    """FLOPs the F(2x2,3x3) kernels execute for one phase of a 3x3 stride-1
    pad-1 layer: 16 products of Cin x Cout per 2x2 output tile (the forward,
    the flipped-filter input gradient and the adjoint weight gradient alike)."""
    tiles = xs[0] * ((xs[2] + 1) // 2) * ((xs[3] + 1) // 2)
    return 2.0 * 16 * tiles * xs[1] * cout


class Launcher:
    """Runs ABI calls on one stream, optionally bracketing each with HIP events."""

    def __init__(self, mx, stream):
        self.mx = mx
        self.stream = stream
        self.timing = False
        self.pending = []  # (label, flops, bytes, start, end)

    def run(self, label, flops, nbytes, fn):
        if not self.timing:
            fn()
            return
        s, e = self.mx.Event(), self.mx.Event()
        s.record(self.stream)
        fn()
        e.record(self.stream)
        self.pending.append((label, flops, nbytes, s, e))

    def collect(self):
        agg = defaultdict(lambda: [0, 0.0, 0.0, 0.0])  # launches, ms, flops, bytes
        for label, flops, nbytes, s, e in self.pending:
            a = agg[label]
            a[0] += 1
            a[1] += s.elapsed_ms(e)
            a[2] += flops
            a[3] += nbytes
        self.pending = []
        return agg


def build_c3(torch, mx, L, batch, winograd=True):
    """Per-layer buffers and the list of launches of one C3 step, its
    direct-convolution FLOPs and the FLOPs its kernels execute (Winograd
    phases count their 16 products per tile)."""
    g = torch.Generator(device="cuda").manual_seed(0)
    calls, total, executed = [], 0.0, 0.0
    for name, xs, cout, k, stride, pad in resnet50_convs(batch):
        flops, (oh, ow) = conv_flops(xs, cout, k, stride, pad)
        d = mx.conv_desc(xs, (cout, xs[1], k, k), (stride, stride), (pad, pad))
        x = torch.randn(xs, device="cuda", generator=g)
        w = torch.randn((cout, xs[1], k, k), device="cuda", generator=g) * math.sqrt(2.0 / (cout * k * k))
        dy = torch.randn((xs[0], cout, oh, ow), device="cuda", generator=g)
        y, dw = torch.empty_like(dy), torch.empty_like(w)
        dx = torch.empty_like(x) if name != "stem" else None
        fwd_algo = mx.ALGO_WINOGRAD if (winograd and k == 3 and stride == 1) else mx.ALGO_IMPLICIT_GEMM
        phase_flops = winograd_flops(xs, cout) if fwd_algo == mx.ALGO_WINOGRAD else flops
        fname = ("winograd_forward" if fwd_algo == mx.ALGO_WINOGRAD
                 else mx.conv2d_kernel_name(d, mx.MX_CONV_FORWARD, fwd_algo))
        st = L.stream
        calls.append((fname, flops, 0, lambda d=d, x=x, w=w, y=y, a=fwd_algo: mx.conv2d_forward(d, x, w, None, y, a, st)))
        if dx is not None:
            # The input gradient of a 3x3 stride-1 layer is itself a 3x3
            # stride-1 convolution (of dy with the flipped filter): Winograd too.
            dx_algo = fwd_algo
            dname = ("winograd_dinput" if dx_algo == mx.ALGO_WINOGRAD
                     else mx.conv2d_kernel_name(d, mx.MX_CONV_DINPUT, dx_algo))
            calls.append((dname, flops, 0,
                          lambda d=d, dy=dy, w=w, dx=dx, a=dx_algo: mx.conv2d_backward_input(d, dy, w, dx, a, st)))
            total += flops
            executed += phase_flops
        # ... and so is its weight gradient, through the adjoint of the transform.
        dw_algo = fwd_algo
        wname = ("winograd_dweight" if dw_algo == mx.ALGO_WINOGRAD
                 else mx.conv2d_kernel_name(d, mx.MX_CONV_DWEIGHT, dw_algo))
        calls.append((wname, flops, 0,
                      lambda d=d, x=x, dy=dy, dw=dw, a=dw_algo: mx.conv2d_backward_weight(d, x, dy, dw, None, a, st)))
        total += 2 * flops
        executed += 2 * phase_flops
    return calls, total, executed


# C1 routing: forward and dInput (both 3x3 stride-1 correlations) and the
# weight gradient (the transform's adjoint, dBias in the same launch) on
# Winograd F(2x2,3x3), the fastest correct kernels for this layer (rel 1e-3
# parity).  C1_IMPLICIT keeps every phase on the implicit GEMM (rel 1e-4
# parity) for comparison.
C1_ROUTED = ("winograd", "winograd", "winograd")
C1_IMPLICIT = ("implicit_gemm", "implicit_gemm", "implicit_gemm")


def build_c1(torch, mx, L, routing=C1_ROUTED):
    g = torch.Generator().manual_seed(0)
    xs, cout = (8, 64, 56, 56), 64
    x = torch.randn(xs, generator=g)
    w = torch.empty(cout, 64, 3, 3)
    torch.nn.init.kaiming_uniform_(w, a=math.sqrt(5), generator=g)
    b = torch.empty(cout).uniform_(-1 / 24, 1 / 24, generator=g)
    dy = torch.randn(8, cout, 56, 56, generator=g)
    host = dict(x=x, w=w, b=b, dy=dy)
    X, W, B, DY = (t.cuda() for t in (x, w, b, dy))
    d = mx.conv_desc(xs, w.shape, (1, 1), (1, 1))
    Y, DX, DW, DB = torch.empty_like(DY), torch.empty_like(X), torch.empty_like(W), torch.empty_like(B)
    flops, _ = conv_flops(xs, cout, 3, 1, 1)
    st = L.stream
    code = {"winograd": mx.ALGO_WINOGRAD, "implicit_gemm": mx.ALGO_IMPLICIT_GEMM}
    af, ax, aw = (code[a] for a in routing)

    def label(phase, algo, wino_name):
        return wino_name if algo == mx.ALGO_WINOGRAD else mx.conv2d_kernel_name(d, phase, algo)

    # The backward is one library call (dx, dw, db), as the reference's
    # convolution_backward is one operator; with both gradients on Winograd
    # it is one launch for this layer.
    calls = [(label(mx.MX_CONV_FORWARD, af, "winograd_forward"), flops, 0,
              lambda: mx.conv2d_forward(d, X, W, B, Y, af, st))]
    if ax == aw == mx.ALGO_WINOGRAD:
        calls.append(("winograd_backward", 2 * flops, 0,
                      lambda: mx.conv2d_backward(d, X, W, DY, DX, DW, DB, ax, aw, st)))
    else:  # the same two launches mx_conv2d_backward makes, timed apart
        calls += [(label(mx.MX_CONV_DINPUT, ax, "winograd_dinput"), flops, 0,
                   lambda: mx.conv2d_backward_input(d, DY, W, DX, ax, st)),
                  (label(mx.MX_CONV_DWEIGHT, aw, "winograd_dweight"), flops, 0,
                   lambda: mx.conv2d_backward_weight(d, X, DY, DW, DB, aw, st))]
    executed = sum(winograd_flops(xs, cout) if a == mx.ALGO_WINOGRAD else flops for a in (af, ax, aw))
    return calls, 3 * flops, host, dict(y=Y, dx=DX, dw=DW, db=DB), executed


def build_c2(torch, mx, L):
    g = torch.Generator(device="cuda").manual_seed(0)
    M, K, N = 8192, 4096, 4096
    X = torch.randn(M, K, device="cuda", generator=g)
    W = (torch.rand(N, K, device="cuda", generator=g) * 2 - 1) / 64
    b = (torch.rand(N, device="cuda", generator=g) * 2 - 1) / 64
    dY = torch.randn(M, N, device="cuda", generator=g)
    Y, dX, dW, db = torch.empty(M, N, device="cuda"), torch.empty_like(X), torch.empty_like(W), torch.empty_like(b)
    f = 2.0 * M * N * K
    st = L.stream
    calls = [
        ("gemm addmm X.W^T+b", f, 0, lambda: mx.gemm(X, W.t(), Y, bias=b, beta=1.0, stream=st)),
        ("gemm dX=dY.W", f, 0, lambda: mx.gemm(dY, W, dX, stream=st)),
        ("gemm dW=dY^T.X", f, 0, lambda: mx.gemm(dY.t(), X, dW, stream=st)),
        ("sum db=dY.sum(0)", 0, 4.0 * M * N, lambda: mx.sum_mid(db, dY, 1, M, N, st)),
    ]
    return calls, 3 * f


def build_c5(torch, mx, L):
    import numpy as np
    rng = np.random.default_rng(0)
    sizes = np.exp(rng.uniform(math.log(64), math.log(4194304), 250)).astype(np.int64)
    g = torch.Generator(device="cuda").manual_seed(0)
    P = [torch.randn(int(n), device="cuda", generator=g) * 0.02 for n in sizes]
    G = [torch.randn(int(n), device="cuda", generator=g) * 1e-3 for n in sizes]
    M = [torch.zeros(int(n), device="cuda") for n in sizes]
    V = [torch.zeros(int(n), device="cuda") for n in sizes]
    numel = int(sizes.sum())
    state = {"step": 0}
    st = L.stream

    def step():
        state["step"] += 1
        mx.adamw_step(P, G, M, V, lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01,
                      steps=[state["step"]] * len(P), stream=st)

    for _ in range(10):  # warm the moments as the configuration states
        step()
    return [("adamw_kernel", 0, 28.0 * numel, step)], numel, sizes


def build_c4_ops(torch, mx, L):
    """The normalisation / activation / resampling / softmax kernels of the C4
    step at its largest shapes, each launch priced at its algorithmic HBM
    bytes (every input read once, every output written once)."""
    g = torch.Generator(device="cuda").manual_seed(0)
    st = L.stream
    big = (16, 128, 64, 64)  # level-0 activations
    n = math.prod(big)
    x = torch.randn(big, device="cuda", generator=g) * 2 + 0.5
    dy = torch.randn(big, device="cuda", generator=g)
    y = torch.empty_like(x)
    dx = torch.empty_like(x)
    gamma = torch.rand(128, device="cuda", generator=g) + 0.5
    beta = torch.randn(128, device="cuda", generator=g)
    mean = torch.empty(16, 32, device="cuda")
    rstd = torch.empty(16, 32, device="cuda")
    dg = torch.empty(128, device="cuda")
    db = torch.empty(128, device="cuda")
    up_in = torch.randn(16, 256, 32, 32, device="cuda", generator=g)  # upsample into level 0
    up_out = torch.empty(16, 256, 64, 64, device="cuda")
    up_grad = torch.empty_like(up_in)
    att = torch.randn(64, 256, 256, device="cuda", generator=g) * 3  # attention scores at 16x16
    att_y = torch.empty_like(att)
    att_dx = torch.empty_like(att)
    att_dy = torch.randn(64, 256, 256, device="cuda", generator=g)
    mx.group_norm_forward(x, gamma, beta, 32, 1e-5, y, mean, rstd, stream=st)
    calls = [
        ("group_norm_forward", 0, 8.0 * n,
         lambda: mx.group_norm_forward(x, gamma, beta, 32, 1e-5, y, mean, rstd, stream=st)),
        ("group_norm_backward", 0, 12.0 * n,
         lambda: mx.group_norm_backward(dy, x, mean, rstd, gamma, 32, dx, dg, db, stream=st)),
        ("silu_forward", 0, 8.0 * n, lambda: mx.unary(mx.UNARY_SILU, x, y, stream=st)),
        ("silu_backward", 0, 12.0 * n, lambda: mx.unary_backward(mx.UNARY_SILU_GRAD, dy, x, dx, stream=st)),
        ("upsample_nearest2d", 0, 4.0 * (up_in.numel() + up_out.numel()),
         lambda: mx.upsample_nearest2d(up_in, up_out, 2.0, 2.0, stream=st)),
        ("upsample_nearest2d_backward", 0, 4.0 * (up_in.numel() + up_out.numel()),
         lambda: mx.upsample_nearest2d_backward(up_out, up_grad, 2.0, 2.0, stream=st)),
        ("softmax_forward", 0, 8.0 * att.numel(), lambda: mx.softmax(att, -1, att_y, stream=st)),
        ("softmax_backward", 0, 12.0 * att.numel(), lambda: mx.softmax_backward(att_dy, att_y, -1, att_dx, stream=st)),
    ]
    return calls


def run_c4_ops(torch, mx, L):
    """Each C4 normalisation / activation op at its largest shape: 20 calls
    back to back between one pair of HIP events, priced at its algorithmic
    bytes."""
    ops = {}
    for label, _, nbytes, fn in build_c4_ops(torch, mx, L):
        us = back_to_back_us(torch, fn, 20, 3)
        gbs = nbytes / (us * 1e-6) / 1e9
        ops[label] = {"avg_us": round(us, 2), "algorithmic_gb_s": round(gbs, 1),
                      "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    return {"workload": "C4 normalisation / activation kernels at the step's largest shapes: GroupNorm32 and SiLU "
                        "on 16x128x64x64, 2x nearest 16x256x32x32->64x64, softmax over 64x256x256 scores; per op "
                        "20 back-to-back calls between one pair of HIP events (a call's launches and the gaps "
                        "between them), algorithmic bytes (inputs read once, outputs written once)", "ops": ops}


def run_c4(torch, steps, warmup, log):
    """The C4 U-Net training step (forward, MSE loss, backward, fused AdamW) on
    the "vulkan" device at batch 16, 64x64; GEMM FLOPs of convolutions and
    attention bmm over the whole step time."""
    import torch_vulkan as tv
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import unet_c4 as U
    model = U.make_model().to("vulkan")
    x, t = U.make_inputs()
    x, t = x.to("vulkan"), t.to("vulkan")
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, weight_decay=0.01, fused=True)
    flops = U.step_flops(model, x)

    def step():
        U.train_step_loss(model, x, t)
        opt.step()

    for _ in range(warmup):
        step()
    tv.synchronize()
    before = tv.execution_stats()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    tv.synchronize()
    dt = (time.perf_counter() - t0) / steps
    after = tv.execution_stats()
    fallbacks = after["cpu_fallback_calls"] - before["cpu_fallback_calls"]
    reads = after["host_reads"] - before["host_reads"]
    params = sum(p.numel() for p in model.parameters())
    out = {"workload": "C4: diffusion U-Net training step (GroupNorm32/SiLU ResBlocks, width 128 x (1,2,2,4), "
                       "4-head bmm attention at 16x16, MSE, fused AdamW), batch 16, 3x64x64, on the vulkan device",
           "ms_per_step": round(dt * 1e3, 3), "value": round(flops / dt / 1e12, 3), "unit": "TFLOP/s",
           "gflop_per_step": round(flops / 1e9, 1), "params": params,
           "cpu_fallback_calls_per_step": fallbacks / steps, "host_reads_per_step": reads / steps}
    out.update(c4_kernel_table(tv, step, steps))
    del model, opt, x, t
    return out


def c4_kernel_table(tv, step, steps):
    """The same training steps again with HIP events around every
    convolution, GEMM / bmm and AdamW call on its stream
    (TORCH_VULKAN_PROFILE_TIMESTAMPS=1): per kernel label the calls per step,
    time per call and algorithmic TFLOP/s (direct-convolution / 2*M*N*K
    FLOPs of the phases the call computes), the conv/GEMM kernel-summed rate
    and the roofline of the kernel that takes the most time.  A call's time
    covers all of its dispatches (weight packing, split-K sums)."""
    os.environ["TORCH_VULKAN_PROFILE_TIMESTAMPS"] = "1"
    try:
        step()
        tv.synchronize()
        tv.reset_gpu_timing_stats()
        for _ in range(steps):
            step()
        tv.synchronize()
        stats = tv.gpu_timing_stats()
    finally:
        os.environ.pop("TORCH_VULKAN_PROFILE_TIMESTAMPS", None)
        tv.reset_gpu_timing_stats()
    rows = []
    for name, v in stats.items():
        if not v["samples"]:
            continue
        ms = v["shader_ms"]
        ex = v.get("executed_flops", v["flops"])
        row = {"kernel": name, "calls_per_step": round(v["samples"] / steps, 2),
               "ms_per_step": round(ms / steps, 4), "avg_us": round(1000 * ms / v["samples"], 2)}
        if v["flops"] > 0 and ms > 0:
            # tflop_s at direct-convolution / GEMM FLOPs; the fraction of peak
            # at the FLOPs the kernels execute (Winograd: 16 products per 2x2
            # tile instead of 36).
            row["tflop_s"] = round(v["flops"] / (ms * 1e-3) / 1e12, 3)
            row["executed_tflop_s"] = round(ex / (ms * 1e-3) / 1e12, 3)
            row["frac_of_fp32_peak"] = round(row["executed_tflop_s"] / PEAK_FP32_TFLOPS, 4)
        rows.append((ms, v["flops"], v["samples"], row, ex))
    rows.sort(key=lambda r: -r[0])
    mm = [r for r in rows if r[1] > 0]
    gemm_ms = sum(r[0] for r in mm)
    gemm_flops = sum(r[1] for r in mm)
    gemm_exec = sum(r[4] for r in mm)
    res = {"kernel_table": [r[3] for r in rows[:16]],
           "timed_ms_per_step": round(sum(r[0] for r in rows) / steps, 3),
           "conv_gemm_ms_per_step": round(gemm_ms / steps, 3)}
    if mm:
        ms, fl, n, row, ex = mm[0]
        achieved = ex / n / (ms / n * 1e-3) / 1e12
        res["conv_gemm_kernel_tflop_s"] = round(gemm_flops / (gemm_ms * 1e-3) / 1e12, 3)
        res["conv_gemm_executed_tflop_s"] = round(gemm_exec / (gemm_ms * 1e-3) / 1e12, 3)
        res["conv_gemm_frac_of_fp32_peak_executed"] = round(res["conv_gemm_executed_tflop_s"] / PEAK_FP32_TFLOPS, 4)
        res["roofline"] = {"bound": "mfma", "kernel": row["kernel"], "achieved": round(achieved, 3),
                           "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
                           "flops_counted": "executed (Winograd: 16 products per 2x2 tile)",
                           "traffic": None, "launches": n, "avg_launch_us": row["avg_us"],
                           "timing": "HIP events around each call on its stream"}
    return res


def run_streams(torch, reps=5):
    """Copy / compute overlap on the "vulkan" device: a 256 MiB upload from
    page-locked host memory (non_blocking) on a copy stream beside two one-tile
    GEMMs (64x64 output, K = 2^19: one workgroup for milliseconds) on a
    compute stream, then two such GEMMs on two streams.  Each figure is the
    best of `reps` runs timed on the host between device synchronisations."""
    import torch_vulkan as tv

    def timed(fn):
        best = float("inf")
        for _ in range(reps):
            tv.synchronize()
            t0 = time.perf_counter()
            fn()
            tv.synchronize()
            best = min(best, time.perf_counter() - t0)
        return 1e3 * best

    g = torch.Generator().manual_seed(3)
    a = torch.randn(64, 1 << 19, generator=g).to("vulkan")
    b = torch.randn(1 << 19, 64, generator=g).to("vulkan")
    host = torch.randn(64 << 20, generator=g).pin_memory()
    dst = torch.empty(64 << 20, device="vulkan")
    s1, s2 = tv.Stream(), tv.Stream()
    for s in (s1, s2):
        s.wait_stream(tv.current_stream())

    def upload():
        with tv.stream(s2):
            dst.copy_(host, non_blocking=True)

    def gemms(streams):
        for s in streams:
            with tv.stream(s):
                a @ b

    t_copy = timed(upload)
    t_gemm = timed(lambda: gemms((s1, s1)))
    t_both = timed(lambda: (upload(), gemms((s1, s1))))
    t_two = timed(lambda: gemms((s1, s2)))
    out = {"workload": "stream overlap: 256 MiB non_blocking upload from pinned memory on a copy stream beside "
                       "two one-tile GEMMs (64x64, K=2^19) on a compute stream; then the two GEMMs on two streams",
           "copy_ms": round(t_copy, 3), "h2d_gb_s": round(4 * (64 << 20) / (t_copy * 1e-3) / 1e9, 1),
           "gemms_one_stream_ms": round(t_gemm, 3), "copy_beside_gemms_ms": round(t_both, 3),
           "copy_hidden_frac": round((t_copy + t_gemm - t_both) / t_copy, 3),
           "gemms_two_streams_ms": round(t_two, 3), "two_stream_speedup": round(t_gemm / t_two, 3)}
    del a, b, host, dst
    return out


def run_stream_probes(torch, numel, reps=20):
    """The AdamW access pattern with trivial arithmetic (4 reads + 3 writes per
    element, in place), the same pattern with AdamW's per-element update, a
    plain copy and a 4-stream read sweep over buffers of C5's size, from
    libmxprobe.so; GB/s from HIP events on the current stream."""
    import ctypes as C
    lib = C.CDLL(os.path.join(REPO, "libmxprobe.so"))
    lib.mxp_stream.argtypes = [C.c_int, C.POINTER(C.c_void_p), C.c_int64, C.c_int, C.c_void_p]
    lib.mxp_stream.restype = C.c_int
    n = numel // 4096 * 4096
    bufs = [torch.full((n,), 0.5, device="cuda") for _ in range(4)] + [torch.empty(1 << 16, device="cuda")]
    ptrs = (C.c_void_p * 5)(*[b.data_ptr() for b in bufs])
    st = torch.cuda.current_stream()
    out = {}
    for name, kind, bpe in (("adamw_mix_4r3w", 2, 28), ("adamw_math_4r3w", 3, 28), ("copy", 0, 8),
                            ("read_4_streams", 1, 16)):
        for _ in range(3):
            assert lib.mxp_stream(kind, ptrs, n, 32, st.cuda_stream) == 0
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(reps):
            lib.mxp_stream(kind, ptrs, n, 32, st.cuda_stream)
        e1.record(st)
        e1.synchronize()
        out[name] = round(bpe * n / (e0.elapsed_time(e1) / reps * 1e-3) / 1e9, 1)
    del bufs
    torch.cuda.empty_cache()
    return out


def run_probe_sweep(torch, numel, reps=20):
    """The 4-read / 3-write in-place mix of run_stream_probes over buffers of
    C5's size under each memory schedule of libmxprobe.so's mxp_mix_sweep:
    float4 per stream per thread per chunk (vec), next chunk's loads before
    this chunk's stores (prefetch), contiguous runs of chunks per workgroup
    instead of round-robin (contig), and workgroups per CU.  GB/s counts 28
    bytes per element; rows sorted fastest first."""
    import ctypes as C
    lib = C.CDLL(os.path.join(REPO, "libmxprobe.so"))
    lib.mxp_mix_sweep.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_void_p), C.c_int64, C.c_int, C.c_void_p]
    lib.mxp_mix_sweep.restype = C.c_int
    n = numel // 8192 * 8192
    bufs = [torch.full((n,), 0.5, device="cuda") for _ in range(4)]
    ptrs = (C.c_void_p * 4)(*[b.data_ptr() for b in bufs])
    st = torch.cuda.current_stream()
    rows = []
    for vec in (1, 2, 4, 8):
        for prefetch in (0, 1):
            for contig in (0, 1):
                for per_cu in (1, 2, 4, 8, 16, 32):
                    for _ in range(3):
                        assert lib.mxp_mix_sweep(vec, prefetch, contig, ptrs, n, per_cu, st.cuda_stream) == 0
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(st)
                    for _ in range(reps):
                        lib.mxp_mix_sweep(vec, prefetch, contig, ptrs, n, per_cu, st.cuda_stream)
                    e1.record(st)
                    e1.synchronize()
                    rows.append({"vec": vec, "prefetch": prefetch, "contig": contig, "wg_per_cu": per_cu,
                                 "gb_s": round(28 * n / (e0.elapsed_time(e1) / reps * 1e-3) / 1e9, 1)})
    del bufs
    torch.cuda.empty_cache()
    return {"elements": n, "reps": reps, "rows": sorted(rows, key=lambda r: -r["gb_s"])}


def rule_sweep_layers(kind):
    """3x3 layers for run_rule_sweep as (batch, height, width, cin, cout,
    padding).  "grid": square images, padding 1, power-of-two channels, at
    most 1.2e9 multiply-adds per filter tap.  "random": 70 seeded layers with
    non-square images, padding 0 / 1 / 2 and channel counts that are not
    powers of two."""
    import itertools
    import random
    if kind == "grid":
        shapes = [(1, 14), (4, 7), (2, 8), (1, 16), (2, 14), (8, 7), (4, 16), (4, 14), (16, 8), (8, 16), (8, 14),
                  (16, 16), (8, 28), (16, 28), (8, 56), (16, 56), (32, 56)]
        out = []
        for (n, hw), ci, co in itertools.product(shapes, (32, 64, 128, 256, 512, 1024), (32, 64, 128, 256, 512)):
            if 2e6 <= n * hw * hw * ci * co <= 1.2e9:
                out.append((n, hw, hw, ci, co, 1))
        return out
    rng = random.Random(11)
    out = []
    while len(out) < 70:
        n = rng.choice([1, 2, 3, 4, 6, 8, 12, 16, 24])
        h = rng.choice([6, 9, 10, 12, 15, 20, 24, 30, 40])
        w = rng.choice([h, h + 3, max(4, h - 2)])
        ci, co = rng.choice([48, 96, 192, 384, 768]), rng.choice([48, 96, 192, 384, 768])
        pad = rng.choice([1, 1, 1, 0, 2])
        pos = n * (h + 2 * pad - 2) * (w + 2 * pad - 2)
        if 200 <= pos <= 40000 and pos * ci * co <= 1.5e9:
            out.append((n, h, w, ci, co, pad))
    return out


def run_rule_sweep(torch, mx, kind):
    """AUTO's Winograd rule for 3x3 stride-1 layers against both algorithms
    forced: per layer and phase the kernel time of the implicit GEMM and of
    Winograd (best of 3 rounds of 5 back-to-back calls) and the algorithm
    AUTO selects; then, per phase, the summed time of AUTO's choices and of a
    plain position cut (1024 positions for the forward / input gradient, 2048
    for the weight gradient) as a percentage above the per-layer best."""
    st = torch.cuda.current_stream().cuda_stream
    phases = {"fwd": mx.MX_CONV_FORWARD, "dx": mx.MX_CONV_DINPUT, "dw": mx.MX_CONV_DWEIGHT}
    totals = {p: [0.0, 0.0, 0.0] for p in phases}  # best, auto, position cut

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        best = 1e9
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(300_000)
            e0.record()
            for _ in range(5):
                fn()
            e1.record()
            e1.synchronize()
            best = min(best, e0.elapsed_time(e1) / 5 * 1e3)
        return best

    for n, h, w, ci, co, pad in rule_sweep_layers(kind):
        d = mx.conv_desc((n, ci, h, w), (co, ci, 3, 3), (1, 1), (pad, pad))
        x = torch.randn(n, ci, h, w, device="cuda")
        wt = torch.randn(co, ci, 3, 3, device="cuda") * 0.05
        y = torch.empty(n, co, d.oh, d.ow, device="cuda")
        dy, dx = torch.randn_like(y), torch.empty_like(x)
        dw, db = torch.empty_like(wt), torch.empty(co, device="cuda")
        calls = {"fwd": lambda a: mx.conv2d_forward(d, x, wt, None, y, a, st),
                 "dx": lambda a: mx.conv2d_backward_input(d, dy, wt, dx, a, st),
                 "dw": lambda a: mx.conv2d_backward_weight(d, x, dy, dw, db, a, st)}
        pos = n * d.oh * d.ow
        row = {"n": n, "h": h, "w": w, "cin": ci, "cout": co, "pad": pad, "positions": pos}
        for name, phase in phases.items():
            ig = timed(lambda: calls[name](mx.ALGO_IMPLICIT_GEMM))
            wi = timed(lambda: calls[name](mx.ALGO_WINOGRAD))
            auto_wino = mx.conv2d_select(d, phase) == mx.ALGO_WINOGRAD
            cut_wino = pos >= (2048 if name == "dw" else 1024)
            t = totals[name]
            t[0] += min(ig, wi)
            t[1] += wi if auto_wino else ig
            t[2] += wi if cut_wino else ig
            row[name] = {"implicit_gemm_us": round(ig, 1), "winograd_us": round(wi, 1),
                         "auto": "winograd" if auto_wino else "implicit_gemm"}
        print(json.dumps(row), flush=True)
    return {"sweep": kind, "above_best_pct": {p: {"auto": round(100 * (t[1] / t[0] - 1), 2),
                                                  "position_cut": round(100 * (t[2] / t[0] - 1), 2)}
                                              for p, t in totals.items()}}


def plan_sweep_layers():
    """(x shape, cout, k, stride, pad, source) of the planner sweep: the 53
    ResNet-50 convolutions at batch 64 (C3) and the small C1 / C4 layers."""
    layers = {}
    for _, xs, cout, k, stride, pad in resnet50_convs(64):
        layers.setdefault((xs, cout, k, stride, pad), "c3")
    for xs, co, k, s, pad in [((8, 64, 56, 56), 64, 3, 1, 1), ((16, 256, 16, 16), 768, 1, 1, 0),
                              ((16, 768, 16, 16), 256, 1, 1, 0), ((16, 256, 8, 8), 512, 1, 1, 0),
                              ((16, 1024, 8, 8), 512, 1, 1, 0), ((16, 128, 64, 64), 128, 3, 2, 1),
                              ((16, 256, 16, 16), 256, 3, 2, 1), ((16, 256, 16, 16), 256, 1, 1, 0),
                              ((16, 384, 64, 64), 128, 1, 1, 0), ((16, 512, 32, 32), 256, 1, 1, 0),
                              ((16, 256, 32, 32), 256, 3, 2, 1), ((16, 128, 32, 32), 256, 1, 1, 0),
                              ((16, 256, 16, 16), 512, 1, 1, 0)]:
        layers.setdefault((xs, co, k, s, pad), "small")
    return [(*key, src) for key, src in layers.items()]


def run_blas_compare(torch, mx):
    """Each distinct 1x1 stride-1 layer of C3 (batch 64) run two ways on the
    same operands, best of 3 rounds of 20 back-to-back calls: the forward and
    the input gradient through this library's implicit GEMM, and the same
    products as torch.matmul batched over the images (hipBLASLt on this
    image): y[n] = W x[n] and dx[n] = W^T dy[n].  Reports per-layer times,
    TFLOP/s and the largest difference between the two results."""
    st = torch.cuda.current_stream().cuda_stream

    def timed(fn, n=20):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        best = 1e9
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(n):
                fn()
            e1.record()
            e1.synchronize()
            best = min(best, e0.elapsed_time(e1) / n * 1e3)
        return best

    rows, seen = [], set()
    sums = defaultdict(float)
    for name, xs, cout, k, stride, pad in resnet50_convs(64):
        if k != 1 or stride != 1 or (xs, cout) in seen:
            continue
        seen.add((xs, cout))
        n, cin, h, w = xs
        g = torch.Generator(device="cuda").manual_seed(len(rows))
        x = torch.randn(xs, device="cuda", generator=g)
        wt = torch.randn(cout, cin, device="cuda", generator=g) / math.sqrt(cin)
        dy = torch.randn(n, cout, h, w, device="cuda", generator=g)
        d = mx.conv_desc(xs, (cout, cin, 1, 1), (1, 1), (0, 0))
        w4 = wt.view(cout, cin, 1, 1)
        y, y_ref = torch.empty_like(dy), torch.empty_like(dy)
        dx, dx_ref = torch.empty_like(x), torch.empty_like(x)
        wT = wt.t().contiguous()
        t = {"fwd_ours_us": timed(lambda: mx.conv2d_forward(d, x, w4, None, y, mx.ALGO_IMPLICIT_GEMM, st)),
             "fwd_blas_us": timed(lambda: torch.matmul(wt, x.view(n, cin, h * w), out=y_ref.view(n, cout, h * w))),
             "dx_ours_us": timed(lambda: mx.conv2d_backward_input(d, dy, w4, dx, mx.ALGO_IMPLICIT_GEMM, st)),
             "dx_blas_us": timed(lambda: torch.matmul(wT, dy.view(n, cout, h * w), out=dx_ref.view(n, cin, h * w)))}
        flops = 2.0 * n * h * w * cin * cout
        row = {"layer": name, "shape": f"{cin}->{cout} {h}x{w}", "gflop": round(flops / 1e9, 3)}
        for key, us in t.items():
            row[key] = round(us, 1)
            row[key.replace("_us", "_tflops")] = round(flops / us / 1e6, 1)
            sums[key] += us
        row["fwd_max_diff"] = float((y - y_ref).abs().max())
        row["dx_max_diff"] = float((dx - dx_ref).abs().max())
        rows.append(row)
        print(json.dumps(row), flush=True)
        del x, dy, y, y_ref, dx, dx_ref
    return {"metric": "1x1 conv: implicit GEMM vs torch.matmul (hipBLASLt)", "layers": rows,
            "sums_us": {k: round(v, 1) for k, v in sums.items()}}


def miopen_c3_step(torch, find, progress=True):
    """The C3 step (53 layers, forward + dInput + dWeight, batch 64) through
    PyTorch-ROCm's own convolutions, which call MIOpen: immediate mode
    (torch's default heuristics) or, with `find`, cudnn.benchmark = True
    (every layer's solvers searched on its first call; several minutes, one
    progress line per layer on stderr).  Returns (best ms per step over 3
    rounds of 5 steps, setup seconds, the step function)."""
    torch.backends.cudnn.benchmark = bool(find)
    g = torch.Generator(device="cuda").manual_seed(0)
    layers = []
    for name, xs, cout, k, stride, pad in resnet50_convs(64):
        oh = (xs[2] + 2 * pad - k) // stride + 1
        x = torch.randn(xs, device="cuda", generator=g)
        w = torch.randn((cout, xs[1], k, k), device="cuda", generator=g) * math.sqrt(2.0 / (cout * k * k))
        dy = torch.randn((xs[0], cout, oh, oh), device="cuda", generator=g)
        layers.append((name, x, w, dy, stride, pad))
    conv_bwd = torch.ops.aten.convolution_backward

    def layer_torch(name, x, w, dy, s, p):
        torch.nn.functional.conv2d(x, w, None, s, p)
        conv_bwd(dy, x, w, None, (s, s), (p, p), (1, 1), False, (0, 0), 1, (name != "stem", True, False))

    t0 = time.time()
    for lay in layers:
        layer_torch(*lay)
        torch.cuda.synchronize()
        if progress:
            print(f"[miopen] {lay[0]} ready at {time.time() - t0:.1f} s", file=sys.stderr, flush=True)
    setup_s = time.time() - t0

    def step():
        for lay in layers:
            layer_torch(*lay)

    ms = best_step_ms(torch, step)
    torch.backends.cudnn.benchmark = False
    return ms, setup_s


def run_mfma_probe(torch):
    """The engine clock under sustained FP32 matrix load: register-only MFMA
    chains (libmxprobe.so's mxp_mfma_chain) on every CU, three workgroups per
    CU, about 5 ms per launch, launched one after another from idle (after 2 s
    without GPU work).  Per launch: TFLOP/s from HIP events and the median
    engine clock over workgroups (cycle counter against the 100 MHz real-time
    counter).  Alternates the two FP32 MFMA shapes on random operands, then
    one launch of each on zeros."""
    import ctypes as C
    import numpy as np
    lib = C.CDLL(os.path.join(REPO, "libmxprobe.so"))
    lib.mxp_mfma_chain.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    st = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks, iters = 3 * cus, 2000
    out = torch.empty(blocks * 256, device="cuda")
    clk = torch.zeros(2 * blocks, dtype=torch.int64, device="cuda")
    rand = torch.randn(1 << 20, device="cuda")
    zero = torch.zeros(1 << 20, device="cuda")
    torch.cuda.synchronize()
    time.sleep(2.0)
    rows = []
    plan = [(shape, "randn") for _ in range(6) for shape in (0, 1)] + [(0, "zeros"), (1, "zeros")]
    for i, (shape, data) in enumerate(plan):
        inp = rand if data == "randn" else zero
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        assert lib.mxp_mfma_chain(shape, C.c_void_p(inp.data_ptr()), C.c_void_p(out.data_ptr()), blocks, iters,
                                  C.c_void_p(clk.data_ptr()), C.c_void_p(st)) == 0
        e1.record()
        e1.synchronize()
        ms = e0.elapsed_time(e1)
        c = clk.cpu().numpy().reshape(-1, 2).astype(np.float64)
        ghz = float(np.median(c[:, 0] / (c[:, 1] / 100e6) / 1e9))
        tf = blocks * 4 * iters * 131072.0 / ms / 1e9
        rows.append({"launch": i, "mfma": "32x32x2" if shape == 0 else "16x16x4", "operands": data,
                     "ms": round(ms, 3), "tflops": round(tf, 1), "frac_of_157.3": round(tf / PEAK_FP32_TFLOPS, 3),
                     "clock_ghz": round(ghz, 3)})
        print(json.dumps(rows[-1]), file=sys.stderr, flush=True)
    return {"metric": "FP32 MFMA chains from idle: TFLOP/s and engine clock per launch", "launches": rows}


def torch_rocm_c2_c5(torch):
    """C2's step and C5's AdamW step through PyTorch-ROCm's own kernels on the
    CUDA device, on tensors of the same shapes and distributions: addmm / mm
    (hipBLASLt) and sum for C2; torch._fused_adamw_ (the kernel behind
    torch.optim.AdamW(fused=True)) for C5, after the same 10 warm-up steps.
    Vendor / framework baselines beside the components, not the product
    path."""
    import numpy as np
    out = {}
    g = torch.Generator(device="cuda").manual_seed(0)
    M, K, N = 8192, 4096, 4096
    X = torch.randn(M, K, device="cuda", generator=g)
    W = (torch.rand(N, K, device="cuda", generator=g) * 2 - 1) / 64
    b = (torch.rand(N, device="cuda", generator=g) * 2 - 1) / 64
    dY = torch.randn(M, N, device="cuda", generator=g)
    Y, dX, dW = torch.empty(M, N, device="cuda"), torch.empty_like(X), torch.empty_like(W)

    def c2():
        torch.addmm(b, X, W.t(), out=Y)
        torch.mm(dY, W, out=dX)
        torch.mm(dY.t(), X, out=dW)
        dY.sum(0)

    ms = best_step_ms(torch, c2)
    out["c2"] = {"ms_per_step": round(ms, 4), "value": round(3 * 2.0 * M * N * K / ms / 1e9, 3), "unit": "TFLOP/s",
                 "kernels": "torch.addmm / torch.mm (hipBLASLt) + sum"}
    del X, W, b, dY, Y, dX, dW
    rng = np.random.default_rng(0)
    sizes = np.exp(rng.uniform(math.log(64), math.log(4194304), 250)).astype(np.int64)
    P = [torch.randn(int(n), device="cuda", generator=g) * 0.02 for n in sizes]
    G = [torch.randn(int(n), device="cuda", generator=g) * 1e-3 for n in sizes]
    Mo = [torch.zeros(int(n), device="cuda") for n in sizes]
    V = [torch.zeros(int(n), device="cuda") for n in sizes]
    steps = [torch.zeros((), device="cuda") for _ in sizes]

    def c5():
        torch._foreach_add_(steps, 1)
        torch._fused_adamw_(P, G, Mo, V, [], steps, lr=1e-3, beta1=0.9, beta2=0.999, weight_decay=0.01, eps=1e-8,
                            amsgrad=False, maximize=False)

    for _ in range(10):
        c5()
    ms = best_step_ms(torch, c5, steps=10)
    numel = int(sizes.sum())
    out["c5"] = {"ms_per_step": round(ms, 4), "value": round(28.0 * numel / ms / 1e6, 1), "unit": "GB/s",
                 "kernels": "torch._fused_adamw_ (+ one _foreach_add_ for the step counters)"}
    return out


def best_step_ms(torch, step, rounds=3, steps=5):
    best = 1e9
    for _ in range(rounds):
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        e1.synchronize()
        best = min(best, e0.elapsed_time(e1) / steps)
    return best


def run_miopen_compare(torch, mx, find):
    """The C3 step through PyTorch-ROCm's MIOpen convolutions (miopen_c3_step)
    beside the same step through this library, in one process on the same
    data, best of 3 rounds of 5 steps each way."""
    L = Launcher(mx, torch.cuda.current_stream().cuda_stream)
    calls, total, _ = build_c3(torch, mx, L, 64)

    def ours():
        for c in calls:
            c[3]()

    ms_miopen, setup_s = miopen_c3_step(torch, find)
    ms_ours = best_step_ms(torch, ours)
    return {"metric": "C3 step: this library vs PyTorch-ROCm convolutions (MIOpen)",
            "miopen_mode": "find (cudnn.benchmark = True)" if find else "immediate (torch default)",
            "miopen_setup_s": round(setup_s, 1), "gflop_per_step": round(total / 1e9, 2),
            "ours_ms": round(ms_ours, 3), "ours_tflops": round(total / ms_ours / 1e9, 1),
            "miopen_ms": round(ms_miopen, 3), "miopen_tflops": round(total / ms_miopen / 1e9, 1),
            "speedup": round(ms_miopen / ms_ours, 3)}


def run_plan_sweep(torch, mx):
    """The convolution planner against every (tile, K split) plan: each
    implicit-GEMM phase of the sweep's layers (phases AUTO sends to Winograd
    are skipped) timed under every plan MX_CONV_PLAN can force (best of 3
    rounds of 4 back-to-back calls), and the planner's own pick.  Reports,
    per source, the summed time of the planner's picks and of the best plan
    per layer phase."""
    st = torch.cuda.current_stream().cuda_stream
    algo = mx.ALGO_IMPLICIT_GEMM
    totals = defaultdict(lambda: [0.0, 0.0])

    def timed(fn):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        best = 1e9
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda._sleep(200_000)
            e0.record()
            for _ in range(4):
                fn()
            e1.record()
            e1.synchronize()
            best = min(best, e0.elapsed_time(e1) / 4 * 1e3)
        return best

    try:
        for xs, co, k, s, pad, src in plan_sweep_layers():
            d = mx.conv_desc(xs, (co, xs[1], k, k), (s, s), (pad, pad))
            x = torch.randn(xs, device="cuda")
            w = torch.randn(co, xs[1], k, k, device="cuda") * 0.05
            y = torch.empty(xs[0], co, d.oh, d.ow, device="cuda")
            dy, dx = torch.randn_like(y), torch.empty_like(x)
            dw, db = torch.empty_like(w), torch.empty(co, device="cuda")
            phases = [(mx.MX_CONV_FORWARD, "fwd", lambda: mx.conv2d_forward(d, x, w, None, y, algo, st)),
                      (mx.MX_CONV_DINPUT, "dx", lambda: mx.conv2d_backward_input(d, dy, w, dx, algo, st)),
                      (mx.MX_CONV_DWEIGHT, "dw", lambda: mx.conv2d_backward_weight(d, x, dy, dw, db, algo, st))]
            for phase, name, fn in phases:
                if (name == "dx" and xs[1] == 3) or mx.conv2d_select(d, phase) != algo:
                    continue
                os.environ.pop("MX_CONV_PLAN", None)
                plan = mx.conv2d_plan(d, phase, algo)
                auto = f"{plan['tile']},{plan['splits']}"
                times = {auto: timed(fn)}
                for tile in range(6):
                    for splits in (1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64, 96, 128):
                        os.environ["MX_CONV_PLAN"] = f"{tile},{splits}"
                        try:
                            p = mx.conv2d_plan(d, phase, algo)
                        except mx.MXError:
                            continue
                        key = f"{p['tile']},{p['splits']}"
                        if p["tile"] == tile and key not in times:
                            times[key] = timed(fn)
                os.environ.pop("MX_CONV_PLAN", None)
                best = min(times, key=times.get)
                totals[src][0] += times[auto]
                totals[src][1] += times[best]
                print(json.dumps({"source": src, "x": xs, "cout": co, "k": k, "stride": s, "pad": pad, "phase": name,
                                  "planner": auto, "planner_us": round(times[auto], 2), "best": best,
                                  "best_us": round(times[best], 2)}), flush=True)
    finally:
        os.environ.pop("MX_CONV_PLAN", None)
    return {"planner_above_best_pct": {src: round(100 * (t[0] / t[1] - 1), 2) for src, t in totals.items()},
            "planner_us": {src: round(t[0], 1) for src, t in totals.items()},
            "best_us": {src: round(t[1], 1) for src, t in totals.items()}}


def back_to_back_us(torch, fn, reps, warmup):
    """Average microseconds per call of `reps` calls issued back to back on the
    current stream between one pair of HIP events.  A spin kernel queued
    before the first event keeps the GPU busy while the host issues the calls,
    so a call shorter than its Python issue time is timed at the GPU's pace,
    not the host's."""
    for _ in range(warmup):
        fn()
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(2_000_000)
    e0.record(st)
    for _ in range(reps):
        fn()
    e1.record(st)
    e1.synchronize()
    return 1000.0 * e0.elapsed_time(e1) / reps


def run_steps(torch, L, calls, steps, warmup, timing):
    for _ in range(warmup):
        for c in calls:
            c[3]()
    torch.cuda.synchronize()
    L.timing = timing
    t0 = time.perf_counter()
    for _ in range(steps):
        for label, flops, nbytes, fn in calls:
            L.run(label, flops, nbytes, fn)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    L.timing = False
    return dt, (L.collect() if timing else {})


def roofline_from(agg, bound, wino_exec_ratio=None):
    """Dominant kernel (most total time) among single-kernel launch classes.

    A Winograd call is two launches (the filter transform or the range sum
    beside the main kernel) and its FLOPs are quoted as the direct
    convolution's; it is the roofline class only when every call is
    Winograd, and then it is priced at its executed FLOPs (the direct count
    times wino_exec_ratio)."""
    best = None
    for label, (n, ms, flops, nbytes) in agg.items():
        if label.startswith("winograd"):
            continue
        if best is None or ms > best[1][1]:
            best = (label, (n, ms, flops, nbytes))
    whole_call = best is None
    if whole_call:
        best = max(agg.items(), key=lambda kv: kv[1][1])
    label, (n, ms, flops, nbytes) = best
    if whole_call:
        flops *= wino_exec_ratio
    avg_us = 1000.0 * ms / n
    if bound == "mfma":
        achieved = flops / n / (avg_us * 1e-6) / 1e12
        peak, unit = PEAK_FP32_TFLOPS, "TFLOP/s"
    else:
        achieved = nbytes / n / (avg_us * 1e-6) / 1e9
        peak, unit = PEAK_HBM_GBS, "GB/s"
    out = {"bound": bound, "kernel": label, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
           "frac": round(achieved / peak, 4), "traffic": None, "launches": n, "avg_launch_us": round(avg_us, 3)}
    if whole_call:
        out["note"] = ("one Winograd call: its main kernel and the launch beside it (filter transform or "
                       "range sum), at the executed (Winograd) FLOPs")
    return out


def breakdown(agg):
    out = {}
    for label, (n, ms, flops, nbytes) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        e = {"launches": n, "total_ms": round(ms, 3), "avg_us": round(1000 * ms / n, 2)}
        if flops:
            e["tflops"] = round(flops / (ms * 1e-3) / 1e12, 2)
        if nbytes:
            e["gbs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        out[label] = e
    return out


# ------------------------------------------------------------------ CPU baseline
def cgroup_cpu_quota():
    """CPUs the process's cgroup grants (cgroup v2 cpu.max or v1 cfs quota), or None."""
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()
        if quota != "max":
            return max(1, int(int(quota) // int(period)))
    except Exception:  # noqa: BLE001 (no cgroup v2 file: try v1)
        pass
    try:
        quota = int(open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us").read())
        period = int(open("/sys/fs/cgroup/cpu/cpu.cfs_period_us").read())
        if quota > 0:
            return max(1, quota // period)
    except Exception:  # noqa: BLE001
        pass
    return None


def cpu_setup(torch):
    """Give CPU PyTorch one thread per core this process may run on -- the
    affinity mask, capped by the cgroup's CPU quota where one is set (more
    threads than granted CPUs would only time-slice) -- and describe the host."""
    affinity = len(os.sched_getaffinity(0))
    quota = cgroup_cpu_quota()
    cores = min(affinity, quota) if quota else affinity
    torch.set_num_threads(cores)
    model = None
    lscpu = {}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        lscpu = {k.strip(): v.strip() for k, v in (l.split(":", 1) for l in out.splitlines() if ":" in l)}
        model = lscpu.get("Model name")
    except Exception:  # noqa: BLE001 (lscpu missing: fall back to /proc/cpuinfo)
        pass
    cpuinfo = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                if cpuinfo:
                    break  # the first processor's block is enough
                continue
            k, v = line.split(":", 1)
            cpuinfo.setdefault(k.strip(), v.strip())
    except Exception:  # noqa: BLE001
        pass
    if model is None:
        model = cpuinfo.get("model name", "unknown")
    # Virtual machines often report only "AMD EPYC": family / model / stepping
    # (family 25 is Zen 3-4, 26 Zen 5), clocks and caches tell hosts apart.
    host = {"family": cpuinfo.get("cpu family"), "model": cpuinfo.get("model"), "stepping": cpuinfo.get("stepping"),
            "mhz": cpuinfo.get("cpu MHz"), "max_mhz": lscpu.get("CPU max MHz"), "l3": lscpu.get("L3 cache"),
            "sockets": lscpu.get("Socket(s)"), "hypervisor": lscpu.get("Hypervisor vendor"),
            "avx512": "avx512f" in cpuinfo.get("flags", "")}
    return {"cores": cores, "threads": torch.get_num_threads(), "cpu_model": model, "affinity": affinity,
            "cgroup_quota": quota, "cpu_host": {k: v for k, v in host.items() if v not in (None, "")}}


def cpu_time(fn, warmup, reps):
    """Median wall time of fn over reps runs after warmup runs (time.perf_counter)."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_c1(torch, host):
    """C1 on CPU PyTorch: F.conv2d + autograd (forward, dInput, dWeight, dBias) on
    the same seeded inputs."""
    F = torch.nn.functional
    x, w, b = (host[k].clone().requires_grad_() for k in ("x", "w", "b"))

    def step():
        y = F.conv2d(x, w, b, 1, 1)
        torch.autograd.grad(y, (x, w, b), host["dy"])

    t, n = cpu_time(step, 2, 9)
    flops, _ = conv_flops(tuple(host["x"].shape), w.shape[0], 3, 1, 1)
    return {"value": round(3 * flops / t / 1e12, 4), "unit": "TFLOP/s", "ms_per_step": round(1e3 * t, 3),
            "sample": f"the full C1 step (forward + dInput + dWeight + dBias), median of {n} after 2 warm-ups"}


def cpu_c2(torch):
    """C2 on CPU PyTorch: addmm forward, dX, dW, db at 8192 x 4096 x 4096, and
    the two transposed-input products, on seeded inputs of the same shapes."""
    g = torch.Generator().manual_seed(0)
    M, K, N = 8192, 4096, 4096
    X = torch.randn(M, K, generator=g)
    W = (torch.rand(N, K, generator=g) * 2 - 1) / 64
    b = (torch.rand(N, generator=g) * 2 - 1) / 64
    dY = torch.randn(M, N, generator=g)

    def step():
        torch.addmm(b, X, W.t())
        torch.mm(dY, W)
        torch.mm(dY.t(), X)
        dY.sum(0)

    t, n = cpu_time(step, 1, 3)
    t_xtg, _ = cpu_time(lambda: torch.mm(X.t(), dY), 1, 3)
    t_xwt, _ = cpu_time(lambda: torch.mm(X, W.t()), 1, 3)
    f = 2.0 * M * N * K
    return {"value": round(3 * f / t / 1e12, 4), "unit": "TFLOP/s", "ms_per_step": round(1e3 * t, 3),
            "transposed": {"X^T.G": round(f / t_xtg / 1e12, 4), "X.W^T": round(f / t_xwt / 1e12, 4)},
            "sample": f"the full C2 step (addmm forward, dX, dW, db), median of {n} after 1 warm-up; "
                      "transposed-input products timed alone (TFLOP/s)"}


def cpu_c4(torch, batch=4, reps=3):
    """The C4 U-Net training step on CPU PyTorch (forward, MSE, backward,
    AdamW fused=True on the CPU) at a reduced batch."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    import unet_c4 as U
    model = U.make_model()
    x, t = U.make_inputs(batch=batch)
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, weight_decay=0.01, fused=True)
    flops = U.step_flops(model, x)

    def step():
        U.train_step_loss(model, x, t)
        opt.step()

    tt, n = cpu_time(step, 1, reps)
    return {"value": round(flops / tt / 1e12, 4), "unit": "TFLOP/s", "ms_per_step": round(1e3 * tt, 2),
            "sample": f"the same U-Net step at batch {batch} instead of 16 ({flops / 1e9:.1f} GFLOP), "
                      f"median of {n} after 1 warm-up"}


def cpu_c5(torch, sizes):
    """torch.optim.AdamW on CPU over the same 250 tensor shapes, foreach=False,
    foreach=True and fused=True; the fastest is the baseline."""
    g = torch.Generator().manual_seed(0)
    numel = int(sum(int(n) for n in sizes))
    out = {}
    for name, kw in (("foreach=False", dict(foreach=False)), ("foreach=True", dict(foreach=True)),
                     ("fused=True", dict(fused=True))):
        ps = [torch.nn.Parameter(torch.randn(int(n), generator=g) * 0.02) for n in sizes]
        for p_ in ps:
            p_.grad = torch.randn(p_.shape, generator=g) * 1e-3
        opt = torch.optim.AdamW(ps, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, **kw)
        t, n = cpu_time(opt.step, 2, 5)
        out[name] = {"ms_per_step": round(1e3 * t, 2), "gb_s": round(28.0 * numel / t / 1e9, 2)}
        del ps, opt
    best = min(out, key=lambda k: out[k]["ms_per_step"])
    return {"value": out[best]["gb_s"], "unit": "GB/s", "ms_per_step": out[best]["ms_per_step"], "variant": best,
            "variants": out,
            "sample": f"one AdamW step over all {numel} elements (250 tensors), median of 5 after 2 warm-ups per "
                      f"variant; the fastest ({best}) is the baseline"}


def cpu_conv_stack(torch, batch, reps):
    F = torch.nn.functional
    g = torch.Generator().manual_seed(0)
    layers = []
    total = 0.0
    for name, xs, cout, k, stride, pad in resnet50_convs(batch):
        flops, (oh, ow) = conv_flops(xs, cout, k, stride, pad)
        x = torch.randn(xs, generator=g).requires_grad_(name != "stem")
        w = torch.randn(cout, xs[1], k, k, generator=g).requires_grad_()
        dy = torch.randn(xs[0], cout, oh, ow, generator=g)
        layers.append((x, w, dy, stride, pad))
        total += flops * (3 if name != "stem" else 2)

    def one():
        for x, w, dy, s, p in layers:
            y = F.conv2d(x, w, None, s, p)
            torch.autograd.grad(y, [t for t in (x, w) if t.requires_grad], dy)

    one()  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    times.sort()
    return total / times[len(times) // 2] / 1e12, total, times


# ------------------------------------------------------------------ HBM traffic (PMC)
def kernel_class(name: str) -> str:
    """Demangled dispatch name -> the label bench uses for its launch class."""
    import re
    name = name.replace("conv_dx_phases_kernel", "conv_dx_kernel")  # fused stride phases: the same tile class
    for kind in ("conv_fwd_kernel", "conv_dx_kernel", "conv_dw_kernel"):
        if kind in name:
            m = re.search(r"Cfg<(\d+), (\d+), (\d+),", name)
            return f"{kind}<{m.group(1)}x{m.group(2)}x{m.group(3)}>" if m else kind
    m = re.search(r"(?:mx::)?(?:\(anonymous namespace\)::)?(\w+_kernel)", name)
    return m.group(1) if m else name[:60]


def read_pmc(directory: str, counter: str):
    """[(dispatch id, kernel name, KiB)] from a rocprofv3 --pmc CSV directory."""
    import csv
    import glob
    rows = []
    for path in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(path)):
            if r["Counter_Name"] == counter:
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return rows


def pmc_summary(fetch_dir, write_dir, copy_fetch_dir, copy_write_dir):
    """Per launch class: mean HBM bytes read and written per dispatch, each
    scaled so the calibration copy reads/writes exactly its 1 GiB."""
    copy_bytes = COPY_FLOATS * 4
    cf = [kib for _, name, kib in read_pmc(copy_fetch_dir, "FETCH_SIZE") if "copy" in name.lower()]
    cw = [kib for _, name, kib in read_pmc(copy_write_dir, "WRITE_SIZE") if "copy" in name.lower()]
    f_scale = copy_bytes / (1024.0 * max(cf)) if cf else 1.0
    w_scale = copy_bytes / (1024.0 * max(cw)) if cw else 1.0
    agg = defaultdict(lambda: [0, 0.0, 0, 0.0])
    for _, name, kib in read_pmc(fetch_dir, "FETCH_SIZE"):
        a = agg[kernel_class(name)]
        a[0] += 1
        a[1] += kib * 1024.0 * f_scale
    for _, name, kib in read_pmc(write_dir, "WRITE_SIZE"):
        a = agg[kernel_class(name)]
        a[2] += 1
        a[3] += kib * 1024.0 * w_scale
    out = {"fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4), "kernels": {}}
    for label, (nf, fb, nw, wb) in sorted(agg.items(), key=lambda kv: -(kv[1][1] + kv[1][3])):
        if nf and nw:
            out["kernels"][label] = {"dispatches": nf, "read_bytes": round(fb / nf), "write_bytes": round(wb / nw),
                                     "bytes_per_launch": round(fb / nf + wb / nw)}
    return out


def sq_summary(directory, xcds=8, cus=256):
    """Markdown table of SQ counters per launch class from a rocprofv3 --pmc
    CSV directory (SQ_* with GRBM_GUI_ACTIVE): mean per dispatch, and derived
    figures -- kernel cycles (GRBM_GUI_ACTIVE sums the XCDs), MFMA busy as a
    share of every SIMD's cycles (SQ_VALU_MFMA_BUSY_CYCLES sums the SIMDs:
    each instruction's matrix-core cycles) and the share of wave-resident
    cycles spent waiting on dependencies (SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES)."""
    import csv
    import glob
    vals = defaultdict(lambda: defaultdict(list))
    for path in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(path)):
            vals[kernel_class(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    names = ["SQ_WAVES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_VALU_MFMA_BUSY_CYCLES",
             "SQ_WAVE_CYCLES", "SQ_WAIT_INST_ANY", "SQ_BUSY_CU_CYCLES", "GRBM_GUI_ACTIVE"]
    out = ["| launch class | dispatches | " + " | ".join(n.replace("SQ_", "") for n in names) +
           " | kernel us | MFMA busy | waiting |", "|---|" + "---:|" * (len(names) + 4)]
    for k, c in sorted(vals.items(), key=lambda kv: -sum(kv[1].get("SQ_VALU_MFMA_BUSY_CYCLES", [0]))):
        m = {n: sum(v) / len(v) for n, v in c.items()}
        if not m.get("SQ_WAVES"):
            continue
        cyc = m.get("GRBM_GUI_ACTIVE", 0) / xcds
        busy = m.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) / (4 * cus * cyc) if cyc else 0
        wait = m.get("SQ_WAIT_INST_ANY", 0) / m["SQ_WAVE_CYCLES"] if m.get("SQ_WAVE_CYCLES") else 0
        out.append(f"| `{k}` | {len(c.get('SQ_WAVES', []))} | " + " | ".join(f"{m.get(n, 0):.0f}" for n in names) +
                   f" | {cyc / 2400:.1f} | {100 * busy:.1f}% | {100 * wait:.1f}% |")
    return "\n".join(out)


WINOGRAD_KERNELS = ("filter_kernel", "wino_ws_kernel", "wino_ws16_kernel",   # fused path
                    "wino_filter_kernel", "wino_input_kernel", "wino_output_kernel", "gemm_kernel")
# First dispatch of a Winograd call: its filter transform, or the fused
# kernel itself when that transforms the filter (no filter launch before it).
WINOGRAD_CALL_START = ("filter_kernel", "wino_filter_kernel")
BEFORE_HELPERS = ("conv_fwd_pack_kernel", "conv_dx_pack_kernel")       # run before their tile kernel
AFTER_HELPERS = ("conv_dw_finalize_kernel", "conv_sum_splits_kernel")   # run after it


PHASE_MARKER = "spin_kernel"   # torch.cuda._sleep's kernel, issued once between the headline and the components


def stats_table(stats_csv, steps_run, top=25):
    """Markdown tables from a rocprofv3 --stats kernel_stats.csv (or from a
    --kernel-trace CSV, up to the headline's end marker): time per step of
    each launch class (all instantiations of a kernel template together), then
    the top kernel instantiations."""
    import csv
    import re
    rows = list(csv.DictReader(open(stats_csv)))
    if rows and "Start_Timestamp" in rows[0]:
        # a --kernel-trace CSV: the headline phase only, aggregated per kernel
        rows.sort(key=lambda r: int(r["Start_Timestamp"]))
        agg = defaultdict(lambda: [0, 0])
        for r in rows:
            if PHASE_MARKER in r["Kernel_Name"]:
                break
            a = agg[r["Kernel_Name"]]
            a[0] += 1
            a[1] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        rows = [{"Name": k, "Calls": str(n), "TotalDurationNs": str(t)} for k, (n, t) in agg.items()]
    steps_run = float(steps_run)
    cls = defaultdict(lambda: [0, 0.0])
    for r in rows:
        c = cls[kernel_class(r["Name"]).split("<")[0]]
        c[0] += int(r["Calls"])
        c[1] += float(r["TotalDurationNs"])
    total = sum(t for _, t in cls.values())
    out = [f"Kernel time {total / 1e6 / steps_run:.3f} ms per step over {steps_run:g} steps.", "",
           "| launch class | ms/step | calls/step | avg us | % |", "|---|---:|---:|---:|---:|"]
    for k, (n, t) in sorted(cls.items(), key=lambda kv: -kv[1][1])[:top]:
        out.append(f"| `{k}` | {t / 1e6 / steps_run:.3f} | {n / steps_run:.1f} | {t / n / 1e3:.1f} | "
                   f"{100 * t / total:.2f} |")

    def short(n):
        n = re.sub(r"mx::(conv::|mfma::)?(\(anonymous namespace\)::)?", "", n).replace("void ", "")
        n = re.sub(r"\((ConvArgs|GemmArgs|WinoArgs)\)$", "", n)
        return ("torch: " + n.split("<")[0].split("(")[0]) if "at::native" in n else n[:120]
    out += ["", "| kernel | calls | total us | avg us | % |", "|---|---:|---:|---:|---:|"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"]))[:top]:
        t = float(r["TotalDurationNs"])
        out.append(f"| `{short(r['Name'])}` | {r['Calls']} | {t / 1e3:.1f} | {t / int(r['Calls']) / 1e3:.2f} | "
                   f"{100 * t / total:.2f} |")
    return "\n".join(out)


def trace_summary(trace_csv, bench_log):
    """Per bench launch class: the kernel time of one ABI call from a rocprofv3
    --kernel-trace CSV of a bench.py run, comparable with that run's live
    `avg_us`.  An ABI call can issue several dispatches (weight packing, one
    GEMM per dInput stride phase, zero phases, the split-K sum); helper
    dispatches are charged to the call's tile kernel (packing to the next one,
    split sums and zero phases to the previous one), Winograd's kernels to
    "winograd_forward" or, when the run also routed input gradients there,
    alternately to "winograd_forward" and "winograd_dinput" (C3 issues a
    layer's forward call, then its dInput call; each call starts with a
    filter transform), and the class total is divided by the number of calls
    the run made (warm-up + untimed + event-timed steps)."""
    import csv
    res = [json.loads(l) for l in open(bench_log) if l.startswith("{")][-1]
    steps_run = res["warmup"] + 2 * res["steps"]
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    # the headline phase ends at the marker dispatch main() issues before the components
    end = next((i for i, r in enumerate(rows) if PHASE_MARKER in r["Kernel_Name"]), len(rows))
    rows = rows[:end]
    seq = [(kernel_class(r["Kernel_Name"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
           for r in rows]
    owner = [None] * len(seq)
    last_tile = None
    wino_dx = "winograd_dinput" in res["kernels"]
    wino_calls = 0
    for i, (label, _) in enumerate(seq):
        if label in ("wino_dw_kernel", "wino_dw_ws_kernel"):
            # the Winograd weight gradient; its range sum follows as a helper
            owner[i] = last_tile = "winograd_dweight"
        elif label in WINOGRAD_KERNELS:
            wino_calls += label in WINOGRAD_CALL_START or (
                label in ("wino_ws_kernel", "wino_ws16_kernel") and (i == 0 or seq[i - 1][0] != "filter_kernel"))
            owner[i] = "winograd_dinput" if (wino_dx and wino_calls % 2 == 0) else "winograd_forward"
        elif label in AFTER_HELPERS or label == "conv_dx_zero_kernel":
            owner[i] = last_tile
        elif label not in BEFORE_HELPERS:
            owner[i] = last_tile = label
    nxt = None
    for i in range(len(seq) - 1, -1, -1):
        label = seq[i][0]
        if label in BEFORE_HELPERS or (label == "conv_dx_zero_kernel" and owner[i] is None):
            owner[i] = nxt
        elif owner[i] is not None and not owner[i].startswith("winograd"):
            nxt = owner[i]
    agg = defaultdict(float)
    for (label, us), own in zip(seq, owner):
        agg[own or label] += us
    out = {}
    for label, live in res["kernels"].items():
        calls = live["launches"] // res["steps"] * steps_run
        if label in agg and calls:
            out[label] = {"calls": calls, "trace_total_us": round(agg[label], 1),
                          "trace_avg_us_per_call": round(agg[label] / calls, 2), "live_avg_us": live["avg_us"]}
    return out


def run_copy(torch, steps, warmup):
    x = torch.ones(COPY_FLOATS, device="cuda")
    y = torch.empty_like(x)
    for _ in range(warmup):
        y.copy_(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        y.copy_(x)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    return {"workload": "copy: 1 GiB device-to-device (PMC calibration)", "ms_per_step": round(dt * 1e3, 4),
            "value": round(2 * 4 * COPY_FLOATS / dt / 1e9, 1), "unit": "GB/s"}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=["c3", "c1", "c4", "c4ops", "c5", "copy"], default="c3",
                    help="c4 / c4ops / c5 run only that component (for profiling); the headline stays C3")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"),
                    help="summarise four rocprofv3 --pmc output directories into per-kernel HBM bytes")
    ap.add_argument("--trace-summary", nargs=2, metavar=("KERNEL_TRACE_CSV", "BENCH_LOG"),
                    help="kernel time per ABI call of each launch class from a rocprofv3 kernel trace of a "
                         "bench.py run, next to that run's live per-call time")
    ap.add_argument("--sq-summary", metavar="PMC_DIR",
                    help="markdown table of SQ counters (and MFMA busy share) per launch class from a --pmc CSV dir")
    ap.add_argument("--stats-table", nargs=2, metavar=("KERNEL_STATS_CSV", "STEPS_RUN"),
                    help="markdown tables (per launch class, per kernel) from a rocprofv3 --stats CSV")
    ap.add_argument("--probe-sweep", action="store_true",
                    help="sweep the 4-read / 3-write probe's memory schedule at C5's size (one JSON object)")
    ap.add_argument("--rule-sweep", choices=["grid", "random"],
                    help="time both algorithms on 3x3 stride-1 layers in every phase against AUTO's Winograd rule")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="FP32 MFMA chains from idle: TFLOP/s and engine clock per launch")
    ap.add_argument("--miopen-compare", choices=["immediate", "find"],
                    help="time the C3 step against PyTorch-ROCm's MIOpen convolutions")
    ap.add_argument("--blas-compare", action="store_true",
                    help="time C3's 1x1 stride-1 forwards and input gradients against torch.matmul (hipBLASLt)")
    ap.add_argument("--plan-sweep", action="store_true",
                    help="time every (tile, K split) plan of the convolution planner against its own picks")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-components", action="store_true")
    ap.add_argument("--no-winograd", action="store_true", help="route C3's 3x3 stride-1 layers (all three phases) to implicit GEMM")
    args = ap.parse_args(argv)
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary), indent=1))
        return 0
    if args.trace_summary:
        print(json.dumps(trace_summary(*args.trace_summary), indent=1))
        return 0
    if args.sq_summary:
        print(sq_summary(args.sq_summary))
        return 0
    if args.stats_table:
        print(stats_table(*args.stats_table))
        return 0
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); the multi-GPU "
              "sharding is a design (DESIGN.md), not a measured path.", file=sys.stderr)
        return 2

    import torch
    from torch_vulkan import mx

    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    mx.lib()
    stream = torch.cuda.current_stream().cuda_stream
    L = Launcher(mx, stream)
    log = lambda *a: print("[bench]", *a, file=sys.stderr, flush=True)  # noqa: E731

    if args.mfma_probe:
        print(json.dumps(run_mfma_probe(torch)), flush=True)
        return 0
    if args.miopen_compare:
        print(json.dumps(run_miopen_compare(torch, mx, args.miopen_compare == "find")), flush=True)
        return 0
    if args.blas_compare:
        print(json.dumps(run_blas_compare(torch, mx)), flush=True)
        return 0
    if args.plan_sweep:
        print(json.dumps(run_plan_sweep(torch, mx)), flush=True)
        return 0
    if args.rule_sweep:
        print(json.dumps(run_rule_sweep(torch, mx, args.rule_sweep)), flush=True)
        return 0
    if args.probe_sweep:
        _, numel, _ = build_c5(torch, mx, L)
        print(json.dumps(run_probe_sweep(torch, numel)), flush=True)
        return 0
    if args.workload == "copy":
        print(json.dumps(run_copy(torch, args.steps, args.warmup)), flush=True)
        return 0
    if args.workload == "c4":
        print(json.dumps(run_c4(torch, args.steps, args.warmup, log)), flush=True)
        return 0
    if args.workload == "c4ops":
        print(json.dumps(run_c4_ops(torch, mx, L)), flush=True)
        return 0
    if args.workload == "c5":
        calls, numel, _ = build_c5(torch, mx, L)
        dt, _ = run_steps(torch, L, calls, args.steps, args.warmup, timing=False)
        print(json.dumps({"workload": "C5 only (PMC passes)", "ms_per_step": round(1e3 * dt / args.steps, 4),
                          "value": round(28.0 * numel / (dt / args.steps) / 1e9, 1), "unit": "GB/s"}), flush=True)
        return 0

    # ---------------- headline
    if args.workload == "c3":
        calls, flops_step, executed_step = build_c3(torch, mx, L, 64, winograd=not args.no_winograd)
        config = {"workload": "C3: ResNet-50 v1.5 conv stack (53 convs) fwd+dInput+dWeight, batch 64, 224x224, "
                              + ("3x3/s1 layers (forward, dInput, dWeight) via Winograd F(2x2,3x3)" if not args.no_winograd
                                 else "all phases implicit-GEMM MFMA"),
                  "global_batch": 64, "image": 224, "layers": 53, "gflop_per_step": round(flops_step / 1e9, 2),
                  "executed_gflop_per_step": round(executed_step / 1e9, 2)}
    else:
        calls, flops_step, _, _, executed_step = build_c1(torch, mx, L)
        config = {"workload": "C1: Conv2D 8x64x56x56, 64->64 3x3 s1 p1, fwd+dInput+dWeight+dBias",
                  "global_batch": 8, "gflop_per_step": round(flops_step / 1e9, 4),
                  "executed_gflop_per_step": round(executed_step / 1e9, 4)}
    log("headline built:", config["workload"])
    dt, _ = run_steps(torch, L, calls, args.steps, args.warmup, timing=False)
    ms_step = 1000 * dt / args.steps
    value = flops_step / (dt / args.steps) / 1e12
    log(f"headline: {ms_step:.3f} ms/step, {value:.2f} TFLOP/s")
    _, agg = run_steps(torch, L, calls, args.steps, 0, timing=True)
    roof = roofline_from(agg, "mfma", executed_step / flops_step)
    if args.workload == "c3" and not args.no_winograd and os.path.exists(TRAFFIC_FILE):
        traffic = json.load(open(TRAFFIC_FILE)).get("kernels", {}).get(roof["kernel"])
        if traffic:
            roof["traffic"] = traffic["bytes_per_launch"]
            roof["traffic_source"] = os.path.relpath(TRAFFIC_FILE, REPO)
    result = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded randn / kaiming inputs)",
        "config": config, "frac_of_fp32_peak": round(value / PEAK_FP32_TFLOPS, 4),
        # The same step priced at the FLOPs its kernels execute (Winograd
        # phases at 16 products per 2x2 tile instead of 36).
        "frac_of_fp32_peak_executed": round(executed_step / (dt / args.steps) / 1e12 / PEAK_FP32_TFLOPS, 4),
        "roofline": roof,
        "kernels": breakdown(agg),
    }
    del calls
    torch.cuda.empty_cache()
    torch.cuda._sleep(1)   # marks the end of the headline phase in a kernel trace (PHASE_MARKER)

    # ---------------- components
    cpu_inputs = {}
    if not args.no_components:
        comps = {}
        for key, builder in (("c1", build_c1), ("c1_implicit", lambda t, m, l: build_c1(t, m, l, C1_IMPLICIT)),
                             ("c2", build_c2), ("c5", build_c5)):
            built = builder(torch, mx, L)
            calls_c, work = built[0], built[1]
            if key == "c1":
                cpu_inputs["c1"] = built[2]
            if key == "c5":
                cpu_inputs["c5"] = built[2]
            # C1 steps are ~60 us: 200 of them keep the timed region above 10 ms,
            # and as many untimed ones before it bring the clocks and caches to
            # their steady state (after 3 warm-up steps the first 200 timed
            # ones ran 59.7 us each against 57.2-57.7 for every later 200).
            steps = (max(args.steps, 200) if key.startswith("c1") else max(args.steps, 20)) if key != "c2" else args.steps
            warm = steps if key.startswith("c1") else 3
            dt, _ = run_steps(torch, L, calls_c, steps, warm, timing=False)
            _, agg_c = run_steps(torch, L, calls_c, steps, 0, timing=True)
            ms = 1000 * dt / steps
            if key == "c5":
                gbs = 28.0 * work / (dt / steps) / 1e9
                roof = roofline_from(agg_c, "hbm")
                if os.path.exists(TRAFFIC_C5_FILE):
                    tr = json.load(open(TRAFFIC_C5_FILE)).get("kernels", {}).get("adamw_kernel")
                    if tr:
                        roof["traffic"] = tr["bytes_per_launch"]
                        roof["traffic_source"] = os.path.relpath(TRAFFIC_C5_FILE, REPO)
                ceiling = run_stream_probes(torch, work)
                comps[key] = {"workload": f"C5: multi-tensor AdamW, 250 tensors, {work} elements, 28 B/elem",
                              "ms_per_step": round(ms, 4), "value": round(gbs, 1), "unit": "GB/s",
                              "frac_of_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                              "stream_probes_gb_s": ceiling,
                              "frac_of_4r3w_probe": round(gbs / ceiling["adamw_mix_4r3w"], 4),
                              "frac_of_4r3w_math_probe": round(gbs / ceiling["adamw_math_4r3w"], 4),
                              "roofline": roof, "kernels": breakdown(agg_c)}
            else:
                desc = {"c1": "C1: Conv2D 8x64x56x56 3x3 fwd+dX+dW+dB; every phase on Winograd F(2x2,3x3), "
                              "the planner's AUTO choice for this layer (parity asserted at rel 1e-4 / abs 1e-5), "
                              "dX, dW and dBias in one backward call (one launch beside the range sum)",
                        "c1_implicit": "C1 with every phase on the implicit GEMM (rel 1e-4 parity)",
                        "c2": "C2: Linear addmm 8192x4096x4096 fwd + dX + dW + db"}[key]
                comps[key] = {"workload": desc, "ms_per_step": round(ms, 4),
                              "value": round(work / (dt / steps) / 1e12, 3), "unit": "TFLOP/s",
                              "frac_of_fp32_peak": round(work / (dt / steps) / 1e12 / PEAK_FP32_TFLOPS, 4),
                              "roofline": roofline_from(agg_c, "mfma", built[4] / work if key.startswith("c1") else None),
                              "kernels": breakdown(agg_c)}
                if key.startswith("c1"):
                    comps[key]["frac_of_fp32_peak_executed"] = round(
                        built[4] / (dt / steps) / 1e12 / PEAK_FP32_TFLOPS, 4)
            log(key, comps[key]["value"], comps[key]["unit"])
            del calls_c, built
            torch.cuda.empty_cache()
        comps["c4_ops"] = run_c4_ops(torch, mx, L)
        log("c4_ops", {k: v["algorithmic_gb_s"] for k, v in comps["c4_ops"]["ops"].items()})
        torch.cuda.empty_cache()
        comps["c4"] = run_c4(torch, max(3, min(args.steps, 10)), 3, log)
        log("c4", comps["c4"]["ms_per_step"], "ms/step", comps["c4"]["value"], "TFLOP/s; conv/GEMM kernels",
            comps["c4"].get("conv_gemm_kernel_tflop_s"), "TFLOP/s (executed",
            comps["c4"].get("conv_gemm_executed_tflop_s"), "); roofline", comps["c4"].get("roofline"))
        comps["streams"] = run_streams(torch)
        log("streams", comps["streams"])
        if args.workload == "c3" and not args.no_winograd:
            # The headline step through PyTorch-ROCm's own convolutions (MIOpen,
            # torch's default immediate mode) on this box: a vendor-library
            # baseline, not the product path.
            try:
                ms_m, setup_s = miopen_c3_step(torch, False, progress=False)
                comps["miopen"] = {
                    "workload": "C3 step through torch.nn.functional.conv2d + aten.convolution_backward on the "
                                "CUDA device (MIOpen, immediate mode: torch's default)",
                    "ms_per_step": round(ms_m, 4), "value": round(flops_step / ms_m / 1e9, 3), "unit": "TFLOP/s",
                    "setup_s": round(setup_s, 1), "headline_ms_per_step": round(ms_step, 4),
                    "miopen_over_headline_time": round(ms_m / ms_step, 3)}
            except Exception as e:  # a baseline only: never fail the bench on it
                comps["miopen"] = {"error": f"{type(e).__name__}: {e}"}
            log("miopen", comps["miopen"])
            torch.cuda.empty_cache()
        try:
            for key, v in torch_rocm_c2_c5(torch).items():
                v["this_library_over_torch_rocm"] = round(comps[key]["value"] / v["value"], 3)
                comps[key]["torch_rocm"] = v
                log(key, "torch-rocm", v)
        except Exception as e:  # a baseline only: never fail the bench on it
            log("torch-rocm baselines failed:", f"{type(e).__name__}: {e}")
        torch.cuda.empty_cache()
        result["components"] = comps

    # ---------------- CPU baselines (bounded samples, same seeded inputs)
    # CPU PyTorch is the reference's CPU implementation of these ops (its
    # tests compare against it); the reference's own build cannot run here.
    if not args.no_cpu_baseline and args.workload == "c3":
        host = cpu_setup(torch)
        log("cpu baselines on", host)
        tflops, sample_flops, times = cpu_conv_stack(torch, 4, 3)
        result["cpu_baseline"] = {
            "value": round(tflops, 4), "unit": "TFLOP/s", "cores": host["threads"], "kind": "reference",
            "cpu_model": host["cpu_model"], "cpu_host": host["cpu_host"], "affinity_cores": host["affinity"],
            "cgroup_cpu_quota": host["cgroup_quota"],
            "sample": f"CPU PyTorch {torch.__version__} F.conv2d + autograd over the same 53-layer stack at batch 4 "
                      f"instead of 64 ({sample_flops / 1e9:.1f} GFLOP per pass, median of {len(times)} passes "
                      f"after 1 warm-up, {host['threads']} threads)",
            "gpu_over_cpu": round(value / tflops, 1),
        }
        log("cpu baseline c3", result["cpu_baseline"]["value"], "TFLOP/s")
        if not args.no_components:
            base = {"cores": host["threads"], "kind": "reference", "cpu_model": host["cpu_model"]}
            for key, fn in (("c1", lambda: cpu_c1(torch, cpu_inputs["c1"])), ("c2", lambda: cpu_c2(torch)),
                            ("c4", lambda: cpu_c4(torch)), ("c5", lambda: cpu_c5(torch, cpu_inputs["c5"]))):
                cb = dict(base, **fn())
                comps[key]["cpu_baseline"] = cb
                comps[key]["cpu_baseline"]["gpu_over_cpu"] = round(comps[key]["value"] / cb["value"], 1)
                log(f"cpu baseline {key}", cb["value"], cb["unit"])
            comps["c1_implicit"]["cpu_baseline"] = comps["c1"]["cpu_baseline"]
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
