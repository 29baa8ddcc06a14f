"""Kernel-variant coverage shared by the GPU parity tests and the CPU planner test.

Every kernel instantiation the library can launch is named by its planner
(`mx_conv2d_plan` / `mx_gemm_variant`: tile, operand loaders, split-K,
epilogue flags).  This module lists

* the cases the GPU parity tests run (`tests/test_gpu_plans.py`), each with the
  environment that forces its plan (`MX_CONV_PLAN`, `MX_GEMM_TILE`,
  `MX_WINOGRAD_FUSED`, `MX_WINOGRAD_FILTER`, `MX_WINOGRAD_T16`, `MX_WINO_DW_WS`,
  `TORCH_VULKAN_CONV_WORKSPACE_MB`), and
* every call the benchmark configurations make (C1 single layer, C2 Linear,
  C3 ResNet-50 conv stack, C4 U-Net step), with the algorithm bench.py or the
  "vulkan" device requests,

so `tests/test_plan_coverage.py` can check on the host that each variant the
configurations use is one a parity test runs.  The reference forces every
tile of its planner on its dispatch geometries in the same way
(tests/test_conv_dispatch.py:20-82) and sizes a test to reach its large GEMM
kernel (tests/test_fused_addmm.py:7-33).

Plans depend on operand shape, layout and alignment, not on the batch size
(except through split feasibility), so the parity cases use small batches of
the configurations' own layer shapes.
"""
from __future__ import annotations

import contextlib
import os

# ------------------------------------------------------------------ conv cases
# x shape, output channels, kernel, stride, padding, dilation, groups
REFERENCE_GEOMETRIES = [  # tests/test_conv_dispatch.py:20-47
    ((1, 7, 1, 15), 7, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 1, 17), 9, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 15, 1, 31), 15, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 17, 1, 33), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 31, 1, 63), 31, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 33, 1, 65), 33, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 12, 14), 17, (9, 9), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 13, 15), 17, (10, 10), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 14, 16), 17, (11, 11), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 15, 17), 17, (12, 12), (1, 1), (0, 0), (1, 1), 1),
    ((2, 18, 19, 23), 34, (3, 5), (2, 1), (2, 3), (2, 1), 2),
    ((1, 5, 11, 13), 15, (3, 5), (1, 2), (1, 4), (1, 2), 5),
    ((2, 6, 15, 19), 9, (3, 5), (1, 1), (3, 4), (2, 3), 3),
    ((1, 5, 11, 13), 15, (3, 5), (1, 1), (2, 4), (2, 2), 5),
    ((1, 9, 17, 23), 17, (3, 5), (2, 3), (3, 2), (2, 1), 1),
    ((1, 9, 1, 255), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 1, 256), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 1, 257), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1),
]


def resnet50_layers(batch):
    """(name, x_shape, cout, k, stride, pad) of the 53 ResNet-50 v1.5 convolutions."""
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


def _geometry(xs, cout, k, s, p, batch):
    return ((batch,) + tuple(xs[1:]), cout, (k, k), (s, s), (p, p), (1, 1), 1)


def c3_geometries(batch=2):
    """Distinct layer shapes of the C3 stack at a test batch, raised where the
    output plane is small so the weight gradient still has at least 512
    positions to split (7x7 planes: batch 11)."""
    seen, out = set(), []
    for _, xs, cout, k, s, p in resnet50_layers(batch):
        oh = (xs[2] + 2 * p - k) // s + 1
        b = max(batch, -(-512 // (oh * oh)))
        g = _geometry(xs, cout, k, s, p, b)
        if g not in seen:
            seen.add(g)
            out.append(g)
    return out


def c4_conv_geometries(calls, batch=2):
    """Distinct conv shapes of captured C4 calls, at a test batch."""
    seen, out = set(), []
    for c in calls:
        if c["kind"] != "conv":
            continue
        xs, cout, k, stride, padding, dilation, groups = c["geometry"]
        g = ((batch,) + tuple(xs[1:]), cout, tuple(k), stride, padding, dilation, groups)
        if g not in seen:
            seen.add(g)
            out.append(g)
    return out


# Forced implicit-GEMM plans: every tile of the menu (conv::Tile order:
# 256x128, 128x256, 128x128, 64x256, 256x64, 64x64), each with no split, two
# splits and as many as the shape allows.  A tile a phase cannot use (256x64
# for forward / dInput, the 256-wide-column tiles for a gathered dWeight)
# leaves that phase to its planner, which the variant names record.
CONV_TILES = list(range(6))
SPLITS = (1, 2, 512)


def conv_plan_env(tile, splits):
    return {"MX_CONV_PLAN": f"{tile},{splits}"}


# Winograd: fused (ragged and even channel slabs) and unfused passes with every
# GEMM tile, in one pass or in image chunks under a small workspace budget.
WINOGRAD_GEOMETRIES = [
    ((2, 64, 14, 14), 64, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((3, 20, 9, 11), 24, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((2, 32, 8, 8), 32, (3, 3), (1, 1), (0, 0), (1, 1), 2),
    ((5, 128, 7, 7), 128, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((8, 64, 8, 8), 64, (3, 3), (1, 1), (1, 1), (1, 1), 1),  # 1 MiB budget: two image chunks
]
WINOGRAD_MODES = [
    {"MX_WINOGRAD_FUSED": "1", "MX_WINOGRAD_FILTER": "0", "MX_WINOGRAD_T16": "0"},
    {"MX_WINOGRAD_FUSED": "1", "MX_WINOGRAD_FILTER": "0", "MX_WINOGRAD_T16": "1"},
    {"MX_WINOGRAD_FUSED": "1", "MX_WINOGRAD_FILTER": "1"},
    {"MX_WINO_DW_WS": "0"},
    {"MX_WINO_DW_WS": "1"},
    {},
    *[{"MX_WINOGRAD_FUSED": "0", "MX_GEMM_TILE": str(t)} for t in range(4)],
    *[{"MX_WINOGRAD_FUSED": "0", "MX_GEMM_TILE": str(t), "TORCH_VULKAN_CONV_WORKSPACE_MB": "1"} for t in range(4)],
    {"TORCH_VULKAN_CONV_WORKSPACE_MB": "0"},
]

# ------------------------------------------------------------------ GEMM cases
# Shapes with K >= 1024 and M, N off every tile boundary; the first keeps the
# 16-byte operand modes (multiples of four), the second forces scalar modes.
GEMM_SHAPES = [(300, 516, 1028), (301, 517, 1029), (68, 132, 2052)]
GEMM_LAYOUTS = ["nn", "tn", "nt", "tt"]
GEMM_BIAS = ["none", "col", "matrix"]
GEMM_TILES = [0, 1, 2, 3]


@contextlib.contextmanager
def env(values):
    """Temporarily set environment variables (the planners read them per call)."""
    old = {k: os.environ.get(k) for k in values}
    os.environ.update({k: str(v) for k, v in values.items()})
    try:
        yield
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


class Shaped:
    """Shape / stride / offset stand-in for a tensor (what mx.gemm_desc reads)."""

    def __init__(self, shape, stride, offset=0):
        self.shape, self._stride, self._offset = tuple(shape), tuple(stride), offset

    def dim(self):
        return len(self.shape)

    def stride(self, i=None):
        return self._stride if i is None else self._stride[i]

    def storage_offset(self):
        return self._offset

    def expand(self, *sizes):
        sizes = sizes[0] if len(sizes) == 1 and isinstance(sizes[0], (tuple, list)) else sizes
        pad = len(sizes) - len(self.shape)
        st = [0] * pad + list(self._stride)
        sh = [1] * pad + list(self.shape)
        return Shaped(sizes, [0 if sh[i] == 1 and sizes[i] != 1 else st[i] for i in range(len(sizes))], self._offset)

    def t(self):
        return Shaped(self.shape[::-1], self._stride[::-1], self._offset)


def contiguous(shape):
    st, acc = [], 1
    for s in reversed(shape):
        st.append(acc)
        acc *= s
    return Shaped(shape, list(reversed(st)))


def layout_operands(m, n, k, layout, batch=None):
    """A [m, k] and B [k, n] as row-major ("n") or transposed views ("t")."""
    pre = (batch,) if batch else ()

    def mat(r, c, trans):
        if not trans:
            return contiguous(pre + (r, c))
        base = contiguous(pre + (c, r))
        st = base.stride()
        return Shaped(pre + (r, c), st[:-2] + (st[-1], st[-2]))

    return mat(m, k, layout[0] == "t"), mat(k, n, layout[1] == "t")


# ------------------------------------------------------------------ configuration calls
def c1_calls():
    """C1 as bench.py runs it: one 3x3 layer, forward + dInput + dWeight + dBias,
    every phase on Winograd (dBias in the weight-gradient launch); and the same
    layer with every phase on the implicit GEMM (its comparison line)."""
    g = ((8, 64, 56, 56), 64, (3, 3), (1, 1), (1, 1), (1, 1), 1)
    routed = [("winograd", 0), ("winograd", 1), ("winograd", 2)]
    implicit = [("implicit_gemm", ph) for ph in (0, 1, 2)]
    return [{"kind": "conv", "geometry": g, "phase": ph, "algo": a, "with_bias": True} for a, ph in routed + implicit]


def c2_calls():
    """C2's GEMMs as (label, A, B, C, bias, beta): Linear forward addmm(b, X, W^T),
    dX = dY W, dW = dY^T X, and the transposed-input variants X^T G and X W^T."""
    M, K, N = 8192, 4096, 4096
    X, W, dY = contiguous((M, K)), contiguous((N, K)), contiguous((M, N))
    b = contiguous((N,))
    return [
        ("addmm X.W^T+b", X, W.t(), contiguous((M, N)), b, 1.0),
        ("dX=dY.W", dY, W, contiguous((M, K)), None, 0.0),
        ("dW=dY^T.X", dY.t(), X, contiguous((N, K)), None, 0.0),
        ("X^T.G", X.t(), dY, contiguous((K, N)), None, 0.0),
        ("X.W^T", X, W.t(), contiguous((M, N)), None, 0.0),
    ]


def c3_calls(batch=64):
    """C3 as bench.py runs it: 3x3 stride-1 layers on Winograd in all three
    phases, the rest on the implicit GEMM; no bias; the stem has no dInput."""
    out = []
    for name, xs, cout, k, s, p in resnet50_layers(batch):
        g = _geometry(xs, cout, k, s, p, batch)
        algo = "winograd" if (k == 3 and s == 1) else "implicit_gemm"
        for ph in (0, 1, 2):
            if name == "stem" and ph == 1:
                continue
            out.append({"kind": "conv", "geometry": g, "phase": ph, "algo": algo, "with_bias": False})
    return out


def c4_calls(batch=16, image=64):
    """Conv and GEMM calls of one C4 training step, captured from the U-Net on
    the meta device (shapes and strides only, as the "vulkan" device receives
    them through aten.convolution / convolution_backward / bmm / mm)."""
    import torch
    from torch.nn import functional as F
    from torch.utils._python_dispatch import TorchDispatchMode

    import unet_c4 as U

    aten = torch.ops.aten
    calls = []

    def shaped(t):
        return Shaped(t.shape, t.stride(), t.storage_offset())

    class Capture(TorchDispatchMode):
        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            kwargs = kwargs or {}
            if func is aten.convolution.default:
                x, w, bias, stride, padding, dilation, transposed, _, groups = args
                calls.append({"kind": "conv", "x": tuple(x.shape), "w": tuple(w.shape), "stride": tuple(stride),
                              "padding": tuple(padding), "dilation": tuple(dilation), "groups": groups,
                              "phases": [0], "with_bias": bias is not None})
            elif func is aten.convolution_backward.default:
                _, x, w, bias_sizes, stride, padding, dilation, _, _, groups, mask = args
                phases = [ph for ph, on in zip((1, 2), mask[:2]) if on]
                calls.append({"kind": "conv", "x": tuple(x.shape), "w": tuple(w.shape), "stride": tuple(stride),
                              "padding": tuple(padding), "dilation": tuple(dilation), "groups": groups,
                              "phases": phases, "with_bias": bool(mask[2])})
            elif func in (aten.bmm.default, aten.mm.default):
                a, b = args[0], args[1]
                c = contiguous(tuple(a.shape[:-1]) + (b.shape[-1],))
                calls.append({"kind": "gemm", "label": str(func), "a": shaped(a), "b": shaped(b), "c": c,
                              "bias": None, "beta": 0.0})
            elif func in (aten.addmm.default, aten.baddbmm.default):
                bias, a, b = args[0], args[1], args[2]
                c = contiguous(tuple(a.shape[:-1]) + (b.shape[-1],))
                calls.append({"kind": "gemm", "label": str(func), "a": shaped(a), "b": shaped(b), "c": c,
                              "bias": shaped(bias), "beta": float(kwargs.get("beta", 1.0))})
            return func(*args, **kwargs)

    model = U.make_model().to("meta")
    x = torch.empty(batch, 3, image, image, device="meta")
    t = torch.empty(batch, 3, image, image, device="meta")
    with Capture():
        loss = F.mse_loss(model(x), t)
        loss.backward()
    out = []
    for c in calls:
        if c["kind"] == "conv":
            g = (c["x"], c["w"][0], c["w"][2:], c["stride"], c["padding"], c["dilation"], c["groups"])
            for ph in c["phases"]:
                out.append({"kind": "conv", "geometry": g, "phase": ph, "algo": "auto",
                            "with_bias": c["with_bias"] and ph != 1})
        else:
            out.append(c)
    return out
