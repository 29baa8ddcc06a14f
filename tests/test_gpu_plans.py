"""GPU parity of every kernel variant the planners can pick, forced one by one.

The case lists live in tests/plan_cases.py; tests/test_plan_coverage.py checks
on the host that they include every variant the C1-C4 configurations launch.
Each case runs through the C ABI (libmx.so) with its plan forced by the
environment the planners read per call:

* convolutions: every tile of the implicit-GEMM menu with no split, two splits
  and as many as the shape and workspace budget allow (MX_CONV_PLAN), forward,
  dInput, dWeight with and without the fused dBias, on the reference's 17
  dispatch geometries (tests/test_conv_dispatch.py:20-82 forces every tile on
  them the same way) and on every distinct layer shape of C3 and C4;
* Winograd F(2x2,3x3): fused, unfused with each GEMM tile, unfused in image
  chunks under a 1 MiB budget, and the no-scratch budget, all three phases;
* GEMM: every tile (MX_GEMM_TILE) on four operand layouts, plain / batched,
  no bias / column bias / matrix bias, K >= 1024 with M and N off every tile
  boundary (the reference sizes tests/test_fused_addmm.py:7-33 to reach its
  large register kernel in the same spirit).

References are float64 CPU torch on the same seeded inputs; the tolerance is
the north star's rel 1e-4 / abs 1e-5 (rel 1e-3 for Winograd) under the
magnitude model of tests/helpers.py, evaluated on the device.
"""
from __future__ import annotations

import math

import pytest
import torch

import plan_cases as P
from helpers import ATOL, RTOL, WINOGRAD_RTOL, conv_refs, gemm_mag

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mx():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from torch_vulkan import mx as m
    m.lib()
    return m


def stream():
    return torch.cuda.current_stream().cuda_stream


def check_dev(actual, ref, mag, rtol, atol, what):
    """|actual - ref| <= rtol |ref| + atol max(1, mag), elementwise on the device."""
    err = (actual.double() - ref).abs()
    bound = rtol * ref.abs() + atol * mag.clamp_min(1.0)
    bad = ~(err <= bound)
    nbad = int(bad.sum())
    if nbad:
        i = int(torch.nonzero(bad.flatten())[0])
        raise AssertionError(
            f"{what}: {nbad}/{bad.numel()} elements out of bound; first at {i}: actual="
            f"{actual.flatten()[i].item():.9g} ref={ref.flatten()[i].item():.9g} "
            f"max err/bound={float((err / bound).max()):.3g}")


def conv_inputs(g, seed):
    xs, cout, k, s, p, dil, groups = g
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(xs, generator=gen)
    w = torch.randn((cout, xs[1] // groups, *k), generator=gen) / math.sqrt(xs[1] // groups * k[0] * k[1])
    b = torch.randn(cout, generator=gen) * 0.1
    return x, w, b


def geom_id(g):
    xs, cout, k, s, p, dil, groups = g
    return f"{'x'.join(map(str, xs))}-{cout}-k{k[0]}x{k[1]}-s{s[0]}{s[1]}-p{p[0]}{p[1]}-d{dil[0]}{dil[1]}-g{groups}"


class ConvCase:
    """Seeded inputs, device buffers and float64 references of one geometry."""

    def __init__(self, mx, g):
        xs, cout, k, s, p, dil, groups = g
        self.d = mx.conv_desc(xs, (cout, xs[1] // groups, *k), s, p, dil, groups)
        x, w, b = conv_inputs(g, seed=sum(xs) + cout + k[0])
        dy = torch.randn((xs[0], cout, self.d.oh, self.d.ow), generator=torch.Generator().manual_seed(7))
        refs = conv_refs(x, w, b, dy, s, p, dil, groups)
        self.refs = {n: (r.cuda(), m.cuda()) for n, (r, m) in refs.items()}
        self.x, self.w, self.b, self.dy = (t.cuda() for t in (x, w, b, dy))
        self.y = torch.empty(self.refs["y"][0].shape, device="cuda")
        self.dx = torch.empty(xs, device="cuda")
        self.dw = torch.empty(w.shape, device="cuda")
        self.db = torch.empty(cout, device="cuda")

    def run(self, mx, phase, algo, with_bias, rtol, what):
        for t in (self.y, self.dx, self.dw, self.db):
            t.fill_(float("nan"))  # nothing stale can pass
        if phase == 0:
            mx.conv2d_forward(self.d, self.x, self.w, self.b, self.y, algo, stream())
            outs = [("y", self.y)]
        elif phase == 1:
            mx.conv2d_backward_input(self.d, self.dy, self.w, self.dx, algo, stream())
            outs = [("dx", self.dx)]
        else:
            mx.conv2d_backward_weight(self.d, self.x, self.dy, self.dw, self.db if with_bias else None, algo,
                                      stream())
            outs = [("dw", self.dw)] + ([("db", self.db)] if with_bias else [])
        for name, got in outs:
            ref, mag = self.refs[name]
            check_dev(got, ref, mag, rtol, ATOL, f"{what} {name}")


CONV_GEOMS = P.REFERENCE_GEOMETRIES + P.c3_geometries() + P.c4_conv_geometries(P.c4_calls())
FORCED = [{}] + [P.conv_plan_env(t, s) for t in P.CONV_TILES for s in P.SPLITS]
PHASES = ((0, False), (1, False), (2, False), (2, True))


@pytest.mark.parametrize("g", CONV_GEOMS, ids=[geom_id(g) for g in CONV_GEOMS])
def test_conv_forced_plans(mx, g):
    """Each distinct implicit-GEMM plan of the geometry (auto and every forced
    tile x split), every phase, against float64 CPU torch."""
    case = ConvCase(mx, g)
    seen = set()
    for forced in FORCED:
        with P.env(forced):
            for ph, wb in PHASES:
                plan = mx.conv2d_plan(case.d, ph, mx.ALGO_IMPLICIT_GEMM, wb)
                key = (ph, wb, plan["variant"], plan["splits"], plan["span"])
                if key in seen:
                    continue
                seen.add(key)
                print(f"[plans] {geom_id(g)} {forced} phase {ph} bias {wb}: {plan}", flush=True)
                case.run(mx, ph, mx.ALGO_IMPLICIT_GEMM, wb, RTOL, f"{forced} phase {ph} {plan}")
    torch.cuda.synchronize()


WINO_GEOMS = P.WINOGRAD_GEOMETRIES + [g for g in P.c3_geometries() if g[2] == (3, 3) and g[3] == (1, 1)]


@pytest.mark.parametrize("g", WINO_GEOMS, ids=[geom_id(g) for g in WINO_GEOMS])
def test_winograd_modes(mx, g):
    case = ConvCase(mx, g)
    seen = set()
    for mode in P.WINOGRAD_MODES:
        with P.env(mode):
            for ph in (0, 1, 2):
                plan = mx.conv2d_plan(case.d, ph, mx.ALGO_WINOGRAD, False)
                key = (ph, plan["variant"], plan["workspace_bytes"])
                if key in seen:
                    continue
                seen.add(key)
                print(f"[plans] {geom_id(g)} {mode} phase {ph}: {plan}", flush=True)
                case.run(mx, ph, mx.ALGO_WINOGRAD, False, WINOGRAD_RTOL, f"{mode} phase {ph} {plan}")
    torch.cuda.synchronize()


def gemm_operand(rows, cols, trans, batch, gen):
    """[batch,] rows x cols as a row-major matrix or a transposed view."""
    pre = (batch,) if batch else ()
    if not trans:
        return torch.randn(pre + (rows, cols), generator=gen)
    return torch.randn(pre + (cols, rows), generator=gen).transpose(-1, -2)


def to_dev(t):
    """Device copy with the same strides (a transposed view stays a view)."""
    if t.is_contiguous():
        return t.cuda()
    return t.transpose(-1, -2).contiguous().cuda().transpose(-1, -2)


@pytest.mark.parametrize("shape", P.GEMM_SHAPES, ids=["x".join(map(str, s)) for s in P.GEMM_SHAPES])
@pytest.mark.parametrize("layout", P.GEMM_LAYOUTS)
@pytest.mark.parametrize("batch", [None, 3], ids=["2d", "b3"])
def test_gemm_forced_tiles(mx, shape, layout, batch):
    m, n, k = shape
    gen = torch.Generator().manual_seed(m + n + k + (batch or 0))
    a = gemm_operand(m, k, layout[0] == "t", batch, gen)
    b = gemm_operand(k, n, layout[1] == "t", batch, gen)
    biases = {"none": None, "col": torch.randn(n, generator=gen), "matrix": torch.randn(m, n, generator=gen)}
    A, B = to_dev(a), to_dev(b)
    prod = a.double() @ b.double()
    mag0 = gemm_mag(a, b)
    c = torch.empty(((batch,) if batch else ()) + (m, n), device="cuda")
    for kind, bias in biases.items():
        beta = 1.0 if bias is not None else 0.0
        ref = prod + (bias.double() if bias is not None else 0.0)
        mag = mag0 + (bias.double().abs() if bias is not None else 0.0)
        ref_d, mag_d = ref.cuda(), mag.expand_as(ref).contiguous().cuda()
        bias_d = bias.cuda() if bias is not None else None
        for tile in P.GEMM_TILES:
            with P.env({"MX_GEMM_TILE": tile}):
                name = mx.gemm_variant(mx.gemm_desc(A, B, c, bias=bias_d, beta=beta))
                c.fill_(float("nan"))
                mx.gemm(A, B, c, bias=bias_d, beta=beta, stream=stream())
                check_dev(c, ref_d, mag_d, RTOL, ATOL, f"tile {tile} bias {kind} {name}")
    torch.cuda.synchronize()
