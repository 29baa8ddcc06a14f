"""Planner coverage on the host: every kernel instantiation the benchmark
configurations launch (C1, C2, C3 at batch 64, the C4 U-Net step at batch 16)
is one that a GPU parity case of tests/test_gpu_plans.py runs.

Variants come from the library's own planners (mx_conv2d_plan,
mx_gemm_variant) evaluated without a GPU (the plans only need shapes, strides,
alignment and the CU count, 256 on MI355X), under the same forcing environment
the GPU test sets.  The workspace budget is part of the plan, so its tests live
here too (ports of /root/reference/tests/test_conv_dispatch.py:255-309).
"""
from __future__ import annotations

import functools

import pytest

import plan_cases as P


@pytest.fixture(scope="module")
def mx():
    from torch_vulkan import mx as m
    m.lib()
    return m


def conv_desc(mx, g):
    xs, cout, k, s, p, dil, groups = g
    return mx.conv_desc(xs, (cout, xs[1] // groups, *k), s, p, dil, groups)


def algo_code(mx, name):
    return {"auto": mx.ALGO_AUTO, "implicit_gemm": mx.ALGO_IMPLICIT_GEMM, "winograd": mx.ALGO_WINOGRAD}[name]


def conv_variants(mx, g, phase, algo, with_bias):
    info = mx.conv2d_plan(conv_desc(mx, g), phase, algo, with_bias)
    return set(info["variant"].split())


def gemm_variant(mx, a, b, c, bias=None, beta=0.0):
    return mx.gemm_variant(mx.gemm_desc(a, b, c, bias=bias, beta=beta))


@functools.lru_cache(maxsize=None)
def variants_under_parity():
    """Variants the GPU parity cases of test_gpu_plans.py run."""
    from torch_vulkan import mx
    mx.lib()
    out = set()
    geoms = P.REFERENCE_GEOMETRIES + P.c3_geometries() + P.c4_conv_geometries(P.c4_calls())
    for g in geoms:
        for forced in [{}] + [P.conv_plan_env(t, s) for t in P.CONV_TILES for s in P.SPLITS]:
            with P.env(forced):
                for ph in (0, 1, 2):
                    for wb in ((False, True) if ph == 2 else (False,)):
                        out |= conv_variants(mx, g, ph, mx.ALGO_IMPLICIT_GEMM, wb)
    for g in P.WINOGRAD_GEOMETRIES + [g for g in P.c3_geometries() if g[2] == (3, 3) and g[3] == (1, 1)]:
        for mode in P.WINOGRAD_MODES:
            with P.env(mode):
                for ph in (0, 1, 2):
                    out |= conv_variants(mx, g, ph, mx.ALGO_WINOGRAD, False)
    for (m, n, k) in P.GEMM_SHAPES:
        for layout in P.GEMM_LAYOUTS:
            for batch in (None, 3):
                a, b = P.layout_operands(m, n, k, layout, batch)
                c = P.contiguous(((batch,) if batch else ()) + (m, n))
                for bias_kind in P.GEMM_BIAS:
                    bias = None if bias_kind == "none" else (P.contiguous((n,)) if bias_kind == "col"
                                                             else P.contiguous((m, n)))
                    for tile in P.GEMM_TILES:
                        with P.env({"MX_GEMM_TILE": tile}):
                            out.add(gemm_variant(mx, a, b, c, bias, 1.0 if bias is not None else 0.0))
    return out


def needed_variants(mx):
    """(variant, where) for every call of the benchmark configurations."""
    out = []
    for cfg, calls in (("C1", P.c1_calls()), ("C3", P.c3_calls()), ("C4", P.c4_calls())):
        for c in calls:
            if c["kind"] == "conv":
                for v in conv_variants(mx, c["geometry"], c["phase"], algo_code(mx, c["algo"]), c["with_bias"]):
                    out.append((v, f"{cfg} conv {c['geometry']} phase {c['phase']}"))
            else:
                out.append((gemm_variant(mx, c["a"], c["b"], c["c"], c["bias"], c["beta"]), f"{cfg} {c['label']}"))
    for label, a, b, c, bias, beta in P.c2_calls():
        out.append((gemm_variant(mx, a, b, c, bias, beta), f"C2 {label}"))
    return out


def test_every_configuration_variant_is_parity_tested(mx):
    tested = variants_under_parity()
    missing = sorted({(v, where) for v, where in needed_variants(mx) if v not in tested})
    assert not missing, "kernel variants without a parity case:\n  " + "\n  ".join(f"{v}  <- {w}" for v, w in missing)


def test_tile_menu_is_fully_tested(mx):
    """Every tile of each implicit-GEMM kernel appears in some tested variant."""
    tested = " ".join(variants_under_parity())
    for kind, tiles in (("conv_fwd_kernel", ["256x128x16", "128x256x16", "128x128x16", "64x256x16", "64x64x16"]),
                        ("conv_dx_kernel", ["256x128x16", "128x256x16", "128x128x16", "64x256x16", "64x64x16"]),
                        ("conv_dw_kernel", ["256x128x16", "128x256x16", "128x128x16", "64x256x16", "256x64x16",
                                            "64x64x32"]),
                        ("gemm_kernel", ["256x128x16", "128x256x16", "128x128x16", "64x64x16"])):
        for t in tiles:
            assert f"{kind}<{t}," in tested, f"{kind}<{t}> is not exercised by any parity case"


# ------------------------------------------------------------------ workspace budget
BUDGET_CASES = [  # /root/reference/tests/test_conv_dispatch.py:255-258
    ((1, 48, 64, 64), 96, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((1, 64, 64, 31), 128, (3, 5), (1, 2), (2, 3), (2, 1), 2),
]


@pytest.mark.parametrize("g", BUDGET_CASES)
@pytest.mark.parametrize("budget_mb", [1, 64])
def test_weight_split_fits_workspace(mx, g, budget_mb):
    """A forced many-way dWeight split shrinks to the budget; its partials
    cover the positions exactly and fit; the natural plan is kept when it fits."""
    d = conv_desc(mx, g)
    xs, cout, k, _, _, _, groups = g
    weight_bytes = cout * (xs[1] // groups) * k[0] * k[1] * 4
    positions = xs[0] * d.oh * d.ow
    with P.env({"TORCH_VULKAN_CONV_WORKSPACE_MB": budget_mb, "MX_CONV_PLAN": "5,512"}):
        plan = mx.conv2d_plan(d, mx.MX_CONV_DWEIGHT, mx.ALGO_IMPLICIT_GEMM, with_bias=False)
    parts, span = plan["splits"], plan["span"]
    assert 2 <= parts and span % 32 == 0
    assert (parts - 1) * span < positions <= parts * span
    assert plan["workspace_bytes"] == parts * weight_bytes <= budget_mb << 20
    with P.env({"TORCH_VULKAN_CONV_WORKSPACE_MB": 4096, "MX_CONV_PLAN": "5,512"}):
        free = mx.conv2d_plan(d, mx.MX_CONV_DWEIGHT, mx.ALGO_IMPLICIT_GEMM, with_bias=False)
    if free["workspace_bytes"] <= budget_mb << 20:
        assert plan == free
    else:
        assert parts < free["splits"] and span > free["span"]


def test_zero_workspace_plans_have_no_scratch(mx):
    with P.env({"TORCH_VULKAN_CONV_WORKSPACE_MB": 0}):
        for g in BUDGET_CASES + P.c3_geometries(batch=8):
            for ph in (0, 1, 2):
                for algo in (mx.ALGO_IMPLICIT_GEMM, mx.ALGO_WINOGRAD):
                    try:
                        plan = mx.conv2d_plan(conv_desc(mx, g), ph, algo, with_bias=True)
                    except mx.MXError as e:
                        assert e.status == mx.MX_ERR_UNSUPPORTED  # Winograd not applicable to this layer
                        continue
                    assert plan["workspace_bytes"] == 0 and plan["splits"] == 1, (g, ph, plan)


def test_forced_split_rejects_zero_workspace(mx):
    """/root/reference/tests/test_conv_dispatch.py:302-313."""
    d = mx.conv_desc((1, 9, 1, 257), (17, 9, 1, 1))
    with P.env({"TORCH_VULKAN_CONV_WORKSPACE_MB": 0, "MX_CONV_PLAN": "5,2"}):
        with pytest.raises(mx.MXError, match="[Ww]orkspace") as e:
            mx.conv2d_plan(d, mx.MX_CONV_DWEIGHT, mx.ALGO_IMPLICIT_GEMM)
    assert e.value.status == mx.MX_ERR_WORKSPACE
    with P.env({"TORCH_VULKAN_CONV_WORKSPACE_MB": 0, "MX_CONV_PLAN": "5,1"}):
        assert mx.conv2d_plan(d, mx.MX_CONV_DWEIGHT, mx.ALGO_IMPLICIT_GEMM)["splits"] == 1


@pytest.mark.parametrize("value", ["-1", "4097", "12x", " "])
def test_workspace_knob_is_validated(mx, value):
    d = mx.conv_desc((1, 9, 1, 257), (17, 9, 1, 1))
    with P.env({"TORCH_VULKAN_CONV_WORKSPACE_MB": value}):
        with pytest.raises(mx.MXError, match="TORCH_VULKAN_CONV_WORKSPACE_MB"):
            mx.conv2d_plan(d, mx.MX_CONV_DWEIGHT, mx.ALGO_IMPLICIT_GEMM)


def test_budget_bounds_every_configuration_call(mx):
    """At the default 64 MiB budget no C3 / C4 call plans more scratch."""
    for c in P.c3_calls() + [c for c in P.c4_calls() if c["kind"] == "conv"]:
        plan = mx.conv2d_plan(conv_desc(mx, c["geometry"]), c["phase"], algo_code(mx, c["algo"]), c["with_bias"])
        assert plan["workspace_bytes"] <= 64 << 20, (c, plan)
