"""Warp-specialized Winograd weight gradient at several range counts, and the
combined backward entry point.

The kernel splits the output tiles into ranges whose partials a finalize
launch sums in a fixed order; with whole 64 x 32 channel blocks it stages
each partial in LDS and writes it as 16-byte rows.  These cases check dW and
dB against float64 CPU torch (rel 1e-3, the Winograd bound of
tests/helpers.py; dB at rel 1e-4), with and without dBias, for run-to-run
bit identity, and on a second stream.  The reference's weight gradient is
the direct / tiled one (conv2d_backward_weight_tiled_body.glsl, finalize
conv2d_backward_weight_finalize.comp); the Winograd weight gradient is this
build's, pinned here and in oracle/winograd.py.
"""
import math

import pytest
import torch

from helpers import WINOGRAD_RTOL, assert_close_mag, conv_refs

pytestmark = pytest.mark.gpu

# x shape, output channels, groups: C1's layer (98 ranges, 16-byte rows),
# uneven ranges, two filter groups, a few ranges, a ragged channel block
# (scalar stores).
CASES = [((8, 64, 56, 56), 64, 1), ((3, 64, 20, 22), 128, 1), ((4, 128, 14, 14), 128, 2), ((5, 64, 9, 13), 64, 1),
         ((2, 40, 12, 12), 48, 1)]


@pytest.fixture(scope="module")
def mx():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from torch_vulkan import mx as m
    m.lib()
    return m


@pytest.mark.parametrize("case", CASES, ids=[f"w{i}" for i in range(len(CASES))])
def test_winograd_dweight_ranges(mx, case):
    xs, cout, groups = case
    g = torch.Generator().manual_seed(sum(xs) + cout)
    x = torch.randn(xs, generator=g)
    w = torch.randn(cout, xs[1] // groups, 3, 3, generator=g) / math.sqrt(9 * xs[1] // groups)
    d = mx.conv_desc(xs, w.shape, (1, 1), (1, 1), (1, 1), groups)
    dy = torch.randn(xs[0], cout, d.oh, d.ow, generator=g)
    refs = conv_refs(x, w, torch.zeros(cout), dy, (1, 1), (1, 1), (1, 1), groups)
    plan = mx.conv2d_plan(d, mx.MX_CONV_DWEIGHT, mx.ALGO_WINOGRAD)
    print(f"[wino_dw] {case}: {plan}", flush=True)
    assert plan["variant"].startswith("wino_dw_ws_kernel")
    X, DY = x.cuda(), dy.cuda()
    st = torch.cuda.current_stream().cuda_stream
    first = None
    for with_db in (True, False):
        dw = torch.full(w.shape, float("nan"), device="cuda")
        db = torch.full((cout,), float("nan"), device="cuda") if with_db else None
        mx.conv2d_backward_weight(d, X, DY, dw, db, mx.ALGO_WINOGRAD, st)
        assert_close_mag(dw, *refs["dw"], rtol=WINOGRAD_RTOL, what=f"dw db={with_db}")
        if with_db:
            assert_close_mag(db, *refs["db"], what="db")
        first = dw.clone() if first is None else first
    side = torch.cuda.Stream()
    for stream in (torch.cuda.current_stream(), side, torch.cuda.current_stream()):
        with torch.cuda.stream(stream):
            dw = torch.empty(w.shape, device="cuda")
            db = torch.empty(cout, device="cuda")
            mx.conv2d_backward_weight(d, X, DY, dw, db, mx.ALGO_WINOGRAD, stream.cuda_stream)
        stream.synchronize()
        assert torch.equal(dw, first), "the weight gradient differs between calls"


# The combined backward entry point (mx_conv2d_backward): one launch for both
# Winograd gradients where its rule picks it (C1's layer, small layers) or
# where MX_WINOGRAD_BWD=1 forces it, the two calls otherwise; bit-identical to
# mx_conv2d_backward_input + mx_conv2d_backward_weight in every case.
# x shape, output channels, padding, MX_WINOGRAD_BWD, MX_WINOGRAD_FILTER
BWD_CASES = [((8, 64, 56, 56), 64, (1, 1), "auto", "auto"), ((8, 64, 56, 56), 64, (1, 1), "1", "0"),
             ((3, 33, 17, 15), 40, (1, 1), "auto", "auto"), ((4, 128, 14, 14), 128, (1, 1), "1", "auto"),
             ((2, 64, 16, 16), 128, (0, 0), "1", "1"), ((2, 40, 12, 12), 48, (2, 2), "1", "auto"),
             ((2, 64, 16, 16), 64, (1, 1), "0", "auto")]


@pytest.mark.parametrize("case", BWD_CASES, ids=[f"b{i}" for i in range(len(BWD_CASES))])
def test_combined_backward_matches_separate_calls(mx, case, monkeypatch):
    xs, cout, pad, mode, filt = case
    if mode != "auto":
        monkeypatch.setenv("MX_WINOGRAD_BWD", mode)
    if filt != "auto":
        monkeypatch.setenv("MX_WINOGRAD_FILTER", filt)
    g = torch.Generator().manual_seed(sum(xs) + cout + pad[0])
    x = torch.randn(xs, generator=g)
    w = torch.randn(cout, xs[1], 3, 3, generator=g) / math.sqrt(9 * xs[1])
    d = mx.conv_desc(xs, w.shape, (1, 1), pad)
    dy = torch.randn(xs[0], cout, d.oh, d.ow, generator=g)
    refs = conv_refs(x, w, torch.zeros(cout), dy, (1, 1), pad, (1, 1), 1)
    X, W, DY = x.cuda(), w.cuda(), dy.cuda()
    st = torch.cuda.current_stream().cuda_stream
    A = mx.ALGO_WINOGRAD
    shapes = (xs, w.shape, (cout,))
    for mask in ((1, 1, 1), (1, 1, 0), (1, 0, 0), (0, 1, 1), (0, 0, 1)):
        # the separate calls: dx alone, then dw and / or db in one weight call
        sep = [torch.empty(sh, device="cuda") if m else None for sh, m in zip(shapes, mask)]
        if sep[0] is not None:
            mx.conv2d_backward_input(d, DY, W, sep[0], A, st)
        if sep[1] is not None or sep[2] is not None:
            mx.conv2d_backward_weight(d, X, DY, sep[1], sep[2], A, st)
        out = [torch.full(sh, float("nan"), device="cuda") if m else None for sh, m in zip(shapes, mask)]
        mx.conv2d_backward(d, X, W, DY, *out, A, A, st)
        torch.cuda.synchronize()
        for name, got, want in zip(("dx", "dw", "db"), out, sep):
            if got is not None:
                assert torch.equal(got, want), f"{case} mask {mask}: {name} differs from the separate call"
                assert_close_mag(got, *refs[name], rtol=WINOGRAD_RTOL if name != "db" else 1e-4, what=name)


def test_combined_backward_other_algorithms(mx):
    """Implicit-GEMM gradients through the combined entry point: the two calls."""
    xs, cout = (2, 32, 12, 12), 48
    g = torch.Generator().manual_seed(5)
    x, w = torch.randn(xs, generator=g), torch.randn(cout, 32, 3, 3, generator=g) / 17
    d = mx.conv_desc(xs, w.shape, (2, 2), (1, 1))
    dy = torch.randn(xs[0], cout, d.oh, d.ow, generator=g)
    refs = conv_refs(x, w, torch.zeros(cout), dy, (2, 2), (1, 1), (1, 1), 1)
    dx, dw, db = torch.empty(xs, device="cuda"), torch.empty(w.shape, device="cuda"), torch.empty(cout, device="cuda")
    mx.conv2d_backward(d, x.cuda(), w.cuda(), dy.cuda(), dx, dw, db, mx.ALGO_AUTO, mx.ALGO_AUTO,
                       torch.cuda.current_stream().cuda_stream)
    for name, got in (("dx", dx), ("dw", dw), ("db", db)):
        assert_close_mag(got, *refs[name], what=name)
