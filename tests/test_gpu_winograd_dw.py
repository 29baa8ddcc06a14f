"""Warp-specialized Winograd weight gradient at several range counts.

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
        assert_close_mag(dw, *refs["dw"], rtol=WINOGRAD_RTOL, atol=1e-4, what=f"dw db={with_db}")
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
