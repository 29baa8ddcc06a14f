"""bench.py's host-side helpers (no GPU): the roofline class picker."""
import importlib.util
import os

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(REPO, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_roofline_prefers_single_kernel_classes(bench):
    # label: (launches, total ms, direct FLOPs, bytes)
    agg = {"winograd_dweight": (10, 0.40, 1e10, 0), "conv_fwd_kernel<64x64x16>": (10, 0.30, 1e10, 0)}
    r = bench.roofline_from(agg, "mfma", 0.5)
    assert r["kernel"] == "conv_fwd_kernel<64x64x16>"
    assert r["achieved"] == pytest.approx(1e9 / 30e-6 / 1e12, rel=1e-3)
    assert "note" not in r


def test_roofline_whole_winograd_call_at_executed_flops(bench):
    agg = {"winograd_forward": (10, 0.20, 1e10, 0), "winograd_dweight": (10, 0.40, 1e10, 0)}
    r = bench.roofline_from(agg, "mfma", 0.5)
    assert r["kernel"] == "winograd_dweight"
    # 1e9 direct FLOPs per call at half executed, 40 us per call
    assert r["achieved"] == pytest.approx(0.5e9 / 40e-6 / 1e12, rel=1e-3)
    assert r["avg_launch_us"] == pytest.approx(40.0)
    assert "Winograd" in r["note"]
