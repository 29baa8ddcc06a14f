"""The C-ABI library on the CPU (no GPU calls): it loads, exports every entry
point include/mx.h declares, and its host-side validation and planning behave
like the reference's (csrc/ops/convolution.cpp:101-156 checks before any
launch; forced-but-inapplicable algorithms raise, :472-473)."""
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def mx():
    from torch_vulkan import mx as m
    m.lib()
    return m


def header_symbols():
    text = open(os.path.join(REPO, "include", "mx.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(mx):
    syms = header_symbols()
    assert len(syms) >= 40
    missing = [s for s in syms if not hasattr(mx.lib(), s)]
    assert not missing, missing
    assert sorted(mx.EXPORTS) == syms, "ctypes binding and header disagree"


def test_library_links_torch_hip_runtime_only():
    import subprocess
    so = os.path.join(REPO, "pytorch-vulkan_amd", "torch_vulkan", "libmx.so")
    out = subprocess.run(["readelf", "-d", so], capture_output=True, text=True).stdout
    assert "libamdhip64" in out and "torch/lib" in out


def test_link_resolves_without_the_wheels_hip_runtime(tmp_path):
    """With a torch wheel that ships no HIP runtime (CPU-only torch) libmx.so
    links ROCm's: the link of the built objects succeeds against an empty
    torch lib directory and the library's rpath then points at ROCm."""
    import glob
    import subprocess
    import sys
    sys.path.insert(0, os.path.join(REPO, "pytorch-vulkan_amd"))
    import build
    objs = sorted(glob.glob(os.path.join(REPO, "pytorch-vulkan_amd", "_build", "mx_*.o")))
    if len(objs) < len(build.MX_SOURCES):
        pytest.skip("objects not built (run build.py first)")
    empty = tmp_path / "torch_lib"
    empty.mkdir()
    runtime = build.hip_runtime_dir(str(empty))
    assert runtime != str(empty) and glob.glob(os.path.join(runtime, "libamdhip64.so*"))
    out = tmp_path / "libmx.so"
    build.link_mx(objs, out, runtime)
    dyn = subprocess.run(["readelf", "-d", str(out)], capture_output=True, text=True).stdout
    assert "libamdhip64" in dyn and runtime in dyn and "torch/lib" not in dyn
    ldd = subprocess.run(["ldd", str(out)], capture_output=True, text=True).stdout
    assert "not found" not in ldd and runtime in ldd


def test_conv_check_fills_output_shape(mx):
    d = mx.conv_desc((8, 64, 56, 56), (64, 64, 3, 3), (1, 1), (1, 1))
    assert (d.oh, d.ow) == (56, 56)
    d = mx.conv_desc((64, 3, 224, 224), (64, 3, 7, 7), (2, 2), (3, 3))
    assert (d.oh, d.ow) == (112, 112)


@pytest.mark.parametrize("xs,ws,kw,msg", [
    ((1, 2, 2, 2), (3, 2, 3, 3), dict(stride=(2, 2)), "effective kernel exceeds padded input"),
    ((1, 4, 5, 5), (3, 2, 1, 1), dict(groups=3), "invalid shapes"),
    ((1, 1, 1, 1), (1, 1, 1, 1), dict(stride=(2147483647, 2147483647), padding=(2147483647, 2147483647)),
     "int32 coordinates"),
])
def test_conv_validation_errors(mx, xs, ws, kw, msg):
    with pytest.raises(mx.MXError, match=msg):
        mx.conv_desc(xs, ws, kw.get("stride", (1, 1)), kw.get("padding", (0, 0)), (1, 1), kw.get("groups", 1))


def test_planner_mirrors_reference_heuristic(mx):
    """The reference's candidates (csrc/ops/convolution.cpp:423-482) except
    for dense 3x3 stride-1 layers, which AUTO routes to Winograd in every
    phase above the measured break-even sizes."""
    dense = mx.conv_desc((8, 64, 56, 56), (64, 64, 3, 3), (1, 1), (1, 1))
    for phase in (mx.MX_CONV_FORWARD, mx.MX_CONV_DINPUT, mx.MX_CONV_DWEIGHT):
        assert mx.conv2d_select(dense, phase) == mx.ALGO_WINOGRAD
    assert mx.conv2d_select(dense, mx.MX_CONV_DBIAS) == mx.ALGO_REDUCE
    dense5 = mx.conv_desc((8, 64, 56, 56), (64, 64, 3, 5), (1, 1), (1, 2))
    assert mx.conv2d_select(dense5, mx.MX_CONV_FORWARD) == mx.ALGO_IMPLICIT_GEMM
    assert mx.conv2d_select(dense5, mx.MX_CONV_DINPUT) == mx.ALGO_IMPLICIT_GEMM
    assert mx.conv2d_select(dense5, mx.MX_CONV_DWEIGHT) == mx.ALGO_IMPLICIT_GEMM
    strided = mx.conv_desc((8, 64, 56, 56), (64, 64, 3, 3), (2, 2), (1, 1))
    assert mx.conv2d_select(strided, mx.MX_CONV_FORWARD) == mx.ALGO_IMPLICIT_GEMM
    # Break-even sizes.  Forward / dInput: 16384 output positions, or 512 when
    # the channel walk (cin forward, cout dInput) is at most 4x the channels
    # produced.  dWeight: 2^25 multiply-adds per filter tap (positions x cin
    # per group x cout).
    b1 = mx.conv_desc((1, 64, 32, 32), (64, 64, 3, 3), (1, 1), (1, 1))     # 1024 positions
    assert mx.conv2d_select(b1, mx.MX_CONV_FORWARD) == mx.ALGO_WINOGRAD
    assert mx.conv2d_select(b1, mx.MX_CONV_DINPUT) == mx.ALGO_WINOGRAD
    assert mx.conv2d_select(b1, mx.MX_CONV_DWEIGHT) == mx.ALGO_IMPLICIT_GEMM
    b512 = mx.conv_desc((2, 64, 16, 16), (64, 64, 3, 3), (1, 1), (1, 1))   # 512 positions
    assert mx.conv2d_select(b512, mx.MX_CONV_FORWARD) == mx.ALGO_WINOGRAD
    b511 = mx.conv_desc((1, 64, 7, 73), (64, 64, 3, 3), (1, 1), (1, 1))    # 511 positions
    assert mx.conv2d_select(b511, mx.MX_CONV_FORWARD) == mx.ALGO_IMPLICIT_GEMM
    walk = mx.conv_desc((16, 1024, 8, 8), (32, 1024, 3, 3), (1, 1), (1, 1))  # walk 32x the outputs
    assert mx.conv2d_select(walk, mx.MX_CONV_FORWARD) == mx.ALGO_IMPLICIT_GEMM
    assert mx.conv2d_select(walk, mx.MX_CONV_DINPUT) == mx.ALGO_WINOGRAD   # walks 32 output channels
    four = mx.conv_desc((16, 512, 8, 8), (128, 512, 3, 3), (1, 1), (1, 1))   # walk exactly 4x
    assert mx.conv2d_select(four, mx.MX_CONV_FORWARD) == mx.ALGO_WINOGRAD
    five = mx.conv_desc((16, 640, 8, 8), (128, 640, 3, 3), (1, 1), (1, 1))   # 5x
    assert mx.conv2d_select(five, mx.MX_CONV_FORWARD) == mx.ALGO_IMPLICIT_GEMM
    many = mx.conv_desc((16, 1024, 32, 32), (32, 1024, 3, 3), (1, 1), (1, 1))  # 16384 positions
    assert mx.conv2d_select(many, mx.MX_CONV_FORWARD) == mx.ALGO_WINOGRAD
    dx_walk = mx.conv_desc((16, 32, 8, 8), (1024, 32, 3, 3), (1, 1), (1, 1))   # dInput walks 1024
    assert mx.conv2d_select(dx_walk, mx.MX_CONV_DINPUT) == mx.ALGO_IMPLICIT_GEMM
    assert mx.conv2d_select(dx_walk, mx.MX_CONV_FORWARD) == mx.ALGO_WINOGRAD
    deep = mx.conv_desc((16, 512, 8, 8), (512, 512, 3, 3), (1, 1), (1, 1))  # C4's 8x8 level: 2^28
    assert mx.conv2d_select(deep, mx.MX_CONV_DWEIGHT) == mx.ALGO_WINOGRAD
    at = mx.conv_desc((8, 64, 16, 16), (256, 64, 3, 3), (1, 1), (1, 1))     # 2048 x 64 x 256 = 2^25
    assert mx.conv2d_select(at, mx.MX_CONV_DWEIGHT) == mx.ALGO_WINOGRAD
    below = mx.conv_desc((8, 64, 16, 16), (255, 64, 3, 3), (1, 1), (1, 1))  # one output channel fewer
    assert mx.conv2d_select(below, mx.MX_CONV_DWEIGHT) == mx.ALGO_IMPLICIT_GEMM
    thin_many = mx.conv_desc((8, 32, 16, 16), (64, 32, 3, 3), (1, 1), (1, 1))  # 2048 positions, 2^22
    assert mx.conv2d_select(thin_many, mx.MX_CONV_FORWARD) == mx.ALGO_WINOGRAD
    assert mx.conv2d_select(thin_many, mx.MX_CONV_DWEIGHT) == mx.ALGO_IMPLICIT_GEMM
    grouped_w = mx.conv_desc((16, 512, 8, 8), (512, 256, 3, 3), (1, 1), (1, 1), (1, 1), 2)  # per group 2^27
    assert mx.conv2d_select(grouped_w, mx.MX_CONV_DWEIGHT) == mx.ALGO_WINOGRAD
    small = mx.conv_desc((1, 256, 14, 14), (256, 256, 3, 3), (1, 1), (1, 1))  # 196 positions
    for phase in (mx.MX_CONV_FORWARD, mx.MX_CONV_DINPUT, mx.MX_CONV_DWEIGHT):
        assert mx.conv2d_select(small, phase) == mx.ALGO_IMPLICIT_GEMM
    thin = mx.conv_desc((16, 16, 64, 64), (64, 16, 3, 3), (1, 1), (1, 1))     # 16 input channels
    assert mx.conv2d_select(thin, mx.MX_CONV_FORWARD) == mx.ALGO_IMPLICIT_GEMM
    wide_pad = mx.conv_desc((8, 64, 56, 56), (64, 64, 3, 3), (1, 1), (3, 3))  # padding beyond 2
    for phase in (mx.MX_CONV_FORWARD, mx.MX_CONV_DINPUT, mx.MX_CONV_DWEIGHT):
        assert mx.conv2d_select(wide_pad, phase) == mx.ALGO_IMPLICIT_GEMM
    grouped = mx.conv_desc((2, 128, 64, 64), (128, 16, 3, 3), (1, 1), (1, 1), (1, 1), 8)
    assert mx.conv2d_select(grouped, mx.MX_CONV_FORWARD) == mx.ALGO_WINOGRAD
    tiny = mx.conv_desc((1, 1, 4, 4), (2, 1, 1, 1))
    assert mx.conv2d_select(tiny, mx.MX_CONV_FORWARD) == mx.ALGO_DIRECT
    # 3-channel input conv and output head: every phase on the MFMA GEMM
    for x_shape, w_shape in (((16, 3, 64, 64), (128, 3, 3, 3)), ((16, 128, 64, 64), (3, 128, 3, 3))):
        d = mx.conv_desc(x_shape, w_shape, (1, 1), (1, 1))
        for phase in (mx.MX_CONV_FORWARD, mx.MX_CONV_DINPUT, mx.MX_CONV_DWEIGHT):
            assert mx.conv2d_select(d, phase) == mx.ALGO_IMPLICIT_GEMM


def test_depthwise_selection(mx):
    """Depthwise forward: AUTO for groups == cin >= 8 (csrc/ops/convolution.cpp:462),
    forced only where groups == cin (:361), never for a gradient."""
    dw = mx.conv_desc((2, 32, 28, 28), (64, 1, 3, 3), (1, 1), (1, 1), (1, 1), 32)
    assert mx.conv2d_select(dw, mx.MX_CONV_FORWARD) == mx.ALGO_DEPTHWISE
    assert mx.conv2d_kernel_name(dw, mx.MX_CONV_FORWARD) == "conv_depthwise_kernel"
    small = mx.conv_desc((1, 4, 8, 8), (4, 1, 3, 3), (1, 1), (1, 1), (1, 1), 4)
    assert mx.conv2d_select(small, mx.MX_CONV_FORWARD) == mx.ALGO_DIRECT
    assert mx.conv2d_select(small, mx.MX_CONV_FORWARD, mx.ALGO_DEPTHWISE) == mx.ALGO_DEPTHWISE
    grouped = mx.conv_desc((1, 16, 8, 8), (16, 8, 3, 3), (1, 1), (1, 1), (1, 1), 2)
    with pytest.raises(mx.MXError, match="depthwise"):
        mx.conv2d_select(grouped, mx.MX_CONV_FORWARD, mx.ALGO_DEPTHWISE)
    for phase in (mx.MX_CONV_DINPUT, mx.MX_CONV_DWEIGHT):
        with pytest.raises(mx.MXError):
            mx.conv2d_select(dw, phase, mx.ALGO_DEPTHWISE)
    with pytest.raises(mx.MXError, match="unknown algorithm"):
        mx.conv2d_select(dw, mx.MX_CONV_FORWARD, 9)


def test_forced_inapplicable_algorithm_raises(mx):
    strided = mx.conv_desc((1, 8, 9, 9), (8, 8, 3, 3), (2, 2), (1, 1))
    with pytest.raises(mx.MXError, match="winograd"):
        mx.conv2d_select(strided, mx.MX_CONV_FORWARD, mx.ALGO_WINOGRAD)
    with pytest.raises(mx.MXError):
        mx.conv2d_select(strided, mx.MX_CONV_DINPUT, mx.ALGO_WINOGRAD)
    # Winograd input gradients: 3x3 stride 1 with padding <= 2, only on request.
    same = mx.conv_desc((1, 8, 9, 9), (8, 8, 3, 3), (1, 1), (1, 1))
    assert mx.conv2d_select(same, mx.MX_CONV_DINPUT, mx.ALGO_WINOGRAD) == mx.ALGO_WINOGRAD
    assert mx.conv2d_select(same, mx.MX_CONV_DINPUT) == mx.ALGO_IMPLICIT_GEMM
    wide = mx.conv_desc((1, 8, 9, 9), (8, 8, 3, 3), (1, 1), (3, 3))
    with pytest.raises(mx.MXError, match="winograd"):
        mx.conv2d_select(wide, mx.MX_CONV_DINPUT, mx.ALGO_WINOGRAD)
    assert mx.conv2d_select(same, mx.MX_CONV_DWEIGHT, mx.ALGO_WINOGRAD) == mx.ALGO_WINOGRAD
    assert mx.conv2d_select(wide, mx.MX_CONV_DWEIGHT, mx.ALGO_WINOGRAD) == mx.ALGO_WINOGRAD
    assert mx.conv2d_select(same, mx.MX_CONV_DWEIGHT) == mx.ALGO_IMPLICIT_GEMM
    with pytest.raises(mx.MXError, match="winograd"):
        mx.conv2d_select(strided, mx.MX_CONV_DWEIGHT, mx.ALGO_WINOGRAD)
    assert mx.conv2d_kernel_name(same, mx.MX_CONV_DWEIGHT, mx.ALGO_WINOGRAD) in ("wino_dw_kernel", "wino_dw_ws_kernel")
    with pytest.raises(mx.MXError):
        mx.conv2d_select(strided, mx.MX_CONV_FORWARD, mx.ALGO_REDUCE)


def test_dweight_split_plan(mx):
    c1 = mx.conv_desc((8, 64, 56, 56), (64, 64, 3, 3), (1, 1), (1, 1))
    splits, span, ws = mx.dweight_plan(c1)
    assert splits >= 2 and span % 16 == 0 and splits * span >= 8 * 56 * 56 > (splits - 1) * span
    assert ws > 0
    small = mx.conv_desc((1, 9, 1, 64), (17, 9, 1, 1))
    assert mx.dweight_plan(small)[0] == 1


def test_kernel_names(mx):
    c1 = mx.conv_desc((8, 64, 56, 56), (64, 64, 3, 3), (1, 1), (1, 1))
    assert mx.conv2d_kernel_name(c1, mx.MX_CONV_FORWARD, mx.ALGO_IMPLICIT_GEMM).startswith("conv_fwd_kernel<")
    assert mx.conv2d_kernel_name(c1, mx.MX_CONV_DWEIGHT, mx.ALGO_IMPLICIT_GEMM).startswith("conv_dw_kernel<")
    assert mx.conv2d_kernel_name(c1, mx.MX_CONV_FORWARD, mx.ALGO_WINOGRAD).startswith("wino")
    # Winograd names are the kernels that carry the call (profiler names),
    # taken from the plan's variant.
    for phase in (mx.MX_CONV_FORWARD, mx.MX_CONV_DINPUT, mx.MX_CONV_DWEIGHT):
        variant = mx.conv2d_plan(c1, phase, mx.ALGO_WINOGRAD)["variant"]
        name = mx.conv2d_kernel_name(c1, phase, mx.ALGO_WINOGRAD)
        assert variant.startswith(name) and name in ("wino_ws_kernel", "wino_ws16_kernel", "wino_dw_ws_kernel",
                                                     "wino_dw_kernel"), (phase, name, variant)
    # C1's two Winograd gradients (AUTO's choice) run as one launch; the
    # implicit GEMM's do not.
    assert mx.conv2d_backward_one_launch(c1, mx.ALGO_WINOGRAD, mx.ALGO_WINOGRAD)
    assert mx.conv2d_backward_one_launch(c1, mx.ALGO_AUTO, mx.ALGO_AUTO)
    assert not mx.conv2d_backward_one_launch(c1, mx.ALGO_IMPLICIT_GEMM, mx.ALGO_IMPLICIT_GEMM)
    assert not mx.conv2d_backward_one_launch(c1, mx.ALGO_WINOGRAD, mx.ALGO_IMPLICIT_GEMM)


def test_gemm_rejects_bad_descriptor(mx):
    import ctypes as C
    d = mx.GemmDesc(batch=1, m=-1, n=2, k=2)
    with pytest.raises(mx.MXError, match="negative"):
        mx.check(mx.lib().mx_gemm_f32(C.byref(d), None, None, None, None, None))
    d = mx.GemmDesc(batch=1, m=2, n=2, k=2, bias_kind=7)
    with pytest.raises(mx.MXError, match="bias kind"):
        mx.check(mx.lib().mx_gemm_f32(C.byref(d), None, None, None, None, None))


def test_adamw_rejects_invalid_hyperparameters(mx):
    import ctypes as C
    hp = mx.AdamWHParams(lr=1e-3, beta1=1.0, beta2=0.999, eps=1e-8, weight_decay=0.0)
    with pytest.raises(mx.MXError, match="invalid hyperparameters"):
        mx.check(mx.lib().mx_adamw_step(None, 0, C.byref(hp), None, None))
    hp.beta1 = 0.9
    t = (mx.AdamWTensor * 1)()
    t[0].numel, t[0].step = 4, 0
    t[0].param = t[0].grad = t[0].exp_avg = t[0].exp_avg_sq = 16
    with pytest.raises(mx.MXError, match="step must be positive"):
        mx.check(mx.lib().mx_adamw_step(t, 1, C.byref(hp), None, None))


def test_last_error_is_thread_local_and_cleared(mx):
    d = mx.ConvDesc(n=1, cin=1, h=1, w=1, cout=1, kh=3, kw=3, sh=1, sw=1, ph=0, pw=0, dh=1, dw=1, groups=1)
    import ctypes as C
    assert mx.lib().mx_conv2d_check(C.byref(d)) != mx.MX_OK
    assert mx.lib().mx_last_error()
    ok = mx.ConvDesc(n=1, cin=1, h=3, w=3, cout=1, kh=3, kw=3, sh=1, sw=1, ph=0, pw=0, dh=1, dw=1, groups=1)
    assert mx.lib().mx_conv2d_check(C.byref(ok)) == mx.MX_OK
    assert mx.lib().mx_last_error() == b""


def test_conv_entry_points_reject_null_descriptor(mx):
    """Every convolution entry point returns MX_ERR_INVALID for a null
    descriptor (before touching the device), as for any other bad argument."""
    import ctypes as C
    L = mx.lib()
    algo = C.c_int()
    info = mx.ConvPlanInfo() if hasattr(mx, "ConvPlanInfo") else None
    buf = C.create_string_buffer(64)
    n1, n2, n3 = C.c_int64(), C.c_int64(), C.c_int64()
    calls = [
        lambda: L.mx_conv2d_select(None, mx.MX_CONV_FORWARD, mx.ALGO_AUTO, C.byref(algo)),
        lambda: L.mx_conv2d_forward(None, None, None, None, None, mx.ALGO_AUTO, None),
        lambda: L.mx_conv2d_backward_input(None, None, None, None, mx.ALGO_AUTO, None),
        lambda: L.mx_conv2d_backward_weight(None, None, None, None, None, mx.ALGO_AUTO, None),
        lambda: L.mx_conv2d_backward_bias(None, None, None, None),
        lambda: L.mx_conv2d_backward(None, None, None, None, None, None, None, mx.ALGO_AUTO, mx.ALGO_AUTO, None),
        lambda: L.mx_conv2d_backward_weight_noalloc(None, None, None, None, None, mx.ALGO_AUTO, None),
        lambda: L.mx_conv2d_kernel_name(None, mx.MX_CONV_FORWARD, mx.ALGO_AUTO, buf, len(buf)),
        lambda: L.mx_conv2d_backward_one_launch(None, mx.ALGO_AUTO, mx.ALGO_AUTO, 1, C.byref(algo)),
        lambda: L.mx_conv2d_dweight_plan(None, C.byref(n1), C.byref(n2), C.byref(n3)),
    ]
    if info is not None:
        calls.append(lambda: L.mx_conv2d_plan(None, mx.MX_CONV_FORWARD, mx.ALGO_AUTO, 0, C.byref(info)))
    for call in calls:
        with pytest.raises(mx.MXError, match="null (descriptor|argument)"):
            mx.check(call())


def test_tile_knob_changes_the_plan(mx, monkeypatch):
    """TORCH_VULKAN_CONV_TILE (csrc/ops/convolution.cpp:411-414) reaches the
    planner: C1's forward moves to the named tile of this build's menu, a
    fixed-3x3 name on a 1x1 layer plans the base tile under AUTO and is
    rejected when the tiled algorithm is forced, and an unknown name raises
    the reference's message."""
    d = mx.conv_desc((8, 64, 56, 56), (64, 64, 3, 3), (1, 1), (1, 1))
    tiles = {}
    for name in ("base", "wide", "tall", "register", "register3", "register3_hoist"):
        monkeypatch.setenv("TORCH_VULKAN_CONV_TILE", name)
        tiles[name] = mx.conv2d_plan(d, mx.MX_CONV_FORWARD, mx.ALGO_IMPLICIT_GEMM)["tile"]
        assert mx.conv2d_plan(d, mx.MX_CONV_DINPUT, mx.ALGO_IMPLICIT_GEMM)["tile"] >= 0
        assert mx.conv2d_plan(d, mx.MX_CONV_DWEIGHT, mx.ALGO_IMPLICIT_GEMM)["tile"] >= 0
    assert len({tiles[n] for n in ("base", "wide", "tall", "register")}) == 4, tiles
    assert tiles["register3_hoist"] == tiles["register"]
    monkeypatch.setenv("TORCH_VULKAN_CONV_TILE", "register3")
    pointwise = mx.conv_desc((8, 64, 56, 56), (64, 64, 1, 1))
    assert mx.conv2d_plan(pointwise, mx.MX_CONV_FORWARD)["tile"] == tiles["base"]
    with pytest.raises(mx.MXError, match="tiled_register3 exceeds"):
        mx.conv2d_select(pointwise, mx.MX_CONV_FORWARD, mx.ALGO_IMPLICIT_GEMM)
    monkeypatch.setenv("TORCH_VULKAN_CONV_TILE", "huge")
    with pytest.raises(mx.MXError, match="TORCH_VULKAN_CONV_TILE must be auto/base/wide/tall/register"):
        mx.conv2d_select(d, mx.MX_CONV_FORWARD)
    monkeypatch.setenv("TORCH_VULKAN_CONV_TILE", "auto")
    auto = mx.conv2d_plan(d, mx.MX_CONV_FORWARD)["tile"]
    monkeypatch.delenv("TORCH_VULKAN_CONV_TILE")
    assert mx.conv2d_plan(d, mx.MX_CONV_FORWARD)["tile"] == auto


def test_gemm_kernel_class_reaches_the_tile_choice(mx):
    """mx_gemm_desc.kernel, the counterpart of TORCH_VULKAN_MM_KERNEL
    (csrc/ops/mm.cpp:299-307): 'tiled' forces the 64x64 tile, 'register' keeps
    the large tiles even where the cost model would pick the small one."""
    def variant(m, n, k, kernel):
        d = mx.GemmDesc(batch=1, m=m, n=n, k=k, a_stride_m=k, a_stride_k=1, b_stride_k=n, b_stride_n=1, ldc=n,
                        alpha=1.0, kernel=kernel)
        return mx.gemm_variant(d)
    assert variant(8192, 4096, 4096, 1).startswith("gemm_kernel<64x64")
    assert not variant(8192, 4096, 4096, 0).startswith("gemm_kernel<64x64")
    assert not variant(8192, 4096, 4096, 2).startswith("gemm_kernel<64x64")
    assert variant(64, 64, 64, 0).startswith("gemm_kernel<64x64")
    assert not variant(64, 64, 64, 2).startswith("gemm_kernel<64x64")
    import ctypes as C
    d = mx.GemmDesc(batch=1, m=4, n=4, k=4, a_stride_m=4, a_stride_k=1, b_stride_k=4, b_stride_n=1, ldc=4, kernel=7)
    buf = C.create_string_buffer(64)
    with pytest.raises(mx.MXError, match="kernel class"):
        mx.check(mx.lib().mx_gemm_variant(C.byref(d), C.c_void_p(256), C.c_void_p(256), buf, 64))


def test_implicit_gemm_group_limit(mx):
    """The implicit GEMM runs one grid-z slice per group: past 65535 groups
    AUTO takes the direct kernels and a forced implicit GEMM is refused with a
    clear error, before any launch."""
    many = mx.conv_desc((1, 140000, 4, 4), (70000, 2, 3, 3), (1, 1), (1, 1), (1, 1), 70000)
    for phase in (mx.MX_CONV_FORWARD, mx.MX_CONV_DINPUT, mx.MX_CONV_DWEIGHT):
        assert mx.conv2d_select(many, phase) != mx.ALGO_IMPLICIT_GEMM
        with pytest.raises(mx.MXError, match="at most 65535 groups"):
            mx.conv2d_select(many, phase, mx.ALGO_IMPLICIT_GEMM)
    fine = mx.conv_desc((1, 40000, 4, 4), (20000, 2, 3, 3), (2, 2), (1, 1), (1, 1), 20000)
    assert mx.conv2d_select(fine, mx.MX_CONV_DINPUT, mx.ALGO_IMPLICIT_GEMM) == mx.ALGO_IMPLICIT_GEMM
