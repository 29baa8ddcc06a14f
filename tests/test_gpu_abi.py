"""GPU parity through the C ABI (include/mx.h) against CPU PyTorch on the same
seeded inputs.

Device buffers are torch ROCm tensors (plumbing only); every product call goes
through libmx.so via ctypes on torch's current stream.  Tolerances
(tests/helpers.py): rel 1e-4 / abs 1e-5 for direct convolution, GEMM and
AdamW, with the absolute part scaled by the magnitude of the summed terms;
rel 1e-3 for Winograd F(2x2,3x3).  References are float64 CPU results.
"""
import math

import pytest
import torch

from helpers import ATOL, RTOL, WINOGRAD_RTOL, assert_close_mag, conv_refs, gemm_mag

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mx():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from torch_vulkan import mx as m
    m.lib()
    return m


def dev(t):
    return t.to("cuda")


def stream():
    return torch.cuda.current_stream().cuda_stream


def close(actual, expected, rtol=RTOL, atol=ATOL, mag=None, what=""):
    assert_close_mag(actual, expected, mag, rtol=rtol, atol=atol, what=what)


# ------------------------------------------------------------------ GEMM
GEMM_SHAPES = [(1, 1, 1), (2, 2, 2), (64, 64, 64), (100, 37, 129), (256, 512, 512), (257, 255, 63), (1024, 768, 96),
               (3, 1000, 17), (2048, 2560, 64), (2049, 2047, 131)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
@pytest.mark.parametrize("layout", ["nn", "tn", "nt", "tt"])
def test_gemm_layouts(mx, m, n, k, layout):
    g = torch.Generator().manual_seed(m * 7 + n * 3 + k)
    a = torch.randn(m, k, generator=g) if layout[0] == "n" else torch.randn(k, m, generator=g).t()
    b = torch.randn(k, n, generator=g) if layout[1] == "n" else torch.randn(n, k, generator=g).t()
    da = dev(a.contiguous()) if layout[0] == "n" else dev(a.t().contiguous()).t()
    db = dev(b.contiguous()) if layout[1] == "n" else dev(b.t().contiguous()).t()
    c = torch.empty(m, n, device="cuda")
    mx.gemm(da, db, c, stream=stream())
    close(c, a.double() @ b.double(), mag=gemm_mag(a, b))


def test_gemm_known_answer(mx):
    a = dev(torch.tensor([[1.0, 2.0], [3.0, 4.0]]))
    b = dev(torch.tensor([[5.0, 6.0], [7.0, 8.0]]))
    c = torch.empty(2, 2, device="cuda")
    mx.gemm(a, b, c, stream=stream())
    assert torch.equal(c.cpu(), torch.tensor([[19.0, 22.0], [43.0, 50.0]]))


@pytest.mark.parametrize("beta,alpha", [(1.0, 1.0), (0.25, 0.8), (-0.5, 1.5)])
def test_addmm_bias_epilogue(mx, beta, alpha):
    g = torch.Generator().manual_seed(11)
    x, w, b = torch.randn(256, 512, generator=g), torch.randn(512, 512, generator=g), torch.randn(512, generator=g)
    c = torch.empty(256, 512, device="cuda")
    mx.gemm(dev(x), dev(w), c, bias=dev(b), alpha=alpha, beta=beta, stream=stream())
    close(c, beta * b.double() + alpha * (x.double() @ w.double()), mag=gemm_mag(x, w, alpha, beta, b))


def test_addmm_beta_zero_ignores_nan_bias(mx):
    x, w = torch.randn(64, 32), torch.randn(32, 48)
    b = torch.full((48,), float("nan"))
    c = torch.empty(64, 48, device="cuda")
    mx.gemm(dev(x), dev(w), c, bias=dev(b), beta=0.0, stream=stream())
    close(c, x.double() @ w.double(), mag=gemm_mag(x, w))


def test_gemm_k_zero(mx):
    c = torch.full((5, 7), 3.0, device="cuda")
    mx.gemm(torch.empty(5, 0, device="cuda"), torch.empty(0, 7, device="cuda"), c, stream=stream())
    assert torch.count_nonzero(c).item() == 0


@pytest.mark.parametrize("bsz,m,k,n", [(5, 17, 9, 33), (64, 256, 64, 256), (64, 256, 256, 64), (3, 1, 1, 1)])
def test_bmm_strided(mx, bsz, m, k, n):
    g = torch.Generator().manual_seed(bsz + m + k + n)
    a = torch.randn(bsz, m, k, generator=g)
    bt = torch.randn(bsz, n, k, generator=g)  # transposed right operand (a view)
    c = torch.empty(bsz, m, n, device="cuda")
    mx.gemm(dev(a), dev(bt).transpose(1, 2), c, stream=stream())
    close(c, a.double() @ bt.double().transpose(1, 2), mag=gemm_mag(a, bt.transpose(1, 2)))


@pytest.mark.parametrize("bias_shape", [(6, 40, 24), (1, 40, 24), (6, 1, 24), (24,)])
def test_bmm_batched_bias_stride(mx, bias_shape):
    """MX_BIAS_MATRIX / COL with a bias batch stride (0 when broadcast), incl. K = 0."""
    g = torch.Generator().manual_seed(len(bias_shape) + bias_shape[0])
    a, b = torch.randn(6, 40, 19, generator=g), torch.randn(6, 19, 24, generator=g)
    bias = torch.randn(bias_shape, generator=g)
    c = torch.empty(6, 40, 24, device="cuda")
    kind = mx.BIAS_COL if len(bias_shape) == 1 else mx.BIAS_MATRIX
    mx.gemm(dev(a), dev(b), c, bias=dev(bias), alpha=0.5, beta=-2.0, bias_kind=kind, stream=stream())
    ref = -2.0 * bias.double() + 0.5 * (a.double() @ b.double())
    close(c, ref.expand(6, 40, 24), mag=2.0 * bias.double().abs().expand(6, 40, 24) + 0.5 * gemm_mag(a, b))
    c0 = torch.empty(6, 40, 24, device="cuda")
    mx.gemm(torch.empty(6, 40, 0, device="cuda"), torch.empty(6, 0, 24, device="cuda"), c0, bias=dev(bias),
            beta=3.0, bias_kind=kind, stream=stream())
    assert torch.allclose(c0.cpu(), (3.0 * bias).expand(6, 40, 24))


def test_gemm_offset_view(mx):
    big = torch.randn(300, 200)
    a = big[7:107, 3:67]
    b = torch.randn(64, 50)
    dbig = dev(big)
    c = torch.empty(100, 50, device="cuda")
    mx.gemm(dbig[7:107, 3:67], dev(b), c, stream=stream())
    close(c, a.double() @ b.double(), mag=gemm_mag(a, b))


# ------------------------------------------------------------------ conv
CONV_CASES = [
    # x shape, cout, kernel, stride, padding, dilation, groups
    ((8, 64, 56, 56), 64, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((1, 7, 1, 15), 7, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 33, 1, 65), 33, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 13, 14), 17, (10, 10), (1, 1), (0, 0), (1, 1), 1),
    ((2, 18, 19, 23), 34, (3, 5), (2, 1), (2, 3), (2, 1), 2),
    ((1, 5, 11, 13), 15, (3, 5), (1, 2), (1, 4), (1, 2), 5),
    ((2, 6, 15, 19), 9, (3, 5), (1, 1), (3, 4), (2, 3), 3),
    ((1, 9, 17, 23), 17, (3, 5), (2, 3), (3, 2), (2, 1), 1),
    ((1, 9, 1, 255), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 1, 256), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((1, 9, 1, 257), 17, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((2, 3, 32, 32), 16, (7, 7), (2, 2), (3, 3), (1, 1), 1),
    ((2, 128, 14, 14), 256, (1, 1), (2, 2), (0, 0), (1, 1), 1),
    # 16-byte operand paths: unpadded 1x1 stride 1 with H*W % 4 == 0
    ((3, 64, 12, 12), 128, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((2, 32, 8, 6), 48, (1, 1), (1, 1), (0, 0), (1, 1), 2),
    ((4, 64, 28, 28), 64, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    ((2, 256, 14, 14), 512, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    # H*W % 4 != 0 and Cin % 4 != 0: scalar operand paths
    ((2, 6, 7, 7), 10, (1, 1), (1, 1), (0, 0), (1, 1), 1),
    # dInput stride phases: zero phases, one-to-one phase, 1/2-tap phases,
    # stride 3 with dilation 2, stride 2 with dilation 2
    ((2, 64, 16, 16), 128, (1, 1), (2, 2), (0, 0), (1, 1), 1),
    # 1x1 stride 2: the phase GEMM zero-fills its 2x2 blocks (odd H: the last
    # block has one row); odd W keeps the separate fill
    ((2, 32, 15, 12), 48, (1, 1), (2, 2), (0, 0), (1, 1), 1),
    ((1, 16, 10, 9), 16, (1, 1), (2, 2), (0, 0), (1, 1), 1),
    ((2, 64, 16, 16), 64, (3, 3), (2, 2), (1, 1), (1, 1), 1),
    ((1, 8, 20, 20), 8, (5, 5), (3, 3), (2, 2), (2, 2), 1),
    ((1, 8, 15, 15), 8, (3, 3), (2, 2), (2, 2), (2, 2), 1),
    # channel-blocked gathered K order (channels per group a multiple of 16):
    # grouped, strided + grouped, dilated
    ((2, 32, 9, 9), 64, (3, 3), (1, 1), (1, 1), (1, 1), 2),
    ((2, 64, 10, 10), 32, (3, 3), (2, 2), (1, 1), (1, 1), 2),
    ((1, 16, 12, 12), 16, (3, 3), (1, 1), (2, 2), (2, 2), 1),
    # small-channel layers of the C4 U-Net: 3-channel input conv and output head
    ((2, 3, 64, 64), 128, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((2, 128, 64, 64), 3, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    # 20000 groups at stride 2: four dInput phases x 20000 groups pass the
    # 65535 grid-z limit of one fused phase launch, so the phases split
    ((1, 40000, 4, 4), 20000, (3, 3), (2, 2), (1, 1), (1, 1), 20000),
]


def conv_inputs(xs, cout, kernel, groups, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(xs, generator=g)
    w = torch.randn((cout, xs[1] // groups, *kernel), generator=g) * (1.0 / math.sqrt(xs[1] // groups * kernel[0] * kernel[1]))
    b = torch.randn(cout, generator=g) * 0.1
    return x, w, b


@pytest.mark.parametrize("algo", ["implicit_gemm", "direct"])
@pytest.mark.parametrize("case", CONV_CASES, ids=[f"c{i}" for i in range(len(CONV_CASES))])
def test_conv_all_phases(mx, case, algo):
    xs, cout, kernel, stride, padding, dilation, groups = case
    if algo == "direct" and xs[0] * xs[2] * xs[3] > 4096 and cout >= 64:
        pytest.skip("direct dWeight is a serial per-weight loop; covered on small cases")
    A = mx.ALGO_IMPLICIT_GEMM if algo == "implicit_gemm" else mx.ALGO_DIRECT
    x, w, b = conv_inputs(xs, cout, kernel, groups, seed=sum(xs) + cout)
    d = mx.conv_desc(xs, w.shape, stride, padding, dilation, groups)
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(5))
    refs = conv_refs(x, w, b, dy, stride, padding, dilation, groups)
    X, W, B, DY = dev(x), dev(w), dev(b), dev(dy)
    y = torch.empty(dy.shape, device="cuda")
    dx = torch.empty(xs, device="cuda")
    dw = torch.empty(w.shape, device="cuda")
    dbias = torch.empty(cout, device="cuda")
    mx.conv2d_forward(d, X, W, B, y, A, stream())
    mx.conv2d_backward_input(d, DY, W, dx, A, stream())
    mx.conv2d_backward_weight(d, X, DY, dw, dbias, A if A != mx.ALGO_DIRECT else mx.ALGO_DIRECT, stream())
    for name, got in (("y", y), ("dx", dx), ("dw", dw), ("db", dbias)):
        ref, mag = refs[name]
        close(got, ref, mag=mag, what=name)


@pytest.mark.parametrize("case", [((3, 64, 12, 12), 128, (1, 1), (1, 1), (0, 0), (1, 1), 1),
                                  ((2, 64, 16, 16), 64, (3, 3), (2, 2), (1, 1), (1, 1), 1)])
def test_conv_unaligned_views(mx, case):
    """Operands at a 4-byte offset from 16-byte alignment take the scalar paths."""
    xs, cout, kernel, stride, padding, dilation, groups = case
    x, w, b = conv_inputs(xs, cout, kernel, groups, seed=11)
    d = mx.conv_desc(xs, w.shape, stride, padding, dilation, groups)
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(6))
    refs = conv_refs(x, w, b, dy, stride, padding, dilation, groups)

    def shifted(t):
        buf = torch.empty(t.numel() + 1, device="cuda")
        buf[1:] = t.reshape(-1).to("cuda")
        return buf[1:].view(t.shape)

    X, W, DY = shifted(x), shifted(w), shifted(dy)
    assert X.data_ptr() % 16 != 0
    y = torch.empty(dy.shape, device="cuda")
    dx = torch.empty(xs, device="cuda")
    dw = torch.empty(w.shape, device="cuda")
    dbias = torch.empty(cout, device="cuda")
    A = mx.ALGO_IMPLICIT_GEMM
    mx.conv2d_forward(d, X, W, dev(b), y, A, stream())
    mx.conv2d_backward_input(d, DY, W, dx, A, stream())
    mx.conv2d_backward_weight(d, X, DY, dw, dbias, A, stream())
    for name, got in (("y", y), ("dx", dx), ("dw", dw), ("db", dbias)):
        ref, mag = refs[name]
        close(got, ref, mag=mag, what=name)


@pytest.mark.parametrize("case", [((5, 32, 12, 10), 48, (3, 3), (1, 1), (1, 1), (1, 1), 1),
                                  ((5, 6, 9, 9), 10, (3, 3), (2, 2), (1, 1), (1, 1), 1),
                                  ((5, 64, 8, 8), 32, (1, 1), (1, 1), (0, 0), (1, 1), 1)])
def test_conv_batch_chunks(mx, case, monkeypatch):
    """Operands past the loaders' 32-bit byte range run as several launches over
    image chunks (dWeight summed over chunks); MX_CONV_BUFFER_LIMIT lowers that
    range so 5 images split 2 + 2 + 1."""
    xs, cout, kernel, stride, padding, dilation, groups = case
    x, w, b = conv_inputs(xs, cout, kernel, groups, seed=21)
    d = mx.conv_desc(xs, w.shape, stride, padding, dilation, groups)
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(8))
    refs = conv_refs(x, w, b, dy, stride, padding, dilation, groups)
    per_img = 4 * max(xs[1] * xs[2] * xs[3], cout * d.oh * d.ow)
    monkeypatch.setenv("MX_CONV_BUFFER_LIMIT", str(2 * per_img + 3))
    X, W, B, DY = dev(x), dev(w), dev(b), dev(dy)
    y = torch.empty(dy.shape, device="cuda")
    dx = torch.empty(xs, device="cuda")
    dw = torch.empty(w.shape, device="cuda")
    dbias = torch.empty(cout, device="cuda")
    A = mx.ALGO_IMPLICIT_GEMM
    mx.conv2d_forward(d, X, W, B, y, A, stream())
    mx.conv2d_backward_input(d, DY, W, dx, A, stream())
    mx.conv2d_backward_weight(d, X, DY, dw, dbias, A, stream())
    for name, got in (("y", y), ("dx", dx), ("dw", dw), ("db", dbias)):
        ref, mag = refs[name]
        close(got, ref, mag=mag, what=name)


# Winograd geometries: input channels that are not a multiple of the 8-channel
# slab (3, 12), output channels that are not a multiple of the 64-channel
# block (24, 70) or span several (130), odd output sizes (half tiles), tile
# counts off the 32-tile block, padding 0 and 2, groups.
WINO_CASES = [
    CONV_CASES[0],
    ((2, 16, 9, 11), 24, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((1, 32, 8, 8), 32, (3, 3), (1, 1), (0, 0), (1, 1), 4),
    ((2, 3, 10, 10), 130, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((3, 12, 7, 9), 70, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((2, 64, 14, 14), 64, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((1, 16, 6, 6), 8, (3, 3), (1, 1), (2, 2), (1, 1), 1),
    ((2, 24, 5, 4), 48, (3, 3), (1, 1), (1, 1), (1, 1), 3),
]


@pytest.mark.parametrize("fused", ["1", "0"], ids=["fused", "unfused"])
@pytest.mark.parametrize("case", WINO_CASES, ids=[f"w{i}" for i in range(len(WINO_CASES))])
def test_conv_winograd_forward(mx, monkeypatch, case, fused):
    monkeypatch.setenv("MX_WINOGRAD_FUSED", fused)
    xs, cout, kernel, stride, padding, dilation, groups = case
    x, w, b = conv_inputs(xs, cout, kernel, groups, seed=3)
    d = mx.conv_desc(xs, w.shape, stride, padding, dilation, groups)
    dy = torch.zeros((xs[0], cout, d.oh, d.ow))
    yref, mag = conv_refs(x, w, b, dy, stride, padding, dilation, groups)["y"]
    y = torch.empty(yref.shape, device="cuda")
    mx.conv2d_forward(d, dev(x), dev(w), dev(b), y, mx.ALGO_WINOGRAD, stream())
    close(y, yref, rtol=WINOGRAD_RTOL, mag=mag, what="winograd y")


def test_conv_winograd_batch_chunks(mx, monkeypatch):
    """A batch past the operand bound runs as several launches (bound lowered
    so three images need three launches)."""
    xs, cout = (3, 16, 12, 10), 40
    x, w, b = conv_inputs(xs, cout, (3, 3), 1, seed=8)
    d = mx.conv_desc(xs, w.shape, (1, 1), (1, 1), (1, 1), 1)
    monkeypatch.setenv("MX_CONV_BUFFER_LIMIT", str(4 * max(16 * 12 * 10, cout * d.oh * d.ow) + 5))
    monkeypatch.setenv("MX_WINOGRAD_FUSED", "1")
    dy = torch.zeros((xs[0], cout, d.oh, d.ow))
    yref, mag = conv_refs(x, w, b, dy, (1, 1), (1, 1), (1, 1), 1)["y"]
    y = torch.empty(yref.shape, device="cuda")
    mx.conv2d_forward(d, dev(x), dev(w), dev(b), y, mx.ALGO_WINOGRAD, stream())
    close(y, yref, rtol=WINOGRAD_RTOL, mag=mag, what="winograd chunked y")


@pytest.mark.parametrize("fused", ["1", "0"], ids=["fused", "unfused"])
@pytest.mark.parametrize("case", WINO_CASES, ids=[f"w{i}" for i in range(len(WINO_CASES))])
def test_conv_winograd_dinput(mx, monkeypatch, case, fused):
    """Input gradient of a 3x3 stride-1 layer through Winograd (dy convolved
    with the flipped, channel-swapped filter at padding 2 - p) against float64
    CPU torch at the Winograd tolerance; dx starts as NaN so every element
    must be written."""
    monkeypatch.setenv("MX_WINOGRAD_FUSED", fused)
    xs, cout, kernel, stride, padding, dilation, groups = case
    x, w, b = conv_inputs(xs, cout, kernel, groups, seed=11)
    d = mx.conv_desc(xs, w.shape, stride, padding, dilation, groups)
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(12))
    ref, mag = conv_refs(x, w, b, dy, stride, padding, dilation, groups)["dx"]
    dx = torch.full(ref.shape, float("nan"), device="cuda")
    mx.conv2d_backward_input(d, dev(dy), dev(w), dx, mx.ALGO_WINOGRAD, stream())
    close(dx, ref, rtol=WINOGRAD_RTOL, mag=mag, what="winograd dx")


# Tensors smaller than one patch row or whose rows straddle the tensor's
# ends: the weight gradient's row loads give way to element loads there.
WINO_DW_CASES = WINO_CASES + [
    ((1, 1, 1, 2), 1, (3, 3), (1, 1), (1, 1), (1, 1), 1),
    ((1, 2, 3, 3), 1, (3, 3), (1, 1), (2, 2), (1, 1), 1),
    ((2, 1, 5, 3), 3, (3, 3), (1, 1), (1, 2), (1, 1), 1),
]


@pytest.mark.parametrize("case", WINO_DW_CASES, ids=[f"w{i}" for i in range(len(WINO_DW_CASES))])
def test_conv_winograd_dweight(mx, case):
    """Weight gradient (and the bias gradient beside it) of a 3x3 stride-1
    layer through the Winograd adjoint against float64 CPU torch at the
    Winograd tolerance; outputs start as NaN so every element must be written."""
    xs, cout, kernel, stride, padding, dilation, groups = case
    x, w, b = conv_inputs(xs, cout, kernel, groups, seed=21)
    d = mx.conv_desc(xs, w.shape, stride, padding, dilation, groups)
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(22))
    refs = conv_refs(x, w, b, dy, stride, padding, dilation, groups)
    dw = torch.full(w.shape, float("nan"), device="cuda")
    db = torch.full(b.shape, float("nan"), device="cuda")
    mx.conv2d_backward_weight(d, dev(x), dev(dy), dw, db, mx.ALGO_WINOGRAD, stream())
    close(dw, refs["dw"][0], rtol=WINOGRAD_RTOL, mag=refs["dw"][1], what="winograd dw")
    close(db, refs["db"][0], mag=refs["db"][1], what="db beside winograd dw")


def test_conv_winograd_dweight_large_k(mx):
    """C1's layer (8x64x56x56, K = 6272 tiles over many ranges summed by the
    finalize) through the Winograd adjoint."""
    xs, cout = (8, 64, 56, 56), 64
    x, w, b = conv_inputs(xs, cout, (3, 3), 1, seed=23)
    d = mx.conv_desc(xs, w.shape, (1, 1), (1, 1), (1, 1), 1)
    dy = torch.randn((8, cout, 56, 56), generator=torch.Generator().manual_seed(24))
    ref, mag = conv_refs(x, w, None, dy, (1, 1), (1, 1), (1, 1), 1)["dw"]
    dw = torch.full(w.shape, float("nan"), device="cuda")
    mx.conv2d_backward_weight(d, dev(x), dev(dy), dw, None, mx.ALGO_WINOGRAD, stream())
    close(dw, ref, rtol=WINOGRAD_RTOL, mag=mag, what="winograd dw (C1)")


def test_conv_winograd_dweight_batch_chunks(mx, monkeypatch):
    """Winograd weight gradient of a batch past the operand bound: the
    per-slice gradients are summed in slice order."""
    xs, cout = (3, 40, 12, 10), 24
    x, w, b = conv_inputs(xs, cout, (3, 3), 1, seed=25)
    d = mx.conv_desc(xs, w.shape, (1, 1), (1, 1), (1, 1), 1)
    monkeypatch.setenv("MX_CONV_BUFFER_LIMIT", str(4 * max(40 * 12 * 10, cout * d.oh * d.ow) + 5))
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(26))
    refs = conv_refs(x, w, b, dy, (1, 1), (1, 1), (1, 1), 1)
    dw = torch.full(w.shape, float("nan"), device="cuda")
    db = torch.full(b.shape, float("nan"), device="cuda")
    mx.conv2d_backward_weight(d, dev(x), dev(dy), dw, db, mx.ALGO_WINOGRAD, stream())
    close(dw, refs["dw"][0], rtol=WINOGRAD_RTOL, mag=refs["dw"][1], what="winograd chunked dw")
    close(db, refs["db"][0], mag=refs["db"][1], what="chunked db")


def test_conv_winograd_dweight_one_range(mx, monkeypatch):
    """No workspace for partials: one tile range of 1798 tiles, which the
    kernel decodes in several table chunks (the last one ragged), with ragged
    input- and output-channel blocks; dBias comes out of the same launch."""
    xs, cout = (2, 16, 58, 62), 24
    x, w, b = conv_inputs(xs, cout, (3, 3), 1, seed=27)
    d = mx.conv_desc(xs, w.shape, (1, 1), (1, 1), (1, 1), 1)
    monkeypatch.setenv("TORCH_VULKAN_CONV_WORKSPACE_MB", "0")
    assert mx.conv2d_plan(d, mx.MX_CONV_DWEIGHT, mx.ALGO_WINOGRAD, True)["variant"] == "wino_dw_kernel"
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(28))
    refs = conv_refs(x, w, b, dy, (1, 1), (1, 1), (1, 1), 1)
    dw = torch.full(w.shape, float("nan"), device="cuda")
    db = torch.full(b.shape, float("nan"), device="cuda")
    mx.conv2d_backward_weight(d, dev(x), dev(dy), dw, db, mx.ALGO_WINOGRAD, stream())
    close(dw, refs["dw"][0], rtol=WINOGRAD_RTOL, mag=refs["dw"][1], what="winograd dw, one range")
    close(db, refs["db"][0], mag=refs["db"][1], what="db beside winograd dw, one range")


def test_conv_winograd_dinput_batch_chunks(mx, monkeypatch):
    """Winograd input gradient of a batch past the operand bound (lowered so
    three images take three launches)."""
    xs, cout = (3, 40, 12, 10), 16
    x, w, b = conv_inputs(xs, cout, (3, 3), 1, seed=13)
    d = mx.conv_desc(xs, w.shape, (1, 1), (1, 1), (1, 1), 1)
    monkeypatch.setenv("MX_CONV_BUFFER_LIMIT", str(4 * max(40 * 12 * 10, cout * d.oh * d.ow) + 5))
    monkeypatch.setenv("MX_WINOGRAD_FUSED", "1")
    dy = torch.randn((xs[0], cout, d.oh, d.ow), generator=torch.Generator().manual_seed(14))
    ref, mag = conv_refs(x, w, b, dy, (1, 1), (1, 1), (1, 1), 1)["dx"]
    dx = torch.full(ref.shape, float("nan"), device="cuda")
    mx.conv2d_backward_input(d, dev(dy), dev(w), dx, mx.ALGO_WINOGRAD, stream())
    close(dx, ref, rtol=WINOGRAD_RTOL, mag=mag, what="winograd chunked dx")


def test_conv_closed_form_1x1(mx):
    # w = 2, b = 1 -> y = 2x + 1; dx = 0.5 * w-sum per input channel for dy = 0.25.
    x = torch.randn(2, 1, 5, 7)
    d = mx.conv_desc(x.shape, (1, 1, 1, 1))
    y = torch.empty(2, 1, 5, 7, device="cuda")
    mx.conv2d_forward(d, dev(x), dev(torch.full((1, 1, 1, 1), 2.0)), dev(torch.ones(1)), y, mx.ALGO_IMPLICIT_GEMM, stream())
    assert torch.equal(y.cpu(), 2 * x + 1)
    dx = torch.empty_like(y)
    mx.conv2d_backward_input(d, dev(torch.full((2, 1, 5, 7), 0.25)), dev(torch.full((1, 1, 1, 1), 2.0)), dx,
                             mx.ALGO_IMPLICIT_GEMM, stream())
    assert torch.equal(dx.cpu(), torch.full((2, 1, 5, 7), 0.5))


def test_conv_dbias_only(mx):
    dy = torch.randn(4, 8, 6, 6)
    d = mx.conv_desc((4, 3, 6, 6), (8, 3, 1, 1))
    db = torch.empty(8, device="cuda")
    mx.conv2d_backward_bias(d, dev(dy), db, stream())
    close(db, dy.double().sum((0, 2, 3)), mag=dy.double().abs().sum((0, 2, 3)))


# ------------------------------------------------------------------ AdamW
def test_adamw_matches_torch_cpu(mx):
    lengths = [1, 257, 513, 5, 2049, 2, 65, 0, 117, 4056, 16, 1 << 20]
    g = torch.Generator().manual_seed(7521)
    ps = [torch.randn(n, generator=g) for n in lengths]
    cpu = [torch.nn.Parameter(p.clone()) for p in ps]
    opts = dict(lr=0.0017, betas=(0.79, 0.933), eps=1e-7, weight_decay=0.014)
    ref = torch.optim.AdamW(cpu, foreach=False, **opts)
    P = [dev(p) for p in ps]
    G = [torch.empty_like(p) for p in P]
    M = [torch.zeros_like(p) for p in P]
    V = [torch.zeros_like(p) for p in P]
    for step in range(1, 9):
        grads = [torch.randn(n, generator=g) * 0.03 for n in lengths]
        for c, gr in zip(cpu, grads):
            c.grad = gr.clone()
        ref.step()
        for Gi, gr in zip(G, grads):
            Gi.copy_(gr)
        n = mx.adamw_step(P, G, M, V, lr=opts["lr"], beta1=0.79, beta2=0.933, eps=1e-7, weight_decay=0.014,
                          steps=[step] * len(P), stream=stream())
        assert n == 1
    for c, p, m, v in zip(cpu, P, M, V):
        close(p, c.detach(), rtol=RTOL, atol=ATOL)
        if c.numel():
            st = ref.state[c]
            close(m, st["exp_avg"])
            close(v, st["exp_avg_sq"])


def test_adamw_alias_runs_sequentially(mx):
    p = dev(torch.linspace(0.2, 0.9, 257))
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    g1, g2 = dev(torch.full((257,), 0.025)), dev(torch.full((257,), -0.04))
    n = mx.adamw_step([p, p], [g1, g2], [m, m], [v, v], lr=0.003, beta1=0.8, beta2=0.93, eps=1e-7,
                      weight_decay=0.02, steps=[1, 2], stream=stream())
    assert n == 2
    ref = torch.nn.Parameter(torch.linspace(0.2, 0.9, 257))
    opt = torch.optim.AdamW([ref], lr=0.003, betas=(0.8, 0.93), eps=1e-7, weight_decay=0.02, foreach=False)
    for gv in (0.025, -0.04):
        ref.grad = torch.full((257,), gv)
        opt.step()
    close(p, ref.detach(), rtol=4e-5, atol=4e-5)


# ------------------------------------------------------------------ sum
@pytest.mark.parametrize("outer,reduce,inner", [(1, 8192, 4096), (3, 5, 7), (4, 100000, 1), (1, 1, 1)])
def test_sum_mid(mx, outer, reduce, inner):
    x = torch.randn(outer, reduce, inner)
    out = torch.empty(outer, inner, device="cuda")
    mx.sum_mid(out, dev(x), outer, reduce, inner, stream())
    close(out, x.double().sum(1), mag=x.double().abs().sum(1))
