"""HIP path vs the oracle on the committed golden fixtures, through the C ABI.

For every fixture case the GPU result is checked against the oracle
(oracle/oracle.c) computed on the same inputs, and the oracle is itself pinned
to CPU PyTorch by tests/test_oracle_*.py.  Tolerances are the tolerance model of
tests/helpers.py (rel 1e-4 / abs 1e-5 scaled by the summed-term magnitude;
rel 1e-3 for Winograd); the AdamW kernel performs the oracle's float
operations in the same order and must agree to 1e-6 relative.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from helpers import WINOGRAD_RTOL, assert_close_mag

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
CONV = np.load(os.path.join(HERE, "golden", "conv.npz"))
GEMM = np.load(os.path.join(HERE, "golden", "gemm.npz"))
ADAM = np.load(os.path.join(HERE, "golden", "adamw.npz"))
CONV_CASES = sorted({k.split("/")[0] for k in CONV.files if not k.startswith("meta")})


@pytest.fixture(scope="module")
def mx():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    from torch_vulkan import mx as m
    m.lib()
    return m


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def stream():
    return torch.cuda.current_stream().cuda_stream


def t(a):
    return torch.from_numpy(np.asarray(a))


@pytest.mark.parametrize("algo", ["implicit_gemm", "direct"])
@pytest.mark.parametrize("name", CONV_CASES)
def test_conv_fixture_vs_oracle(mx, name, algo):
    g = {k.split("/", 1)[1]: CONV[k] for k in CONV.files if k.startswith(name + "/")}
    s = g["params"]
    stride, padding, dilation, groups = tuple(s[0:2]), tuple(s[2:4]), tuple(s[4:6]), int(s[6])
    A = mx.ALGO_IMPLICIT_GEMM if algo == "implicit_gemm" else mx.ALGO_DIRECT
    x, w, dy, b = g["x"], g["w"], g["dy"], g.get("b")
    d = mx.conv_desc(x.shape, w.shape, stride, padding, dilation, groups)
    y = torch.empty(dy.shape, device="cuda")
    dx = torch.empty(x.shape, device="cuda")
    dw = torch.empty(w.shape, device="cuda")
    db = torch.empty(w.shape[0], device="cuda")
    X, W, DY = dev(x), dev(w), dev(dy)
    mx.conv2d_forward(d, X, W, dev(b) if b is not None else None, y, A, stream())
    mx.conv2d_backward_input(d, DY, W, dx, A, stream())
    mx.conv2d_backward_weight(d, X, DY, dw, db, A, stream())
    yo, my = oracle.conv2d_forward(x, w, b, stride, padding, dilation, groups)
    back = oracle.conv2d_backward(x, w, dy, stride, padding, dilation, groups)
    assert_close_mag(y, t(yo), t(my), what=f"{name} y")
    for key, got in (("dx", dx), ("dw", dw), ("db", db)):
        assert_close_mag(got, t(back[key][0]), t(back[key][1]), what=f"{name} {key}")


@pytest.mark.parametrize("name", [c for c in CONV_CASES if c.startswith("winograd")])
def test_winograd_fixture_vs_oracle(mx, name):
    g = {k.split("/", 1)[1]: CONV[k] for k in CONV.files if k.startswith(name + "/")}
    s = g["params"]
    stride, padding, groups = tuple(s[0:2]), tuple(s[2:4]), int(s[6])
    d = mx.conv_desc(g["x"].shape, g["w"].shape, stride, padding, (1, 1), groups)
    y = torch.empty(g["dy"].shape, device="cuda")
    mx.conv2d_forward(d, dev(g["x"]), dev(g["w"]), dev(g["b"]), y, mx.ALGO_WINOGRAD, stream())
    yo, my = oracle.conv2d_forward(g["x"], g["w"], g["b"], stride, padding, (1, 1), groups, winograd=True)
    assert_close_mag(y, t(yo), t(my), rtol=WINOGRAD_RTOL, what=name)


@pytest.mark.parametrize("shape", ["addmm_5_7_11", "addmm_32_64_19", "addmm_128_256_128"])
@pytest.mark.parametrize("j", [0, 1, 2])
def test_addmm_fixture_vs_oracle(mx, shape, j):
    lhs, rhs, bias = GEMM[f"{shape}/lhs"], GEMM[f"{shape}/rhs"], GEMM[f"{shape}/bias"]
    beta, alpha = (float(v) for v in GEMM[f"{shape}/coef{j}"])
    c = torch.empty(lhs.shape[0], rhs.shape[1], device="cuda")
    mx.gemm(dev(lhs), dev(rhs), c, bias=dev(bias), alpha=alpha, beta=beta, stream=stream())
    ref, mag = oracle.gemm(lhs, rhs, bias, alpha=alpha, beta=beta)
    assert_close_mag(c, t(ref), t(mag), what=shape)


@pytest.mark.parametrize("key", [k.split("/")[0] for k in GEMM.files if k.startswith("bmm_") and k.endswith("/a")])
def test_bmm_fixture_vs_oracle(mx, key):
    a, b = GEMM[f"{key}/a"], GEMM[f"{key}/b"]
    c = torch.empty(a.shape[0], a.shape[1], b.shape[2], device="cuda")
    mx.gemm(dev(a), dev(b), c, stream=stream())
    ref, mag = oracle.gemm(a, b)
    assert_close_mag(c, t(ref), t(mag), what=key)


@pytest.mark.parametrize("key", ["traj_3", "traj_4_5", "traj_64_65"])
def test_adamw_trajectory_vs_oracle(mx, key):
    hp = dict(lr=0.005, beta1=0.8, beta2=0.91, eps=1e-6, weight_decay=0.031)
    p = ADAM[f"{key}/p0"].copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    P, M, V = dev(p.ravel()), dev(m.ravel()), dev(v.ravel())
    for i in range(8):
        g = ADAM[f"{key}/g{i}"]
        oracle.adamw_step(p, g.copy(), m, v, step=i + 1, **hp)
        mx.adamw_step([P], [dev(g.ravel())], [M], [V], steps=[i + 1], stream=stream(), **hp)
        for name, gpu, ref in (("p", P, p), ("m", M, m), ("v", V, v)):
            np.testing.assert_allclose(gpu.cpu().numpy(), ref.ravel(), rtol=1e-6, atol=1e-9,
                                       err_msg=f"{key} {name} step {i + 1}")


@pytest.mark.parametrize("ams", [0, 1])
def test_adamw_multitensor_fixture_one_launch(mx, ams):
    """The lengths list with missing gradients: each step is one launch over
    the tensors that have gradients; final state equals CPU torch's."""
    key = f"multi_ams{ams}"
    n = 11
    P = [dev(ADAM[f"{key}/p0_{i}"]) for i in range(n)]
    M = [torch.zeros_like(p) for p in P]
    V = [torch.zeros_like(p) for p in P]
    X = [torch.zeros_like(p) for p in P]
    steps = [0] * n
    for it in range(9):
        idx = [i for i in range(n) if (i + it) % 13 != 0]
        for i in idx:
            steps[i] += 1
        grads = [dev(ADAM[f"{key}/g{it}_{i}"]) for i in idx]
        launches = mx.adamw_step([P[i] for i in idx], grads, [M[i] for i in idx], [V[i] for i in idx],
                                 lr=.0017, beta1=.79, beta2=.933, eps=1e-7, weight_decay=.014,
                                 steps=[steps[i] for i in idx], max_exp_avg_sqs=[X[i] for i in idx] if ams else None,
                                 stream=stream())
        assert launches == 1
    for i in range(n):
        np.testing.assert_allclose(P[i].cpu().numpy(), ADAM[f"{key}/p_{i}"], rtol=1e-4, atol=1e-5)
        if f"{key}/exp_avg_{i}" in ADAM.files:
            np.testing.assert_allclose(M[i].cpu().numpy(), ADAM[f"{key}/exp_avg_{i}"], rtol=1e-4, atol=1e-5)
            np.testing.assert_allclose(V[i].cpu().numpy(), ADAM[f"{key}/exp_avg_sq_{i}"], rtol=1e-4, atol=1e-5)
