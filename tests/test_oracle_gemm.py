"""Pins the GEMM oracle (oracle_gemm in oracle/oracle.c) on the CPU.

Checks: the reference's known answer [[1,2],[3,4]]x[[5,6],[7,8]] =
[[19,22],[43,50]] (tests/test_mm.py:29-35), CPU PyTorch golden fixtures for
addmm (tests/test_fused_addmm.py shapes and coefficients) and bmm
(tests/test_native_bmm.py shapes), strided/offset views, the NaN-safe
beta == 0 rule (matmul_strided_reg_bias.comp:96), K == 0, the closed form
dW = X^T g (tests/test_training_step.py:6-17), and per-batch bmm == mm.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from helpers import assert_close_mag

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "gemm.npz"))


def test_known_answer():
    c, _ = oracle.gemm(GOLD["known/a"], GOLD["known/b"])
    np.testing.assert_array_equal(c, [[19, 22], [43, 50]])
    np.testing.assert_array_equal(GOLD["known/c"], [[19, 22], [43, 50]])


@pytest.mark.parametrize("shape", ["addmm_5_7_11", "addmm_32_64_19", "addmm_128_256_128"])
@pytest.mark.parametrize("j", [0, 1, 2])
def test_addmm_matches_cpu_torch(shape, j):
    lhs, rhs, bias = GOLD[f"{shape}/lhs"], GOLD[f"{shape}/rhs"], GOLD[f"{shape}/bias"]
    beta, alpha = GOLD[f"{shape}/coef{j}"]
    c, mag = oracle.gemm(lhs, rhs, bias, alpha=alpha, beta=beta)
    np.testing.assert_allclose(c, GOLD[f"{shape}/out64_{j}"], rtol=1e-10, atol=1e-10 * (1 + mag.max()))
    assert_close_mag(torch.from_numpy(GOLD[f"{shape}/out32_{j}"]), torch.from_numpy(c), torch.from_numpy(mag),
                     what=shape)


@pytest.mark.parametrize("key", [k.split("/")[0] for k in GOLD.files if k.startswith("bmm_") and k.endswith("/a")])
def test_bmm_matches_cpu_torch_and_per_batch_mm(key):
    a, b = GOLD[f"{key}/a"], GOLD[f"{key}/b"]
    c, mag = oracle.gemm(a, b)
    np.testing.assert_allclose(c, GOLD[f"{key}/out64"], rtol=1e-10, atol=1e-10 * (1 + mag.max()))
    assert_close_mag(torch.from_numpy(GOLD[f"{key}/out32"]), torch.from_numpy(c), torch.from_numpy(mag), what=key)
    for z in range(a.shape[0]):
        cz, _ = oracle.gemm(a[z], b[z])
        np.testing.assert_array_equal(cz, c[z])


def test_strided_views_transposes_and_offsets():
    rng = np.random.default_rng(5)
    base = rng.standard_normal((40, 50)).astype(np.float32)
    w = rng.standard_normal((30, 20)).astype(np.float32)
    a = base[3:33, 7:47:2].T          # transposed, offset, stride-2 columns
    ref = a.astype(np.float64) @ w.astype(np.float64)
    c, _ = oracle.gemm(a, w)
    np.testing.assert_allclose(c, ref, rtol=1e-12, atol=1e-12)
    bt = rng.standard_normal((3, 9, 30)).astype(np.float32)
    c3, _ = oracle.gemm(np.broadcast_to(a[None], (3, 20, 30)), bt.transpose(0, 2, 1))
    np.testing.assert_allclose(c3, np.einsum("mk,bnk->bmn", a.astype(np.float64), bt.astype(np.float64)), rtol=1e-12,
                               atol=1e-12)


def test_beta_zero_ignores_nan_bias_and_k_zero():
    a, b = np.ones((4, 3), np.float32), np.ones((3, 5), np.float32)
    c, _ = oracle.gemm(a, b, np.full(5, np.nan, np.float32), beta=0.0)
    np.testing.assert_array_equal(c, np.full((4, 5), 3.0))
    c, _ = oracle.gemm(np.ones((4, 0), np.float32), np.ones((0, 5), np.float32))
    np.testing.assert_array_equal(c, np.zeros((4, 5)))
    c, _ = oracle.gemm(np.ones((4, 0), np.float32), np.ones((0, 5), np.float32), np.arange(5, dtype=np.float32),
                       beta=2.0)
    np.testing.assert_array_equal(c, np.broadcast_to(2.0 * np.arange(5), (4, 5)))


def test_linear_weight_gradient_closed_form():
    # tests/test_training_step.py:6-17: for y = x W^T, dW = g^T x.
    x = np.arange(12, dtype=np.float32).reshape(3, 4) / 7
    g = (np.arange(6, dtype=np.float32).reshape(3, 2) - 2) / 3
    dw, _ = oracle.gemm(g.T, x)
    np.testing.assert_allclose(dw, g.T.astype(np.float64) @ x.astype(np.float64), rtol=1e-12)


def test_planted_transpose_mistake_is_rejected():
    lhs, rhs = GOLD["addmm_32_64_19/lhs"], GOLD["addmm_32_64_19/rhs"]
    c, mag = oracle.gemm(lhs, rhs)
    wrong = c.copy()
    wrong[:, [0, 1]] = wrong[:, [1, 0]]  # two swapped output columns
    with pytest.raises(AssertionError):
        assert_close_mag(torch.from_numpy(wrong), torch.from_numpy(c), torch.from_numpy(mag))
