"""Pins the AdamW oracle (oracle_adamw_step / oracle_partition) on the CPU.

Checks: CPU torch.optim.AdamW(foreach=False) golden trajectories
(tests/test_fused_adamw.py hyperparameters and seed) and the
tests/test_multitensor_adamw.py lengths list with missing gradients, plain and
AMSGrad; the closed form of the first step from zero state
(p1 = p0(1 - lr wd) - lr g / (|g| + eps)); g = 0 leaves only the decay;
NaN propagation of the AMSGrad maximum (adamw_fused_amsgrad.comp:30-34); the
launch grouping and alias rule of csrc/ops/multitensor_plan.h:22-48 with
tests/test_multitensor_adamw.py:49-112's expectations; a planted mistake.
"""
import os

import numpy as np
import pytest
import torch

import oracle

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "adamw.npz"))
HP = dict(lr=0.005, beta1=0.8, beta2=0.91, eps=1e-6, weight_decay=0.031)


@pytest.mark.parametrize("key", ["traj_3", "traj_4_5", "traj_64_65"])
def test_trajectory_matches_torch_single_tensor(key):
    p = GOLD[f"{key}/p0"].copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    for i in range(8):
        oracle.adamw_step(p, GOLD[f"{key}/g{i}"].copy(), m, v, step=i + 1, **HP)
        # Same float operations in the same order: within a few ulp of torch
        # (its scalar tail loop may contract differently from the vector body).
        for name, arr in (("p", p), ("m", m), ("v", v)):
            np.testing.assert_allclose(arr, GOLD[f"{key}/{name}{i + 1}"], rtol=1e-6, atol=1e-9,
                                       err_msg=f"{key} {name} step {i + 1}")


@pytest.mark.parametrize("ams", [0, 1])
def test_multitensor_lengths_list_matches_torch(ams):
    key = f"multi_ams{ams}"
    n = 11
    P = [GOLD[f"{key}/p0_{i}"].copy() for i in range(n)]
    M = [np.zeros_like(p) for p in P]
    V = [np.zeros_like(p) for p in P]
    X = [np.zeros_like(p) for p in P]
    steps = [0] * n
    opts = dict(lr=.0017, beta1=.79, beta2=.933, eps=1e-7, weight_decay=.014)
    for it in range(9):
        for i in range(n):
            g = GOLD[f"{key}/g{it}_{i}"]
            if g.size == 0 and P[i].size != 0 or (g.size == 0 and (i + it) % 13 == 0):
                continue  # missing gradient: torch skips the parameter
            steps[i] += 1
            oracle.adamw_step(P[i], g.copy(), M[i], V[i], step=steps[i], vmax=X[i] if ams else None, **opts)
    for i in range(n):
        np.testing.assert_allclose(P[i], GOLD[f"{key}/p_{i}"], rtol=1e-6, atol=1e-9)
        if f"{key}/exp_avg_{i}" in GOLD.files:
            np.testing.assert_allclose(M[i], GOLD[f"{key}/exp_avg_{i}"], rtol=1e-6, atol=1e-9)
            np.testing.assert_allclose(V[i], GOLD[f"{key}/exp_avg_sq_{i}"], rtol=1e-6, atol=1e-9)
            assert steps[i] == int(GOLD[f"{key}/step_{i}"])
            if ams:
                np.testing.assert_allclose(X[i], GOLD[f"{key}/max_exp_avg_sq_{i}"], rtol=1e-6, atol=1e-9)


def test_first_step_closed_form_and_zero_gradient():
    rng = np.random.default_rng(1)
    p0 = rng.standard_normal(1000).astype(np.float32)
    g = rng.standard_normal(1000).astype(np.float32)
    p = p0.copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    lr, wd, eps = 1e-3, 0.01, 1e-8
    oracle.adamw_step(p, g, m, v, lr=lr, beta1=0.9, beta2=0.999, eps=eps, weight_decay=wd, step=1)
    closed = p0.astype(np.float64) * (1 - lr * wd) - lr * g / (np.abs(g) + eps)
    np.testing.assert_allclose(p, closed, rtol=2e-6, atol=1e-9)
    p = p0.copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    oracle.adamw_step(p, np.zeros_like(p), m, v, lr=lr, beta1=0.9, beta2=0.999, eps=eps, weight_decay=wd, step=1)
    np.testing.assert_array_equal(p, p0 * np.float32(1 - lr * wd))


def test_amsgrad_max_propagates_nan():
    p = np.ones(4, np.float32)
    g = np.array([0.1, np.nan, 0.2, -0.3], np.float32)
    m, v, x = np.zeros(4, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32)
    oracle.adamw_step(p, g, m, v, vmax=x, step=1, **HP)
    assert np.isnan(x[1]) and not np.isnan(x[[0, 2, 3]]).any()
    assert np.isnan(p[1])
    ref = torch.maximum(torch.tensor([0.0, float("nan")]), torch.tensor([1.0, 2.0]))
    assert torch.isnan(ref[1]) and ref[0] == 1.0


def test_partition_alias_rule():
    # Independent tensors: the reference groups 8 per dispatch (ceil(11/8) = 2,
    # tests/test_multitensor_adamw.py:49-70); this build's launches are
    # unbounded (one launch).
    none = np.zeros((11, 11), np.uint8)
    assert oracle.partition(none, slots=8) == [0, 8]
    assert oracle.partition(none, slots=0) == [0]
    # The same parameter listed twice must update sequentially
    # (tests/test_multitensor_adamw.py:73-112): two launches.
    alias = np.zeros((2, 2), np.uint8)
    alias[0, 1] = alias[1, 0] = 1
    assert oracle.partition(alias) == [0, 1]
    chain = np.zeros((5, 5), np.uint8)
    chain[1, 3] = 1
    assert oracle.partition(chain) == [0, 3]


def test_sequential_alias_semantics_match_torch():
    ref = torch.nn.Parameter(torch.linspace(.2, .9, 257))
    opt = torch.optim.AdamW([ref], lr=.003, betas=(.8, .93), eps=1e-7, weight_decay=.02, foreach=False)
    for gv in (.025, -.04):
        ref.grad = torch.full_like(ref, gv)
        opt.step()
    p = np.linspace(.2, .9, 257, dtype=np.float32)
    p = torch.linspace(.2, .9, 257).numpy().copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    for step, gv in ((1, .025), (2, -.04)):
        oracle.adamw_step(p, np.full_like(p, gv), m, v, lr=.003, beta1=.8, beta2=.93, eps=1e-7, weight_decay=.02,
                          step=step)
    np.testing.assert_allclose(p, ref.detach().numpy(), rtol=1e-6, atol=1e-7)


def test_planted_mistake_bias_correction_is_detected():
    key = "traj_4_5"
    p = GOLD[f"{key}/p0"].copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    oracle.adamw_step(p, GOLD[f"{key}/g0"].copy(), m, v, step=2, **HP)  # wrong step -> wrong bias correction
    with pytest.raises(AssertionError):
        np.testing.assert_allclose(p, GOLD[f"{key}/p1"], rtol=1e-4, atol=1e-5)
