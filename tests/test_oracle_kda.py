"""Pins for the KDA oracle (CPU only).

Each check would fail under a plausible restatement mistake:
* recurrence vs an explicit-matrix statement of the delta rule
  (S_t = (I - b k k^T) Diag(e^g) S_{t-1} + b k v^T, ops_kda.py:6-9) -> sign /
  order-of-decay / post-update-output errors;
* chunk form vs recurrence (the reference's own invariant,
  run_correctness.py:103-133, at its 1e-6 fp32 tolerance) -> WY/UT mistakes,
  wrong decay direction (ops_kda.py:521-534), mask diagonal (ops_kda.py:396-408);
* special cases with closed forms (beta=0 pure decay; beta=1, g=0 exact write);
* GVA head sharing, padding/causality, the g clamp;
* the hand-written gradients against central finite differences of the
  forward in fp64, every coordinate (the reference's gradient test,
  run_correctness.py:765-833, samples 8 per tensor at the same 1e-6 bar);
* the torch-CPU restatement (``oracle.kda_torch``, the CPU baseline's) against
  the numpy one and the recurrence in fp64, GVA and padding included.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.common import l2_normalize, logsigmoid, sigmoid
from oracle.kda import chunk_kda, delta_rule_matrix_form, recurrent_kda, recurrent_kda_grad
from oracle.kda_torch import chunk_kda as chunk_kda_torch


def _inputs(rng, B, T, H, HV, K, V, gscale=1.0):
    q = l2_normalize(rng.standard_normal((B, T, H, K)))
    k = l2_normalize(rng.standard_normal((B, T, H, K)))
    v = rng.standard_normal((B, T, HV, V))
    g = logsigmoid(rng.standard_normal((B, T, HV, K))) * gscale
    beta = sigmoid(rng.standard_normal((B, T, HV)))
    return q, k, v, g, beta


def test_recurrent_matches_matrix_form():
    rng = np.random.default_rng(1)
    q, k, v, g, beta = _inputs(rng, 2, 23, 2, 4, 8, 5)
    S0 = rng.standard_normal((2, 4, 8, 5))
    o1, s1 = recurrent_kda(q, k, v, g, beta, initial_state=S0, compute=np.float64)
    o2, s2 = delta_rule_matrix_form(q, k, v, g, beta, initial_state=S0)
    assert np.abs(o1 - o2).max() < 1e-12
    assert np.abs(s1 - s2).max() < 1e-12


@pytest.mark.parametrize("T,C", [(64, 64), (100, 16), (130, 64), (7, 64)])
def test_chunk_matches_recurrent_fp64(T, C):
    rng = np.random.default_rng(T)
    q, k, v, g, beta = _inputs(rng, 2, T, 2, 4, 16, 8)
    S0 = 0.1 * rng.standard_normal((2, 4, 16, 8))
    o1, s1 = recurrent_kda(q, k, v, g, beta, initial_state=S0, compute=np.float64)
    o2, s2 = chunk_kda(q, k, v, g, beta, initial_state=S0, chunk_size=C, compute=np.float64)
    assert o2.shape == o1.shape
    assert np.abs(o1 - o2).max() < 1e-10
    assert np.abs(s1 - s2).max() < 1e-10


def test_chunk_vs_recurrent_fp32_reference_tolerance():
    # shapes and generators of run_correctness.py:103-133 (tolerance 1e-6 fp32)
    rng = np.random.default_rng(0)
    B, T, H, K, V = 2, 128, 4, 32, 32
    q = l2_normalize(rng.standard_normal((B, T, H, K))).astype(np.float32)
    k = l2_normalize(rng.standard_normal((B, T, H, K))).astype(np.float32)
    v = (0.1 * rng.standard_normal((B, T, H, V))).astype(np.float32)
    g = (-0.05 * rng.random((B, T, H, K))).astype(np.float32)
    beta = (0.2 * rng.random((B, T, H))).astype(np.float32)
    o1, s1 = recurrent_kda(q, k, v, g, beta)
    o2, s2 = chunk_kda(q, k, v, g, beta, chunk_size=64)
    assert np.abs(o1 - o2).max() < 1e-6
    assert np.abs(s1 - s2).max() < 1e-6


def test_beta_zero_is_pure_decay():
    rng = np.random.default_rng(2)
    B, T, H, K, V = 1, 9, 1, 6, 3
    q, k, v, g, _ = _inputs(rng, B, T, H, H, K, V)
    beta = np.zeros((B, T, H))
    S0 = rng.standard_normal((B, H, K, V))
    o, s = recurrent_kda(q, k, v, g, beta, initial_state=S0, scale=0.5, compute=np.float64)
    G = np.cumsum(np.maximum(g, -10.0), axis=1)
    for t in range(T):
        St = np.exp(G[0, t, 0])[:, None] * S0[0, 0]
        assert np.allclose(o[0, t, 0], 0.5 * q[0, t, 0] @ St, atol=1e-12)
    assert np.allclose(s[0, 0], np.exp(G[0, -1, 0])[:, None] * S0[0, 0], atol=1e-12)
    o2, s2 = chunk_kda(q, k, v, g, beta, initial_state=S0, scale=0.5, chunk_size=4,
                       compute=np.float64)
    assert np.abs(o2 - o).max() < 1e-12 and np.abs(s2 - s).max() < 1e-12


def test_beta_one_writes_value_exactly():
    # with beta=1 and g=0 the delta rule overwrites: k_t^T S_t = v_t
    rng = np.random.default_rng(3)
    B, T, H, K, V = 1, 5, 1, 8, 4
    q, k, v, _, _ = _inputs(rng, B, T, H, H, K, V)
    g = np.zeros((B, T, H, K))
    beta = np.ones((B, T, H))
    S0 = rng.standard_normal((B, H, K, V))
    St = S0.copy()
    for t in range(T):
        _, St = recurrent_kda(q[:, t:t + 1], k[:, t:t + 1], v[:, t:t + 1], g[:, t:t + 1],
                              beta[:, t:t + 1], initial_state=St, compute=np.float64)
        assert np.allclose(k[0, t, 0] @ St[0, 0], v[0, t, 0], atol=1e-12)


def test_gva_matches_repeated_heads():
    rng = np.random.default_rng(4)
    B, T, H, HV, K, V = 1, 40, 2, 4, 8, 8
    q, k, v, g, beta = _inputs(rng, B, T, H, HV, K, V)
    o1, s1 = chunk_kda(q, k, v, g, beta, chunk_size=16, compute=np.float64)
    qr, kr = np.repeat(q, 2, axis=2), np.repeat(k, 2, axis=2)
    o2, s2 = chunk_kda(qr, kr, v, g, beta, chunk_size=16, compute=np.float64)
    assert np.abs(o1 - o2).max() < 1e-12 and np.abs(s1 - s2).max() < 1e-12


def test_causality_and_padding():
    rng = np.random.default_rng(5)
    q, k, v, g, beta = _inputs(rng, 1, 70, 2, 2, 8, 8)
    o_full, _ = chunk_kda(q, k, v, g, beta, chunk_size=32, compute=np.float64)
    o_pre, s_pre = chunk_kda(q[:, :45], k[:, :45], v[:, :45], g[:, :45], beta[:, :45],
                             chunk_size=32, compute=np.float64)
    assert np.abs(o_full[:, :45] - o_pre).max() < 1e-12
    # continuing from the prefix state reproduces the rest (state carry)
    o_rest, _ = chunk_kda(q[:, 45:], k[:, 45:], v[:, 45:], g[:, 45:], beta[:, 45:],
                          initial_state=s_pre, chunk_size=32, compute=np.float64)
    assert np.abs(o_full[:, 45:] - o_rest).max() < 1e-10


def test_g_clamp():
    rng = np.random.default_rng(6)
    q, k, v, g, beta = _inputs(rng, 1, 20, 1, 1, 4, 4)
    g = g - 15.0
    o1, _ = recurrent_kda(q, k, v, g, beta, g_clamp_min=-10.0, compute=np.float64)
    o2, _ = recurrent_kda(q, k, v, np.maximum(g, -10.0), beta, g_clamp_min=-np.inf,
                          compute=np.float64)
    o3, _ = recurrent_kda(q, k, v, g, beta, g_clamp_min=-np.inf, compute=np.float64)
    assert np.abs(o1 - o2).max() < 1e-14
    assert np.abs(o1 - o3).max() > 1e-6


def test_t_zero():
    rng = np.random.default_rng(7)
    q, k, v, g, beta = _inputs(rng, 2, 0, 1, 1, 4, 4)
    S0 = rng.standard_normal((2, 1, 4, 4))
    o, s = chunk_kda(q, k, v, g, beta, initial_state=S0)
    assert o.shape == (2, 0, 1, 4)
    assert np.allclose(s, S0)


def test_bf16_round_matches_torch_conversion():
    """``bf16_round`` is torch's float32 -> bfloat16 conversion (round to
    nearest even, NaN kept), on random values, random bit patterns and the
    special values."""
    import torch

    from oracle.common import bf16_round
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(200_000) * 1e3).astype(np.float32),
        rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
        np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 3.3895314e38, -3.3895314e38, 1e-40,
                  -1e-40, 1.00390625, 1.01171875], np.float32)])
    got = bf16_round(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _fd_check(q, k, v, g, beta, s0, W_o, W_s, scale, clamp):
    """Largest error of recurrent_kda_grad against central differences of
    L = sum(o * W_o) + sum(S_T * W_s) over every input coordinate, relative to
    |num| + |ana| + 1e-2: the differences carry ~1e-10 of rounding noise, so a
    gradient of 1e-5 cannot be resolved to 1e-6 relative, while a dropped or
    wrong term moves a gradient by its own size."""
    def loss(q, k, v, g, beta, s0):
        o, S = recurrent_kda(q, k, v, g, beta, scale=scale, initial_state=s0, g_clamp_min=clamp,
                             compute=np.float64)
        return float((o * W_o).sum() + (S * W_s).sum())

    grads = recurrent_kda_grad(q, k, v, g, beta, W_o, scale=scale, initial_state=s0,
                               ds_final=W_s, g_clamp_min=clamp)
    args = [q, k, v, g, beta, s0]
    eps, worst = 1e-6, 0.0
    for i, (x, gx) in enumerate(zip(args, grads)):
        assert gx.shape == x.shape
        for idx in np.ndindex(*x.shape):
            orig = x[idx]
            x[idx] = orig + eps
            lp = loss(*args)
            x[idx] = orig - eps
            lm = loss(*args)
            x[idx] = orig
            num = (lp - lm) / (2 * eps)
            rel = abs(num - gx[idx]) / (abs(num) + abs(gx[idx]) + 1e-2)
            worst = max(worst, rel)
    return worst


def test_recurrent_grad_matches_finite_differences():
    """The reference's gradient test shape (B=1, T=16, H=2, K=V=4, fp64, small
    gates and betas), here with an initial state and a final-state cotangent."""
    rng = np.random.default_rng(6)
    B, T, H, K, V = 1, 16, 2, 4, 4
    q = rng.standard_normal((B, T, H, K))
    k = rng.standard_normal((B, T, H, K))
    v = rng.standard_normal((B, T, H, V))
    g = -rng.random((B, T, H, K)) * 0.1
    beta = rng.random((B, T, H)) * 0.2
    s0 = rng.standard_normal((B, H, K, V)) * 0.1
    W_o = rng.standard_normal((B, T, H, V))
    W_s = rng.standard_normal((B, H, K, V))
    assert _fd_check(q, k, v, g, beta, s0, W_o, W_s, None, -10.0) < 1e-6


def test_recurrent_grad_gva_and_clamp():
    """GVA (2 value heads per key head): dq, dk sum over the value heads; gate
    entries below the clamp get zero gradient (kept 0.5 away from the kink so
    the differences do not straddle it); explicit scale."""
    rng = np.random.default_rng(11)
    B, T, H, HV, K, V = 2, 9, 1, 2, 4, 3
    q, k, v, g, beta = _inputs(rng, B, T, H, HV, K, V)
    g = np.where(rng.random(g.shape) < 0.3, -10.5 - rng.random(g.shape), g)
    s0 = rng.standard_normal((B, HV, K, V)) * 0.1
    W_o = rng.standard_normal((B, T, HV, V))
    W_s = rng.standard_normal((B, HV, K, V))
    assert _fd_check(q, k, v, g, beta, s0, W_o, W_s, 0.7, -10.0) < 1e-6
    dg = recurrent_kda_grad(q, k, v, g, beta, W_o, scale=0.7, initial_state=s0, ds_final=W_s)[3]
    assert np.all(dg[g < -10.0] == 0) and np.any(dg[g >= -10.0] != 0)


@pytest.mark.parametrize("B,T,H,HV,K,V,C", [(2, 200, 2, 4, 32, 16, 64), (1, 37, 1, 1, 16, 8, 16),
                                            (1, 130, 2, 2, 64, 64, 64)])
def test_torch_restatement_matches(B, T, H, HV, K, V, C):
    import torch
    rng = np.random.default_rng(T + K)
    q, k, v, g, beta = _inputs(rng, B, T, H, HV, K, V, gscale=3.0)
    S0 = 0.02 * rng.standard_normal((B, HV, K, V))
    o1, s1 = chunk_kda(q, k, v, g, beta, initial_state=S0, chunk_size=C, compute=np.float64)
    o2, s2 = chunk_kda_torch(q, k, v, g, beta, initial_state=S0, chunk_size=C,
                             dtype=torch.float64)
    assert np.abs(o1 - o2.numpy()).max() < 1e-12 * max(1.0, np.abs(o1).max())
    assert np.abs(s1 - s2.numpy()).max() < 1e-12 * max(1.0, np.abs(s1).max())
    o3, s3 = recurrent_kda(q, k, v, g, beta, initial_state=S0, compute=np.float64)
    assert np.abs(o3 - o2.numpy()).max() < 1e-9
