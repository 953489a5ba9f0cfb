"""KDA oracle: numpy restatement of the reference delta rule (test only).

Functions
---------
``recurrent_kda``  restates ``naive_recurrent_kda`` (``ops_kda.py:175-267``):
    per token ``S <- S * exp(g_t)``; ``S += (b_t k_t) (x) (v_t - k_t^T S)``;
    ``o_t = (scale q_t)^T S`` with the post-update state (``:253-258``).
``chunk_kda``      restates ``naive_chunk_kda`` (``ops_kda.py:340-536``):
    right-pad to a multiple of the chunk (``:375-382``), in-chunk cumsum of the
    clamped gate (``:388-394``), the per-column build of A with
    ``clamp(max=50)`` on the decay exponent (``:409-417``), the triangular
    solve and ``(A + I) diag(beta)`` (``:418-421``), ``w``/``u`` (``:423-424``),
    and the sequential chunk loop (``:509-535``).
``recurrent_kda_grad``  the reverse-mode gradients of ``recurrent_kda``, pinned by
    central finite differences of ``recurrent_kda`` in fp64.
``delta_rule_matrix_form``  an independent fp64 statement of the recurrence
    as explicit matrices, ``S_t = (I - b k k^T) Diag(exp g) S_{t-1} + b k v^T``
    (module docstring, ``ops_kda.py:6-9``), used only to pin ``recurrent_kda``.

All functions take float arrays (bf16 inputs are passed as their exact float32
values) and compute in ``compute`` precision (float32 mirrors the reference's
fp32 compute dtype, ``ops_kda.py:125-127``). GVA: q/k heads are repeated
``HV // H`` times (``ops_kda.py:226-227,386-387``).
"""

from __future__ import annotations

import numpy as np


def _prep_common(q, k, v, g, beta, scale, compute):
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    if HV % H:
        raise ValueError("HV must be divisible by H")
    G = HV // H
    if scale is None:
        scale = K ** -0.5
    q = np.repeat(np.asarray(q, compute), G, axis=2) * compute(scale)
    k = np.repeat(np.asarray(k, compute), G, axis=2)
    return (q, k, np.asarray(v, compute), np.asarray(g, compute),
            np.asarray(beta, compute), B, T, HV, K, V)


def recurrent_kda(q, k, v, g, beta, scale=None, initial_state=None,
                  g_clamp_min=-10.0, compute=np.float32):
    """Per-token recurrence; returns ``(o [B,T,HV,V], S [B,HV,K,V])``."""
    q, k, v, g, beta, B, T, HV, K, V = _prep_common(q, k, v, g, beta, scale, compute)
    if g_clamp_min > -np.inf:
        g = np.maximum(g, compute(g_clamp_min))
    S = np.zeros((B, HV, K, V), compute)
    if initial_state is not None:
        S = S + np.asarray(initial_state, compute)
    o = np.zeros((B, T, HV, V), compute)
    for t in range(T):
        S = S * np.exp(g[:, t])[..., None]
        kS = np.einsum('bhk,bhkv->bhv', k[:, t], S)
        S = S + np.einsum('bhk,bhv->bhkv', beta[:, t][..., None] * k[:, t], v[:, t] - kS)
        o[:, t] = np.einsum('bhk,bhkv->bhv', q[:, t], S)
    return o, S


def delta_rule_matrix_form(q, k, v, g, beta, scale=None, initial_state=None,
                           g_clamp_min=-10.0):
    """fp64 explicit-matrix recurrence (independent pin for the oracle)."""
    q, k, v, g, beta, B, T, HV, K, V = _prep_common(q, k, v, g, beta, scale, np.float64)
    if g_clamp_min > -np.inf:
        g = np.maximum(g, g_clamp_min)
    S = np.zeros((B, HV, K, V))
    if initial_state is not None:
        S = S + np.asarray(initial_state, np.float64)
    o = np.zeros((B, T, HV, V))
    eye = np.eye(K)
    for b in range(B):
        for h in range(HV):
            St = S[b, h].copy()
            for t in range(T):
                kt = k[b, t, h][:, None]
                P = eye - beta[b, t, h] * (kt @ kt.T)
                St = P @ np.diag(np.exp(g[b, t, h])) @ St + beta[b, t, h] * kt @ v[b, t, h][None, :]
                o[b, t, h] = St.T @ q[b, t, h]
            S[b, h] = St
    return o, S


def _forward_substitution_unit_lower(N):
    """Solve ``(I - N) X = N`` for strictly-lower ``N`` (batched, last 2 dims).

    Restates ``torch.linalg.solve_triangular(I - A, A, upper=False)``
    (``ops_kda.py:418-420``) by row-wise forward substitution.
    """
    C = N.shape[-1]
    X = np.zeros_like(N)
    for r in range(C):
        acc = N[..., r, :].copy()
        if r:
            acc += np.einsum('...c,...cj->...j', N[..., r, :r], X[..., :r, :])
        X[..., r, :] = acc
    return X


def chunk_kda(q, k, v, g, beta, scale=None, initial_state=None, chunk_size=64,
              g_clamp_min=-10.0, compute=np.float32):
    """Chunkwise WY form; returns ``(o [B,T,HV,V], S [B,HV,K,V])``."""
    q, k, v, g, beta, B, T, HV, K, V = _prep_common(q, k, v, g, beta, scale, compute)
    S = np.zeros((B, HV, K, V), compute)
    if initial_state is not None:
        S = S + np.asarray(initial_state, compute)
    if T == 0:
        return np.zeros((B, 0, HV, V), compute), S
    C = chunk_size
    pad = (-T) % C
    if pad:
        def _p(x):
            w = [(0, 0)] * x.ndim
            w[1] = (0, pad)
            return np.pad(x, w)
        q, k, v, g, beta = map(_p, (q, k, v, g, beta))
    Tp = T + pad
    NT = Tp // C

    def to_chunks(x):  # [B, Tp, HV, ...] -> [B, HV, NT, C, ...]
        x = x.reshape(B, NT, C, HV, *x.shape[3:])
        return np.moveaxis(x, 3, 1)

    q, k, v, g = (to_chunks(x) for x in (q, k, v, g))
    beta = to_chunks(beta)
    if g_clamp_min > -np.inf:
        g = np.maximum(g, compute(g_clamp_min))
    g = np.cumsum(g, axis=-2, dtype=compute)

    # A[..., j, i] = sum_k k_j exp(min(g_j - g_i, 50)) k_i   (ops_kda.py:409-415);
    # only the strictly lower part (j > i) survives the mask of :417, so only
    # those rows are formed (the same arithmetic per element)
    A = np.zeros(g.shape[:-1] + (C,), compute)
    for i in range(C - 1):
        gd = np.minimum(g[..., i + 1:, :] - g[..., i:i + 1, :], compute(50.0))
        A[..., i + 1:, i] = (k[..., i + 1:, :] * np.exp(gd) * k[..., i:i + 1, :]).sum(-1)
    A = A * beta[..., None]
    upper_incl = np.triu(np.ones((C, C), bool), 0)
    A = -np.where(upper_incl, compute(0), A)
    X = _forward_substitution_unit_lower(A)
    A = (X + np.eye(C, dtype=compute)) * beta[..., None, :]
    w = A @ (np.exp(g) * k)
    u = A @ v

    # Aqk[..., r, c] = sum_k q_r exp(min(g_r - g_c, 50)) k_c for r >= c, zero
    # above the diagonal (ops_kda.py:515-517), for all chunks at once, column
    # by column (the same arithmetic per element)
    Aqk_all = np.zeros(g.shape[:-1] + (C,), compute)
    for c in range(C):
        diff = np.minimum(g[..., c:, :] - g[..., c:c + 1, :], compute(50.0))
        Aqk_all[..., c:, c] = (q[..., c:, :] * np.exp(diff) * k[..., c:c + 1, :]).sum(-1)
    o = np.zeros((B, HV, NT, C, V), compute)
    for n in range(NT):
        q_i, k_i, u_i, g_i, w_i = q[:, :, n], k[:, :, n], u[:, :, n], g[:, :, n], w[:, :, n]
        Aqk = Aqk_all[:, :, n]
        v_i = u_i - w_i @ S
        o[:, :, n] = (q_i * np.exp(g_i)) @ S + Aqk @ v_i
        S = S * np.exp(g_i[:, :, -1])[..., None]
        S = S + np.einsum('bhck,bhcv->bhkv', np.exp(g_i[:, :, -1:] - g_i) * k_i, v_i)
    o = o.reshape(B, HV, Tp, V).transpose(0, 2, 1, 3)[:, :T]
    return np.ascontiguousarray(o), S


def recurrent_kda_grad(q, k, v, g, beta, d_o, scale=None, initial_state=None, ds_final=None,
                       g_clamp_min=-10.0, compute=np.float64):
    """Gradients of ``recurrent_kda`` (the backward of ``naive_recurrent_kda``,
    ``ops_kda.py:175-267``, which the reference takes from autograd and checks
    in ``run_correctness.py:765-833``) for the cotangents ``d_o = dL/do``
    ``[B,T,HV,V]`` and ``ds_final = dL/dS_T`` ``[B,HV,K,V]`` (or ``None``).

    Reverse-mode pass written out by hand: the forward states are kept, then
    per token, last first, with ``a = exp(max(g, clamp))``, ``Sd = a S``,
    ``u = v - Sd^T k``, ``d = beta u``, ``S' = Sd + k d^T``, ``o = S'^T (scale q)``::

        dSt = dS + q^ do^T;   dq^ = S' do;   dd = dSt^T k;   du = beta dd
        dv = du;   dbeta = dd . u;   dk = dSt d - Sd du
        dSd = dSt - k du^T;   dg = rowsum(dSd * Sd) (0 where g < clamp);   dS = a dSd

    q and k are shared by the ``HV // H`` value heads of a key head, so their
    gradients sum over them. Returns ``(dq, dk, dv, dg, dbeta, ds0)``.
    """
    B, T, H, K = np.shape(q)
    G = np.shape(v)[2] // H
    sc = K ** -0.5 if scale is None else scale
    qh, kh, v, g_raw, beta, B, T, HV, K, V = _prep_common(q, k, v, g, beta, sc, compute)
    g = np.maximum(g_raw, compute(g_clamp_min)) if g_clamp_min > -np.inf else g_raw
    d_o = np.asarray(d_o, compute)
    S = np.zeros((B, HV, K, V), compute)
    if initial_state is not None:
        S = S + np.asarray(initial_state, compute)
    a = np.exp(g)
    Sds, us = [], []
    for t in range(T):
        Sd = S * a[:, t][..., None]
        u = v[:, t] - np.einsum('bhk,bhkv->bhv', kh[:, t], Sd)
        S = Sd + np.einsum('bhk,bhv->bhkv', kh[:, t], beta[:, t][..., None] * u)
        Sds.append(Sd)
        us.append(u)
    dS = np.zeros((B, HV, K, V), compute) if ds_final is None else np.array(ds_final, compute)
    dqh = np.zeros_like(qh)
    dkh = np.zeros_like(kh)
    dv = np.zeros_like(v)
    dg = np.zeros_like(g)
    dbeta = np.zeros_like(beta)
    for t in range(T - 1, -1, -1):
        Sd, u = Sds[t], us[t]
        d = beta[:, t][..., None] * u
        Sp = Sd + np.einsum('bhk,bhv->bhkv', kh[:, t], d)
        dSt = dS + np.einsum('bhk,bhv->bhkv', qh[:, t], d_o[:, t])
        dqh[:, t] = np.einsum('bhkv,bhv->bhk', Sp, d_o[:, t])
        dd = np.einsum('bhkv,bhk->bhv', dSt, kh[:, t])
        du = beta[:, t][..., None] * dd
        dv[:, t] = du
        dbeta[:, t] = (dd * u).sum(-1)
        dkh[:, t] = (np.einsum('bhkv,bhv->bhk', dSt, d)
                     - np.einsum('bhkv,bhv->bhk', Sd, du))
        dSd = dSt - np.einsum('bhk,bhv->bhkv', kh[:, t], du)
        dg[:, t] = (dSd * Sd).sum(-1)
        dS = dSd * a[:, t][..., None]
    if g_clamp_min > -np.inf:
        dg = np.where(g_raw >= compute(g_clamp_min), dg, compute(0))
    dq = dqh.reshape(B, T, H, G, K).sum(3) * compute(sc)
    dk = dkh.reshape(B, T, H, G, K).sum(3)
    return dq, dk, dv, dg, dbeta, dS
