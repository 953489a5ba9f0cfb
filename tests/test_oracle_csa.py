"""Pins for the CSA / HCA / decode-cache oracle (CPU only).

Each check is an independent statement of what the mathematics fixes, chosen
so that a plausible restatement mistake fails one of them:

* compression: per-(block, channel) loops of the softmax-gated sums of the
  paper's Eqs. 11-12 / 22-23 (``2606.19348v1.txt:474-488,639-644``), the
  block-0 rule of the overlapped branch and its causality
  (``run_correctness.py:701-762``) -> wrong branch pairing, wrong softmax axis;
* block mask: window-close counts (``run_correctness.py:1145-1163``);
* indexer: loop logits (ReLU per head, weighted head sum), selection by an
  explicit sort on (-logit, index), -1 padding, ``w_idx=None`` == ones,
  ``topk=0`` (``run_correctness.py:1095-1264``);
* joint softmax + sink: a per-(token, head) fp64 loop of
  p_i = e^{s_i} / (sum_j e^{s_j} + e^{sink}) over the selected / compressed and
  window rows (the independent formula of ``run_correctness.py:2530-2707``);
* causality under future perturbations (``:1937-2155``), T < m' (``:3360-3403``),
  topk = 0 (``:3297-3357``);
* decode caches == the full-sequence operator row by row
  (``run_correctness.py:4731-4830``), ring contents (``:4872-4894``).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import csa as O
from oracle.caches import CSACacheOracle, HCACacheOracle
from oracle.common import l2_normalize


def _rn(rng, *s, scale=1.0):
    return scale * rng.standard_normal(s)


def _softmax_list(xs):
    mx = max(xs)
    e = [math.exp(x - mx) for x in xs]
    s = sum(e)
    return [v / s for v in e]


def test_compress_kv_bruteforce():
    rng = np.random.default_rng(0)
    B, T, c, m = 2, 12, 3, 4
    C, Z, Bp = _rn(rng, B, T, c), _rn(rng, B, T, c), _rn(rng, m, c, scale=0.3)
    out = O.compress_kv(C, Z, Bp, m, compute=np.float64)
    for b in range(B):
        for i in range(T // m):
            for ch in range(c):
                w = _softmax_list([Z[b, i * m + j, ch] + Bp[j, ch] for j in range(m)])
                ref = sum(w[j] * C[b, i * m + j, ch] for j in range(m))
                assert abs(out[b, i, ch] - ref) < 1e-12


def test_compress_overlapped_bruteforce_and_causality():
    rng = np.random.default_rng(1)
    B, T, c, m = 2, 16, 3, 4
    Ca, Cb, Za, Zb = (_rn(rng, B, T, c) for _ in range(4))
    Ba, Bb = _rn(rng, m, c, scale=0.3), _rn(rng, m, c, scale=0.3)
    out = O.compress_kv_overlapped(Ca, Cb, Za, Zb, Ba, Bb, m, compute=np.float64)
    for b in range(B):
        for i in range(T // m):
            for ch in range(c):
                logits = [Za[b, i * m + j, ch] + Ba[j, ch] for j in range(m)]
                vals = [Ca[b, i * m + j, ch] for j in range(m)]
                if i > 0:  # block i mixes Ca_i with Cb_{i-1}; block 0 has no b-branch
                    logits += [Zb[b, (i - 1) * m + j, ch] + Bb[j, ch] for j in range(m)]
                    vals += [Cb[b, (i - 1) * m + j, ch] for j in range(m)]
                w = _softmax_list(logits)
                assert abs(out[b, i, ch] - sum(a * v for a, v in zip(w, vals))) < 1e-12
    # causality: changing block 2's tokens leaves blocks 0..1 alone; changing
    # Cb of block 1 moves block 2 but not block 1
    Ca2 = Ca.copy()
    Ca2[:, 2 * m:3 * m] += 1.0
    out2 = O.compress_kv_overlapped(Ca2, Cb, Za, Zb, Ba, Bb, m, compute=np.float64)
    assert np.array_equal(out2[:, :2], out[:, :2]) and not np.allclose(out2[:, 2], out[:, 2])
    Cb2 = Cb.copy()
    Cb2[:, m:2 * m] += 1.0
    out3 = O.compress_kv_overlapped(Ca, Cb2, Za, Zb, Ba, Bb, m, compute=np.float64)
    assert np.array_equal(out3[:, :2], out[:, :2]) and not np.allclose(out3[:, 2], out[:, 2])


def test_causal_block_mask_counts():
    for m in (1, 3, 4):
        T = 13
        nb = T // m
        mask = O.causal_block_mask(T, nb, m)
        for t in range(T):
            vis = [b for b in range(nb) if mask[t, b]]
            # a block becomes visible at the token that closes it
            assert vis == list(range(min(nb, (t + 1) // m)))


def _brute_logits(q, k, w, scale, normalize):
    B, T, Hh, D = q.shape
    nb = k.shape[1]
    if normalize:
        q, k = l2_normalize(q), l2_normalize(k)
    out = np.zeros((B, T, nb))
    for b in range(B):
        for t in range(T):
            for n in range(nb):
                s = 0.0
                for h in range(Hh):
                    dot = sum(q[b, t, h, d] * k[b, n, d] for d in range(D))
                    s += (1.0 if w is None else w[b, t, h]) * max(scale * dot, 0.0)
                out[b, t, n] = s
    return out


@pytest.mark.parametrize("normalize", [True, False])
def test_indexer_bruteforce(normalize):
    rng = np.random.default_rng(2)
    B, T, Hh, D, nb, m, topk = 2, 9, 2, 4, 4, 2, 3
    q, k, w = _rn(rng, B, T, Hh, D), _rn(rng, B, nb, D), _rn(rng, B, T, Hh)
    mask = O.causal_block_mask(T, nb, m)
    scale = 1.0 if normalize else D ** -0.5
    lg = O.indexer_logits(q, k, w, None, mask, normalize, compute=np.float64)
    ref = _brute_logits(q, k, w, scale, normalize)
    ref = np.where(mask[None], ref, -np.inf)
    np.testing.assert_allclose(lg, ref, rtol=1e-12, atol=1e-12)
    idx = O.lightning_indexer(q, k, w, topk, None, mask, normalize, compute=np.float64)
    for b in range(B):
        for t in range(T):
            order = sorted(range(nb), key=lambda n: (-ref[b, t, n], n))[:topk]
            exp = [n if np.isfinite(ref[b, t, n]) else -1 for n in order]
            exp += [-1] * (topk - len(exp))
            assert list(idx[b, t]) == exp
    # w_idx=None is all-ones weights; topk=0 gives an empty selection; ties by index
    np.testing.assert_allclose(
        O.indexer_logits(q, k, None, None, mask, normalize, compute=np.float64),
        O.indexer_logits(q, k, np.ones_like(w), None, mask, normalize, compute=np.float64))
    assert O.lightning_indexer(q, k, w, 0, None, mask, normalize).shape == (B, T, 0)
    tie = O.topk_desc_lowest_index(np.array([[1.0, 3.0, 3.0, 0.0, 3.0]]), 4)
    assert list(tie[0]) == [1, 2, 4, 0]


def _joint_loop(rows_s, rows_v, sink):
    """sum_i p_i v_i with p_i = e^{s_i}/(sum e^{s_j} + e^{sink}); 0 with no rows."""
    if not rows_s:
        return np.zeros(rows_v.shape[-1] if hasattr(rows_v, 'shape') else 0)
    terms = list(rows_s) + ([sink] if sink is not None else [])
    mx = max(terms)
    den = sum(math.exp(x - mx) for x in terms)
    return sum(math.exp(s - mx) / den * v for s, v in zip(rows_s, rows_v))


def _csa_inputs(rng, B, T, c, cI, nh, nIh):
    Ca, Cb, Za, Zb = (_rn(rng, B, T, c) for _ in range(4))
    Ki, Zi = _rn(rng, B, T, cI), _rn(rng, B, T, cI)
    q, qi, wi = _rn(rng, B, T, nh, c), _rn(rng, B, T, nIh, cI), _rn(rng, B, T, nIh)
    return Ca, Cb, Za, Zb, Ki, Zi, q, qi, wi


@pytest.mark.parametrize("sink", [True, False])
def test_csa_core_joint_softmax_loop(sink):
    rng = np.random.default_rng(3)
    B, T, c, cI, nh, nIh, m, topk, win = 1, 11, 4, 3, 2, 2, 2, 3, 3
    Ca, Cb, Za, Zb, Ki, Zi, q, qi, wi = _csa_inputs(rng, B, T, c, cI, nh, nIh)
    Ba, Bb, Bi = _rn(rng, m, c), _rn(rng, m, c), _rn(rng, m, cI)
    sk = _rn(rng, nh) if sink else None
    out, idx = O.csa_core(Ca, Cb, Za, Zb, Ki, Zi, q, qi, wi, Ba, Bb, Bi, m=m, topk=topk,
                          sliding_window=win, sink_logits=sk, compute=np.float64,
                          return_indices=True)
    Tp = T + (-T) % m
    pad = lambda x: np.concatenate([x, np.zeros((B, Tp - T) + x.shape[2:])], 1)  # noqa: E731
    Cn = l2_normalize(O.compress_kv_overlapped(pad(Ca), pad(Cb), pad(Za), pad(Zb), Ba, Bb, m,
                                               compute=np.float64))
    Cl = l2_normalize(Ca)
    qn = l2_normalize(q)
    for t in range(T):
        sel = [int(n) for n in idx[0, t] if n >= 0]
        assert all(n < (t + 1) // m for n in sel)  # only visible blocks
        wpos = list(range(max(0, t - win + 1), t + 1))
        for h in range(nh):
            s = [float(qn[0, t, h] @ Cn[0, n]) for n in sel] + \
                [float(qn[0, t, h] @ Cl[0, p]) for p in wpos]
            v = [Cn[0, n] for n in sel] + [Cl[0, p] for p in wpos]
            ref = _joint_loop(s, v, None if sk is None else float(sk[h]))
            np.testing.assert_allclose(out[0, t, h], ref, rtol=1e-10, atol=1e-12)


def test_hca_core_joint_softmax_loop_and_short_T():
    rng = np.random.default_rng(4)
    B, T, c, nh, m2, win = 1, 13, 4, 2, 4, 3
    C, Z, q = _rn(rng, B, T, c), _rn(rng, B, T, c), _rn(rng, B, T, nh, c)
    Bp, sk = _rn(rng, m2, c), _rn(rng, nh)
    out = O.hca_core(C, Z, q, Bp, m2=m2, sliding_window=win, sink_logits=sk, compute=np.float64)
    Tp = T + (-T) % m2
    pad = lambda x: np.concatenate([x, np.zeros((B, Tp - T) + x.shape[2:])], 1)  # noqa: E731
    Cn = l2_normalize(O.compress_kv(pad(C), pad(Z), Bp, m2, compute=np.float64))
    Cl, qn = l2_normalize(C), l2_normalize(q)
    for t in range(T):
        blocks = list(range((t + 1) // m2))
        wpos = list(range(max(0, t - win + 1), t + 1))
        for h in range(nh):
            s = [float(qn[0, t, h] @ Cn[0, n]) for n in blocks] + \
                [float(qn[0, t, h] @ Cl[0, p]) for p in wpos]
            v = [Cn[0, n] for n in blocks] + [Cl[0, p] for p in wpos]
            np.testing.assert_allclose(out[0, t, h], _joint_loop(s, v, float(sk[h])),
                                       rtol=1e-10, atol=1e-12)
    # T < m2: no compressed block is visible, only the window contributes
    short = O.hca_core(C[:, :3], Z[:, :3], q[:, :3], Bp, m2=m2, sliding_window=0,
                       sink_logits=sk, compute=np.float64)
    assert np.all(short == 0)


def test_causality_csa_hca():
    rng = np.random.default_rng(5)
    B, T, c, cI, nh, nIh, m, t0 = 1, 16, 4, 3, 2, 2, 4, 9
    args = list(_csa_inputs(rng, B, T, c, cI, nh, nIh))
    W = [_rn(rng, m, c), _rn(rng, m, c), _rn(rng, m, cI)]
    kw = dict(m=m, topk=2, sliding_window=3, sink_logits=_rn(rng, nh), compute=np.float64)
    base = O.csa_core(*args, *W, **kw)
    pert = [a.copy() for a in args]
    for a in pert:
        a[:, t0 + 1:] += _rn(rng, *a[:, t0 + 1:].shape)
    moved = O.csa_core(*pert, *W, **kw)
    np.testing.assert_array_equal(moved[:, :t0 + 1], base[:, :t0 + 1])
    assert not np.allclose(moved[:, t0 + 1:], base[:, t0 + 1:])
    C, Z, q = args[0], args[2], args[6]
    hk = dict(m2=m, sliding_window=3, sink_logits=kw['sink_logits'], compute=np.float64)
    hb = O.hca_core(C, Z, q, W[0], **hk)
    hm = O.hca_core(pert[0], pert[2], pert[6], W[0], **hk)
    np.testing.assert_array_equal(hm[:, :t0 + 1], hb[:, :t0 + 1])


def test_topk_zero_is_window_only():
    rng = np.random.default_rng(6)
    B, T, c, cI, nh, nIh, m = 1, 8, 4, 3, 2, 2, 2
    args = _csa_inputs(rng, B, T, c, cI, nh, nIh)
    W = [_rn(rng, m, c), _rn(rng, m, c), _rn(rng, m, cI)]
    sk = _rn(rng, nh)
    a = O.csa_core(*args, *W, m=m, topk=0, sliding_window=3, sink_logits=sk, compute=np.float64)
    # the same as an all-empty selection
    b = O.csa_core(*args, *W, m=m, topk=2, sliding_window=3, sink_logits=sk, compute=np.float64,
                   indices=np.full((B, T, 2), -1))
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-14)
    # no window and no selection: zero output
    z = O.csa_core(*args, *W, m=m, topk=0, sliding_window=0, sink_logits=sk, compute=np.float64)
    assert np.all(z == 0)


def test_cache_oracles_match_full_sequence():
    rng = np.random.default_rng(7)
    B, T, c, cI, nh, nIh, m, win = 2, 19, 4, 3, 2, 2, 3, 4
    Ca, Cb, Za, Zb, Ki, Zi, q, qi, wi = _csa_inputs(rng, B, T, c, cI, nh, nIh)
    Ba, Bb, Bi, sk = _rn(rng, m, c), _rn(rng, m, c), _rn(rng, m, cI), _rn(rng, nh)
    full = O.csa_core(Ca, Cb, Za, Zb, Ki, Zi, q, qi, wi, Ba, Bb, Bi, m=m, topk=64,
                      sliding_window=win, sink_logits=sk)
    cache = CSACacheOracle(B, c, cI, m, win, 'fp32')
    for t in range(T):
        sl = slice(t, t + 1)
        cache.append_step(Ca[:, sl], Cb[:, sl], Za[:, sl], Zb[:, sl], Ki[:, sl], Zi[:, sl],
                          Ba, Bb, Bi)
        o = cache.forward_step(l2_normalize(q[:, sl]), qi[:, sl], wi[:, sl], topk=64,
                               sink_logits=sk)
        np.testing.assert_allclose(o[:, 0], full[:, t], rtol=1e-5, atol=1e-6)
        assert cache.n_blocks == (t + 1) // m
    ring = np.stack(cache.ring, axis=1)
    np.testing.assert_allclose(ring, l2_normalize(Ca[:, T - win:]).astype(np.float32),
                               rtol=1e-6)
    C, Z = Ca, Za
    hfull = O.hca_core(C, Z, q, Ba, m2=m, sliding_window=win, sink_logits=sk)
    hc = HCACacheOracle(B, c, m, win, 'fp32')
    hc.append_step(C[:, :7], Z[:, :7], Ba)  # bulk prefill, then single tokens
    for t in range(7, T):
        hc.append_step(C[:, t:t + 1], Z[:, t:t + 1], Ba)
        o = hc.forward_step(l2_normalize(q[:, t:t + 1]), sink_logits=sk)
        np.testing.assert_allclose(o[:, 0], hfull[:, t], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("win,sink,topk", [(8, True, 5), (0, False, 3), (16, True, 0)])
def test_csa_core_at_equals_csa_core_rows(win, sink, topk):
    """The query-sliced restatement gives csa_core's rows, its selection and logits."""
    rng = np.random.default_rng(win + topk)
    B, T, c, cI, nh, nIh, m = 2, 64, 16, 8, 3, 2, 4
    r = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    args = (r(B, T, c), r(B, T, c), r(B, T, c), r(B, T, c), r(B, T, cI), r(B, T, cI),
            r(B, T, nh, c), r(B, T, nIh, cI), r(B, T, nIh))
    par = (0.1 * r(m, c), 0.1 * r(m, c), 0.1 * r(m, cI))
    kw = dict(m=m, topk=topk, sliding_window=win, sink_logits=r(nh) if sink else None,
              normalize_qk=True)
    full, idx_full = O.csa_core(*args, *par, return_indices=True, **kw)
    Q = np.array([0, 3, 17, 40, 63])
    out, idx, lg = O.csa_core_at(*args, *par, queries=Q, **kw)
    np.testing.assert_allclose(out, full[:, Q], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(idx, idx_full[:, Q])
    out2, _, _ = O.csa_core_at(*args, *par, queries=Q, indices=idx, **kw)
    np.testing.assert_array_equal(out2, out)


@pytest.mark.parametrize("win,sink", [(8, True), (0, False)])
def test_hca_core_at_equals_hca_core_rows(win, sink):
    """The query-sliced HCA restatement gives hca_core's rows."""
    rng = np.random.default_rng(win + 3)
    B, T, c, nh, m2 = 2, 64, 16, 3, 8
    r = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    C, Z, q, Bp = r(B, T, c), r(B, T, c), r(B, T, nh, c), 0.1 * r(m2, c)
    sk = r(nh) if sink else None
    full = O.hca_core(C, Z, q, Bp, m2=m2, sliding_window=win, sink_logits=sk)
    Q = np.array([0, 5, 7, 8, 31, 63])
    out = O.hca_core_at(C, Z, q, Bp, m2=m2, queries=Q, sliding_window=win, sink_logits=sk)
    np.testing.assert_allclose(out, full[:, Q], rtol=1e-5, atol=1e-6)
    out2 = O.hca_core_at(C, Z, q, Bp, m2=m2, queries=Q, sliding_window=win, sink_logits=sk,
                         C_comp=O.compress_kv(C, Z, Bp, m2))
    np.testing.assert_array_equal(out2, out)


def _fd_worst(loss, args, grads):
    """Largest |central difference - gradient| / (|num| + |ana| + 1e-2) over
    every coordinate of every argument (the floor absorbs the ~1e-10 rounding
    noise of the differences; a dropped or wrong term moves a gradient by its
    own size)."""
    worst = 0.0
    for name, x in args.items():
        for idx in np.ndindex(*x.shape):
            orig = x[idx]
            x[idx] = orig + 1e-6
            lp = loss()
            x[idx] = orig - 1e-6
            lm = loss()
            x[idx] = orig
            num = (lp - lm) / 2e-6
            a = grads[name][idx]
            worst = max(worst, abs(num - a) / (abs(num) + abs(a) + 1e-2))
    return worst


@pytest.mark.parametrize("T,win,sink,local", [(10, 3, True, False), (12, 0, False, False),
                                              (8, 5, True, True)])
def test_hca_core_grad_matches_finite_differences(T, win, sink, local):
    """``hca_core_grad`` (queries, compression inputs, window rows, sink) against
    central differences of ``hca_core`` in fp64, every coordinate; T=10 pads to
    a multiple of m2=4."""
    from oracle.csa import hca_core_grad
    rng = np.random.default_rng(T + win)
    B, m2, nh, c = 1, 4, 2, 4
    a = dict(C=rng.standard_normal((B, T, c)), Z=rng.standard_normal((B, T, c)),
             q=rng.standard_normal((B, T, nh, c)), B_pos=rng.standard_normal((m2, c)) * 0.3)
    if sink:
        a["sink_logits"] = rng.standard_normal(nh)
    if local:
        a["C_local_raw"] = rng.standard_normal((B, T, c))
    W = rng.standard_normal((B, T, nh, c))
    kw = dict(m2=m2, sliding_window=win, scale=1.3)

    def loss():
        return float((O.hca_core(compute=np.float64, **kw, **a) * W).sum())

    g = hca_core_grad(d_out=W, **kw, **a)
    assert set(g) == set(a)
    assert _fd_worst(loss, a, g) < 1e-6


def test_compress_kv_grad_matches_finite_differences():
    from oracle.csa import compress_kv_grad
    rng = np.random.default_rng(2)
    B, T, c, m = 2, 12, 3, 4
    a = dict(C=rng.standard_normal((B, T, c)), Z=rng.standard_normal((B, T, c)),
             B_pos=rng.standard_normal((m, c)))
    W = rng.standard_normal((B, T // m, c))

    def loss():
        return float((O.compress_kv(a["C"], a["Z"], a["B_pos"], m, np.float64) * W).sum())

    dC, dZ, dB = compress_kv_grad(a["C"], a["Z"], a["B_pos"], m, W)
    assert _fd_worst(loss, a, dict(C=dC, Z=dZ, B_pos=dB)) < 1e-6


def test_compress_overlapped_grad_matches_finite_differences():
    from oracle.csa import compress_kv_overlapped_grad
    rng = np.random.default_rng(5)
    B, T, c, m = 1, 12, 3, 4
    a = {k: rng.standard_normal((B, T, c)) for k in ("Ca", "Cb", "Za", "Zb")}
    a.update(Ba=rng.standard_normal((m, c)), Bb=rng.standard_normal((m, c)))
    W = rng.standard_normal((B, T // m, c))

    def loss():
        return float((O.compress_kv_overlapped(a["Ca"], a["Cb"], a["Za"], a["Zb"], a["Ba"], a["Bb"],
                                               m, np.float64) * W).sum())

    g = compress_kv_overlapped_grad(a["Ca"], a["Cb"], a["Za"], a["Zb"], a["Ba"], a["Bb"], m, W)
    assert _fd_worst(loss, a, dict(zip(("Ca", "Cb", "Za", "Zb", "Ba", "Bb"), g))) < 1e-6


@pytest.mark.parametrize("norm,win,sink", [(True, 3, True), (False, 0, False), (False, 5, True)])
def test_csa_attn_grad_matches_finite_differences(norm, win, sink):
    """``csa_attn_grad`` with a fixed selection (including -1 slots and a
    query whose every slot is unused) against central differences of
    ``csa_core(indices=...)`` in fp64; ``slot`` against the derivative of the
    loss along a rescaling of each selected row in the gather (one query's
    attention restated from the oracle's joint softmax)."""
    from oracle.csa import csa_attn_grad
    rng = np.random.default_rng(7 + win)
    B, T, c, m, nh, topk, cI, nIh = 1, 12, 4, 4, 2, 2, 4, 1
    a = {k: rng.standard_normal((B, T, c)) for k in ("Ca", "Cb", "Za", "Zb")}
    a.update(q=rng.standard_normal((B, T, nh, c)), Ba=rng.standard_normal((m, c)) * 0.3,
             Bb=rng.standard_normal((m, c)) * 0.3)
    if sink:
        a["sink_logits"] = rng.standard_normal(nh)
    nb = T // m
    idx = np.full((B, T, topk), -1)
    for t in range(T):
        vis = (t + 1) // m
        if vis and t != 9:
            pick = rng.choice(vis, size=min(vis, topk), replace=False)
            idx[0, t, :len(pick)] = pick
    W = rng.standard_normal((B, T, nh, c))
    dummy = dict(K_idx=np.zeros((B, T, cI)), Z_idx=np.zeros((B, T, cI)),
                 q_idx=np.zeros((B, T, nIh, cI)), w_idx=np.zeros((B, T, nIh)),
                 B_idx=np.zeros((m, cI)))
    kw = dict(m=m, topk=topk, sliding_window=win, normalize_qk=norm, indices=idx)

    def loss():
        return float((O.csa_core(a["Ca"], a["Cb"], a["Za"], a["Zb"], dummy["K_idx"], dummy["Z_idx"],
                                 a["q"], dummy["q_idx"], dummy["w_idx"], a["Ba"], a["Bb"],
                                 dummy["B_idx"], sink_logits=a.get("sink_logits"),
                                 compute=np.float64, **kw) * W).sum())

    g = csa_attn_grad(a["Ca"], a["Cb"], a["Za"], a["Zb"], a["q"], a["Ba"], a["Bb"], idx, W, m=m,
                      sliding_window=win, sink_logits=a.get("sink_logits"), normalize_qk=norm)
    assert _fd_worst(loss, a, g) < 1e-6
    assert nb == 3 and np.all(g["slot"][idx < 0] == 0)
    # slot: d L / d alpha where selected row k of query t enters (as key and
    # value) scaled by 1 + alpha; the attention of that one query, restated
    # from the oracle's pieces
    from oracle.common import l2_normalize as l2n
    raw = O.compress_kv_overlapped(a["Ca"], a["Cb"], a["Za"], a["Zb"], a["Ba"], a["Bb"], m, np.float64)
    Cn = l2n(raw) if norm else raw
    qn = l2n(a["q"]) if norm else a["q"]
    sc = 1.0 if norm else c ** -0.5
    Cl = l2n(a["Ca"]) if norm else a["Ca"]
    sk = a.get("sink_logits")

    def q_loss(t, k, alpha):
        rows = [Cn[0, j] * (1 + alpha if kk == k else 1) for kk, j in enumerate(idx[0, t]) if j >= 0]
        rows += [Cl[0, u] for u in range(max(0, t - win + 1), t + 1)] if win else []
        if not rows:
            return 0.0
        V = np.stack(rows)
        s = np.einsum('hd,jd->hj', qn[0, t], V) * sc
        pr = O.joint_softmax_csa(s[None], np.ones_like(s[None], bool),
                                 None if sk is None else sk.reshape(1, nh, 1))[0]
        return float((np.einsum('hj,jd->hd', pr, V) * W[0, t]).sum())

    for t in range(T):
        for k in range(topk):
            if idx[0, t, k] >= 0:
                num = (q_loss(t, k, 1e-6) - q_loss(t, k, -1e-6)) / 2e-6
                ana = g["slot"][0, t, k]
                assert abs(num - ana) <= 1e-6 * (abs(num) + abs(ana) + 1e-2), (t, k, num, ana)
