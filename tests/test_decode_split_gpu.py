"""Split decode kernels (``kch_csa_decode`` / ``kch_hca_decode``) vs the CPU
oracle at cache sizes that take several indexer ranges and many attention
slices (needs a ROCm GPU).

* indices: the oracle's selection (``oracle.csa``, fp64 logits of the same
  stored key rows, ties by ascending index) under the rule of
  ``selection_check``: a row may differ only at a near-tie within twice the
  fp32-level logit bound ``eps``; engineered exact ties must follow the
  lowest-index rule;
* outputs: the joint softmax with sink over the selected rows and the ring,
  in fp64 (the sink formula of ``run_correctness.py:2530-2707``), atol 2e-3 +
  rtol 2e-2 (keys and values are bf16 rows).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.common import bf16_round, l2_normalize
from oracle.csa import indexer_logits, topk_desc_lowest_index
from selection_check import check_selection, logit_eps

pytestmark = pytest.mark.gpu


def close(name, got, ref, rtol=2e-2, atol=2e-3):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), name
    bad = np.abs(got - ref) > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{name}: {bad.sum()} bad, max err {np.abs(got - ref).max():.3e}"


def joint_ref(q, rows, sink):
    """q [nh, c] unit rows, rows [n, c] unit rows: sum_i p_i rows_i with
    p_i = e^{s_i} / (sum_j e^{s_j} + e^{sink}); zero without rows."""
    nh, c = q.shape
    if rows.shape[0] == 0:
        return np.zeros((nh, c))
    s = q.astype(np.float64) @ rows.T.astype(np.float64)
    mx = np.maximum(s.max(-1, keepdims=True), sink[:, None])
    e = np.exp(s - mx)
    den = e.sum(-1, keepdims=True) + np.exp(sink[:, None] - mx)
    return (e / den) @ rows.astype(np.float64)


def run_csa(dev, kraw, q, qi, wi, crow, ring, sink, topk, nIh, cI, normalize=True, key_dt=torch.bfloat16):
    """kraw [B, nb, cI] (key rows as cached), crow [B, nb, c] unit bf16 rows."""
    from kch import _lib
    B, nb = kraw.shape[:2]
    nh, c = q.shape[1], q.shape[2]
    lib = _lib.load()
    kr = torch.from_numpy(kraw).to(dev, key_dt)
    kinv = kr.float().norm(dim=-1).clamp_min(1e-12).reciprocal() if normalize else None
    kv = torch.from_numpy(crow).to(dev, torch.bfloat16) if nb else None
    rg = torch.from_numpy(ring).to(dev, torch.bfloat16) if ring.shape[1] else None
    qd = torch.from_numpy(q).to(dev)
    qid = torch.from_numpy(qi).to(dev)
    wid = torch.from_numpy(wi).to(dev)
    sk = torch.from_numpy(sink).to(dev)
    out = torch.empty(B, nh, c, device=dev)
    idx = torch.empty(B, max(topk, 1), device=dev, dtype=torch.int32)
    nbytes = lib.kch_decode_ws_bytes(B, nb, nh, c, topk, ring.shape[1], 1)
    ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
    _lib.call("kch_csa_decode", _lib.ptr(qd), _lib.ptr(qid), _lib.ptr(wid), _lib.ptr(kv), nb * c,
              _lib.ptr(kr), nb * cI, _lib.ptr(kinv), nb, _lib.ptr(rg), ring.shape[1] * c,
              ring.shape[1], _lib.ptr(sk), _lib.ptr(out), _lib.ptr(idx) if topk else None, B, nb,
              nh, c, nIh, cI, topk, 1.0, 1.0 if normalize else cI ** -0.5, 0, int(normalize), 0,
              _lib.dtype_code("t", key_dt), 0, _lib.ptr(ws), nbytes, _lib.stream_of(qd))
    torch.cuda.synchronize()
    return out.cpu().numpy(), idx.cpu().numpy()[:, :topk], kr.float().cpu().numpy()


def make_csa(rng, B, nb, c, cI, nh, nIh, win):
    kraw = rng.standard_normal((B, nb, cI)).astype(np.float32)
    crow = bf16_round(l2_normalize(rng.standard_normal((B, nb, c)))).astype(np.float32)
    ring = bf16_round(l2_normalize(rng.standard_normal((B, win, c)))).astype(np.float32)
    q = l2_normalize(rng.standard_normal((B, nh, c))).astype(np.float32)
    qi = rng.standard_normal((B, nIh, cI)).astype(np.float32)
    wi = rng.standard_normal((B, nIh)).astype(np.float32)
    sink = rng.standard_normal(nh).astype(np.float32)
    return kraw, crow, ring, q, qi, wi, sink


def sel_eps(qi, kr_used, wi, normalize):
    """The logit bound of ``selection_check`` per sequence; unnormalised rows
    scale it by the largest ``|q_h| |k_n| / sqrt(cI)``."""
    eps = logit_eps(wi, qi.shape[1])
    if normalize:
        return eps
    mag = (np.linalg.norm(qi, axis=-1).max(-1) * np.linalg.norm(kr_used, axis=-1).max(-1)
           * qi.shape[-1] ** -0.5)
    return eps * np.maximum(mag, 1.0)


def check_csa(name, out, idx, kr_used, crow, ring, q, qi, wi, sink, topk, normalize=True):
    B = q.shape[0]
    lg = indexer_logits(qi[:, None], kr_used, wi[:, None], None, None, normalize,
                        compute=np.float64)[:, 0]
    ref_idx = topk_desc_lowest_index(lg, topk)
    rows, differ, near = check_selection(name, idx, ref_idx, lg,
                                         sel_eps(qi, kr_used, wi, normalize), sorted_=True)
    print(f"{name}: {differ} of {rows} selections differ, {near} near-ties")
    for b in range(B):
        got = idx[b]
        sel = got[got >= 0]
        rows = np.concatenate([crow[b][sel], ring[b]], axis=0)
        close(f"{name} out b{b}", out[b], joint_ref(q[b], rows, sink))


@pytest.mark.parametrize("nb,topk", [(20000, 512), (9000, 64), (3000, 512), (700, 1024), (5000, 37)])
def test_csa_decode_multi_range(dev, nb, topk):
    rng = np.random.default_rng(nb + topk)
    B, c, cI, nh, nIh, win = 2, 128, 64, 16, 4, 128
    kraw, crow, ring, q, qi, wi, sink = make_csa(rng, B, nb, c, cI, nh, nIh, win)
    out, idx, kr_used = run_csa(dev, kraw, q, qi, wi, crow, ring, sink, topk, nIh, cI)
    check_csa(f"nb{nb} topk{topk}", out, idx, kr_used, crow, ring, q, qi, wi, sink, topk)


def test_csa_decode_fp32_keys_unnormalised(dev):
    rng = np.random.default_rng(5)
    B, nb, c, cI, nh, nIh, win, topk = 3, 10000, 64, 32, 8, 2, 16, 128
    kraw, crow, ring, q, qi, wi, sink = make_csa(rng, B, nb, c, cI, nh, nIh, win)
    out, idx, kr_used = run_csa(dev, kraw, q, qi, wi, crow, ring, sink, topk, nIh, cI,
                                normalize=False, key_dt=torch.float32)
    check_csa("fp32 keys", out, idx, kr_used, crow, ring, q, qi, wi, sink, topk, normalize=False)


def test_csa_decode_exact_ties_lowest_index(dev):
    """Every block but 100 random ones repeats one key row, so the threshold
    logit is tied many times over three indexer ranges: the tied picks must be
    the lowest block indices."""
    rng = np.random.default_rng(6)
    B, nb, c, cI, nh, nIh, win, topk = 1, 18000, 64, 64, 4, 4, 0, 256
    kraw, crow, ring, q, qi, wi, sink = make_csa(rng, B, nb, c, cI, nh, nIh, win)
    winners = rng.choice(nb, 100, replace=False)
    base = kraw[:, :1].copy()
    kraw[:] = base
    kraw[:, winners] = rng.standard_normal((B, 100, cI)).astype(np.float32)
    tied_at = int(np.setdiff1d(np.arange(nb), winners)[0])
    out, idx, kr_used = run_csa(dev, kraw, q, qi, wi, crow, ring, sink, topk, nIh, cI)
    check_csa("ties", out, idx, kr_used, crow, ring, q, qi, wi, sink, topk)
    lg = indexer_logits(qi[:, None], kr_used, wi[:, None], None, None, True)[:, 0]
    tied = np.nonzero(lg[0] == lg[0][tied_at])[0]
    assert len(tied) >= nb - 100
    tset = set(tied.tolist())
    got_tied = [int(i) for i in idx[0] if int(i) in tset]
    assert got_tied == tied[:len(got_tied)].tolist(), got_tied[:10]


def test_csa_decode_edges(dev):
    rng = np.random.default_rng(7)
    B, c, cI, nh, nIh = 2, 64, 32, 4, 2
    # no cached block: ring only
    kraw, crow, ring, q, qi, wi, sink = make_csa(rng, B, 0, c, cI, nh, nIh, 5)
    out, idx, _ = run_csa(dev, kraw, q, qi, wi, crow, ring, sink, 8, nIh, cI)
    assert (idx == -1).all()
    for b in range(B):
        close("ring only", out[b], joint_ref(q[b], ring[b], sink))
    # blocks, no ring, topk > nb, and topk = 0 with a ring
    kraw, crow, ring, q, qi, wi, sink = make_csa(rng, B, 40, c, cI, nh, nIh, 0)
    out, idx, kr = run_csa(dev, kraw, q, qi, wi, crow, ring, sink, 64, nIh, cI)
    assert (idx[:, 40:] == -1).all() and (np.sort(idx[:, :40], axis=1) == np.arange(40)).all()
    check_csa("topk>nb", out, idx, kr, crow, ring, q, qi, wi, sink, 64)
    kraw, crow, ring, q, qi, wi, sink = make_csa(rng, B, 40, c, cI, nh, nIh, 9)
    out, idx, _ = run_csa(dev, kraw, q, qi, wi, crow, ring, sink, 0, nIh, cI)
    for b in range(B):
        close("topk=0", out[b], joint_ref(q[b], ring[b], sink))


@pytest.mark.parametrize("B,nb,win", [(2, 5000, 128), (3, 37, 16), (1, 0, 7), (2, 300, 0)])
def test_hca_decode_split(dev, B, nb, win):
    from kch import _lib
    rng = np.random.default_rng(nb + win)
    c, nh = 128, 16
    crow = bf16_round(l2_normalize(rng.standard_normal((B, nb, c)))).astype(np.float32)
    ring = bf16_round(l2_normalize(rng.standard_normal((B, win, c)))).astype(np.float32)
    q = rng.standard_normal((B, nh, c)).astype(np.float32)  # normalised in-kernel
    sink = rng.standard_normal(nh).astype(np.float32)
    kv = torch.from_numpy(crow).to(dev, torch.bfloat16) if nb else None
    rg = torch.from_numpy(ring).to(dev, torch.bfloat16) if win else None
    qd = torch.from_numpy(q).to(dev)
    sk = torch.from_numpy(sink).to(dev)
    out = torch.empty(B, nh, c, device=dev)
    nbytes = _lib.load().kch_decode_ws_bytes(B, nb, nh, c, 0, win, 0)
    ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
    _lib.call("kch_hca_decode", _lib.ptr(qd), _lib.ptr(kv), nb * c, _lib.ptr(rg), win * c, win,
              _lib.ptr(sk), _lib.ptr(out), B, nb, nh, c, 1.0, 1, 0, 0, _lib.ptr(ws), nbytes,
              _lib.stream_of(qd))
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    qn = l2_normalize(q)
    for b in range(B):
        rows = np.concatenate([crow[b], ring[b]], axis=0)
        close(f"hca b{b}", o[b], joint_ref(qn[b], rows, sink))


@pytest.mark.parametrize("nb,topk,win", [(300, 64, 128), (2000, 512, 16), (50, 64, 0)])
def test_decode_step_entry_points(dev, nb, topk, win):
    """``kch_csa_decode_step`` / ``kch_hca_decode_step`` (one workgroup per
    sequence, the prefill kernels in ring mode) against the oracle's indexer
    and the fp64 joint softmax."""
    from kch import _lib
    rng = np.random.default_rng(nb + 3 * topk + win)
    B, c, cI, nh, nIh = 2, 128, 64, 16, 4
    kraw, crow, ring, q, qi, wi, sink = make_csa(rng, B, nb, c, cI, nh, nIh, win)
    kn = l2_normalize(kraw.astype(np.float64)).astype(np.float32)  # fp32 unit key rows
    kd = torch.from_numpy(kn).to(dev)
    kv = torch.from_numpy(crow).to(dev, torch.bfloat16)
    rg = torch.from_numpy(ring).to(dev, torch.bfloat16) if win else None
    qd, qid, wid, sk = (torch.from_numpy(a).to(dev) for a in (q, qi, wi, sink))
    out = torch.empty(B, nh, c, device=dev)
    idx = torch.empty(B, topk, device=dev, dtype=torch.int32)
    _lib.call("kch_csa_decode_step", _lib.ptr(qd), _lib.ptr(qid), _lib.ptr(wid), _lib.ptr(kv),
              nb * c, _lib.ptr(kd), nb * cI, _lib.ptr(rg), win * c, win, _lib.ptr(sk),
              _lib.ptr(out), _lib.ptr(idx), B, nb, nh, c, nIh, cI, topk, 1.0, 1.0, 0, 1, 0, 0,
              _lib.stream_of(qd))
    torch.cuda.synchronize()
    check_csa("csa decode_step", out.cpu().numpy(), idx.cpu().numpy(), kn, crow, ring, q, qi, wi,
              sink, topk)
    out_h = torch.empty(B, nh, c, device=dev)
    _lib.call("kch_hca_decode_step", _lib.ptr(qd), _lib.ptr(kv), nb * c, _lib.ptr(rg), win * c, win,
              _lib.ptr(sk), _lib.ptr(out_h), B, nb, nh, c, 1.0, 0, 0, 0, _lib.stream_of(qd))
    torch.cuda.synchronize()
    oh = out_h.cpu().numpy()
    for b in range(B):
        rows = np.concatenate([crow[b], ring[b]], axis=0)
        close(f"hca decode_step b{b}", oh[b], joint_ref(q[b], rows, sink))
