"""The generic CSA / HCA kernels (``kch_gen_*``) against the oracle (needs a
ROCm GPU): float64 inputs, head dims above 128, more than 16 indexer heads
and indexer masks other than the block-causal one.

* float64: every output within 1e-10 of the oracle's float64 arithmetic (the
  reference's own float64 sink test, ``run_correctness.py:2530-2707``, holds
  ``naive_csa`` / ``naive_hca`` to 1e-10), selections equal;
* float32 at wide shapes: the oracle in float32 on the same inputs,
  1e-5 + 1e-4 relative, the attention fed the kernel's selection, the
  selection equal to the oracle's except at a near-tie within 1e-5 of the
  k-th logit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import csa as O
from oracle.common import l2_normalize
from selection_check import check_selection

pytestmark = pytest.mark.gpu


def dev_t(x, dev, dt):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev, dt)


def close(name, got, ref, atol, rtol=0.0):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{name}: {bad.sum()} of {bad.size} off; max abs err {err.max():.3e}"


def test_reference_fp64_sink_case(dev):
    """``run_correctness.py:2530-2707`` on the HIP operators: naive_csa
    (m 8, topk 2, nh 2, nIh 2, c 8, c_I 4, no window, sink [0.5, -0.3],
    normalize_qk) and naive_hca (m2 16, nh 2, c 8, sink [0.7, -0.2]) in
    float64, against the oracle's float64 restatement: within 1e-10."""
    import kch
    torch.manual_seed(14)
    f64 = torch.float64
    B, T, d = 1, 32, 16
    m, topk, nh, nIh, c, c_I, dc = 8, 2, 2, 2, 8, 4, 8
    H = torch.randn(B, T, d, dtype=f64) * 0.1
    W = {n: torch.randn(*s, dtype=f64) * 0.1 for n, s in (
        ("W_aKV", (c, d)), ("W_bKV", (c, d)), ("W_aZ", (c, d)), ("W_bZ", (c, d)),
        ("Ba", (m, c)), ("Bb", (m, c)), ("W_DQ", (dc, d)), ("W_UQ", (c * nh, dc)),
        ("W_IUQ", (c_I * nIh, dc)), ("W_w", (nIh, d)), ("W_KV_idx", (c_I, d)),
        ("W_Z_idx", (c_I, d)), ("B_idx", (m, c_I)))}
    sink = torch.tensor([0.5, -0.3], dtype=f64)
    Wd = {k: v.to(dev) for k, v in W.items()}
    o = kch.naive_csa(H.to(dev), Wd["W_aKV"], Wd["W_bKV"], Wd["W_aZ"], Wd["W_bZ"], Wd["Ba"],
                      Wd["Bb"], Wd["W_DQ"], Wd["W_UQ"], Wd["W_IUQ"], Wd["W_w"], Wd["W_KV_idx"],
                      Wd["W_Z_idx"], Wd["B_idx"], m=m, topk=topk, nh=nh, nIh=nIh, c=c, c_I=c_I,
                      dc=dc, sliding_window=0, sink_logits=sink.to(dev), normalize_qk=True)
    assert o.dtype == f64
    h = H.numpy()
    Wn = {k: v.numpy() for k, v in W.items()}
    lin = lambda x, w: x @ w.T  # noqa: E731
    cQ = lin(h, Wn["W_DQ"])
    ref = O.csa_core(lin(h, Wn["W_aKV"]), lin(h, Wn["W_bKV"]), lin(h, Wn["W_aZ"]),
                     lin(h, Wn["W_bZ"]), lin(h, Wn["W_KV_idx"]), lin(h, Wn["W_Z_idx"]),
                     lin(cQ, Wn["W_UQ"]).reshape(B, T, nh, c),
                     lin(cQ, Wn["W_IUQ"]).reshape(B, T, nIh, c_I), lin(h, Wn["W_w"]),
                     Wn["Ba"], Wn["Bb"], Wn["B_idx"], m=m, topk=topk, sliding_window=0,
                     sink_logits=sink.numpy(), normalize_qk=True, compute=np.float64)
    close("naive_csa fp64", o.cpu().numpy(), ref.reshape(B, T, nh * c), 1e-10)

    B2, T2, d2 = 1, 32, 16
    m2, nh2, c2, dc2 = 16, 2, 8, 16
    H2 = torch.randn(B2, T2, d2, dtype=f64) * 0.1
    W_KV2 = torch.randn(c2, d2, dtype=f64) * 0.1
    W_Z2 = torch.randn(c2, d2, dtype=f64) * 0.1
    B_pos2 = torch.randn(m2, c2, dtype=f64) * 0.1
    W_DQ2 = torch.randn(dc2, d2, dtype=f64) * 0.1
    W_UQ2 = torch.randn(c2 * nh2, dc2, dtype=f64) * 0.1
    sink2 = torch.tensor([0.7, -0.2], dtype=f64)
    o2 = kch.naive_hca(*(x.to(dev) for x in (H2, W_KV2, W_Z2, B_pos2, W_DQ2, W_UQ2)), m2=m2,
                       nh=nh2, c=c2, dc=dc2, sliding_window=0, sink_logits=sink2.to(dev))
    h2 = H2.numpy()
    ref2 = O.hca_core(h2 @ W_KV2.numpy().T, h2 @ W_Z2.numpy().T,
                      ((h2 @ W_DQ2.numpy().T) @ W_UQ2.numpy().T).reshape(B2, T2, nh2, c2),
                      B_pos2.numpy(), m2=m2, sliding_window=0, sink_logits=sink2.numpy(),
                      compute=np.float64)
    close("naive_hca fp64", o2.cpu().numpy(), ref2.reshape(B2, T2, nh2 * c2), 1e-10)


@pytest.mark.parametrize("win,sink,normalize", [(0, False, True), (5, True, True),
                                                (3, True, False)])
def test_fp64_csa_core_and_indices(dev, win, sink, normalize):
    import kch
    rng = np.random.default_rng(3 + win)
    B, T, c, cI, nh, nIh, m, topk = 2, 48, 24, 12, 3, 3, 4, 5
    x = lambda *s: rng.standard_normal(s)  # noqa: E731
    Ca, Cb, Za, Zb = x(B, T, c), x(B, T, c), x(B, T, c), x(B, T, c)
    Ki, Zi = x(B, T, cI), x(B, T, cI)
    q, qi, wi = x(B, T, nh, c), x(B, T, nIh, cI), x(B, T, nIh)
    Ba, Bb, Bi = 0.1 * x(m, c), 0.1 * x(m, c), 0.1 * x(m, cI)
    sk = x(nh) if sink else None
    args = [Ca, Cb, Za, Zb, Ki, Zi, q, qi, wi, Ba, Bb, Bi]
    out, idx = kch.csa_core(*(dev_t(a, dev, torch.float64) for a in args), m=m, topk=topk,
                            sliding_window=win,
                            sink_logits=None if sk is None else dev_t(sk, dev, torch.float64),
                            normalize_qk=normalize, return_indices=True)
    ref, ridx = O.csa_core(*args, m=m, topk=topk, sliding_window=win, sink_logits=sk,
                           normalize_qk=normalize, compute=np.float64, return_indices=True)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    close("csa_core fp64", out.cpu().numpy(), ref, 1e-10)


@pytest.mark.parametrize("win,sink", [(0, False), (7, True)])
def test_fp64_hca_core(dev, win, sink):
    import kch
    rng = np.random.default_rng(11 + win)
    B, T, c, nh, m2 = 2, 64, 20, 3, 8
    C, Z, q = rng.standard_normal((B, T, c)), rng.standard_normal((B, T, c)), \
        rng.standard_normal((B, T, nh, c))
    Bp = 0.1 * rng.standard_normal((m2, c))
    sk = rng.standard_normal(nh) if sink else None
    out = kch.hca_core(*(dev_t(a, dev, torch.float64) for a in (C, Z, q, Bp)), m2=m2,
                       sliding_window=win,
                       sink_logits=None if sk is None else dev_t(sk, dev, torch.float64))
    ref = O.hca_core(C, Z, q, Bp, m2=m2, sliding_window=win, sink_logits=sk, compute=np.float64)
    close("hca_core fp64", out.cpu().numpy(), ref, 1e-10)


def test_fp64_compression(dev):
    import kch
    rng = np.random.default_rng(2)
    B, T, c, m = 2, 40, 9, 5
    Ca, Cb, Za, Zb = (rng.standard_normal((B, T, c)) for _ in range(4))
    Ba, Bb = rng.standard_normal((m, c)), rng.standard_normal((m, c))
    f = lambda a: dev_t(a, dev, torch.float64)  # noqa: E731
    one = kch.csa_compress_kv(f(Ca), f(Za), f(Ba), m)
    two = kch.csa_compress_kv_overlapped(f(Ca), f(Cb), f(Za), f(Zb), f(Ba), f(Bb), m)
    assert one.dtype == two.dtype == torch.float64
    close("compress fp64", one.cpu().numpy(), O.compress_kv(Ca, Za, Ba, m, np.float64), 1e-12)
    close("compress overlapped fp64", two.cpu().numpy(),
          O.compress_kv_overlapped(Ca, Cb, Za, Zb, Ba, Bb, m, np.float64), 1e-12)


@pytest.mark.parametrize("dt", [torch.float64, torch.float32])
def test_indexer_arbitrary_mask(dev, dt):
    """A random boolean mask (not block-causal), broadcast over the batch, with
    soft weights; float64 exact selection, float32 under a 1e-5 near-tie rule."""
    import kch
    rng = np.random.default_rng(5)
    B, T, nb, nIh, cI, topk = 2, 33, 19, 3, 7, 6
    qi, K, wi = (rng.standard_normal(s) for s in ((B, T, nIh, cI), (B, nb, cI), (B, T, nIh)))
    mask = rng.random((T, nb)) < 0.6
    mask[:3] = False  # rows with nothing visible
    f = lambda a: dev_t(a, dev, dt)  # noqa: E731
    idx, soft = kch.csa_lightning_indexer(f(qi), f(K), f(wi), topk,
                                          causal_block_mask=torch.from_numpy(mask).to(dev),
                                          return_soft_weights=True, normalize_qk=True)
    ridx, lg = O.lightning_indexer(qi, K, wi, topk, None, mask, True, np.float64,
                                   return_logits=True)
    got = idx.cpu().numpy()
    if dt == torch.float64:
        assert np.array_equal(got, ridx)
    else:
        check_selection("indexer fp32 mask", got, ridx, lg, 1e-5, sorted_=True)
    fin = np.isfinite(lg)
    mx = np.where(fin, lg, -np.inf).max(-1, keepdims=True)
    e = np.where(fin, np.exp(lg - np.where(np.isfinite(mx), mx, 0)), 0)
    sref = np.where(fin.any(-1, keepdims=True), e / np.maximum(e.sum(-1, keepdims=True), 1e-300), 0)
    close("soft weights", soft.cpu().numpy(), sref, 1e-12 if dt == torch.float64 else 1e-6)


def test_fp32_wide_shapes(dev):
    """c = 160, c_I = 144, nIh = 20 (beyond the MFMA kernels) in float32: the
    CSA core against the oracle fed the kernel's selection; HCA with c = 192."""
    import kch
    rng = np.random.default_rng(8)
    B, T, c, cI, nh, nIh, m, topk, win = 1, 64, 160, 144, 2, 20, 4, 6, 5
    x = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    args = [x(B, T, c), x(B, T, c), x(B, T, c), x(B, T, c), x(B, T, cI), x(B, T, cI),
            x(B, T, nh, c), x(B, T, nIh, cI), x(B, T, nIh), 0.1 * x(m, c), 0.1 * x(m, c),
            0.1 * x(m, cI)]
    sk = x(nh)
    out, idx = kch.csa_core(*(dev_t(a, dev, torch.float32) for a in args), m=m, topk=topk,
                            sliding_window=win, sink_logits=dev_t(sk, dev, torch.float32),
                            normalize_qk=True, return_indices=True)
    got = idx.cpu().numpy().astype(np.int64)
    _, ridx = O.csa_core(*args, m=m, topk=topk, sliding_window=win, sink_logits=sk,
                         normalize_qk=True, compute=np.float64, return_indices=True)
    nb = T // m
    lg = O.indexer_logits(args[7], O.compress_kv(args[4], args[5], args[11], m, np.float64),
                          args[8], None, O.causal_block_mask(T, nb, m), True, np.float64)
    check_selection("wide csa", got, ridx, lg, 1e-5)
    ref = O.csa_core(*args, m=m, topk=topk, sliding_window=win, sink_logits=sk,
                     normalize_qk=True, compute=np.float64, indices=got)
    close("wide csa_core", out.cpu().numpy(), ref, 1e-5, 1e-4)

    c2, m2 = 192, 8
    C, Z, q, Bp = x(B, T, c2), x(B, T, c2), x(B, T, 3, c2), 0.1 * x(m2, c2)
    out2 = kch.hca_core(*(dev_t(a, dev, torch.float32) for a in (C, Z, q, Bp)), m2=m2,
                        sliding_window=win)
    ref2 = O.hca_core(C, Z, q, Bp, m2=m2, sliding_window=win, compute=np.float64)
    close("wide hca_core", out2.cpu().numpy(), ref2, 1e-5, 1e-4)


def test_generic_paths_refuse_gradients(dev):
    import kch
    q = torch.randn(1, 8, 2, 8, dtype=torch.float64, device=dev, requires_grad=True)
    C = torch.randn(1, 8, 8, dtype=torch.float64, device=dev)
    Bp = torch.randn(4, 8, dtype=torch.float64, device=dev)
    with pytest.raises(NotImplementedError, match="gradients are not provided"):
        kch.hca_core(C, C, q, Bp, m2=4)
