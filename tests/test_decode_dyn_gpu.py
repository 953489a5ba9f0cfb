"""Counter-driven decode entry points against the host-planned ones (needs a
ROCm GPU).

``kch_csa_decode_dyn`` / ``kch_hca_decode_dyn`` take the block count and the
window length from a device counter (``n_seen``: nb = (n_seen + 1) / m,
ring_len = min(n_seen + 1, win)) and plan for a block capacity ``cap`` >= nb;
rows past nb hold garbage that must not matter. Against ``kch_csa_decode`` /
``kch_hca_decode`` on the same nb:

* the selection is bit-identical (both are exact top-k with ties to the lower
  block index; the counter-driven step scores in 256-block ranges and selects
  from all keys in one workgroup up to 8192 blocks, and takes the ranges +
  merge path beyond), and also checked against the oracle's indexer (fp64
  logits) under the near-tie rule of ``selection_check``;
* outputs agree to fp32 summation order (the two plan their row groups from
  different row counts).

``kch_csa_cache_append`` / ``kch_hca_cache_append`` one token at a time
against ``append_step`` of the same cache on the same projections: the ring,
the accumulator, the overlapped b-branch rows and the indexer key rows
bit-identical; the compressed rows, their attention keys and the inverse norms
within one rounding of the storage dtype (the norms are summed in another
order, and HCA's long blocks are compressed by a two-pass softmax instead of
the bulk kernel's online one).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.csa import indexer_logits, topk_desc_lowest_index
from selection_check import check_selection, logit_eps
from test_decode_split_gpu import joint_ref, make_csa, run_csa

pytestmark = pytest.mark.gpu


def _pad_rows(a, cap, rng):
    """[B, n, w] -> [B, cap, w] with random rows past n."""
    B, n, w = a.shape
    out = rng.standard_normal((B, cap, w)).astype(np.float32)
    out[:, :n] = a
    return out


def run_csa_dyn(dev, kraw, q, qi, wi, crow, ring, sink, topk, nIh, cI, cap, m, extra, rng):
    from kch import _lib
    B, nb = kraw.shape[:2]
    nh, c = q.shape[1], q.shape[2]
    win = ring.shape[1]
    lib = _lib.load()
    kr = torch.from_numpy(_pad_rows(kraw, cap, rng)).to(dev, torch.bfloat16)
    kinv = kr.float().norm(dim=-1).clamp_min(1e-12).reciprocal()
    kv = torch.from_numpy(_pad_rows(crow, cap, rng)).to(dev, torch.bfloat16)
    rg = torch.from_numpy(ring).to(dev, torch.bfloat16) if win else None
    # q rows inside wider rows (the fused projection layout)
    Q = torch.zeros(B, nh * c + nIh * cI + 8, device=dev, dtype=torch.float32)
    Q[:, :nh * c] = torch.from_numpy(q.reshape(B, -1))
    Q[:, nh * c:nh * c + nIh * cI] = torch.from_numpy(qi.reshape(B, -1))
    W = torch.zeros(B, nIh + 4, device=dev, dtype=torch.float32)
    W[:, :nIh] = torch.from_numpy(wi)
    sk = torch.from_numpy(sink).to(dev)
    out = torch.empty(B, nh, c, device=dev)
    idx = torch.empty(B, topk, device=dev, dtype=torch.int32)
    n_seen = torch.tensor([nb * m - 1 + extra], device=dev, dtype=torch.int32)
    nbytes = lib.kch_decode_dyn_ws_bytes(B, cap, nh, c, topk, win, 1)
    ws = torch.empty(max(nbytes, 256), device=dev, dtype=torch.uint8)
    _lib.call("kch_csa_decode_dyn", _lib.ptr(Q), Q.shape[1], _lib.ptr(Q[:, nh * c:]), Q.shape[1],
              _lib.ptr(W), W.shape[1], _lib.ptr(kv), cap * c, _lib.ptr(kr), cap * cI,
              _lib.ptr(kinv), cap, _lib.ptr(rg), win * c, _lib.ptr(n_seen), m, win, cap,
              _lib.ptr(sk), _lib.ptr(out), _lib.ptr(idx), B, nh, c, nIh, cI, topk, 1.0, 1.0, 0, 1,
              0, _lib.dtype_code("t", torch.bfloat16), 0, _lib.ptr(ws), ws.numel(),
              _lib.stream_of(Q))
    torch.cuda.synchronize()
    return out.cpu().numpy(), idx.cpu().numpy()


@pytest.mark.parametrize("nb,topk,cap,m", [(4096, 512, 8192, 4), (1000, 64, 1024, 4),
                                           (300, 512, 600, 8), (9000, 512, 12000, 4),
                                           (1, 8, 4, 4)])
def test_csa_decode_dyn_matches_planned(dev, nb, topk, cap, m):
    rng = np.random.default_rng(nb + cap)
    B, c, cI, nh, nIh, win = 2, 128, 64, 16, 4, 128
    kraw, crow, ring, q, qi, wi, sink = make_csa(rng, B, nb, c, cI, nh, nIh, win)
    if nb >= 64:
        kraw[:, 40] = kraw[:, 7]    # exact ties: the lower index must win
        kraw[:, 63] = kraw[:, 7]
    for extra in (0, m - 1):
        ring_len = min(nb * m + extra, win)  # min(n_seen + 1, win)
        out_p, idx_p, kr_used = run_csa(dev, kraw, q, qi, wi, crow, ring[:, :ring_len], sink,
                                        topk, nIh, cI)
        out_d, idx_d = run_csa_dyn(dev, kraw, q, qi, wi, crow, ring, sink, topk, nIh, cI, cap, m,
                                   extra, rng)
        assert np.array_equal(idx_d[:, :min(topk, nb)], idx_p[:, :min(topk, nb)]), \
            f"nb={nb}: selections differ"
        assert (idx_d[:, nb:] == -1).all()
        np.testing.assert_allclose(out_d, out_p, rtol=1e-5, atol=1e-6)
    lg = indexer_logits(qi[:, None], kr_used, wi[:, None], None, None, True,
                        compute=np.float64)[:, 0]
    ref = topk_desc_lowest_index(lg, topk)
    check_selection(f"dyn nb={nb}", idx_d, ref, lg, logit_eps(wi, nIh), sorted_=True)
    for b in range(B):
        if nb >= 64 and 7 in ref[b] and 40 not in ref[b]:
            assert 7 in idx_d[b] and 40 not in idx_d[b]


def test_csa_decode_dyn_no_blocks(dev):
    """n_seen = 1 < m - 1: no block yet; the window alone (its first 2 rows)."""
    rng = np.random.default_rng(3)
    B, c, cI, nh, nIh, win, m, cap, topk = 2, 64, 32, 4, 2, 8, 4, 2, 16
    _, _, ring, q, qi, wi, sink = make_csa(rng, B, 1, c, cI, nh, nIh, win)
    kraw = rng.standard_normal((B, 0, cI)).astype(np.float32)
    crow = np.zeros((B, 0, c), np.float32)
    out, idx = run_csa_dyn(dev, kraw, q, qi, wi, crow, ring, sink, topk, nIh, cI, cap, m, 2, rng)
    assert (idx == -1).all()
    for b in range(B):
        np.testing.assert_allclose(out[b], joint_ref(q[b], ring[b][:2], sink), rtol=2e-2, atol=2e-3)


@pytest.mark.parametrize("nb,cap,m2", [(100, 300, 128), (0, 4, 16), (513, 513, 8)])
def test_hca_decode_dyn_matches_planned(dev, nb, cap, m2):
    from kch import _lib
    rng = np.random.default_rng(nb + 7)
    B, c, nh, win = 2, 128, 16, 128
    lib = _lib.load()
    crow = rng.standard_normal((B, cap, c)).astype(np.float32)
    crow /= np.linalg.norm(crow, axis=-1, keepdims=True)
    ring = rng.standard_normal((B, win, c)).astype(np.float32)
    ring /= np.linalg.norm(ring, axis=-1, keepdims=True)
    kv = torch.from_numpy(crow).to(dev, torch.bfloat16)
    rg = torch.from_numpy(ring).to(dev, torch.bfloat16)
    q = torch.randn(B, nh * c + 16, device=dev)
    sink = torch.randn(nh, device=dev)
    extra = m2 - 1 if nb else 5
    n_seen = torch.tensor([max(nb * m2 - 1, 0) + extra], device=dev, dtype=torch.int32)
    ring_len = min(int(n_seen.item()) + 1, win)
    out_d = torch.empty(B, nh, c, device=dev)
    nbytes = lib.kch_decode_dyn_ws_bytes(B, cap, nh, c, 0, win, 0)
    ws = torch.empty(max(nbytes, 256), device=dev, dtype=torch.uint8)
    _lib.call("kch_hca_decode_dyn", _lib.ptr(q), q.shape[1], _lib.ptr(kv), cap * c, _lib.ptr(rg),
              win * c, _lib.ptr(n_seen), m2, win, cap, _lib.ptr(sink), _lib.ptr(out_d), B, nh, c,
              1.0, 1, 0, 0, _lib.ptr(ws), ws.numel(), _lib.stream_of(q))
    qc = q[:, :nh * c].contiguous()
    out_p = torch.empty(B, nh, c, device=dev)
    nbytes = lib.kch_decode_ws_bytes(B, nb, nh, c, 0, ring_len, 0)
    ws2 = torch.empty(max(nbytes, 256), device=dev, dtype=torch.uint8)
    _lib.call("kch_hca_decode", _lib.ptr(qc), _lib.ptr(kv), cap * c, _lib.ptr(rg), win * c,
              ring_len, _lib.ptr(sink), _lib.ptr(out_p), B, nb, nh, c, 1.0, 1, 0, 0,
              _lib.ptr(ws2), ws2.numel(), _lib.stream_of(q))
    torch.cuda.synchronize()
    torch.testing.assert_close(out_d, out_p, rtol=1e-5, atol=1e-6)


def _ulps_close(name, got, ref, dtype):
    got = got.float().cpu().numpy().astype(np.float64)
    ref = ref.float().cpu().numpy().astype(np.float64)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    bad = np.abs(got - ref) > ulp * np.maximum(np.abs(ref), 1e-30) * 1.01
    assert not bad.any(), f"{name}: {bad.sum()} of {bad.size} beyond one rounding"


@pytest.mark.parametrize("kind", ["csa", "hca"])
def test_cache_append_matches_append_step(dev, kind):
    import kch
    from kch import _lib
    torch.manual_seed(5)
    B, c, cI, win = 2, 128, 64, 8
    m = 4 if kind == "csa" else 16
    dt = torch.bfloat16
    W = 4 * c + 2 * cI if kind == "csa" else 2 * c
    T0, steps = 37, 45
    P = torch.randn(B, T0 + steps, W + 8, device=dev).to(dt)
    if kind == "csa":
        Ba, Bb, Bk = (0.1 * torch.randn(m, w, device=dev) for w in (c, c, cI))
        ce = kch.CSADecodingCache(B, c, cI, m, win, dev, dt)
        cd = kch.CSADecodingCache(B, c, cI, m, win, dev, dt)

        def eager(cache, p):
            cache.append_step(*p[..., :W].split([c, c, c, c, cI, cI], -1), Ba, Bb, Bk)
    else:
        Bp = 0.1 * torch.randn(m, c, device=dev)
        ce = kch.HCADecodingCache(B, c, m, win, dev, dt)
        cd = kch.HCADecodingCache(B, c, m, win, dev, dt)

        def eager(cache, p):
            cache.append_step(*p[..., :W].split([c, c], -1), Bp)
    eager(ce, P[:, :T0])
    eager(cd, P[:, :T0])
    n_seen = torch.zeros(1, device=dev, dtype=torch.int32)
    for t in range(T0, T0 + steps):
        eager(ce, P[:, t:t + 1])
        cap = cd._device_buffers()
        if kind == "csa":
            cap = max(cd._C.rows.shape[1], cd._K.rows.shape[1])
            cd._C.ensure(cd.n_blocks, cap)
            cd._K.ensure(cd.n_blocks, cap)
        n_seen.fill_(cd.n_tokens_seen)
        row = P[:, t].contiguous()
        if kind == "csa":
            _lib.call("kch_csa_cache_append", _lib.ptr(row), W + 8, _lib.ptr(cd._acc_buf),
                      _lib.ptr(cd._prev_buf), _lib.ptr(Ba), _lib.ptr(Bb), _lib.ptr(Bk),
                      _lib.ptr(cd._sw._buf), _lib.ptr(cd._C.rows), _lib.ptr(cd._C.keys),
                      _lib.ptr(cd._K.rows), _lib.ptr(cd._K.inv), _lib.ptr(n_seen), B, c, cI, m,
                      win, cap, 1, _lib.dtype_code("t", dt), _lib.stream_of(row))
        else:
            _lib.call("kch_hca_cache_append", _lib.ptr(row), W + 8, _lib.ptr(cd._acc_buf),
                      _lib.ptr(Bp), _lib.ptr(cd._sw._buf), _lib.ptr(cd._C.rows),
                      _lib.ptr(cd._C.keys), _lib.ptr(n_seen), B, c, m, win, cap, 1,
                      _lib.dtype_code("t", dt), _lib.stream_of(row))
        cd._device_advance()
    torch.cuda.synchronize()
    nb = ce.n_blocks
    assert cd.n_blocks == nb == (T0 + steps) // m and cd.n_tokens_seen == ce.n_tokens_seen
    assert cd.accumulator_len == ce.accumulator_len
    assert torch.equal(cd._sw._buf, ce._sw._buf)
    a = ce.accumulator_len
    assert torch.equal(cd._acc_buf[:, :a], ce._acc_buf[:, :a])
    new = slice(T0 // m, nb)  # the blocks completed one token at a time
    _ulps_close(f"{kind} rows", cd._C.rows[:, new], ce._C.rows[:, new], dt)
    _ulps_close(f"{kind} keys", cd._C.keys[:, new], ce._C.keys[:, new], torch.bfloat16)
    if kind == "csa":
        assert torch.equal(cd._prev_buf, ce._prev_buf)
        assert torch.equal(cd._K.rows[:, new], ce._K.rows[:, new])
        torch.testing.assert_close(cd._K.inv[:, new], ce._K.inv[:, new], rtol=1e-6, atol=0)
        # the block rows of the overlapped compression as the bulk kernel computes them
        assert torch.equal(cd._C.rows[:, new], ce._C.rows[:, new])


@pytest.mark.parametrize("kind", ["csa", "hca"])
def test_cache_append_rows_matches_separate_calls(dev, kind):
    """kch_{csa,hca}_cache_append_rows (the append and the query
    up-projection in one launch) against kch_{csa,hca}_cache_append followed
    by kch_linear_rows_fused: the caches and the projected rows bit-identical
    over steps that complete blocks."""
    import kch
    from kch import _lib
    torch.manual_seed(6)
    B, c, cI, win, dc, NQ = 3, 128, 64, 8, 128, 2304
    m = 4 if kind == "csa" else 16
    dt = torch.bfloat16
    code = _lib.dtype_code("t", dt)
    W = 4 * c + 2 * cI if kind == "csa" else 2 * c
    LD = W + dc + 8
    T0, steps = 21, 40
    P = torch.randn(B, T0 + steps, LD, device=dev).to(dt)
    Wq = (torch.randn(NQ, dc, device=dev) / dc ** 0.5).to(dt)
    if kind == "csa":
        Ba, Bb, Bk = (0.1 * torch.randn(m, w, device=dev) for w in (c, c, cI))
        caches = [kch.CSADecodingCache(B, c, cI, m, win, dev, dt) for _ in range(2)]
        for cc in caches:
            cc.append_step(*P[:, :T0, :W].split([c, c, c, c, cI, cI], -1), Ba, Bb, Bk)
    else:
        Bp = 0.1 * torch.randn(m, c, device=dev)
        caches = [kch.HCADecodingCache(B, c, m, win, dev, dt) for _ in range(2)]
        for cc in caches:
            cc.append_step(*P[:, :T0, :W].split([c, c], -1), Bp)
    n_seen = torch.zeros(1, device=dev, dtype=torch.int32)
    for t in range(T0, T0 + steps):
        row = P[:, t].contiguous()
        qs = []
        for i, cd in enumerate(caches):
            cap = cd._device_buffers()
            if kind == "csa":
                cap = max(cd._C.rows.shape[1], cd._K.rows.shape[1])
                cd._C.ensure(cd.n_blocks, cap)
                cd._K.ensure(cd.n_blocks, cap)
            n_seen.fill_(cd.n_tokens_seen)
            q = torch.empty(B, NQ, device=dev, dtype=dt)
            rows = (_lib.ptr(row[:, W:]), LD, _lib.ptr(Wq), dc, _lib.ptr(q), NQ, NQ, dc)
            if kind == "csa":
                cargs = (_lib.ptr(row), LD, _lib.ptr(cd._acc_buf), _lib.ptr(cd._prev_buf),
                         _lib.ptr(Ba), _lib.ptr(Bb), _lib.ptr(Bk), _lib.ptr(cd._sw._buf),
                         _lib.ptr(cd._C.rows), _lib.ptr(cd._C.keys), _lib.ptr(cd._K.rows),
                         _lib.ptr(cd._K.inv), _lib.ptr(n_seen), B, c, cI, m, win, cap, 1)
            else:
                cargs = (_lib.ptr(row), LD, _lib.ptr(cd._acc_buf), _lib.ptr(Bp),
                         _lib.ptr(cd._sw._buf), _lib.ptr(cd._C.rows), _lib.ptr(cd._C.keys),
                         _lib.ptr(n_seen), B, c, m, win, cap, 1)
            if i == 0:
                _lib.call(f"kch_{kind}_cache_append", *cargs, code, _lib.stream_of(row))
                _lib.call("kch_linear_rows_fused", rows[0], LD, rows[2], dc, rows[4], NQ, B, NQ,
                          dc, None, None, 0.0, 0, None, 0, None, code, _lib.stream_of(row))
            else:
                _lib.call(f"kch_{kind}_cache_append_rows", *cargs, *rows, code,
                          _lib.stream_of(row))
            torch.cuda.synchronize()
            cd._device_advance()
            qs.append(q)
        assert torch.equal(qs[0], qs[1]), f"step {t}: projected rows differ"
    a, b = caches
    assert a.n_blocks == b.n_blocks == (T0 + steps) // m
    for x, y in zip(_cache_state(a), _cache_state(b)):
        assert torch.equal(x, y)


def _cache_state(cache):
    """The written part of a decode cache's buffers."""
    nb, acc = cache.n_blocks, cache.accumulator_len
    bufs = [cache._sw._buf, cache._acc_buf[:, :acc], cache._C.rows[:, :nb], cache._C.keys[:, :nb]]
    if hasattr(cache, "_K"):
        bufs += [cache._prev_buf, cache._K.rows[:, :nb], cache._K.inv[:, :nb]]
    return bufs


@pytest.mark.parametrize("d", [2048, 4096, 96])
def test_kda_front_rows_matches_separate_calls(dev, d):
    """kch_kda_front_rows (LayerNorm + conv over [lookback ; h] in the input
    projection's prologue) followed by kch_kda_decode_step_shift, against
    kch_kda_decode_front + kch_linear_rows_fused + kch_kda_decode_step, over
    several tokens: the lookback rows, the projection and the outputs agree to
    the dtype's rounding (the LayerNorm statistics are summed in another order)."""
    from kch import _lib
    torch.manual_seed(7)
    B, H, HV, K, V = 3, 4, 4, 128, 128
    dt = torch.bfloat16
    code = _lib.dtype_code("t", dt)
    NW = 2 * H * K + HV * V + HV + K
    NP = (NW + 7) // 8 * 8
    W = (torch.randn(NW, d, device=dev) / d ** 0.5).to(dt)
    ln_w = 1 + 0.1 * torch.randn(d, device=dev)
    ln_b = 0.1 * torch.randn(d, device=dev)
    conv_w = (0.5 * torch.randn(d, 3, device=dev)).to(dt)
    conv_b = (0.1 * torch.randn(d, device=dev)).to(dt)
    g_up = (torch.randn(HV * K, K, device=dev) / K ** 0.5).to(dt)
    look = [(0.5 * torch.randn(B, 2, d, device=dev)).to(dt) for _ in range(2)]
    look[1].copy_(look[0])
    state = [0.02 * torch.randn(B, HV, K, V, device=dev) for _ in range(2)]
    state[1].copy_(state[0])
    st = _lib.stream_of(W)
    for step in range(4):
        x = torch.randn(B, d, device=dev).to(dt)
        # separate launches
        xc = torch.empty(B, d, device=dev, dtype=dt)
        _lib.call("kch_kda_decode_front", _lib.ptr(x), d, _lib.ptr(ln_w), _lib.ptr(ln_b), 1e-5,
                  _lib.ptr(look[0]), _lib.ptr(conv_w), _lib.ptr(conv_b), _lib.ptr(xc), B, d, code,
                  0, st)
        p0 = torch.empty(B, NP, device=dev, dtype=dt)
        _lib.call("kch_linear_rows_fused", _lib.ptr(xc), d, _lib.ptr(W), d, _lib.ptr(p0), NP, B,
                  NW, d, None, None, 0.0, 0, None, 0, None, code, st)
        o0 = torch.empty(B, HV * V, device=dev, dtype=dt)
        _lib.call("kch_kda_decode_step", _lib.ptr(p0), NP, _lib.ptr(g_up), _lib.ptr(state[0]),
                  _lib.ptr(o0), B, H, HV, K, V, K ** -0.5, 0.5, -10.0, code, st)
        # the front in the projection's prologue, the shift in the step
        h = torch.empty(B, d, device=dev, dtype=dt)
        p1 = torch.empty(B, NP, device=dev, dtype=dt)
        _lib.call("kch_kda_front_rows", _lib.ptr(x), d, _lib.ptr(ln_w), _lib.ptr(ln_b), 1e-5, 0,
                  _lib.ptr(look[1]), _lib.ptr(conv_w), _lib.ptr(conv_b), _lib.ptr(h), _lib.ptr(W),
                  d, _lib.ptr(p1), NP, B, NW, d, code, st)
        o1 = torch.empty(B, HV * V, device=dev, dtype=dt)
        _lib.call("kch_kda_decode_step_shift", _lib.ptr(p1), NP, _lib.ptr(g_up),
                  _lib.ptr(state[1]), _lib.ptr(o1), B, H, HV, K, V, K ** -0.5, 0.5, -10.0,
                  _lib.ptr(look[1]), _lib.ptr(h), d, code, st)
        torch.cuda.synchronize()
        for name, a, b in (("lookback", look[0], look[1]), ("proj", p0[:, :NW], p1[:, :NW]),
                           ("o", o0, o1), ("state", state[0], state[1])):
            torch.testing.assert_close(b.float(), a.float(), rtol=2 ** -6, atol=1e-4,
                                       msg=f"step {step}: {name}")
        exact = (look[0] == look[1]).float().mean().item()
        assert exact > 0.99, f"step {step}: only {exact:.4f} of the lookback bit-identical"
        look[1].copy_(look[0])  # keep the two paths on the same history
        state[1].copy_(state[0])
