"""HIP CSA / HCA kernels vs the CPU oracle (needs a ROCm GPU).

Both sides get the identical bf16 inputs. Tolerances:
* compression (fp32 math on exact bf16 inputs): 1e-5 relative to the row scale;
* indexer: the selection equals the oracle's (fp64 logits, ties by ascending
  index) except at a near-tie of the k-th logit within the kernels' logit
  error bound (``selection_check``), where only blocks within the bound may
  differ; exactly equal logits follow the shared lowest-index rule;
* attention outputs: |hip - ref| <= 2e-3 + 2e-2 |ref| on bf16 outputs, with the
  oracle attention fed the HIP selection (so a near-tie cannot change the set).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import sys

from oracle import csa as O
from oracle.common import bf16_round
from selection_check import check_selection, logit_eps

pytestmark = pytest.mark.gpu


def bf16_dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev, torch.bfloat16)


def host(t):
    return t.float().cpu().numpy()


def close(name, got, ref, rtol=2e-2, atol=2e-3):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    bad = np.abs(got - ref) > atol + rtol * np.abs(ref)
    assert not bad.any(), (f"{name}: {bad.sum()} of {bad.size} outside atol {atol} + rtol {rtol}; "
                           f"max abs err {np.abs(got - ref).max():.3e}")


def check_topk(name, idx_gpu, idx_ref, logits_ref, w_idx, nIh, sorted_=True):
    """Index parity under the kernels' logit error bound (``selection_check``):
    rows may differ from the oracle's only at a near-tie of the k-th logit, by
    blocks within the bound. Prints and returns the fraction of rows that differ."""
    rows, differ, near = check_selection(name, idx_gpu, idx_ref, logits_ref,
                                         logit_eps(w_idx, nIh), sorted_)
    print(f"{name}: {differ} of {rows} rows differ from the oracle ({near} near-ties)",
          file=sys.stderr)
    return differ / rows


def test_indexer_exact_tie_rule(dev):
    """Duplicated key rows give bit-identical logits: ties go to the lower index."""
    import kch
    rng = np.random.default_rng(9)
    B, T, cI, nIh, m, topk = 1, 64, 64, 4, 1, 6
    base = rng.standard_normal((4, cI)).astype(np.float32)
    K = base[rng.integers(0, 4, size=(B, T))]  # 64 blocks, 4 distinct rows
    qi = bf16_dev(rng.standard_normal((B, T, nIh, cI)), dev)
    wi = bf16_dev(rng.standard_normal((B, T, nIh)), dev)
    idx = kch.csa_lightning_indexer(qi, torch.from_numpy(K).to(dev), wi, topk,
                                    normalize_qk=True)
    torch.cuda.synchronize()
    idx_ref, lg = O.lightning_indexer(host(qi), K, host(wi), topk, None, None, True,
                                      return_logits=True)
    # within each group of equal logits the order is ascending block index
    got = idx.cpu().numpy()
    for t in range(T):
        vals = lg[0, t, got[0, t]]
        for j in range(topk - 1):
            if vals[j] == vals[j + 1]:
                assert got[0, t, j] < got[0, t, j + 1]
    assert np.array_equal(got, idx_ref)


def proj_inputs(seed, B, T, c, cI, nh, nIh, m, dev):
    rng = np.random.default_rng(seed)
    r = lambda *s: rng.standard_normal(s)  # noqa: E731
    xs = dict(Ca=r(B, T, c), Cb=r(B, T, c), Za=r(B, T, c), Zb=r(B, T, c), K_idx=r(B, T, cI),
              Z_idx=r(B, T, cI), q=r(B, T, nh, c), q_idx=r(B, T, nIh, cI), w_idx=r(B, T, nIh))
    dv = {k: bf16_dev(v, dev) for k, v in xs.items()}
    hs = {k: host(v) for k, v in dv.items()}
    par = dict(Ba=0.02 * r(m, c), Bb=0.02 * r(m, c), B_idx=0.02 * r(m, cI))
    parf = {k: v.astype(np.float32) for k, v in par.items()}
    pard = {k: torch.from_numpy(v).to(dev) for k, v in parf.items()}
    return dv, hs, pard, parf


@pytest.mark.parametrize("m,c", [(4, 128), (128, 128), (4, 64), (7, 64)])
def test_compress_single(dev, m, c):
    import kch
    B, T = 2, 4 * m * 3
    dv, hs, pard, parf = proj_inputs(m + c, B, T, c, 32, 1, 1, m, dev)
    out = kch.csa_compress_kv(dv["Ca"], dv["Za"], pard["Ba"], m)
    torch.cuda.synchronize()
    ref = O.compress_kv(hs["Ca"], hs["Za"], parf["Ba"], m)
    assert np.abs(host(out) - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("m,c", [(4, 128), (16, 64)])
def test_compress_overlapped(dev, m, c):
    import kch
    B, T = 2, 8 * m
    dv, hs, pard, parf = proj_inputs(3 * m + c, B, T, c, 32, 1, 1, m, dev)
    out = kch.csa_compress_kv_overlapped(dv["Ca"], dv["Cb"], dv["Za"], dv["Zb"], pard["Ba"],
                                         pard["Bb"], m)
    torch.cuda.synchronize()
    ref = O.compress_kv_overlapped(hs["Ca"], hs["Cb"], hs["Za"], hs["Zb"], parf["Ba"], parf["Bb"], m)
    assert np.abs(host(out) - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("m,c,overlap,dt,key_dt", [
    (32, 128, False, "bf16", "bf16"),   # row-parallel kernel, strided rows
    (16, 64, True, "fp32", "fp32"),     # row-parallel, overlapped, fp32 inputs
    (128, 64, False, "fp16", "bf16"),   # row-parallel, long blocks
    (4, 128, True, "bf16", "bf16"),     # lane-parallel kernel (8 rows)
    (5, 64, False, "fp32", "fp32"),     # lane-parallel kernel, odd m
])
def test_compress_key_and_window_outputs(dev, m, c, overlap, dt, key_dt):
    """All compression outputs: raw fp32 blocks, L2-normalised key rows (bf16 or
    fp32) and the per-token window keys L2norm(C_a) (bf16), for both kernels."""
    from kch.ops_csa import _compress, _compress_overlapped
    from oracle.common import l2_normalize
    dts = {"bf16": torch.bfloat16, "fp32": torch.float32, "fp16": torch.float16}
    B, T = 2, 6 * m
    rng = np.random.default_rng(m * 31 + c)
    # strided rows: the four inputs are column slices of one [B, T, 4c + 8] tensor
    big = torch.from_numpy(rng.standard_normal((B, T, 4 * c + 8)).astype(np.float32)).to(dev, dts[dt])
    Ca, Cb, Za, Zb = big[..., :c], big[..., c:2 * c], big[..., 2 * c:3 * c], big[..., 3 * c:4 * c]
    Ba = (0.5 * rng.standard_normal((m, c))).astype(np.float32)
    Bb = (0.5 * rng.standard_normal((m, c))).astype(np.float32)
    key = torch.empty(B, T // m, c, device=dev, dtype=dts[key_dt])
    local = torch.empty(B, T, c, device=dev, dtype=torch.bfloat16)
    if overlap:
        raw = _compress_overlapped("t", Ca, Cb, Za, Zb, torch.from_numpy(Ba).to(dev),
                                   torch.from_numpy(Bb).to(dev), m, key=key, normalize=True,
                                   local=local)
        ref = O.compress_kv_overlapped(host(Ca), host(Cb), host(Za), host(Zb), Ba, Bb, m)
    else:
        raw = _compress("t", Ca, Za, torch.from_numpy(Ba).to(dev), m, key=key, normalize=True,
                        local=local)
        ref = O.compress_kv(host(Ca), host(Za), Ba, m)
    torch.cuda.synchronize()
    assert np.abs(host(raw) - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())
    kref = l2_normalize(ref)
    ktol = 1e-6 if key_dt == "fp32" else 8e-3
    assert np.abs(host(key) - kref).max() <= ktol
    lref = l2_normalize(host(Ca).astype(np.float32))
    assert np.abs(host(local) - lref).max() <= 8e-3


@pytest.mark.parametrize("m,c,overlap,dt", [
    (4, 128, True, "bf16"),    # configs[2]'s CSA compression
    (4, 64, False, "bf16"),    # its indexer keys
    (7, 32, True, "fp32"),
    (5, 128, False, "fp16"),
    (1, 64, True, "bf16"),
])
@pytest.mark.parametrize("key_fmt", [0, 1, 2, 3, 4])
def test_compress_lane_kernel_matches_block_kernel(dev, m, c, overlap, dt, key_fmt):
    """Short blocks with 16-byte aligned rows take the lane-parallel kernel,
    other row strides the one-wave-per-block kernel: the same raw blocks bit for
    bit (the same per-channel arithmetic in the same order), and the same keys
    and window rows up to the norm's summation order (the keys' formats
    decoded: fp32, split bf16, split fp16, chunk-major split fp16, bf16)."""
    from kch._lib import call, ptr, stream_of, dtype_code
    dts = {"bf16": torch.bfloat16, "fp32": torch.float32, "fp16": torch.float16}
    B, T = 3, 37 * m
    nb = T // m
    rng = np.random.default_rng(m * 131 + c + key_fmt)
    wide = torch.from_numpy(rng.standard_normal((B, T, 4 * c + 8)).astype(np.float32)).to(dev, dts[dt])
    odd = torch.empty(B, T, 4 * c + 1, device=dev, dtype=dts[dt])  # unaligned row stride
    odd[..., :4 * c] = wide[..., :4 * c]
    Bab = torch.from_numpy((0.5 * rng.standard_normal((2, m, c))).astype(np.float32)).to(dev)
    kdt = {0: torch.bfloat16, 1: torch.float32, 2: torch.bfloat16, 3: torch.float16,
           4: torch.float16}[key_fmt]
    kw = {0: c, 1: c, 2: 3 * c, 3: 2 * c, 4: 2 * c}[key_fmt]
    krows = nb if key_fmt != 4 else (nb + 15) // 16 * 16
    outs = []
    for src in (wide, odd):
        raw = torch.empty(B, nb, c, device=dev, dtype=torch.float32)
        key = torch.zeros(B, krows, kw, device=dev, dtype=kdt)
        local = torch.empty(B, T, c, device=dev, dtype=torch.bfloat16)
        ld = src.shape[-1]
        Ca, Cb, Za, Zb = (src[..., i * c:(i + 1) * c] for i in range(4))
        if overlap:
            call("kch_compress_overlapped", ptr(Ca), ld, ptr(Cb), ld, ptr(Za), ld, ptr(Zb), ld,
                 ptr(Bab[0]), ptr(Bab[1]), ptr(raw), ptr(key), key_fmt, 1, ptr(local), B, T, m, c,
                 dtype_code("t", src.dtype), stream_of(src))
        else:
            call("kch_compress", ptr(Ca), ld, ptr(Za), ld, ptr(Bab[0]), ptr(raw), ptr(key), key_fmt,
                 1, ptr(local), B, T, m, c, dtype_code("t", src.dtype), stream_of(src))
        outs.append((raw, key, local))
    torch.cuda.synchronize()
    (r0, k0, l0), (r1, k1, l1) = outs
    assert torch.equal(r0.view(torch.int32), r1.view(torch.int32))

    def decode(k):
        k = k.float()
        if key_fmt == 4:  # chunk-major [chunk, part, s, q4, n, i] -> rows [chunk, n, part, s, q4, i]
            k = (k.view(B, krows // 16, 2, c // 32, 4, 16, 8).permute(0, 1, 5, 2, 3, 4, 6)
                 .reshape(B, krows, 2 * c)[:, :nb])
        if key_fmt == 2:
            return k[..., :c] + k[..., c:2 * c] + k[..., 2 * c:]
        if key_fmt in (3, 4):
            return (k[..., :c] + k[..., c:]) / 256.0
        return k
    d = (decode(k0) - decode(k1)).abs().max().item()
    tol = {0: 2.0 ** -8, 1: 1e-6, 2: 1e-6, 3: 1e-6, 4: 1e-6}[key_fmt]
    assert d <= tol, d
    ref = torch.nn.functional.normalize(r0, dim=-1)  # the keys are the unit raw blocks
    assert (decode(k0) - ref).abs().max().item() <= (2.0 ** -8 if key_fmt == 0 else 1e-6)
    assert (l0.float() - l1.float()).abs().max().item() <= 2.0 ** -8


@pytest.mark.parametrize("B,nb,cI,nIh,T_q,topk", [
    (2, 37, 64, 4, 148, 16),     # nb not a multiple of 16 (padded last chunk), two-tile kernel
    (1, 2048, 64, 4, 192, 512),  # configs[2]'s key count and top-k
    (2, 40, 32, 2, 12, 8),       # one-tile kernel (T < 16), two pieces per chunk
    (1, 50, 128, 8, 64, 24),     # 128 channels: eight pieces per chunk
    (1, 4096, 64, 4, 48, 512),   # rows beyond the register selection (configs[4]'s prefill)
])
def test_indexer_chunk_major_keys(dev, B, nb, cI, nIh, T_q, topk):
    """Compression key format 4 holds format 3's fp16 parts chunk-major (checked
    element by element against a host relayout of format 3), and the indexer
    reading them (key_split 3) returns the same logits and indices, bit for
    bit, as from the row-major parts (key_split 2)."""
    from kch.ops_csa import _compress, _indexer
    m = 4
    T = nb * m
    rng = np.random.default_rng(nb * 7 + cI)
    C = bf16_dev(rng.standard_normal((B, T, cI)), dev)
    Z = bf16_dev(rng.standard_normal((B, T, cI)), dev)
    Bp = torch.from_numpy((0.5 * rng.standard_normal((m, cI))).astype(np.float32)).to(dev)
    rows = torch.empty(B, nb, 2 * cI, device=dev, dtype=torch.float16)
    npad = (nb + 15) // 16 * 16
    chunked = torch.zeros(B, npad, 2 * cI, device=dev, dtype=torch.float16)
    _compress("t", C, Z, Bp, m, out_raw=False, key=rows, normalize=True, key_split=2)
    _compress("t", C, Z, Bp, m, out_raw=False, key=chunked, normalize=True, key_split=3)
    torch.cuda.synchronize()
    # host relayout: [B, chunk, n, part, s, q4, i] -> [B, chunk, part, s, q4, n, i]
    r = torch.zeros(B, npad, 2 * cI, dtype=torch.float16)
    r[:, :nb] = rows.cpu()
    expect = (r.view(B, npad // 16, 16, 2, cI // 32, 4, 8).permute(0, 1, 3, 4, 5, 2, 6)
              .reshape(B, npad, 2 * cI))
    assert torch.equal(chunked.cpu().view(torch.int16), expect.view(torch.int16))

    q = bf16_dev(rng.standard_normal((B, T_q, nIh, cI)), dev)
    w = bf16_dev(rng.standard_normal((B, T_q, nIh)), dev)
    pos0 = T - T_q  # the queries are the last T_q positions
    for sorted_ in (True, False):  # unsorted: the lean two-tile launch where LDS allows
        kw = dict(dense=False, pos0=pos0, normalize_q=True, idx64=False, want_logits=True,
                  sorted_=sorted_, nb=nb)
        i_row, l_row = _indexer("t", q, rows, w, topk, 1.0, m, key_split=2, **kw)
        i_chk, l_chk = _indexer("t", q, chunked, w, topk, 1.0, m, key_split=3, **kw)
        torch.cuda.synchronize()
        assert torch.equal(i_row, i_chk), sorted_
        assert torch.equal(l_row.view(torch.int32), l_chk.view(torch.int32)), sorted_
        assert (i_row >= 0).any()


@pytest.mark.parametrize("normalize", [True, False])
@pytest.mark.parametrize("T,m,topk", [(128, 4, 8), (64, 4, 32), (200, 4, 16), (96, 8, 0)])
def test_indexer_matches_oracle(dev, normalize, T, m, topk):
    import kch
    B, cI, nIh = 2, 64, 4
    nb = T // m
    dv, hs, pard, parf = proj_inputs(T + topk, B, T, 64, cI, 1, nIh, m, dev)
    K_ref = O.compress_kv(hs["K_idx"], hs["Z_idx"], parf["B_idx"], m)
    K_dev = torch.from_numpy(K_ref).to(dev)
    cbm = O.causal_block_mask(T, nb, m)
    idx = kch.csa_lightning_indexer(dv["q_idx"], K_dev, dv["w_idx"], topk,
                                    causal_block_mask=torch.from_numpy(cbm).to(dev),
                                    normalize_qk=normalize)
    torch.cuda.synchronize()
    idx_ref, lg = O.lightning_indexer(hs["q_idx"], K_ref, hs["w_idx"], topk, None, cbm,
                                      normalize, compute=np.float64, return_logits=True)
    assert idx.dtype == torch.int64 and tuple(idx.shape) == (B, T, topk)
    if topk:
        check_topk("indexer", idx.cpu().numpy(), idx_ref, lg, hs["w_idx"], nIh)


@pytest.mark.parametrize("nIh", [1, 2, 8, 16])
def test_indexer_head_counts(dev, nIh):
    # the kernel is compiled per head count (the MFMA column is (query, head))
    import kch
    B, T, cI, m, topk = 2, 128, 64, 4, 8
    nb = T // m
    dv, hs, pard, parf = proj_inputs(T + topk + nIh, B, T, 64, cI, 1, nIh, m, dev)
    K_ref = O.compress_kv(hs["K_idx"], hs["Z_idx"], parf["B_idx"], m)
    cbm = O.causal_block_mask(T, nb, m)
    idx = kch.csa_lightning_indexer(dv["q_idx"], torch.from_numpy(K_ref).to(dev), dv["w_idx"],
                                    topk, causal_block_mask=torch.from_numpy(cbm).to(dev),
                                    normalize_qk=True)
    torch.cuda.synchronize()
    idx_ref, lg = O.lightning_indexer(hs["q_idx"], K_ref, hs["w_idx"], topk, None, cbm, True,
                                      compute=np.float64, return_logits=True)
    check_topk("indexer-nIh", idx.cpu().numpy(), idx_ref, lg, hs["w_idx"], nIh)


def test_indexer_soft_weights_and_no_mask(dev):
    import kch
    B, T, cI, nIh, m, topk = 1, 32, 32, 2, 4, 4
    dv, hs, pard, parf = proj_inputs(5, B, T, 64, cI, 1, nIh, m, dev)
    K_ref = O.compress_kv(hs["K_idx"], hs["Z_idx"], parf["B_idx"], m)
    idx, soft = kch.csa_lightning_indexer(dv["q_idx"], torch.from_numpy(K_ref).to(dev), None,
                                          topk, return_soft_weights=True, normalize_qk=True)
    torch.cuda.synchronize()
    idx_ref, lg = O.lightning_indexer(hs["q_idx"], K_ref, None, topk, None, None, True,
                                      compute=np.float64, return_logits=True)
    check_topk("indexer-dense", idx.cpu().numpy(), idx_ref, lg, None, nIh)
    lg = lg.astype(np.float32)
    e = np.exp(lg - lg.max(-1, keepdims=True))
    close("soft", soft.cpu().numpy(), e / e.sum(-1, keepdims=True), rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("win,sink,topk,T", [(16, True, 8, 128), (0, True, 8, 96),
                                             (16, False, 8, 100), (8, True, 0, 64),
                                             (128, True, 512, 256)])
def test_csa_core_matches_oracle(dev, win, sink, topk, T):
    import kch
    B, c, cI, nh, nIh, m = 2, 128, 64, 16, 4, 4
    T = T - T % m
    dv, hs, pard, parf = proj_inputs(win + T + topk, B, T, c, cI, nh, nIh, m, dev)
    sink_v = np.random.default_rng(1).standard_normal(nh).astype(np.float32) if sink else None
    out, idx = kch.csa_core(dv["Ca"], dv["Cb"], dv["Za"], dv["Zb"], dv["K_idx"], dv["Z_idx"],
                            dv["q"], dv["q_idx"], dv["w_idx"], pard["Ba"], pard["Bb"],
                            pard["B_idx"], m=m, topk=topk, sliding_window=win,
                            sink_logits=None if sink_v is None else torch.from_numpy(sink_v).to(dev),
                            normalize_qk=True, return_indices=True)
    torch.cuda.synchronize()
    args = [hs[k] for k in ("Ca", "Cb", "Za", "Zb", "K_idx", "Z_idx", "q", "q_idx", "w_idx")]
    kw = dict(m=m, topk=topk, sliding_window=win, sink_logits=sink_v, normalize_qk=True)
    if topk:
        K_ref = O.compress_kv(hs["K_idx"], hs["Z_idx"], parf["B_idx"], m, compute=np.float64)
        idx_ref, lg = O.lightning_indexer(hs["q_idx"], K_ref, hs["w_idx"], topk, None,
                                          O.causal_block_mask(T, T // m, m), True,
                                          compute=np.float64, return_logits=True)
        check_topk("csa idx", idx.cpu().numpy().astype(np.int64), idx_ref, lg, hs["w_idx"], nIh)
        ref = O.csa_core(*args, parf["Ba"], parf["Bb"], parf["B_idx"],
                         indices=idx.cpu().numpy(), **kw)
    else:
        ref = O.csa_core(*args, parf["Ba"], parf["Bb"], parf["B_idx"], **kw)
    close("csa out", host(out), bf16_round(ref))


@pytest.mark.parametrize("win,sink,m2,T", [(16, True, 16, 160), (0, True, 8, 64),
                                           (32, False, 16, 96), (128, True, 128, 512)])
def test_hca_core_matches_oracle(dev, win, sink, m2, T):
    import kch
    B, c, nh = 2, 128, 16
    rng = np.random.default_rng(T + m2)
    Cd, Zd = bf16_dev(rng.standard_normal((B, T, c)), dev), bf16_dev(rng.standard_normal((B, T, c)), dev)
    qd = bf16_dev(rng.standard_normal((B, T, nh, c)), dev)
    bpos = (0.02 * rng.standard_normal((m2, c))).astype(np.float32)
    sink_v = rng.standard_normal(nh).astype(np.float32) if sink else None
    out = kch.hca_core(Cd, Zd, qd, torch.from_numpy(bpos).to(dev), m2=m2, sliding_window=win,
                       sink_logits=None if sink_v is None else torch.from_numpy(sink_v).to(dev))
    torch.cuda.synchronize()
    ref = O.hca_core(host(Cd), host(Zd), host(qd), bpos, m2=m2, sliding_window=win,
                     sink_logits=sink_v)
    close("hca out", host(out), bf16_round(ref))


def _hca_attn_ref(q, kv, loc, sink, m, win, scale):
    """Dense MQA of ``ops_hca.py:136-194`` over given key rows (oracle pieces)."""
    from oracle.common import l2_normalize
    Bn, T, nh, hd = q.shape
    nb = kv.shape[1]
    qn = l2_normalize(q.astype(np.float32))
    scores = np.einsum('bthd,bnd->bhtn', qn, kv) * np.float32(scale)
    scores = np.where(O.causal_block_mask(T, nb, m)[None, None], scores, -np.inf)
    if win > 0:
        sw, Cw, _ = O.window_scores(qn, loc, win, scale)
        sw = sw.transpose(0, 2, 1, 3)
    else:
        sw, Cw = np.zeros((Bn, nh, T, 0), np.float32), np.zeros((Bn, T, 0, hd), np.float32)
    cat = np.concatenate([scores, sw], -1).astype(np.float32)
    if cat.shape[-1] == 0:
        return np.zeros((Bn, T, nh, hd), np.float32)
    s = None if sink is None else sink.reshape(1, nh, 1, 1)
    p = O.joint_softmax_hca(cat, s)
    return (np.einsum('bhtn,bnd->bthd', p[..., :nb], kv)
            + np.einsum('bhtw,btwd->bthd', p[..., nb:], Cw))


@pytest.mark.parametrize("hd,nh,T,nb,m,win,qdt,odt,scale", [
    (128, 16, 77, 9, 8, 20, "bf16", "bf16", None),  # T not a multiple of the query tile
    (64, 5, 45, 6, 7, 100, "fp32", "fp32", None),  # window longer than the sequence
    (128, 3, 33, 0, 4, 16, "bf16", "fp32", None),  # no compressed block
    (64, 16, 50, 12, 4, 0, "bf16", "bf16", None),  # no window
    (128, 16, 130, 40, 3, 64, "fp16", "fp16", None),  # fp16 queries and output
    (64, 5, 21, 3, 5, 8, "bf16", "bf16", None),  # head count below 16, 16-bit output rows
    (64, 16, 400, 200, 2, 64, "bf16", "bf16", None),  # up to 3 key tiles of 128 rows per query tile
    (128, 8, 300, 150, 2, 100, "bf16", "fp32", None),  # 2 key tiles, rows cut inside a 32-row step
    (128, 16, 96, 12, 8, 40, "bf16", "bf16", -0.7),  # negative score scale
])
def test_hca_attn_abi_shapes(dev, hd, nh, T, nb, m, win, qdt, odt, scale):
    """kch_hca_attn over ragged shapes: query tiles cut by T, head counts below 16,
    head dim 64, empty compressed or window parts, several key tiles, every query /
    output dtype, a negative scale."""
    from kch import _lib
    from oracle.common import l2_normalize
    dts = {"bf16": torch.bfloat16, "fp32": torch.float32, "fp16": torch.float16}
    B = 2
    rng = np.random.default_rng(T * 7 + nb)
    q = torch.from_numpy(rng.standard_normal((B, T, nh, hd)).astype(np.float32)).to(dev, dts[qdt])
    kv = bf16_dev(l2_normalize(rng.standard_normal((B, max(nb, 1), hd)).astype(np.float32)), dev)
    loc = bf16_dev(l2_normalize(rng.standard_normal((B, T, hd)).astype(np.float32)), dev)
    sink = torch.from_numpy(rng.standard_normal(nh).astype(np.float32)).to(dev)
    out = torch.full((B, T, nh, hd), float("nan"), device=dev, dtype=dts[odt])
    code = {"bf16": 1, "fp32": 0, "fp16": 2}
    scale = hd ** -0.5 if scale is None else scale
    _lib.call("kch_hca_attn", _lib.ptr(q), _lib.ptr(kv), _lib.ptr(loc if win > 0 else None),
              _lib.ptr(sink), _lib.ptr(out), B, T, nb, nh, hd, m, win, scale, 1, code[qdt],
              code[odt], _lib.stream_of(q))
    torch.cuda.synchronize()
    ref = _hca_attn_ref(host(q), host(kv)[:, :nb], host(loc), host(sink), m, win, scale)
    close("hca attn", host(out), ref if odt == "fp32" else host(torch.from_numpy(ref).to(dts[odt])))


def _weights(rng, shapes, dev):
    return {k: (rng.standard_normal(s) * s[1] ** -0.5) for k, s in shapes.items()}


def test_naive_csa_end_to_end_plumbing(dev):
    """naive_csa == csa_core on the same GPU projections (padding, split, trim)."""
    import torch.nn.functional as F

    import kch
    B, T, d, c, cI, nh, nIh, dc, m = 2, 70, 64, 128, 64, 16, 4, 32, 4
    rng = np.random.default_rng(3)
    shapes = dict(W_aKV=(c, d), W_bKV=(c, d), W_aZ=(c, d), W_bZ=(c, d), W_DQ=(dc, d),
                  W_UQ=(c * nh, dc), W_IUQ=(cI * nIh, dc), W_w=(nIh, d), W_KV_idx=(cI, d),
                  W_Z_idx=(cI, d))
    W = {k: bf16_dev(v, dev) for k, v in _weights(rng, shapes, dev).items()}
    Ba, Bb = (bf16_dev(0.02 * rng.standard_normal((m, c)), dev) for _ in range(2))
    B_idx = bf16_dev(0.02 * rng.standard_normal((m, cI)), dev)
    H = bf16_dev(rng.standard_normal((B, T, d)), dev)
    sink = torch.from_numpy(rng.standard_normal(nh).astype(np.float32)).to(dev).bfloat16()
    kw = dict(m=m, topk=8, nh=nh, nIh=nIh, c=c, c_I=cI, dc=dc, sliding_window=16,
              sink_logits=sink, normalize_qk=True)
    out, proj = kch.naive_csa(H, W["W_aKV"], W["W_bKV"], W["W_aZ"], W["W_bZ"], Ba, Bb, W["W_DQ"],
                              W["W_UQ"], W["W_IUQ"], W["W_w"], W["W_KV_idx"], W["W_Z_idx"], B_idx,
                              return_projections=True, **kw)
    assert out.shape == (B, T, nh * c) and out.dtype == torch.bfloat16
    assert all(p.shape[1] == T for p in proj)
    Hp = F.pad(H, (0, 0, 0, (-T) % m))
    cat = F.linear(Hp, torch.cat([W[k] for k in ("W_aKV", "W_bKV", "W_aZ", "W_bZ", "W_KV_idx",
                                                 "W_Z_idx")], 0))
    Ca, Cb, Za, Zb, Ki, Zi = cat.split([c, c, c, c, cI, cI], -1)
    cQ = F.linear(Hp, W["W_DQ"])
    core = kch.csa_core(Ca, Cb, Za, Zb, Ki, Zi, F.linear(cQ, W["W_UQ"]).view(B, -1, nh, c),
                        F.linear(cQ, W["W_IUQ"]).view(B, -1, nIh, cI), F.linear(Hp, W["W_w"]),
                        Ba, Bb, B_idx, m=m, topk=8, sliding_window=16, sink_logits=sink,
                        normalize_qk=True)
    torch.cuda.synchronize()
    assert torch.equal(out, core.reshape(B, -1, nh * c)[:, :T])
    assert torch.equal(proj[0], Ca[:, :T])
    # T = 0 and validation
    e = kch.naive_csa(H[:, :0], W["W_aKV"], W["W_bKV"], W["W_aZ"], W["W_bZ"], Ba, Bb, W["W_DQ"],
                      W["W_UQ"], W["W_IUQ"], W["W_w"], W["W_KV_idx"], W["W_Z_idx"], B_idx, **kw)
    assert e.shape == (B, 0, nh * c)
    with pytest.raises(ValueError, match="topk"):
        kch.naive_csa(H, W["W_aKV"], W["W_bKV"], W["W_aZ"], W["W_bZ"], Ba, Bb, W["W_DQ"],
                      W["W_UQ"], W["W_IUQ"], W["W_w"], W["W_KV_idx"], W["W_Z_idx"], B_idx,
                      **{**kw, "topk": -1})


def test_naive_hca_end_to_end_plumbing(dev):
    import torch.nn.functional as F

    import kch
    B, T, d, c, nh, dc, m2 = 2, 100, 64, 128, 16, 32, 16
    rng = np.random.default_rng(4)
    shapes = dict(W_KV=(c, d), W_Z=(c, d), W_DQ=(dc, d), W_UQ=(c * nh, dc))
    W = {k: bf16_dev(v, dev) for k, v in _weights(rng, shapes, dev).items()}
    bpos = bf16_dev(0.02 * rng.standard_normal((m2, c)), dev)
    H = bf16_dev(rng.standard_normal((B, T, d)), dev)
    out, (C, Z) = kch.naive_hca(H, W["W_KV"], W["W_Z"], bpos, W["W_DQ"], W["W_UQ"], m2=m2, nh=nh,
                                c=c, dc=dc, sliding_window=32, return_projections=True)
    Hp = F.pad(H, (0, 0, 0, (-T) % m2))
    CZ = F.linear(Hp, torch.cat([W["W_KV"], W["W_Z"]], 0))
    q = F.linear(F.linear(Hp, W["W_DQ"]), W["W_UQ"]).view(B, -1, nh, c)
    core = kch.hca_core(CZ[..., :c], CZ[..., c:], q, bpos, m2=m2, sliding_window=32)
    torch.cuda.synchronize()
    assert torch.equal(out, core.reshape(B, -1, nh * c)[:, :T])
    assert C.shape == (B, T, c)
    with pytest.raises(TypeError):
        kch.naive_hca(H.long(), W["W_KV"], W["W_Z"], bpos, W["W_DQ"], W["W_UQ"], m2=m2, nh=nh,
                      c=c, dc=dc)
    with pytest.raises(ValueError, match="B_pos"):
        kch.naive_hca(H, W["W_KV"], W["W_Z"], bpos[:1], W["W_DQ"], W["W_UQ"], m2=m2, nh=nh, c=c,
                      dc=dc)
