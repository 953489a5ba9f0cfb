"""Parity at the benchmark configurations' own regimes (needs a ROCm GPU).

* ``configs[1]`` at full length: KDA chunk prefill, bf16, T=4096 (64 chunks
  of 64), K=V=128, S0 ~ 0.02 N(0,1): output and final state against the fp64
  oracle, rtol 2e-2 + atol 2e-3 on every element.
* ``configs[2]``'s selection regime: ``csa_core`` at configs[2]'s own B=4,
  T=8192 (m=4, 2048 blocks, indexer 4 x 64, top-512, window 128 + sink, 16
  heads of 128) on projections of random layer weights, at 384 late queries
  of each sequence (1536 rows; they see 1024-2048 blocks, so the top-512
  binds). The kernel's own logits are checked against the fp64 oracle's
  within ``eps = 1e-6 * sum_h |w_h| + 1e-7`` (``selection_check``: fp32-level,
  from the three-part split-bf16 products); indices are compared with the
  oracle's (fp64 logits, ties by ascending index): a row may differ only
  where its k-th and (k+1)-th logits lie within 2 eps, and then only by
  blocks within 2 eps of the boundary. The mismatch fraction is printed.
  Outputs at those queries are checked against the oracle on the selection
  the kernel made.
* rows beyond the register selection: the indexer at configs[4]'s prefill
  length (T=16384, 4096 blocks) takes the radix select; its unsorted and
  sorted selections hold the same sets, the unsorted rows in ascending
  index, and both match the oracle at 192 late queries under the same bound.
* ``configs[3]`` at full length: ``hca_core`` at T=32768 (B=1; m'=128, 256
  compressed blocks in two key tiles, window 128 + sink, 16 heads of 128) on
  projections of random layer weights, at 448 queries (the first 64, 128
  around the key-tile boundary, the last 256) against ``oracle.csa.hca_core_at``
  in fp64, every element at the bar.
* ``configs[4]``'s shapes: ``HybridDecoding`` (d=2048, 16 x 128 KDA heads,
  CSA as above, HCA m'=128) in bf16 at B=2, prefill of T=2301 = 18 * 128 - 3
  (575 CSA blocks: the top-512 binds), then 8 decode steps on the
  device-driven kernels: the third completes an HCA block (m'=128) and a CSA
  block, the seventh another CSA block. Against ``oracle.hybrid`` layer by
  layer (``composed_check.decode_vs_oracle``: each oracle sub-layer fed the
  residual stream the HIP sub-layer saw, the CSA layer on the selection the
  kernels made). Every element within rtol 2e-2 + atol 2e-3.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from composed_check import decode_vs_oracle
from oracle import csa as OC
from oracle import hybrid as OH
from oracle.kda import chunk_kda
from selection_check import check_logits, check_selection, logit_eps

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-2, 2e-3


def close(name, got, ref, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite output"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    print(f"{name}: max abs err {err.max():.3e}, rel fro {rel:.2e}", file=sys.stderr)
    assert not bad.any(), (f"{name}: {bad.sum()} of {bad.size} beyond atol {atol} + rtol {rtol}; "
                           f"max abs err {err.max():.3e}")


def test_kda_config1_full_length(dev):
    import kch
    B, T, H, K, V = 1, 4096, 2, 128, 128
    g = torch.Generator().manual_seed(11)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    v = torch.randn(B, T, H, V, generator=g)
    gt = torch.nn.functional.logsigmoid(torch.randn(B, T, H, K, generator=g))
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    s0 = 0.02 * torch.randn(B, H, K, V, generator=g)
    xs = [x.to(torch.bfloat16) for x in (q, k, v, gt, beta)]
    o, s = kch.naive_chunk_kda(*[x.to(dev) for x in xs], initial_state=s0.to(dev),
                               output_final_state=True)
    torch.cuda.synchronize()
    o_ref, s_ref = chunk_kda(*[x.double().numpy() for x in xs], initial_state=s0.double().numpy(),
                             chunk_size=64, compute=np.float64)
    close("kda C1 T4096 o", o.float().cpu().numpy(), o_ref)
    close("kda C1 T4096 state", s.cpu().numpy(), s_ref)


def _c2_projections(dev, B, T, seed):
    """configs[2] projections of random weights (bf16, N(0, fan_in^-1/2))."""
    d, c, nh, dc, nIh, cI, m = 2048, 128, 16, 128, 4, 64, 4
    g = torch.Generator().manual_seed(seed)

    def w(o, i):
        return (torch.randn(o, i, generator=g) * i ** -0.5).to(dev, torch.bfloat16)
    W6 = torch.cat([w(c, d), w(c, d), w(c, d), w(c, d), w(cI, d), w(cI, d)], 0)
    W_DQ, W_UQ, W_IUQ, W_w = w(dc, d), w(c * nh, dc), w(cI * nIh, dc), w(nIh, d)
    par = [(0.02 * torch.randn(m, n, generator=g)).to(dev, torch.bfloat16) for n in (c, c, cI)]
    sink = torch.randn(nh, generator=g).to(dev)
    H = torch.randn(B, T, d, generator=g).to(dev, torch.bfloat16)
    with torch.no_grad():
        comb = torch.nn.functional.linear(H, W6)
        Ca, Cb, Za, Zb, Ki, Zi = comb.split([c, c, c, c, cI, cI], -1)
        cQ = torch.nn.functional.linear(H, W_DQ)
        q = torch.nn.functional.linear(cQ, W_UQ).view(B, T, nh, c)
        qi = torch.nn.functional.linear(cQ, W_IUQ).view(B, T, nIh, cI)
        wi = torch.nn.functional.linear(H, W_w)
    return (Ca, Cb, Za, Zb, Ki, Zi, q, qi, wi), par, sink


def test_csa_config2_late_queries(dev):
    import kch
    from kch import ops_csa
    B, T, m, topk, win, cI = 4, 8192, 4, 512, 128, 64
    proj, par, sink = _c2_projections(dev, B, T, seed=21)
    out, idx = kch.csa_core(*proj, *par, m=m, topk=topk, sliding_window=win, sink_logits=sink,
                            normalize_qk=True, return_indices=True)
    # the kernel's own logits: the same compression and indexer launches, with
    # the logits written out
    nb = T // m
    k_split = torch.empty(B, nb, 2 * cI, device=dev, dtype=torch.float16)
    ops_csa._compress("t", proj[4], proj[5], par[2], m, out_raw=False, key=k_split,
                      normalize=True, key_split=2)
    _, lg_dev = ops_csa._indexer("t", proj[7], k_split, proj[8], topk, 1.0, m, dense=False,
                                 normalize_q=True, idx64=False, want_logits=True,
                                 sorted_=True, key_split=2)
    torch.cuda.synchronize()
    Q = np.concatenate([np.arange(4096, 4096 + 128), np.arange(6144, 6144 + 128),
                        np.arange(T - 128, T)])
    lg_k = lg_dev[:, Q].cpu().numpy()
    del lg_dev
    hp = [x.float().cpu().numpy() for x in proj]
    hpar = [x.float().cpu().numpy() for x in par]
    hs = sink.cpu().numpy()
    hidx = idx.cpu().numpy()[:, Q].astype(np.int64)
    hout = out.float().cpu().numpy()[:, Q]
    rows = differ = near = 0
    worst = 0.0
    for b in range(B):
        pb = [x[b:b + 1] for x in hp]
        # the oracle's own selection, on fp64 logits
        _, ref_idx, lg = OC.csa_core_at(*pb, *hpar, m=m, topk=topk, queries=Q,
                                        sliding_window=win, sink_logits=hs, compute=np.float64)
        assert np.all(np.isfinite(lg).sum(-1) >= 1024)   # the top-512 binds at every such query
        eps = logit_eps(pb[8][:, Q], 4)
        worst = max(worst, check_logits(f"C2 logits b{b}", lg_k[b:b + 1], lg, eps))
        r, d, n = check_selection(f"C2 selection b{b}", hidx[b:b + 1], ref_idx, lg, eps,
                                  sorted_=True)
        rows, differ, near = rows + r, differ + d, near + n
        ref_out, _, _ = OC.csa_core_at(*pb, *hpar, m=m, topk=topk, queries=Q,
                                       sliding_window=win, sink_logits=hs,
                                       indices=hidx[b:b + 1])
        close(f"C2 csa_core out (late queries) b{b}", hout[b:b + 1], ref_out)
    print(f"C2 selection: {differ} of {rows} rows differ from the oracle "
          f"({differ / rows:.4f}); {near} rows have a k-th/(k+1)-th gap within 2 eps; "
          f"largest logit error {worst:.3f} eps", file=sys.stderr)


def test_csa_rows_beyond_register_select(dev):
    """Rows longer than the register selection's 2048 blocks (configs[4]'s
    prefill length, T=16384: 4096 blocks) take the radix select: the unsorted
    selection (indices written straight to global memory in ascending order,
    as csa_core's attention takes them) and the sorted one (the indexer
    boundary's order) hold the same sets, and both agree with the oracle at
    late queries within the logit bound."""
    import kch
    from kch import ops_csa
    B, T, m, topk, win, cI = 1, 16384, 4, 512, 128, 64
    proj, par, sink = _c2_projections(dev, B, T, seed=23)
    out, idx = kch.csa_core(*proj, *par, m=m, topk=topk, sliding_window=win, sink_logits=sink,
                            normalize_qk=True, return_indices=True)
    nb = T // m
    k_split = torch.empty(B, nb, 2 * cI, device=dev, dtype=torch.float16)
    ops_csa._compress("t", proj[4], proj[5], par[2], m, out_raw=False, key=k_split,
                      normalize=True, key_split=2)
    sel = {}
    for srt in (False, True):
        sel[srt], _ = ops_csa._indexer("t", proj[7], k_split, proj[8], topk, 1.0, m, dense=False,
                                       normalize_q=True, idx64=False, want_logits=False,
                                       sorted_=srt, key_split=2)
    torch.cuda.synchronize()
    # every row: the same set; unsorted rows in ascending index, padding -1 last
    a = sel[False].cpu().numpy().astype(np.int64)
    s = sel[True].cpu().numpy().astype(np.int64)
    assert np.array_equal(np.sort(a, -1), np.sort(s, -1))
    assert np.array_equal(np.sort(a, -1), np.sort(idx.cpu().numpy().astype(np.int64), -1))
    big = np.iinfo(np.int64).max
    d = np.diff(np.where(a >= 0, a, big), axis=-1)
    assert np.all((d > 0) | ((d == 0) & (a[..., 1:] < 0))), "unsorted rows not ascending"
    Q = np.concatenate([np.arange(8256, 8256 + 64), np.arange(T - 128, T)])
    hp = [x.float().cpu().numpy() for x in proj]
    hpar = [x.float().cpu().numpy() for x in par]
    _, ref_idx, lg = OC.csa_core_at(*hp, *hpar, m=m, topk=topk, queries=Q, sliding_window=win,
                                    sink_logits=sink.cpu().numpy(), compute=np.float64)
    assert np.all(np.isfinite(lg).sum(-1) > 2048)   # the rows the radix select takes
    eps = logit_eps(hp[8][:, Q], 4)
    r, d, n = check_selection("long rows (unsorted)", a[:, Q], ref_idx, lg, eps, sorted_=False)
    r2, d2, _ = check_selection("long rows (sorted)", s[:, Q], ref_idx, lg, eps, sorted_=True)
    print(f"long rows: {d} and {d2} of {r} rows differ from the oracle ({n} near-ties)",
          file=sys.stderr)
    ref_out, _, _ = OC.csa_core_at(*hp, *hpar, m=m, topk=topk, queries=Q, sliding_window=win,
                                   sink_logits=sink.cpu().numpy(), indices=a[:, Q])
    close("long rows csa_core out", out.float().cpu().numpy()[:, Q], ref_out)


def test_hca_config3_full_length(dev):
    import kch
    B, T, d, c, nh, dc, m2, win = 1, 32768, 2048, 128, 16, 128, 128, 128
    g = torch.Generator().manual_seed(41)

    def w(o, i):
        return (torch.randn(o, i, generator=g) * i ** -0.5).to(dev, torch.bfloat16)
    W3 = torch.cat([w(c, d), w(c, d), w(dc, d)], 0)   # W_KV, W_Z, W_DQ
    W_UQ = w(c * nh, dc)
    bpos = 0.02 * torch.randn(m2, c, generator=g)
    sink = torch.randn(nh, generator=g)
    H = torch.randn(B, T, d, generator=g).to(dev, torch.bfloat16)
    with torch.no_grad():
        C, Z, cQ = torch.nn.functional.linear(H, W3).split([c, c, dc], -1)
        q = torch.nn.functional.linear(cQ, W_UQ).view(B, T, nh, c)
        out = kch.hca_core(C, Z, q, bpos.to(dev), m2=m2, sliding_window=win,
                           sink_logits=sink.to(dev))
    torch.cuda.synchronize()
    Q = np.concatenate([np.arange(64), np.arange(16384 - 64, 16384 + 64), np.arange(T - 256, T)])
    qh = np.zeros((B, T, nh, c), np.float32)
    qh[:, Q] = q[:, torch.from_numpy(Q).to(dev)].float().cpu().numpy()
    ref = OC.hca_core_at(C.float().cpu().numpy(), Z.float().cpu().numpy(), qh, bpos.numpy(),
                         m2=m2, queries=Q, sliding_window=win, sink_logits=sink.numpy(),
                         compute=np.float64)
    close("C3 hca_core out (T=32768)", out.float().cpu().numpy()[:, Q], ref)


def c4_cfg():
    import kch
    return kch.HybridConfig(d_model=2048, n_heads_qk=16, n_heads_v=16, head_dim_k=128,
                            head_dim_v=128, kda_chunk_size=64, csa_m=4, csa_topk=512, csa_nh=16,
                            csa_c=128, csa_dc=128, csa_nIh=4, csa_cI=64, csa_sliding_window=128,
                            hca_m2=128, hca_nh=16, hca_c=128, hca_dc=128, hca_sliding_window=128)


def test_hybrid_decoding_config4_shapes(dev):
    import kch
    cfg = c4_cfg()
    torch.manual_seed(31)
    dec = kch.HybridDecoding(cfg=cfg, total_layers=5)
    with torch.no_grad():
        for layer in dec.model.layers:
            if hasattr(layer, 'sink'):
                layer.sink.normal_()
        for n in dec.model.norms:
            n.weight.normal_(1.0, 0.1)
            n.bias.normal_(0.0, 0.1)
    dec = dec.to(dev, torch.bfloat16).eval()
    sd = {k: v.float().cpu().numpy() for k, v in dec.model.state_dict().items()}
    cfgd = {k: getattr(cfg, k) for k in cfg.__dataclass_fields__}
    # the decode steps take tokens 2301..2308: token 2303 completes HCA block 17
    # (m'=128) and CSA block 575, token 2307 CSA block 576
    T0, steps = 18 * 128 - 3, 8
    assert (T0 + 3) % cfg.hca_m2 == 0 and (T0 + 3) % cfg.csa_m == 0
    x = torch.randn(2, T0 + steps, cfg.d_model,
                    generator=torch.Generator().manual_seed(32)).to(dev, torch.bfloat16)
    oracle = OH.HybridDecodingOracle(sd, cfgd, dec.model.layout, "bf16")
    # every decode step on the device-driven kernels
    assert decode_vs_oracle(dec, oracle, x, T0, "C4 HybridDecoding") == steps
