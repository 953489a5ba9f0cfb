"""Shapes between and beyond the kernels' own sizes (needs a ROCm GPU).

The host layer zero-pads what the kernels do not take to their next size:
attention head dims to 64 / 128, indexer key dims to 32 / 64 / 128, indexer
heads to a power of two up to 16 (padded heads weigh 0), the chunk kernels' K
to 64 / 128 and V to a multiple of 64, the recurrent kernel's K to 16 .. 256;
a chunk call with K > 128 runs the recurrence, and more than 16 attention
heads run as groups of 16. Zero channels add nothing to a dot product, a norm
or a KDA state, so the results are those of the unpadded operator; each case
is held to the oracle at the bf16 bar (rtol 2e-2 + atol 2e-3, every element),
CSA on the selection the kernels made after that selection itself passed the
tie-aware index check (``selection_check``).

Shapes: the reference's decode geometry (``HybridDecoding()`` defaults,
``run_decoding.py:642-656``: c = 8, c_I = 4, one indexer head, 2 x 16 KDA
heads), and odd sizes (c = 96, c_I = 48, nIh = 3, nh = 20; KDA K = 32, 48,
192, V = 48).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from composed_check import close, decode_vs_oracle
from oracle import csa as O
from oracle import hybrid as OH
from oracle.common import bf16_round
from oracle.kda import chunk_kda
from selection_check import check_selection, logit_eps

pytestmark = pytest.mark.gpu


def bf16_dev(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev, torch.bfloat16)


def host(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("c,cI,nh,nIh", [(8, 4, 2, 1), (96, 48, 20, 3)])
def test_csa_core_odd_shapes(dev, c, cI, nh, nIh):
    import kch
    B, T, m, topk, win = 2, 96, 4, 6, 8
    rng = np.random.default_rng(c + cI + nh)
    r = lambda *s: rng.standard_normal(s)  # noqa: E731
    names = ("Ca", "Cb", "Za", "Zb", "K_idx", "Z_idx", "q", "q_idx", "w_idx")
    shapes = ((B, T, c),) * 4 + ((B, T, cI),) * 2 + ((B, T, nh, c), (B, T, nIh, cI), (B, T, nIh))
    dv = {k: bf16_dev(r(*s), dev) for k, s in zip(names, shapes)}
    hs = {k: host(v) for k, v in dv.items()}
    par = {k: (0.02 * r(m, w)).astype(np.float32) for k, w in (("Ba", c), ("Bb", c), ("B_idx", cI))}
    sink = r(nh).astype(np.float32)
    out, idx = kch.csa_core(*[dv[k] for k in names],
                            *[torch.from_numpy(par[k]).to(dev) for k in ("Ba", "Bb", "B_idx")],
                            m=m, topk=topk, sliding_window=win,
                            sink_logits=torch.from_numpy(sink).to(dev), normalize_qk=True,
                            return_indices=True)
    torch.cuda.synchronize()
    assert out.shape == (B, T, nh, c)
    K_ref = O.compress_kv(hs["K_idx"], hs["Z_idx"], par["B_idx"], m, compute=np.float64)
    idx_ref, lg = O.lightning_indexer(hs["q_idx"], K_ref, hs["w_idx"], topk, None,
                                      O.causal_block_mask(T, T // m, m), True,
                                      compute=np.float64, return_logits=True)
    rows, differ, _ = check_selection("odd csa idx", idx.cpu().numpy().astype(np.int64), idx_ref,
                                      lg, logit_eps(hs["w_idx"], nIh), sorted_=True)
    print(f"c={c} cI={cI} nh={nh} nIh={nIh}: {differ} of {rows} rows differ", file=sys.stderr)
    ref = O.csa_core(*[hs[k] for k in names], par["Ba"], par["Bb"], par["B_idx"], m=m,
                     topk=topk, sliding_window=win, sink_logits=sink, normalize_qk=True,
                     indices=idx.cpu().numpy())
    close(f"csa c={c} nh={nh}", host(out), bf16_round(ref))


@pytest.mark.parametrize("cI,nIh", [(4, 1), (20, 3)])
def test_indexer_odd_shapes(dev, cI, nIh):
    import kch
    B, T, m, topk = 2, 64, 2, 5
    rng = np.random.default_rng(cI * nIh)
    qi = bf16_dev(rng.standard_normal((B, T, nIh, cI)), dev)
    K = rng.standard_normal((B, T // m, cI)).astype(np.float32)
    wi = bf16_dev(rng.standard_normal((B, T, nIh)), dev)
    mask = O.causal_block_mask(T, T // m, m)
    idx = kch.csa_lightning_indexer(qi, torch.from_numpy(K).to(dev), wi, topk,
                                    causal_block_mask=torch.from_numpy(mask).to(dev),
                                    normalize_qk=True)
    torch.cuda.synchronize()
    idx_ref, lg = O.lightning_indexer(host(qi), K, host(wi), topk, None, mask, True,
                                      compute=np.float64, return_logits=True)
    check_selection("odd indexer", idx.cpu().numpy(), idx_ref, lg, logit_eps(host(wi), nIh),
                    sorted_=True)


@pytest.mark.parametrize("c,nh", [(8, 2), (96, 20)])
def test_hca_core_odd_shapes(dev, c, nh):
    import kch
    B, T, m2, win = 2, 96, 8, 16
    rng = np.random.default_rng(c * nh)
    Cd = bf16_dev(rng.standard_normal((B, T, c)), dev)
    Zd = bf16_dev(rng.standard_normal((B, T, c)), dev)
    qd = bf16_dev(rng.standard_normal((B, T, nh, c)), dev)
    bpos = (0.02 * rng.standard_normal((m2, c))).astype(np.float32)
    sink = rng.standard_normal(nh).astype(np.float32)
    out = kch.hca_core(Cd, Zd, qd, torch.from_numpy(bpos).to(dev), m2=m2, sliding_window=win,
                       sink_logits=torch.from_numpy(sink).to(dev))
    torch.cuda.synchronize()
    assert out.shape == (B, T, nh, c)
    ref = O.hca_core(host(Cd), host(Zd), host(qd), bpos, m2=m2, sliding_window=win,
                     sink_logits=sink)
    close(f"hca c={c} nh={nh}", host(out), bf16_round(ref))


@pytest.mark.parametrize("fn,K,V", [("chunk", 32, 48), ("chunk", 192, 64),
                                    ("recurrent", 48, 40)])
def test_kda_odd_head_dims(dev, fn, K, V):
    import kch
    B, T, H, HV = 2, 150, 2, 4
    g = torch.Generator().manual_seed(K + V)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    v = torch.randn(B, T, HV, V, generator=g)
    gt = torch.nn.functional.logsigmoid(torch.randn(B, T, HV, K, generator=g))
    beta = torch.sigmoid(torch.randn(B, T, HV, generator=g))
    s0 = 0.05 * torch.randn(B, HV, K, V, generator=g)
    xs = [x.to(torch.bfloat16) for x in (q, k, v, gt, beta)]
    op = kch.naive_chunk_kda if fn == "chunk" else kch.naive_recurrent_kda
    o, s = op(*[x.to(dev) for x in xs], initial_state=s0.to(dev), output_final_state=True)
    torch.cuda.synchronize()
    assert o.shape == (B, T, HV, V) and s.shape == (B, HV, K, V)
    o_ref, s_ref = chunk_kda(*[x.double().numpy() for x in xs], initial_state=s0.double().numpy(),
                             chunk_size=64, compute=np.float64)
    close(f"kda {fn} K={K} V={V} o", host(o), o_ref)
    close(f"kda {fn} K={K} V={V} state", host(s), s_ref)


def _randomize(model):
    with torch.no_grad():
        for layer in model.layers:
            if hasattr(layer, 'sink'):
                layer.sink.normal_()
            if hasattr(layer, 'short_conv'):
                layer.short_conv.weight.mul_(3.0)
        for n in model.norms:
            n.weight.normal_(1.0, 0.1)
            n.bias.normal_(0.0, 0.1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hybrid_decoding_reference_defaults(dev, dtype):
    """``HybridDecoding()`` as the reference's decode benchmark builds it: prefill
    then single-token steps, every sub-layer against the teacher-forced oracle."""
    import kch
    torch.manual_seed(41)
    dec = kch.HybridDecoding()
    _randomize(dec.model)
    dec = dec.to(dev, dtype).eval()
    cfg = dec.cfg
    sd = {k: v.float().cpu().numpy() for k, v in dec.model.state_dict().items()}
    oracle = OH.HybridDecodingOracle(sd, {k: getattr(cfg, k) for k in cfg.__dataclass_fields__},
                                     dec.model.layout, 'fp32' if dtype == torch.float32 else 'bf16')
    rng = np.random.default_rng(42)
    x = torch.from_numpy(rng.standard_normal((2, 30, cfg.d_model)).astype(np.float32)).to(
        dev, dtype)
    decode_vs_oracle(dec, oracle, x, 21, f"defaults {dtype}")


def test_hybrid_decoding_wide_odd_heads(dev):
    """Decode caches past the kernels' sizes: 20 CSA / HCA heads of 96, indexer
    keys of 48 with 3 heads (head groups, zero-padded step operands)."""
    import kch
    cfg = kch.HybridConfig(d_model=128, n_heads_qk=2, n_heads_v=2, head_dim_k=64, head_dim_v=64,
                           kda_chunk_size=64, csa_m=4, csa_topk=8, csa_nh=20, csa_c=96,
                           csa_dc=32, csa_nIh=3, csa_cI=48, csa_sliding_window=8, hca_m2=8,
                           hca_nh=20, hca_c=96, hca_dc=32, hca_sliding_window=8)
    torch.manual_seed(43)
    dec = kch.HybridDecoding(cfg=cfg, total_layers=5)
    _randomize(dec.model)
    dec = dec.to(dev, torch.bfloat16).eval()
    sd = {k: v.float().cpu().numpy() for k, v in dec.model.state_dict().items()}
    oracle = OH.HybridDecodingOracle(sd, {k: getattr(cfg, k) for k in cfg.__dataclass_fields__},
                                     dec.model.layout, 'bf16')
    rng = np.random.default_rng(44)
    x = torch.from_numpy(rng.standard_normal((2, 44, cfg.d_model)).astype(np.float32)).to(
        dev, torch.bfloat16)
    decode_vs_oracle(dec, oracle, x, 40, "wide odd heads")
