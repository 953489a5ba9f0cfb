"""Write the golden vectors under ``tests/golden/`` from the reference implementation.

Run in the build container only (``/root/reference`` does not exist on the GPU
box, and nothing that runs there imports this script):

    python tests/golden/make_golden.py

Each fixture records inputs and the reference's outputs for a function whose
result the oracle's other pins (closed forms, invariants, brute force) leave
open: the points where the reference rounds to bfloat16, and ``torch.topk``'s
choice among exactly equal logits.

* ``kda_layer_bf16.npz``  ``KDAHybridLayer.forward_functional`` in bf16
  (``ops_fused.py:391-609``): two calls threading state and conv lookback, the
  first on the chunk path, the second on the recurrent path;
* ``kda_ops_bf16.npz``    ``naive_chunk_kda`` / ``naive_recurrent_kda`` on bf16
  inputs with an fp32 initial state (``ops_kda.py:175-267,464-494``);
* ``csa_hca_bf16.npz``    ``naive_csa`` and ``naive_hca`` in bf16
  (``ops_csa.py:576-1184``, ``ops_hca.py:30-201``) with sink and window;
* ``caches_bf16.npz``     ``CSADecodingCache`` / ``HCADecodingCache`` in bf16
  (``ops_decoding_cache.py:407-1395``): a 37-token bulk append, then ten
  append + forward steps, and the final block stores and ring;
* ``hybrid_bf16.npz``     ``HybridKCHAttention.forward_functional`` in bf16
  (``ops_fused.py:956-1128``) and ``HybridDecoding`` (``run_decoding.py:601-851``,
  with the model swapped for one of this geometry): prefill, then decode steps;
* ``indexer_ties.npz``    ``csa_lightning_indexer`` (``ops_csa.py:330-573``) on
  keys with duplicated rows (exactly equal logits) and ReLU-zero logits;
* ``csa_ste_fp32.npz``    the gradients of ``naive_csa`` in fp32 with the
  straight-through surrogate (``ops_csa.py:1033-1099``), ``ste_mode``
  ``topk_columns`` and ``full_softmax``, of the loss ``sum(out * G)``: every
  weight's, the sink's and H's, with and without ``normalize_qk``.

``python tests/golden/make_golden.py NAME ...`` writes only the named fixtures
(``kda_ops kda_layer csa_hca caches hybrid indexer_ties csa_ste``).

Inputs come from ``numpy.random.default_rng`` with fixed seeds; bf16 tensors
are stored as their 16-bit patterns (``*_bf16`` keys), fp32 tensors as float32.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"


def _import_reference():
    if not os.path.isdir(REF):
        raise SystemExit(f"{REF} is not present: fixtures are generated in the build container")
    if REF not in sys.path:
        sys.path.insert(0, REF)
    import torch  # noqa: F401
    import ops_csa
    import ops_decoding_cache
    import ops_fused
    import ops_hca
    import ops_kda
    import run_decoding
    # every selection the reference makes is recorded (naive_csa calls the
    # indexer through ops_csa's module global, the decode cache through its own)
    real = ops_csa.csa_lightning_indexer

    def recording_indexer(*args, **kwargs):
        res = real(*args, **kwargs)
        SELECTIONS.append((res[0] if isinstance(res, tuple) else res).numpy().astype(np.int64))
        return res
    ops_csa.csa_lightning_indexer = recording_indexer
    ops_decoding_cache.csa_lightning_indexer = recording_indexer
    return ops_kda, ops_csa, ops_hca, ops_decoding_cache, ops_fused, run_decoding


SELECTIONS = []  # int64 index arrays returned by the reference's csa_lightning_indexer


def bits(t):
    """bf16 tensor -> uint16 bit patterns."""
    import torch
    return t.detach().contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def f32(t):
    return t.detach().float().numpy().astype(np.float32)


def to_bf16(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)


def small_cfg_kwargs():
    """Geometry shared by the layer fixtures (every size inside the HIP kernels' coverage)."""
    return dict(d_model=64, n_heads_qk=2, n_heads_v=2, head_dim_k=64, head_dim_v=64,
                kda_chunk_size=64, kda_backend="reference", csa_m=4, csa_topk=6, csa_nh=2,
                csa_c=64, csa_dc=32, csa_nIh=4, csa_cI=32, csa_sliding_window=8, hca_m2=16,
                hca_nh=2, hca_c=64, hca_dc=32, hca_sliding_window=8)


def random_state_dict(module, rng, conv_scale=3.0):
    """N(0, fan_in^-1/2) weights, N(0, 0.02) position biases, N(0, 1) sinks, and
    LayerNorm affine parameters near (1, 0): every parameter bf16-representable."""
    sd = {}
    for name, p in module.state_dict().items():
        shape = tuple(p.shape)
        if name.endswith("sink"):
            a = rng.standard_normal(shape)
        elif name.split(".")[-1] in ("Ba", "Bb", "B_idx", "B_pos"):
            a = 0.02 * rng.standard_normal(shape)
        elif "norms." in name and name.endswith("weight"):
            a = 1.0 + 0.1 * rng.standard_normal(shape)
        elif "norms." in name and name.endswith("bias"):
            a = 0.1 * rng.standard_normal(shape)
        elif "short_conv.weight" in name:
            a = conv_scale * rng.standard_normal(shape) / np.sqrt(3.0)
        elif "short_conv.bias" in name:
            a = 0.1 * rng.standard_normal(shape)
        else:
            a = rng.standard_normal(shape) / np.sqrt(shape[-1])
        sd[name] = np.asarray(to_bf16(a).float().numpy(), np.float32)
    return sd


def load_sd(module, sd):
    import torch
    module.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)


def sd_arrays(prefix, sd):
    return {f"{prefix}{k}": v for k, v in sd.items()}


def make_kda_layer(ref):
    import torch
    _, _, _, _, ops_fused, _ = ref
    rng = np.random.default_rng(101)
    cfg = ops_fused.HybridConfig(**small_cfg_kwargs())
    layer = ops_fused.KDAHybridLayer(cfg)
    sd = random_state_dict(layer, rng)
    load_sd(layer, sd)
    layer = layer.to(torch.bfloat16).eval()
    B, d = 2, cfg.d_model
    x = to_bf16(rng.standard_normal((B, 73, d)))
    out = {"x_bf16": bits(x)}
    with torch.no_grad():
        y1, s1, lb1 = layer.forward_functional(x[:, :70], None, None)
        y2, s2, lb2 = layer.forward_functional(x[:, 70:], s1, lb1)
    out.update(y1_bf16=bits(y1), s1=f32(s1), lb1_bf16=bits(lb1), y2_bf16=bits(y2), s2=f32(s2),
               lb2_bf16=bits(lb2))
    out.update(sd_arrays("w.", sd))
    np.savez_compressed(os.path.join(HERE, "kda_layer_bf16.npz"), **out)


def make_kda_ops(ref):
    import torch
    ops_kda = ref[0]
    rng = np.random.default_rng(102)
    B, T, H, K, V = 1, 100, 2, 64, 64

    def nrm(a):
        return a / np.linalg.norm(a, axis=-1, keepdims=True)
    q = to_bf16(nrm(rng.standard_normal((B, T, H, K))))
    k = to_bf16(nrm(rng.standard_normal((B, T, H, K))))
    v = to_bf16(rng.standard_normal((B, T, H, V)))
    g = to_bf16(-np.logaddexp(0.0, -rng.standard_normal((B, T, H, K))))
    beta = to_bf16(1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H)))))
    s0 = torch.from_numpy((0.02 * rng.standard_normal((B, H, K, V))).astype(np.float32))
    with torch.no_grad():
        oc, sc = ops_kda.naive_chunk_kda(q, k, v, g, beta, initial_state=s0,
                                         output_final_state=True, chunk_size=64)
        orr, sr = ops_kda.naive_recurrent_kda(q, k, v, g, beta, initial_state=s0,
                                              output_final_state=True)
    np.savez_compressed(os.path.join(HERE, "kda_ops_bf16.npz"), q_bf16=bits(q), k_bf16=bits(k),
                        v_bf16=bits(v), g_bf16=bits(g), beta_bf16=bits(beta), s0=f32(s0),
                        o_chunk_bf16=bits(oc), s_chunk=f32(sc), o_rec_bf16=bits(orr),
                        s_rec=f32(sr))


def make_csa_hca(ref):
    import torch
    _, ops_csa, ops_hca, _, _, _ = ref
    rng = np.random.default_rng(103)
    B, T, d, c, nh, dc, nIh, cI, m, m2, win, topk = 2, 50, 64, 64, 2, 32, 4, 32, 4, 16, 8, 6

    def w(o, i):
        return to_bf16(rng.standard_normal((o, i)) / np.sqrt(i))
    H = to_bf16(rng.standard_normal((B, T, d)))
    Wc = {n: w(c, d) for n in ("W_aKV", "W_bKV", "W_aZ", "W_bZ")}
    Wc["Ba"] = to_bf16(0.02 * rng.standard_normal((m, c)))
    Wc["Bb"] = to_bf16(0.02 * rng.standard_normal((m, c)))
    Wc["W_DQ"] = w(dc, d)
    Wc["W_UQ"] = w(c * nh, dc)
    Wc["W_IUQ"] = w(cI * nIh, dc)
    Wc["W_w"] = w(nIh, d)
    Wc["W_KV_idx"] = w(cI, d)
    Wc["W_Z_idx"] = w(cI, d)
    Wc["B_idx"] = to_bf16(0.02 * rng.standard_normal((m, cI)))
    sink = to_bf16(rng.standard_normal(nh))
    names = ("W_aKV", "W_bKV", "W_aZ", "W_bZ", "Ba", "Bb", "W_DQ", "W_UQ", "W_IUQ", "W_w",
             "W_KV_idx", "W_Z_idx", "B_idx")
    SELECTIONS.clear()
    with torch.no_grad():
        oc, proj = ops_csa.naive_csa(H, *[Wc[n] for n in names], m=m, topk=topk, nh=nh, nIh=nIh,
                                     c=c, c_I=cI, dc=dc, sliding_window=win, sink_logits=sink,
                                     use_ste=False, normalize_qk=True, return_projections=True)
    Wh = {"W_KV": w(c, d), "W_Z": w(c, d), "W_DQ": w(dc, d), "W_UQ": w(c * nh, dc),
          "B_pos": to_bf16(0.02 * rng.standard_normal((m2, c)))}
    with torch.no_grad():
        oh = ops_hca.naive_hca(H, Wh["W_KV"], Wh["W_Z"], Wh["B_pos"], Wh["W_DQ"], Wh["W_UQ"],
                               m2=m2, nh=nh, c=c, dc=dc, sliding_window=win, sink_logits=sink)
    assert len(SELECTIONS) == 1
    out = {"H_bf16": bits(H), "sink_bf16": bits(sink), "csa_out_bf16": bits(oc),
           "hca_out_bf16": bits(oh), "csa_idx": SELECTIONS[0]}
    for nme, p in zip(("Ca", "Cb", "Za", "Zb", "K_idx", "Z_idx"), proj):
        out[f"proj.{nme}_bf16"] = bits(p)
    out.update({f"csa.{k}_bf16": bits(v) for k, v in Wc.items()})
    out.update({f"hca.{k}_bf16": bits(v) for k, v in Wh.items()})
    out["meta"] = np.array([B, T, d, c, nh, dc, nIh, cI, m, m2, win, topk], np.int64)
    np.savez_compressed(os.path.join(HERE, "csa_hca_bf16.npz"), **out)


def make_caches(ref):
    import torch
    _, _, _, odc, _, _ = ref
    rng = np.random.default_rng(104)
    B, c, cI, m, m2, win, nh, nIh, topk = 2, 64, 32, 4, 16, 8, 2, 4, 5
    n_pre, n_steps = 37, 10
    n_tot = n_pre + n_steps
    dt = torch.bfloat16

    def r(*s, scale=1.0):
        return to_bf16(scale * rng.standard_normal(s))
    Ca, Cb, Za, Zb = (r(B, n_tot, c) for _ in range(4))
    Ki, Zi = r(B, n_tot, cI), r(B, n_tot, cI)
    Ba, Bb, Bi = r(m, c, scale=0.02), r(m, c, scale=0.02), r(m, cI, scale=0.02)
    C, Z = r(B, n_tot, c), r(B, n_tot, c)
    Bp = r(m2, c, scale=0.02)
    q = F_normalize(torch.from_numpy(rng.standard_normal((B, n_steps, nh, c)).astype(np.float32)))
    qi = torch.from_numpy(rng.standard_normal((B, n_steps, nIh, cI)).astype(np.float32))
    wi = torch.from_numpy(rng.standard_normal((B, n_steps, nIh)).astype(np.float32))
    sink = torch.from_numpy(rng.standard_normal(nh).astype(np.float32))
    csa = odc.CSADecodingCache(B, c, cI, m, win, "cpu", dt)
    hca = odc.HCADecodingCache(B, c, m2, win, "cpu", dt)
    o_csa, o_hca = [], []
    SELECTIONS.clear()
    with torch.no_grad():
        csa.append_step(Ca[:, :n_pre], Cb[:, :n_pre], Za[:, :n_pre], Zb[:, :n_pre],
                        Ki[:, :n_pre], Zi[:, :n_pre], Ba, Bb, Bi)
        hca.append_step(C[:, :n_pre], Z[:, :n_pre], Bp)
        for s in range(n_steps):
            t = n_pre + s
            sl = slice(t, t + 1)
            csa.append_step(Ca[:, sl], Cb[:, sl], Za[:, sl], Zb[:, sl], Ki[:, sl], Zi[:, sl],
                            Ba, Bb, Bi)
            o_csa.append(csa.forward_step(q[:, s:s + 1], qi[:, s:s + 1], wi[:, s:s + 1],
                                          topk=topk, nh=nh, nIh=nIh, scale=1.0,
                                          sink_logits=sink, use_ste=False, normalize_qk=True))
            hca.append_step(C[:, sl], Z[:, sl], Bp)
            o_hca.append(hca.forward_step(q[:, s:s + 1], nh=nh, scale=1.0, sink_logits=sink))
    out = dict(Ca_bf16=bits(Ca), Cb_bf16=bits(Cb), Za_bf16=bits(Za), Zb_bf16=bits(Zb),
               Ki_bf16=bits(Ki), Zi_bf16=bits(Zi), Ba_bf16=bits(Ba), Bb_bf16=bits(Bb),
               Bi_bf16=bits(Bi), C_bf16=bits(C), Z_bf16=bits(Z), Bp_bf16=bits(Bp), q=f32(q),
               qi=f32(qi), wi=f32(wi), sink=f32(sink),
               o_csa=f32(torch.cat(o_csa, 1)), o_hca=f32(torch.cat(o_hca, 1)),
               csa_step_idx=np.concatenate(SELECTIONS, 1),
               csa_C_comp_bf16=bits(csa.C_comp), csa_K_IComp_bf16=bits(csa.K_IComp),
               csa_ring_bf16=bits(csa.sw_buffer.get()), hca_C_comp_bf16=bits(hca.C_comp),
               hca_ring_bf16=bits(hca.sw_buffer.get()),
               meta=np.array([B, c, cI, m, m2, win, nh, nIh, topk, n_pre, n_steps], np.int64))
    np.savez_compressed(os.path.join(HERE, "caches_bf16.npz"), **out)


def F_normalize(t):
    import torch.nn.functional as F
    return F.normalize(t, dim=-1)


def make_hybrid(ref):
    import torch
    _, _, _, _, ops_fused, run_decoding = ref
    rng = np.random.default_rng(105)
    cfg = ops_fused.HybridConfig(**small_cfg_kwargs())
    model = ops_fused.HybridKCHAttention(cfg, total_layers=5)
    sd = random_state_dict(model, rng)
    load_sd(model, sd)
    model = model.to(torch.bfloat16).eval()
    B, T = 2, 70
    x = to_bf16(rng.standard_normal((B, T, cfg.d_model)))
    layer_in = {}  # the residual stream entering each sub-layer (its LayerNorm's input)
    hooks = [n.register_forward_hook(lambda mod, inp, out, i=i: layer_in.__setitem__(i, inp[0]))
             for i, n in enumerate(model.norms)]
    SELECTIONS.clear()
    with torch.no_grad():
        y, states, lbs = model.forward_functional(x, None, [None] * model.n_kda_layers)
    for h in hooks:
        h.remove()
    assert len(SELECTIONS) == 1
    out = {"x_bf16": bits(x), "y_bf16": bits(y), "csa_idx": SELECTIONS[0]}
    for i, xi in layer_in.items():
        out[f"layer_in{i}_bf16"] = bits(xi)
    for i, st in enumerate(states.unbind(0) if torch.is_tensor(states) else states):
        out[f"state{i}"] = f32(st)
    for i, lb in enumerate(lbs):
        out[f"lookback{i}_bf16"] = bits(lb)
    # HybridDecoding of the same weights: prefill 67 tokens, then one token at a time
    dec = run_decoding.HybridDecoding(d_model=cfg.d_model, total_layers=5)
    dec.cfg = cfg
    model2 = ops_fused.HybridKCHAttention(cfg, total_layers=5)
    load_sd(model2, sd)
    dec.model = model2.to(torch.bfloat16).eval()
    dec._csa_caches = [None for layer in dec.model.layers
                       if isinstance(layer, ops_fused.CSAHybridLayer)]
    dec._hca_caches = [None for layer in dec.model.layers
                       if isinstance(layer, ops_fused.HCAHybridLayer)]
    dec.reset()
    ys = []
    SELECTIONS.clear()
    with torch.no_grad():
        ys.append(dec(x[:, :67]))
        for t in range(67, T):
            ys.append(dec(x[:, t:t + 1]))
    out["dec_y_bf16"] = bits(torch.cat(ys, 1))
    # the prefill's selection, then one [B, 1, topk] selection per decode step
    out["dec_prefill_idx"] = SELECTIONS[0]
    out["dec_step_idx"] = np.concatenate(SELECTIONS[1:], 1)
    out["layout"] = np.array([{"kda": 0, "csa": 1, "hca": 2}[k] for k in model.layout], np.int64)
    out.update(sd_arrays("w.", sd))
    np.savez_compressed(os.path.join(HERE, "hybrid_bf16.npz"), **out)


def make_indexer_ties(ref):
    import torch
    ops_csa = ref[1]
    rng = np.random.default_rng(106)
    B, T, nIh, cI, m, topk = 2, 96, 4, 32, 4, 8
    nb = T // m
    base = rng.standard_normal((5, cI)).astype(np.float32)
    k = base[rng.integers(0, 5, size=(B, nb))]          # duplicated rows: equal logits
    q = rng.standard_normal((B, T, nIh, cI)).astype(np.float32)
    w = rng.standard_normal((B, T, nIh)).astype(np.float32)
    t = np.arange(T)[:, None]
    b = np.arange(nb)[None, :]
    mask = torch.from_numpy((t + 1) // m > b)
    SELECTIONS.clear()
    with torch.no_grad():
        idx = ops_csa.csa_lightning_indexer(torch.from_numpy(q), torch.from_numpy(k),
                                            torch.from_numpy(w), topk, causal_block_mask=mask,
                                            normalize_qk=True)
        # ReLU zeros: queries whose heads all score <= 0 against most keys
        idx0 = ops_csa.csa_lightning_indexer(torch.from_numpy(q), torch.from_numpy(k), None,
                                             topk, causal_block_mask=mask, normalize_qk=True)
    np.savez_compressed(os.path.join(HERE, "indexer_ties.npz"), q=q, k=k, w=w,
                        idx=idx.numpy().astype(np.int64), idx_noweights=idx0.numpy().astype(np.int64),
                        meta=np.array([B, T, nIh, cI, m, topk], np.int64))


CSA_STE_NAMES = ("W_aKV", "W_bKV", "W_aZ", "W_bZ", "Ba", "Bb", "W_DQ", "W_UQ", "W_IUQ", "W_w",
                 "W_KV_idx", "W_Z_idx", "B_idx")


def _boundary_tie(H, P, m, topk, nIh, cI, norm):
    """Whether any query's k-th and (k+1)-th indexer logits (fp64, from the
    fp32 projections) are exactly equal: there ``torch.topk``'s choice among
    the tied blocks is unspecified, so such inputs are not used."""
    import torch
    f = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    Hd = f(H)
    K, Z = Hd @ f(P["W_KV_idx"]).T, Hd @ f(P["W_Z_idx"]).T
    B, T, _ = K.shape
    nb = T // m
    wts = torch.softmax(Z.view(B, nb, m, cI) + f(P["B_idx"]), dim=2)
    kc = (wts * K.view(B, nb, m, cI)).sum(2)
    qi = ((Hd @ f(P["W_DQ"]).T) @ f(P["W_IUQ"]).T).view(B, T, nIh, cI)
    wi = Hd @ f(P["W_w"]).T
    if norm:
        kc, qi = torch.nn.functional.normalize(kc, dim=-1), torch.nn.functional.normalize(qi, dim=-1)
    sc = 1.0 if norm else cI ** -0.5
    lg = torch.einsum('bhtn,bth->btn', torch.relu(torch.einsum('bthd,bnd->bhtn', qi, kc) * sc), wi)
    for t in range(T):
        vis = (t + 1) // m
        if vis > topk:
            v = torch.sort(lg[:, t, :vis], dim=-1, descending=True).values
            if bool((v[:, topk - 1] == v[:, topk]).any()):
                return True
    return False


def make_csa_ste(ref):
    """fp32 ``naive_csa`` with ``use_ste=True`` under gradients: for each
    (``normalize_qk``, ``ste_mode``) the output, the selection the indexer made
    and the gradients of ``sum(out * G)``. Inputs whose selection would pass
    through an exact tie at the top-k boundary are skipped (the next seed)."""
    import torch
    _, ops_csa, _, _, _, _ = ref
    for seed in range(211, 400):
        H, P, sink, G = _csa_ste_inputs(seed)
        if not any(_boundary_tie(H, P, 4, 4, 4, 8, norm) for norm in (True, False)):
            break
    else:
        raise SystemExit("no tie-free inputs found")
    B, T, d, c, nh, dc, nIh, cI, m, win, topk = 1, 48, 32, 16, 2, 16, 4, 8, 4, 4, 4
    out = {"H": H, "sink": sink, "G": G, "seed": np.array(seed)}
    out.update({f"w.{k}": v for k, v in P.items()})
    for norm in (True, False):
        for mode in ("topk_columns", "full_softmax"):
            tag = f"{'norm' if norm else 'raw'}.{mode}"
            ts = {k: torch.from_numpy(v).requires_grad_(True) for k, v in P.items()}
            Ht = torch.from_numpy(H).requires_grad_(True)
            st = torch.from_numpy(sink).requires_grad_(True)
            SELECTIONS.clear()
            o = ops_csa.naive_csa(Ht, *[ts[n] for n in CSA_STE_NAMES], m=m, topk=topk, nh=nh,
                                  nIh=nIh, c=c, c_I=cI, dc=dc, sliding_window=win,
                                  sink_logits=st, use_ste=True, ste_mode=mode,
                                  normalize_qk=norm)
            (o * torch.from_numpy(G)).sum().backward()
            assert len(SELECTIONS) == 1
            out[f"{tag}.out"] = f32(o)
            out[f"{tag}.idx"] = SELECTIONS[0]
            out[f"{tag}.dH"] = f32(Ht.grad)
            out[f"{tag}.dsink"] = f32(st.grad)
            for n in CSA_STE_NAMES:
                out[f"{tag}.d{n}"] = f32(ts[n].grad)
    out["meta"] = np.array([B, T, d, c, nh, dc, nIh, cI, m, win, topk], np.int64)
    np.savez_compressed(os.path.join(HERE, "csa_ste_fp32.npz"), **out)


def _csa_ste_inputs(seed):
    rng = np.random.default_rng(seed)
    B, T, d, c, nh, dc, nIh, cI, m = 1, 48, 32, 16, 2, 16, 4, 8, 4
    P = {n: rng.standard_normal((c, d)) / np.sqrt(d) for n in ("W_aKV", "W_bKV", "W_aZ", "W_bZ")}
    P.update(Ba=0.3 * rng.standard_normal((m, c)), Bb=0.3 * rng.standard_normal((m, c)),
             W_DQ=rng.standard_normal((dc, d)) / np.sqrt(d),
             W_UQ=rng.standard_normal((c * nh, dc)) / np.sqrt(dc),
             W_IUQ=rng.standard_normal((cI * nIh, dc)) / np.sqrt(dc),
             W_w=rng.standard_normal((nIh, d)) / np.sqrt(d),
             W_KV_idx=rng.standard_normal((cI, d)) / np.sqrt(d),
             W_Z_idx=rng.standard_normal((cI, d)) / np.sqrt(d),
             B_idx=0.3 * rng.standard_normal((m, cI)))
    P = {k: v.astype(np.float32) for k, v in P.items()}
    H = rng.standard_normal((B, T, d)).astype(np.float32)
    sink = rng.standard_normal(nh).astype(np.float32)
    G = rng.standard_normal((B, T, nh * c)).astype(np.float32)
    return H, P, sink, G


def main():
    import torch
    torch.manual_seed(0)
    torch.set_num_threads(1)
    ref = _import_reference()
    makers = dict(kda_ops=make_kda_ops, kda_layer=make_kda_layer, csa_hca=make_csa_hca,
                  caches=make_caches, hybrid=make_hybrid, indexer_ties=make_indexer_ties,
                  csa_ste=make_csa_ste)
    for name in (sys.argv[1:] or list(makers)):
        makers[name](ref)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f"{f}: {os.path.getsize(os.path.join(HERE, f)) / 1024:.1f} KiB")


if __name__ == "__main__":
    main()
