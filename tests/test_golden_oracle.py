"""The oracle against the reference's own outputs (golden vectors, CPU only).

``tests/golden/*.npz`` hold inputs and outputs of the reference implementation
(written in the build container by ``tests/golden/make_golden.py``). They pin
what the oracle's mathematical checks leave open: where the reference rounds
to bfloat16 (the KDA layer's activation chain, ``ops_fused.py:571-581``; the
projections of ``naive_csa`` / ``naive_hca``; the decode caches' stored rows,
``ops_decoding_cache.py:727-763``), and how the composition threads state.

Bars:

* bf16 outputs: every element within rtol 1e-2 + atol 1e-4 of the reference,
  and at least 98% of them bit-identical (the rest are one-ulp flips where the
  reference's fp32 summation order and numpy's differ before a rounding);
* fp32 states: relative Frobenius error below 1e-5;
* the hybrid stack: each sub-layer on the reference's own residual stream to
  the bf16 bar above; the whole stack (where the one-ulp flips of early layers
  pass through later roundings) to a relative Frobenius error below 5e-3;
* selections: ``torch.topk`` orders exactly equal logits by its internal
  selection order (neither ascending nor descending index: ``indexer_ties.npz``
  shows both), so sets are compared wherever the k-th and (k+1)-th logits
  differ, and the rest of each computation is checked with the reference's
  own selection forced (recorded in the fixtures).

``test_planted_mistakes_fail`` plants plausible mistakes in the oracle
(a dropped bf16 rounding, a dropped term) and checks that these bars catch
each of them.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import caches as OCa
from oracle import csa as OC
from oracle import hybrid as OH
from oracle import kda as OK
from oracle.common import bf16_round

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

SMALL_CFG = dict(d_model=64, n_heads_qk=2, n_heads_v=2, head_dim_k=64, head_dim_v=64,
                 kda_chunk_size=64, csa_m=4, csa_topk=6, csa_nh=2, csa_c=64, csa_dc=32,
                 csa_nIh=4, csa_cI=32, csa_sliding_window=8, hca_m2=16, hca_nh=2, hca_c=64,
                 hca_dc=32, hca_sliding_window=8, kda_decay_scale=0.1, n_kda=3, n_csa=1,
                 n_hca=1)


def load(name):
    return np.load(os.path.join(G, name))


def u2f(b):
    """bf16 bit patterns -> float32 values."""
    return (np.asarray(b).astype(np.uint32) << 16).view(np.float32)


def check_bf16(name, got, ref, min_exact=0.98, rtol=1e-2, atol=1e-4):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    exact = float(np.mean(got == ref))
    assert not bad.any(), f"{name}: {bad.sum()} of {bad.size} beyond tolerance (max {err.max():.3e})"
    assert exact >= min_exact, f"{name}: only {exact:.4f} of the elements bit-identical"
    return exact


def check_f32(name, got, ref, rel=1e-5):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    r = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert r <= rel, f"{name}: relative Frobenius error {r:.2e} > {rel}"


def selection_mismatches(idx, idx_ref, logits, tol=1e-6):
    """(rows whose selected sets differ although the k-th and (k+1)-th logits do
    not tie, rows with such a boundary tie). Also checks that the two
    selections hold the same logit values (any order)."""
    idx = np.asarray(idx, np.int64).reshape(-1, np.shape(idx)[-1])
    idx_ref = np.asarray(idx_ref, np.int64).reshape(idx.shape)
    lg = np.asarray(logits, np.float64).reshape(idx.shape[0], -1)
    bad = tied = 0
    for r in range(idx.shape[0]):
        a, b = idx[r], idx_ref[r]
        assert np.count_nonzero(a >= 0) == np.count_nonzero(b >= 0), f"row {r}: slot counts"
        va = np.sort(lg[r, a[a >= 0]])
        vb = np.sort(lg[r, b[b >= 0]])
        assert va.shape == vb.shape and np.allclose(va, vb, rtol=tol, atol=tol), \
            f"row {r}: selected logits differ"
        row = -np.sort(-lg[r][np.isfinite(lg[r])])
        k = int(np.count_nonzero(b >= 0))
        tie = k < row.size and abs(row[k - 1] - row[k]) <= tol * max(1.0, abs(row[k - 1]))
        tied += int(tie)
        if set(a[a >= 0]) != set(b[b >= 0]) and not tie:
            bad += 1
    return bad, tied


# ----------------------------------------------------------------------------- KDA

def test_kda_ops_golden():
    z = load("kda_ops_bf16.npz")
    q, k, v, g, beta = (u2f(z[n + "_bf16"]) for n in ("q", "k", "v", "g", "beta"))
    o, s = OK.chunk_kda(q, k, v, g, beta, initial_state=z["s0"], chunk_size=64)
    check_bf16("naive_chunk_kda o", bf16_round(o), u2f(z["o_chunk_bf16"]), min_exact=0.999)
    check_f32("naive_chunk_kda state", s, z["s_chunk"])
    o, s = OK.recurrent_kda(q, k, v, g, beta, initial_state=z["s0"])
    check_bf16("naive_recurrent_kda o", bf16_round(o), u2f(z["o_rec_bf16"]), min_exact=0.999)
    check_f32("naive_recurrent_kda state", s, z["s_rec"])


def _kda_layer_run(z):
    W = {k[2:]: z[k] for k in z.files if k.startswith("w.")}
    x = u2f(z["x_bf16"])
    y1, s1, lb1 = OH.kda_layer(x[:, :70], W, SMALL_CFG, None, None, "bf16")
    y2, s2, lb2 = OH.kda_layer(x[:, 70:], W, SMALL_CFG, z["s1"], u2f(z["lb1_bf16"]), "bf16")
    return y1, s1, lb1, y2, s2, lb2


def check_kda_layer(z):
    y1, s1, lb1, y2, s2, lb2 = _kda_layer_run(z)
    check_bf16("kda layer y (chunk call)", y1, u2f(z["y1_bf16"]))
    check_f32("kda layer state (chunk call)", s1, z["s1"])
    np.testing.assert_array_equal(lb1, u2f(z["lb1_bf16"]))
    check_bf16("kda layer y (recurrent call)", y2, u2f(z["y2_bf16"]))
    check_f32("kda layer state (recurrent call)", s2, z["s2"])
    np.testing.assert_array_equal(lb2, u2f(z["lb2_bf16"]))


def test_kda_layer_golden():
    check_kda_layer(load("kda_layer_bf16.npz"))


# ----------------------------------------------------------------------------- CSA / HCA

def _csa_hca_inputs(z):
    B, T, d, c, nh, dc, nIh, cI, m, m2, win, topk = (int(v) for v in z["meta"])
    Wc = {k[4:-5]: u2f(z[k]) for k in z.files if k.startswith("csa.")}
    Wh = {k[4:-5]: u2f(z[k]) for k in z.files if k.startswith("hca.")}
    return (u2f(z["H_bf16"]), u2f(z["sink_bf16"]), Wc, Wh,
            dict(B=B, T=T, c=c, nh=nh, nIh=nIh, cI=cI, m=m, m2=m2, win=win, topk=topk))


def test_naive_csa_hca_golden():
    z = load("csa_hca_bf16.npz")
    H, sink, Wc, Wh, p = _csa_hca_inputs(z)
    kw = dict(m=p["m"], topk=p["topk"], nh=p["nh"], nIh=p["nIh"], c=p["c"], c_I=p["cI"],
              sliding_window=p["win"], sink=sink, dtype="bf16")
    out, proj = OC.naive_csa(H, Wc, indices=z["csa_idx"], **kw)
    check_bf16("naive_csa (reference selection)", out, u2f(z["csa_out_bf16"]), min_exact=0.99)
    for i, n in enumerate(("Ca", "Cb", "Za", "Zb", "K_idx", "Z_idx")):
        check_bf16(f"naive_csa projection {n}", proj[i], u2f(z[f"proj.{n}_bf16"]), min_exact=0.99)
    # the oracle's own selection against the reference's
    Ca, Cb, Za, Zb, Ki, Zi, q, qi, wi = proj
    T = p["T"]
    Tp = T + (-T) % p["m"]
    pad = lambda a: np.pad(a, [(0, 0), (0, Tp - T)] + [(0, 0)] * (a.ndim - 2))  # noqa: E731
    kcomp = OC.compress_kv(pad(Ki), pad(Zi), Wc["B_idx"], p["m"])
    cbm = OC.causal_block_mask(Tp, Tp // p["m"], p["m"])
    lg = OC.indexer_logits(pad(qi), kcomp, pad(wi), None, cbm, True)
    mine = OC.lightning_indexer(pad(qi), kcomp, pad(wi), p["topk"], None, cbm, True)
    bad, tied = selection_mismatches(mine, z["csa_idx"], lg)
    assert bad == 0, f"{bad} selections differ away from ties ({tied} rows tie at the boundary)"
    out, _ = OC.naive_hca(H, Wh, m2=p["m2"], nh=p["nh"], c=p["c"], sliding_window=p["win"],
                          sink=sink, dtype="bf16")
    check_bf16("naive_hca", out, u2f(z["hca_out_bf16"]), min_exact=0.99)


def test_decode_caches_golden():
    z = load("caches_bf16.npz")
    B, c, cI, m, m2, win, nh, nIh, topk, n_pre, n_steps = (int(v) for v in z["meta"])
    g = lambda n: u2f(z[n + "_bf16"])  # noqa: E731
    Ca, Cb, Za, Zb, Ki, Zi = (g(n) for n in ("Ca", "Cb", "Za", "Zb", "Ki", "Zi"))
    C, Z = g("C"), g("Z")
    csa = OCa.CSACacheOracle(B, c, cI, m, win, "bf16")
    hca = OCa.HCACacheOracle(B, c, m2, win, "bf16")
    csa.append_step(Ca[:, :n_pre], Cb[:, :n_pre], Za[:, :n_pre], Zb[:, :n_pre], Ki[:, :n_pre],
                    Zi[:, :n_pre], g("Ba"), g("Bb"), g("Bi"))
    hca.append_step(C[:, :n_pre], Z[:, :n_pre], g("Bp"))
    oc, oh, bad, tied = [], [], 0, 0
    for s in range(n_steps):
        sl = slice(n_pre + s, n_pre + s + 1)
        csa.append_step(Ca[:, sl], Cb[:, sl], Za[:, sl], Zb[:, sl], Ki[:, sl], Zi[:, sl],
                        g("Ba"), g("Bb"), g("Bi"))
        ref_idx = z["csa_step_idx"][:, s:s + 1]
        qs, qis, wis = z["q"][:, s:s + 1], z["qi"][:, s:s + 1], z["wi"][:, s:s + 1]
        oc.append(csa.forward_step(qs, qis, wis, topk=topk, scale=1.0, sink_logits=z["sink"],
                                   normalize_qk=True, indices=ref_idx))
        lg = OC.indexer_logits(qis, csa.K_IComp, wis, None, None, True)
        mine = OC.lightning_indexer(qis, csa.K_IComp, wis, topk, None, None, True)
        b_, t_ = selection_mismatches(mine, ref_idx, lg)
        bad, tied = bad + b_, tied + t_
        hca.append_step(C[:, sl], Z[:, sl], g("Bp"))
        oh.append(hca.forward_step(qs, scale=1.0, sink_logits=z["sink"]))
    assert bad == 0, f"{bad} decode selections differ away from ties ({tied} tied)"
    check_f32("CSADecodingCache.forward_step", np.concatenate(oc, 1), z["o_csa"])
    check_f32("HCADecodingCache.forward_step", np.concatenate(oh, 1), z["o_hca"])
    check_bf16("CSA cache C_comp", csa.C_comp, g("csa_C_comp"), min_exact=0.99)
    check_bf16("CSA cache K_IComp", csa.K_IComp, g("csa_K_IComp"), min_exact=0.99)
    np.testing.assert_array_equal(np.stack(csa.ring, 1), g("csa_ring"))
    check_bf16("HCA cache C_comp", hca.C_comp, g("hca_C_comp"), min_exact=0.99)
    np.testing.assert_array_equal(np.stack(hca.ring, 1), g("hca_ring"))


# ----------------------------------------------------------------------------- composition

def test_hybrid_golden():
    z = load("hybrid_bf16.npz")
    sd = {k[2:]: z[k] for k in z.files if k.startswith("w.")}
    layout = [("kda", "csa", "hca")[i] for i in z["layout"]]
    assert layout == OH.build_layout(SMALL_CFG, 5)
    pos = layout.index("csa")
    x = u2f(z["x_bf16"])
    # each sub-layer on the reference's own residual stream: the strict bar
    xs = [u2f(z[f"layer_in{i}_bf16"]) for i in range(len(layout))]
    np.testing.assert_array_equal(xs[0], x)
    outs, _, _ = OH.hybrid_forward(x, sd, SMALL_CFG, layout, dtype="bf16",
                                   csa_indices={pos: z["csa_idx"]}, layer_inputs=xs)
    for i, kind in enumerate(layout):
        check_bf16(f"HybridKCHAttention layer {i} ({kind})", outs[i],
                   (xs + [u2f(z["y_bf16"])])[i + 1])
    # the whole stack: the same composition, with one-ulp differences of the
    # first layers carried through later bf16 roundings (relative error ~1e-3)
    y, st, lb = OH.hybrid_forward(x, sd, SMALL_CFG, layout, dtype="bf16",
                                  csa_indices={pos: z["csa_idx"]})
    check_f32("HybridKCHAttention y", y, u2f(z["y_bf16"]), rel=5e-3)
    for i in range(3):
        check_f32(f"HybridKCHAttention state {i}", st[i], z[f"state{i}"], rel=5e-3)
        check_f32(f"HybridKCHAttention lookback {i}", lb[i], u2f(z[f"lookback{i}_bf16"]), rel=5e-3)
    orc = OH.HybridDecodingOracle(sd, SMALL_CFG, layout, "bf16")
    T0 = 67
    ys = [orc.step(x[:, :T0], csa_indices={pos: z["dec_prefill_idx"]})]
    for s, t in enumerate(range(T0, x.shape[1])):
        ys.append(orc.step(x[:, t:t + 1], csa_indices={pos: z["dec_step_idx"][:, s:s + 1]}))
    check_f32("HybridDecoding prefill + decode", np.concatenate(ys, 1), u2f(z["dec_y_bf16"]),
              rel=5e-3)


def test_indexer_tie_order_golden():
    """torch.topk among exactly equal logits: neither ascending nor descending
    index (unpinnable). Away from ties the sets agree, and the selected logit
    values agree everywhere."""
    z = load("indexer_ties.npz")
    B, T, nIh, cI, m, topk = (int(v) for v in z["meta"])
    cbm = OC.causal_block_mask(T, T // m, m)
    for w, key in ((z["w"], "idx"), (None, "idx_noweights")):
        lg = OC.indexer_logits(z["q"], z["k"], w, None, cbm, True)
        mine = OC.lightning_indexer(z["q"], z["k"], w, topk, None, cbm, True)
        bad, tied = selection_mismatches(mine, z[key], lg)
        assert bad == 0
        assert tied > 0  # the fixture does exercise boundary ties
    ref = z["idx"].reshape(-1, topk)
    lg = OC.indexer_logits(z["q"], z["k"], z["w"], None, cbm, True).reshape(ref.shape[0], -1)
    asc = desc = 0
    for r in range(ref.shape[0]):
        sel = ref[r][ref[r] >= 0]
        v = lg[r, sel]
        for j in range(len(sel) - 1):
            if v[j] == v[j + 1]:
                asc += int(sel[j] < sel[j + 1])
                desc += int(sel[j] > sel[j + 1])
    assert asc > 0 and desc > 0


# ----------------------------------------------------------------------------- pins catch mistakes

def test_planted_mistakes_fail(monkeypatch):
    """Each plausible mistake in the oracle's bf16 chain fails the golden bars."""
    z = load("kda_layer_bf16.npz")
    check_kda_layer(z)  # the unmodified oracle passes

    def once(x, dtype):  # F.normalize with the norm and quotient kept in fp32
        from oracle.common import round_to
        x = np.asarray(x, np.float64)
        return round_to(x / np.maximum(np.sqrt((x * x).sum(-1, keepdims=True)), 1e-12), dtype)
    silu_plain = OH._silu
    softplus_plain = OH._softplus
    mistakes = {
        "normalise rounded once": lambda: monkeypatch.setattr(OH, "_normalize_lowp", once),
        "decay scale dropped": lambda: monkeypatch.setitem(SMALL_CFG, "kda_decay_scale", 1.0),
        "silu of -x": lambda: monkeypatch.setattr(OH, "_silu", lambda x: silu_plain(-x)),
        "softplus sign": lambda: monkeypatch.setattr(OH, "_softplus",
                                                     lambda x: softplus_plain(-x)),
    }
    for name, plant in mistakes.items():
        plant()
        with pytest.raises(AssertionError):
            check_kda_layer(z)
        monkeypatch.undo()
    check_kda_layer(z)
