"""Gradients of the HIP CSA operators (needs a ROCm GPU).

The reference differentiates ``naive_csa`` with autograd, its top-k selection
held fixed, and adds a straight-through surrogate for the indexer
(``ops_csa.py:1033-1099``; tests ``run_correctness.py:1312-1473``,
``2710-2830``). Checked here:

* ``kch_csa_attn_bwd`` (attention, overlapped compression, window, sink,
  with and without ``normalize_qk``) against ``oracle.csa.csa_attn_grad``
  (pinned by central finite differences on the CPU), including the per-slot
  quantity the surrogate consumes: fp32 within 1e-4 of each tensor's largest
  gradient;
* the whole ``csa_core`` with ``use_ste=True`` against a float64 torch
  statement of the reference's forward with the surrogate identity
  ``kv + (soft_kv - soft_kv.detach())``, differentiated by autograd on the
  CPU on the selection the kernel made: every gradient, indexer inputs
  included, within 1e-4 of its largest entry;
* the reference's contract: ``use_ste`` does not change the forward value, and
  every indexer weight of ``naive_csa`` gets a finite, non-zero gradient;
* ``naive_csa`` in fp32 with ``use_ste=True`` against the reference's own
  gradients (``tests/golden/csa_ste_fp32.npz``, both ``ste_mode`` values,
  with and without ``normalize_qk``): the selection the reference made, and
  every gradient (H, each weight, the sink) within 1e-4 of its largest entry;
* ``full_softmax`` against ``oracle.csa.csa_ste_grad`` (itself pinned by that
  fixture) at a shape with padded channels, and the reference's distinctness
  contract (``run_correctness.py:1588-1731``): the same forward as
  ``topk_columns``, a different and larger indexer gradient.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import ste_fixture as SF
from oracle.csa import csa_attn_grad as o_grad
from oracle.csa import csa_ste_grad as o_ste_grad

pytestmark = pytest.mark.gpu


def _check(name, got, ref, tol_max=1e-4):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite"
    scale = np.abs(ref).max() + 1e-30
    err = np.abs(got - ref).max()
    assert err <= tol_max * scale, f"{name}: max err {err:.3e} of max {scale:.3e}"


def _selection(rng, B, T, m, topk, hole=None):
    idx = np.full((B, T, topk), -1, np.int32)
    for b in range(B):
        for t in range(T):
            vis = (t + 1) // m
            if vis and t != hole:
                pick = rng.choice(vis, size=min(vis, topk), replace=False)
                idx[b, t, :len(pick)] = pick
    return idx


CASES = [
    # B, T, nh, c, m, topk, win, sink, norm
    (2, 64, 4, 64, 4, 8, 8, True, True),
    (1, 128, 16, 128, 8, 4, 0, False, False),
    (1, 48, 2, 16, 4, 3, 5, True, False),      # c padded to 64
    (1, 64, 18, 128, 4, 6, 4, True, True),     # two head groups
    (2, 1040, 3, 64, 8, 16, 24, True, False),  # several query chunks per key tile
]


@pytest.mark.parametrize("B,T,nh,c,m,topk,win,sink,norm", CASES)
def test_attn_grad_matches_oracle(dev, B, T, nh, c, m, topk, win, sink, norm):
    import kch
    rng = np.random.default_rng(T + nh + c + topk)
    X = {k: rng.standard_normal((B, T, c)) for k in ("Ca", "Cb", "Za", "Zb")}
    q = rng.standard_normal((B, T, nh, c))
    Ba, Bb = rng.standard_normal((m, c)) * 0.3, rng.standard_normal((m, c)) * 0.3
    sk = rng.standard_normal(nh) if sink else None
    W = rng.standard_normal((B, T, nh, c))
    idx = _selection(rng, B, T, m, topk, hole=T // 2)
    ref = o_grad(X["Ca"], X["Cb"], X["Za"], X["Zb"], q, Ba, Bb, idx, W, m=m, sliding_window=win,
                 sink_logits=sk, normalize_qk=norm)
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=dev)  # noqa: E731
    g = kch.ops_csa.csa_attn_grad(t(X["Ca"]), t(X["Cb"]), t(X["Za"]), t(X["Zb"]), t(q), t(Ba),
                                  t(Bb), torch.tensor(idx, device=dev), t(W), m=m,
                                  sliding_window=win, sink_logits=None if sk is None else t(sk),
                                  normalize_qk=norm)
    torch.cuda.synchronize()
    for name in ("Ca", "Cb", "Za", "Zb", "q", "Ba", "Bb", "slot") + (("sink_logits",) if sink else ()):
        _check(name, g[name].cpu().numpy(), ref[name])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,nh,c,m,topk,win,sink,norm", [CASES[0], CASES[2], CASES[3]])
def test_attn_grad_half_storage_is_exact(dev, dtype, B, T, nh, c, m, topk, win, sink, norm):
    """bf16 / fp16 q and d_out move in their own dtype where the queries are
    normalised (read and written by the MFMA kernels; fp32 copies otherwise):
    the same bits as the fp32-storage path on the same values, dq rounded to
    nearest even."""
    import kch
    rng = np.random.default_rng(T + nh + c + topk + 7)
    X = {k: rng.standard_normal((B, T, c)) for k in ("Ca", "Cb", "Za", "Zb")}
    q = rng.standard_normal((B, T, nh, c))
    Ba, Bb = rng.standard_normal((m, c)) * 0.3, rng.standard_normal((m, c)) * 0.3
    sk = rng.standard_normal(nh) if sink else None
    W = rng.standard_normal((B, T, nh, c))
    idx = torch.tensor(_selection(rng, B, T, m, topk, hole=T // 2), device=dev)
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=dev)  # noqa: E731
    qh, Wh = t(q).to(dtype), t(W).to(dtype)
    args = [t(X[k]) for k in ("Ca", "Cb", "Za", "Zb")]
    kw = dict(m=m, sliding_window=win, sink_logits=None if sk is None else t(sk),
              normalize_qk=norm, want_gsum=True)
    got = kch.ops_csa.csa_attn_grad(*args, qh, t(Ba), t(Bb), idx, Wh, **kw)
    ref = kch.ops_csa.csa_attn_grad(*args, qh.float(), t(Ba), t(Bb), idx, Wh.float(), **kw)
    torch.cuda.synchronize()
    assert got["q"].dtype == dtype
    assert torch.equal(got["q"], ref["q"].to(dtype)), "dq"
    for name in ref:
        if name != "q":
            assert torch.equal(got[name], ref[name]), name


def _torch_reference(X, idx, *, m, topk, win, sink, norm):
    """The reference's CSA forward (compression ``ops_csa.py:237-305``,
    indexer ``:330-573``, the STE gather ``:1033-1099``, attention with window
    and sink ``:1100-1155``) in float64 torch on the CPU, the selection given."""
    Ca, Cb, Za, Zb, Kx, Zx, q, qi, wi, Ba, Bb, Bi = (X[k] for k in (
        "Ca", "Cb", "Za", "Zb", "K_idx", "Z_idx", "q", "q_idx", "w_idx", "Ba", "Bb", "B_idx"))
    B_, T, c = Ca.shape
    nb = T // m
    nh = q.shape[2]

    def blocks(x):
        return x.reshape(B_, nb, m, x.shape[-1])

    zb_prev = torch.cat([torch.full_like(blocks(Zb)[:, :1], float('-inf')), blocks(Zb)[:, :-1]], 1)
    cb_prev = torch.cat([torch.zeros_like(blocks(Cb)[:, :1]), blocks(Cb)[:, :-1]], 1)
    wts = torch.softmax(torch.cat([blocks(Za) + Ba, zb_prev + Bb], dim=2), dim=2)
    Ccomp = (wts * torch.cat([blocks(Ca), cb_prev], dim=2)).sum(2)
    Kcomp = (torch.softmax(blocks(Zx) + Bi, dim=2) * blocks(Kx)).sum(2)
    cI = Kx.shape[-1]
    qn, Cn = (F.normalize(q, dim=-1), F.normalize(Ccomp, dim=-1)) if norm else (q, Ccomp)
    qin, Kn = (F.normalize(qi, dim=-1), F.normalize(Kcomp, dim=-1)) if norm else (qi, Kcomp)
    scale = 1.0 if norm else c ** -0.5
    iscale = 1.0 if norm else cI ** -0.5
    logits = torch.einsum('bhtn,bth->btn', torch.relu(torch.einsum('bthd,bnd->bhtn', qin, Kn) * iscale), wi)
    tt, nn = torch.arange(T), torch.arange(nb)
    logits = logits.masked_fill(~((tt[:, None] + 1) // m > nn[None, :]), float('-inf'))
    allm = logits.isinf().all(-1, keepdim=True)
    soft = torch.softmax(logits.masked_fill(allm, 0.0), -1).masked_fill(allm, 0.0)
    idx = torch.as_tensor(idx, dtype=torch.long)
    valid = idx >= 0
    isafe = idx.clamp(min=0)
    kv = Cn[torch.arange(B_)[:, None, None], isafe]                             # [B,T,k,c]
    ssel = torch.gather(soft, -1, isafe) * valid.to(soft.dtype)
    soft_kv = ssel.unsqueeze(-1) * kv.detach()
    kv = kv + (soft_kv - soft_kv.detach())
    s = torch.einsum('bthd,btkd->bthk', qn, kv) * scale
    s = s.masked_fill(~valid[:, :, None, :], float('-inf'))
    vals = [kv]
    scores = [s]
    if win:
        Cl = F.normalize(Ca, dim=-1) if norm else Ca
        pad = torch.cat([torch.zeros(B_, win - 1, c, dtype=Ca.dtype), Cl], 1)
        wi_ = torch.arange(T)[:, None] + torch.arange(win)[None, :]
        Cw = pad[:, wi_]                                                          # [B,T,w,c]
        wv = torch.arange(win)[None, :] >= (win - 1 - torch.arange(T)[:, None])
        sw = (torch.einsum('bthd,btwd->bthw', qn, Cw) * scale).masked_fill(~wv[None, :, None, :],
                                                                            float('-inf'))
        vals.append(Cw)
        scores.append(sw)
    cat = torch.cat(scores, -1)
    catv = ~torch.isinf(cat)
    rm = torch.clamp(cat.masked_fill(~catv, float('-inf')).amax(-1, keepdim=True), min=0.0)
    e = torch.exp(cat - rm).masked_fill(~catv, 0.0)
    den = e.sum(-1, keepdim=True)
    if sink is not None:
        den = den + torch.exp(sink.view(1, 1, nh, 1) - rm)
    p = torch.where(den > 0, e / den.clamp_min(1e-300), torch.zeros_like(e))
    out = torch.einsum('bthk,btkd->bthd', p[..., :topk], vals[0])
    if win:
        out = out + torch.einsum('bthw,btwd->bthd', p[..., topk:], vals[1])
    return out


@pytest.mark.parametrize("norm", [False, True])
def test_csa_core_ste_grads_match_torch_reference(dev, norm):
    import kch
    rng = np.random.default_rng(21 + norm)
    B, T, nh, c, m, topk, win, cI, nIh = 1, 64, 2, 64, 4, 4, 6, 32, 2
    shapes = dict(Ca=(B, T, c), Cb=(B, T, c), Za=(B, T, c), Zb=(B, T, c), K_idx=(B, T, cI),
                  Z_idx=(B, T, cI), q=(B, T, nh, c), q_idx=(B, T, nIh, cI), w_idx=(B, T, nIh),
                  Ba=(m, c), Bb=(m, c), B_idx=(m, cI))
    X = {k: rng.standard_normal(s) * (0.3 if k.startswith("B") else 1.0) for k, s in shapes.items()}
    sk = rng.standard_normal(nh)
    W = rng.standard_normal((B, T, nh, c))
    xt = {k: torch.tensor(v, dtype=torch.float32, device=dev, requires_grad=True) for k, v in X.items()}
    st = torch.tensor(sk, dtype=torch.float32, device=dev, requires_grad=True)
    args = [xt[k] for k in ("Ca", "Cb", "Za", "Zb", "K_idx", "Z_idx", "q", "q_idx", "w_idx", "Ba",
                            "Bb", "B_idx")]
    out, idx = kch.csa_core(*args, m=m, topk=topk, sliding_window=win, sink_logits=st,
                            normalize_qk=norm, return_indices=True, use_ste=True)
    (out.double() * torch.tensor(W, device=dev)).sum().backward()
    torch.cuda.synchronize()
    # the same loss through the float64 torch statement, on the kernel's selection
    xr = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in X.items()}
    sr = torch.tensor(sk, dtype=torch.float64, requires_grad=True)
    ref_out = _torch_reference(xr, idx.cpu().numpy(), m=m, topk=topk, win=win, sink=sr, norm=norm)
    # the forward holds its compressed rows in bf16 (2^-9 relative); without
    # normalisation the scores reach |q||k| / sqrt(c) ~ 8, so the outputs move
    # by a few 1e-3 of their largest value
    _check("out", out.detach().cpu().numpy(), ref_out.detach().numpy(), 1e-2)
    (ref_out * torch.tensor(W)).sum().backward()
    for k in X:
        _check(k, xt[k].grad.cpu().numpy(), xr[k].grad.numpy())
    _check("sink", st.grad.cpu().numpy(), sr.grad.numpy())


def test_naive_csa_ste_contract(dev):
    """``run_correctness.py:1312-1473``: ``use_ste`` leaves the forward value
    unchanged, and every indexer weight gets a finite, non-zero gradient."""
    import kch
    torch.manual_seed(42)
    B, T, d = 1, 32, 16
    m, topk, nh, nIh, c, cI, dc = 4, 2, 2, 2, 8, 4, 8
    H = torch.randn(B, T, d, device=dev)
    P = dict(W_aKV=(c, d), W_bKV=(c, d), W_aZ=(c, d), W_bZ=(c, d), Ba=(m, c), Bb=(m, c),
             W_DQ=(dc, d), W_UQ=(c * nh, dc), W_IUQ=(cI * nIh, dc), W_w=(nIh, d),
             W_KV_idx=(cI, d), W_Z_idx=(cI, d), B_idx=(m, cI))
    base = {k: torch.randn(*s) * (0.02 if k.startswith("B") else 0.1) for k, s in P.items()}
    outs = []
    for ste in (False, True):
        ps = {k: v.clone().to(dev).requires_grad_(True) for k, v in base.items()}
        o = kch.naive_csa(H, *[ps[k] for k in P], m=m, topk=topk, nh=nh, nIh=nIh, c=c, c_I=cI,
                          dc=dc, use_ste=ste)
        o.square().sum().backward()
        outs.append((o.detach(), ps))
    assert torch.allclose(outs[0][0], outs[1][0], rtol=0, atol=1e-6)
    for k in ("W_IUQ", "W_w", "W_KV_idx", "W_Z_idx", "B_idx"):
        g = outs[1][1][k].grad
        assert g is not None and torch.isfinite(g).all() and g.abs().sum() > 0, k
        g0 = outs[0][1][k].grad
        assert g0 is None or g0.abs().sum() == 0, k
    for k in ("W_aKV", "W_bKV", "W_aZ", "W_bZ", "W_DQ", "W_UQ", "Ba", "Bb"):
        g = outs[1][1][k].grad
        assert g is not None and torch.isfinite(g).all() and g.abs().sum() > 0, k


@pytest.mark.parametrize("topk,win", [(6, 0), (0, 5)])
def test_attn_grad_sparse_edges(dev, topk, win):
    """A selection wider than the visible blocks (mostly -1 slots), and no
    selection at all (window only)."""
    import kch
    rng = np.random.default_rng(31 + topk)
    B, T, nh, c, m = 1, 16, 2, 64, 4
    X = {k: rng.standard_normal((B, T, c)) for k in ("Ca", "Cb", "Za", "Zb")}
    q = rng.standard_normal((B, T, nh, c))
    Ba, Bb = rng.standard_normal((m, c)) * 0.3, rng.standard_normal((m, c)) * 0.3
    sk = rng.standard_normal(nh)
    W = rng.standard_normal((B, T, nh, c))
    idx = _selection(rng, B, T, m, topk) if topk else np.zeros((B, T, 0), np.int32)
    ref = o_grad(X["Ca"], X["Cb"], X["Za"], X["Zb"], q, Ba, Bb, idx, W, m=m, sliding_window=win,
                 sink_logits=sk, normalize_qk=True)
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=dev)  # noqa: E731
    g = kch.ops_csa.csa_attn_grad(t(X["Ca"]), t(X["Cb"]), t(X["Za"]), t(X["Zb"]), t(q), t(Ba),
                                  t(Bb), torch.tensor(idx, device=dev) if topk else None, t(W),
                                  m=m, sliding_window=win, sink_logits=t(sk), normalize_qk=True)
    torch.cuda.synchronize()
    for name in ("Ca", "Cb", "Za", "Zb", "q", "Ba", "Bb", "sink_logits"):
        _check(name, g[name].cpu().numpy(), ref[name])


@pytest.mark.parametrize("nIh,cI,norm", [(4, 64, True), (4, 64, False), (2, 32, True),
                                         (1, 128, False), (8, 64, True), (3, 48, False)])
def test_ste_kernel_matches_dense_statement(dev, nIh, cI, norm):
    """``kch_csa_ste_bwd`` against the dense torch statement of the same
    surrogate (softmax over every causal block, autograd through the logits
    and the key compression), on a selection with -1 slots; fp32, 1e-4 of each
    tensor's largest gradient. Covers padded heads (3 -> 4) and channels
    (32 -> 64, 48 -> 64)."""
    from kch.ops_csa import _ste_indexer_grads, _ste_indexer_grads_dense
    rng = np.random.default_rng(nIh * cI + norm)
    B, T, m, topk = 2, 256, 4, 16
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=dev)  # noqa: E731
    K = t(rng.standard_normal((B, T, cI)))
    Z = t(rng.standard_normal((B, T, cI)))
    q = t(rng.standard_normal((B, T, nIh, cI)))
    w = t(rng.standard_normal((B, T, nIh)))
    Bi = t(rng.standard_normal((m, cI)) * 0.3)
    idx = torch.tensor(_selection(rng, B, T, m, topk, hole=100), device=dev)
    slot = t(rng.standard_normal((B, T, topk))) * (idx >= 0)
    got = _ste_indexer_grads(K, Z, q, w, Bi, idx, slot, m=m, normalize_qk=norm)
    ref = _ste_indexer_grads_dense(K, Z, q, w, Bi, idx, slot, m=m, normalize_qk=norm)
    torch.cuda.synchronize()
    for name, a, r in zip(("K_idx", "Z_idx", "q_idx", "w_idx", "B_idx"), got, ref):
        _check(name, a.cpu().numpy(), r.cpu().numpy())


@pytest.mark.parametrize("norm,mode", SF.CASES)
def test_naive_csa_ste_grads_match_reference_fixture(dev, norm, mode):
    import kch
    z, meta, W = SF.load()
    t = SF.tag(norm, mode)
    Wt = {k: torch.tensor(v, device=dev, requires_grad=True) for k, v in W.items()}
    H = torch.tensor(z["H"], device=dev, requires_grad=True)
    sk = torch.tensor(z["sink"], device=dev, requires_grad=True)
    with kch.record_selections() as sel:
        out = kch.naive_csa(H, *[Wt[n] for n in SF.NAMES], m=meta["m"], topk=meta["topk"],
                            nh=meta["nh"], nIh=meta["nIh"], c=meta["c"], c_I=meta["cI"],
                            dc=meta["dc"], sliding_window=meta["win"], sink_logits=sk,
                            use_ste=True, ste_mode=mode, normalize_qk=norm)
    (out * torch.tensor(z["G"], device=dev)).sum().backward()
    torch.cuda.synchronize()
    got_idx = sel[0].cpu().numpy().astype(np.int64)
    ref_idx = z[f"{t}.idx"]
    assert got_idx.shape == ref_idx.shape
    for r, (a, b) in enumerate(zip(got_idx.reshape(-1, got_idx.shape[-1]),
                                   ref_idx.reshape(-1, ref_idx.shape[-1]))):
        assert set(a.tolist()) == set(b.tolist()), f"row {r}: {a} vs the reference's {b}"
    _check("out", out.detach().cpu().numpy(), z[f"{t}.out"], 1e-2)
    got = {f"d{n}": Wt[n].grad.cpu().numpy() for n in SF.NAMES}
    got["dH"] = H.grad.cpu().numpy()
    got["dsink"] = sk.grad.cpu().numpy()
    err = SF.worst_rel(got, z, t)
    bad = {k: v for k, v in err.items() if v > 1e-4}
    assert not bad, bad


@pytest.mark.parametrize("norm", [True, False])
def test_csa_core_full_softmax_matches_oracle(dev, norm):
    import kch
    rng = np.random.default_rng(61 + norm)
    B, T, nh, c, m, topk, win, cI, nIh = 2, 64, 3, 40, 4, 5, 6, 24, 3
    shapes = dict(Ca=(B, T, c), Cb=(B, T, c), Za=(B, T, c), Zb=(B, T, c), K_idx=(B, T, cI),
                  Z_idx=(B, T, cI), q=(B, T, nh, c), q_idx=(B, T, nIh, cI), w_idx=(B, T, nIh),
                  Ba=(m, c), Bb=(m, c), B_idx=(m, cI))
    X = {k: rng.standard_normal(s) * (0.3 if k.startswith("B") else 1.0) for k, s in shapes.items()}
    sk = rng.standard_normal(nh)
    Gw = rng.standard_normal((B, T, nh, c))
    names = ("Ca", "Cb", "Za", "Zb", "K_idx", "Z_idx", "q", "q_idx", "w_idx", "Ba", "Bb", "B_idx")
    grads, outs = {}, {}
    for mode in ("topk_columns", "full_softmax"):
        xt = {k: torch.tensor(v, dtype=torch.float32, device=dev, requires_grad=True)
              for k, v in X.items()}
        st = torch.tensor(sk, dtype=torch.float32, device=dev, requires_grad=True)
        out, idx = kch.csa_core(*[xt[k] for k in names], m=m, topk=topk, sliding_window=win,
                                sink_logits=st, normalize_qk=norm, return_indices=True,
                                use_ste=True, ste_mode=mode)
        (out.double() * torch.tensor(Gw, device=dev)).sum().backward()
        torch.cuda.synchronize()
        grads[mode] = {k: xt[k].grad.cpu().numpy() for k in X}
        grads[mode]["sink_logits"] = st.grad.cpu().numpy()
        outs[mode] = out.detach().cpu().numpy()
        if mode == "full_softmax":
            ref = o_ste_grad(*[X[k] for k in names], idx.cpu().numpy(), Gw, m=m,
                             sliding_window=win, sink_logits=sk, normalize_qk=norm,
                             ste_mode=mode)
            for k in list(X) + ["sink_logits"]:
                _check(k, grads[mode][k], ref[k])
    # run_correctness.py:1588-1731: same forward, distinct and larger indexer gradient
    np.testing.assert_array_equal(outs["topk_columns"], outs["full_softmax"])
    for k in ("K_idx", "q_idx", "w_idx"):
        a, b = grads["topk_columns"][k], grads["full_softmax"][k]
        assert np.abs(a - b).max() > 1e-6 * np.abs(b).max(), k
    assert np.abs(grads["full_softmax"]["K_idx"]).sum() > np.abs(grads["topk_columns"]["K_idx"]).sum()


def test_naive_csa_aux_contrastive_raises(dev):
    import kch
    B, T, d, c, nh, dc, nIh, cI, m = 1, 8, 16, 8, 2, 8, 2, 4, 4
    H = torch.randn(B, T, d, device=dev)
    P = dict(W_aKV=(c, d), W_bKV=(c, d), W_aZ=(c, d), W_bZ=(c, d), Ba=(m, c), Bb=(m, c),
             W_DQ=(dc, d), W_UQ=(c * nh, dc), W_IUQ=(cI * nIh, dc), W_w=(nIh, d),
             W_KV_idx=(cI, d), W_Z_idx=(cI, d), B_idx=(m, cI))
    ps = [torch.randn(*s, device=dev) for s in P.values()]
    with pytest.raises(NotImplementedError):
        kch.naive_csa(H, *ps, m=m, topk=2, nh=nh, nIh=nIh, c=c, c_I=cI, dc=dc,
                      ste_mode='aux_contrastive')
