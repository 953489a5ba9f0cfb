"""Gradients of the HIP HCA operators (needs a ROCm GPU).

The reference differentiates ``hca_core`` / ``naive_hca`` with autograd
(``ops_hca.py:30-201``; the hybrid gradient test ``run_correctness.py:
2710-2830`` runs through them). ``kch``'s backward (``kch_hca_attn_bwd``, fp32)
is compared with ``oracle.csa.hca_core_grad``, which is pinned by central
finite differences on the CPU: fp32 inputs within 1e-4 of each tensor's
largest gradient; bf16 inputs within 3e-2 of it plus 3e-2 relative.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.csa import hca_core_grad as o_grad

pytestmark = pytest.mark.gpu


def _make(seed, B, T, nh, c, m2):
    rng = np.random.default_rng(seed)
    C = rng.standard_normal((B, T, c))
    Z = rng.standard_normal((B, T, c))
    q = rng.standard_normal((B, T, nh, c))
    Bp = rng.standard_normal((m2, c)) * 0.3
    sink = rng.standard_normal(nh)
    Cl = rng.standard_normal((B, T, c))
    W = rng.standard_normal((B, T, nh, c))
    return C, Z, q, Bp, sink, Cl, W


def _check(name, got, ref, tol_max, tol_rel=0.0):
    got = np.asarray(got, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite"
    scale = np.abs(ref).max() + 1e-30
    bad = np.abs(got - ref) > tol_max * scale + tol_rel * np.abs(ref)
    assert not bad.any(), (f"{name}: {bad.sum()} of {bad.size} outside; max err "
                           f"{np.abs(got - ref).max():.3e} of max {scale:.3e}")


CASES = [
    # B, T, nh, c, m2, win, sink, local
    (2, 64, 4, 64, 8, 8, True, False),
    (1, 96, 16, 128, 16, 16, False, False),
    (1, 40, 2, 16, 4, 5, True, True),       # c padded to 64; window rows from C_local_raw
    (1, 48, 18, 128, 8, 0, True, False),    # two head groups, no window
    (2, 1056, 3, 64, 32, 40, True, False),  # several query chunks per key tile
]


@pytest.mark.parametrize("B,T,nh,c,m2,win,sink,local", CASES)
def test_core_grad_matches_oracle(dev, B, T, nh, c, m2, win, sink, local):
    import kch
    C, Z, q, Bp, sk, Cl, W = _make(T + nh + c, B, T, nh, c, m2)
    kw = dict(m2=m2, sliding_window=win, scale=0.9)
    ref = o_grad(C, Z, q, Bp, W, sink_logits=sk if sink else None,
                 C_local_raw=Cl if local else None, **kw)
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=dev, requires_grad=True)  # noqa: E731
    Ct, Zt, qt, Bt = t(C), t(Z), t(q), t(Bp)
    st = t(sk) if sink else None
    Clt = t(Cl) if local else None
    out = kch.hca_core(Ct, Zt, qt, Bt, sink_logits=st, C_local_raw=Clt, **kw)
    (out.double() * torch.tensor(W, device=dev)).sum().backward()
    torch.cuda.synchronize()
    pairs = [("C", Ct), ("Z", Zt), ("q", qt), ("B_pos", Bt)]
    if sink:
        pairs.append(("sink_logits", st))
    if local:
        pairs.append(("C_local_raw", Clt))
    for name, x in pairs:
        _check(name, x.grad.cpu().numpy(), ref[name], 1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,nh,c,m2,win,sink,local", [CASES[0], CASES[2], CASES[3]])
def test_core_grad_half_storage_is_exact(dev, dtype, B, T, nh, c, m2, win, sink, local):
    """bf16 / fp16 q and d_out are read, and dq written, by the kernels in
    their own dtype: the same bits as the fp32-storage path (checked against
    the oracle above) run on the same values, dq rounded to nearest even."""
    from kch.ops_hca import hca_core_grad
    C, Z, q, Bp, sk, Cl, W = _make(T + nh + c + 7, B, T, nh, c, m2)
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=dev)  # noqa: E731
    qh, Wh = t(q).to(dtype), t(W).to(dtype)
    kw = dict(m2=m2, sliding_window=win, scale=0.9, sink_logits=t(sk) if sink else None,
              C_local_raw=t(Cl) if local else None)
    got = hca_core_grad(t(C), t(Z), qh, t(Bp), Wh, **kw)
    ref = hca_core_grad(t(C), t(Z), qh.float(), t(Bp), Wh.float(), **kw)
    torch.cuda.synchronize()
    assert got["q"].dtype == dtype
    assert torch.equal(got["q"], ref["q"].to(dtype)), "dq"
    for name in ref:
        if name != "q":
            assert torch.equal(got[name], ref[name]), name


def test_naive_hca_grad_fp32(dev):
    """Whole operator: projections through autograd, the core through its HIP
    backward; the oracle chain rule through the four linear maps."""
    import kch
    rng = np.random.default_rng(3)
    B, T, d, nh, c, dc, m2, win = 1, 70, 48, 4, 64, 32, 8, 8
    H = rng.standard_normal((B, T, d))
    Ws = {k: rng.standard_normal(s) / np.sqrt(s[1]) for k, s in
          dict(W_KV=(c, d), W_Z=(c, d), W_DQ=(dc, d), W_UQ=(c * nh, dc)).items()}
    Bp = rng.standard_normal((m2, c)) * 0.1
    sk = rng.standard_normal(nh)
    G = rng.standard_normal((B, T, nh * c))
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=dev, requires_grad=True)  # noqa: E731
    Ht, Bt, st = t(H), t(Bp), t(sk)
    Wt = {k: t(v) for k, v in Ws.items()}
    out = kch.naive_hca(Ht, Wt["W_KV"], Wt["W_Z"], Bt, Wt["W_DQ"], Wt["W_UQ"], m2=m2, nh=nh,
                        c=c, dc=dc, scale=0.7, sliding_window=win, sink_logits=st)
    (out.double() * torch.tensor(G, device=dev)).sum().backward()
    torch.cuda.synchronize()
    # oracle: pad T to a multiple of m2, project, core gradients, chain rule
    Tp = -(-T // m2) * m2
    Hp = np.concatenate([H, np.zeros((B, Tp - T, d))], axis=1)
    Gp = np.concatenate([G, np.zeros((B, Tp - T, nh * c))], axis=1).reshape(B, Tp, nh, c)
    Cx, Zx, cQ = Hp @ Ws["W_KV"].T, Hp @ Ws["W_Z"].T, Hp @ Ws["W_DQ"].T
    qx = (cQ @ Ws["W_UQ"].T).reshape(B, Tp, nh, c)
    g = o_grad(Cx, Zx, qx, Bp, Gp, m2=m2, sliding_window=win, sink_logits=sk, scale=0.7)
    dq = g["q"].reshape(B, Tp, nh * c)
    dcQ = dq @ Ws["W_UQ"]
    ref = {
        "W_KV": np.einsum("btc,btd->cd", g["C"], Hp), "W_Z": np.einsum("btc,btd->cd", g["Z"], Hp),
        "W_DQ": np.einsum("btc,btd->cd", dcQ, Hp), "W_UQ": np.einsum("btc,btd->cd", dq, cQ),
        "H": (g["C"] @ Ws["W_KV"] + g["Z"] @ Ws["W_Z"] + dcQ @ Ws["W_DQ"])[:, :T],
        "B_pos": g["B_pos"], "sink": g["sink_logits"],
    }
    got = {k: v.grad for k, v in Wt.items()}
    got.update(H=Ht.grad, B_pos=Bt.grad, sink=st.grad)
    for name, r in ref.items():
        _check(name, got[name].cpu().numpy(), r, 2e-4)


def test_naive_hca_grad_bf16(dev):
    """bf16 inputs: gradients in bf16 against fp64 gradients of the same
    bf16-valued weights and input."""
    import kch
    rng = np.random.default_rng(4)
    B, T, d, nh, c, dc, m2, win = 1, 64, 64, 2, 64, 32, 16, 16
    bf = lambda x: torch.tensor(x, dtype=torch.bfloat16)  # noqa: E731
    H = bf(rng.standard_normal((B, T, d)))
    Ws = {k: bf(rng.standard_normal(s) / np.sqrt(s[1])) for k, s in
          dict(W_KV=(c, d), W_Z=(c, d), W_DQ=(dc, d), W_UQ=(c * nh, dc)).items()}
    Bp = bf(rng.standard_normal((m2, c)) * 0.1)
    G = rng.standard_normal((B, T, nh * c))
    Wt = {k: v.to(dev).requires_grad_(True) for k, v in Ws.items()}
    Ht = H.to(dev).requires_grad_(True)
    out = kch.naive_hca(Ht, Wt["W_KV"], Wt["W_Z"], Bp.to(dev), Wt["W_DQ"], Wt["W_UQ"], m2=m2,
                        nh=nh, c=c, dc=dc, sliding_window=win)
    assert out.dtype == torch.bfloat16
    (out.double() * torch.tensor(G, device=dev)).sum().backward()
    torch.cuda.synchronize()
    Hn = H.double().numpy()
    Wn = {k: v.double().numpy() for k, v in Ws.items()}
    Cx, Zx, cQ = Hn @ Wn["W_KV"].T, Hn @ Wn["W_Z"].T, Hn @ Wn["W_DQ"].T
    qx = (cQ @ Wn["W_UQ"].T).reshape(B, T, nh, c)
    g = o_grad(Cx, Zx, qx, Bp.double().numpy(), G.reshape(B, T, nh, c), m2=m2,
               sliding_window=win)
    dq = g["q"].reshape(B, T, nh * c)
    ref_WKV = np.einsum("btc,btd->cd", g["C"], Hn)
    ref_H = g["C"] @ Wn["W_KV"] + g["Z"] @ Wn["W_Z"] + (dq @ Wn["W_UQ"]) @ Wn["W_DQ"]
    assert Wt["W_KV"].grad.dtype == torch.bfloat16
    _check("W_KV", Wt["W_KV"].grad.float().cpu().numpy(), ref_WKV, 3e-2, 3e-2)
    _check("H", Ht.grad.float().cpu().numpy(), ref_H, 3e-2, 3e-2)


def test_no_grad_forward_unchanged(dev):
    """With gradients enabled the forward value is the no-grad forward."""
    import kch
    C, Z, q, Bp, sk, _, _ = _make(8, 1, 64, 4, 64, 8)
    t = lambda x: torch.tensor(x, dtype=torch.bfloat16, device=dev)  # noqa: E731
    args = [t(C), t(Z), t(q), torch.tensor(Bp, dtype=torch.float32, device=dev)]
    kw = dict(m2=8, sliding_window=8, sink_logits=torch.tensor(sk, dtype=torch.float32, device=dev))
    o1 = kch.hca_core(*args, **kw)
    assert o1.grad_fn is None
    o2 = kch.hca_core(*[a.clone().requires_grad_(True) for a in args], **kw)
    assert o2.grad_fn is not None and torch.equal(o1, o2.detach())


@pytest.mark.parametrize("T,m2,win", [(16, 16, 40), (32, 8, 1)])
def test_core_grad_edges(dev, T, m2, win):
    """One block (most queries see none); a window wider than the sequence;
    a one-token window."""
    import kch
    B, nh, c = 1, 2, 64
    C, Z, q, Bp, sk, _, W = _make(T + m2 + win, B, T, nh, c, m2)
    kw = dict(m2=m2, sliding_window=win, scale=1.1)
    ref = o_grad(C, Z, q, Bp, W, sink_logits=sk, **kw)
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=dev, requires_grad=True)  # noqa: E731
    Ct, Zt, qt, Bt, st = t(C), t(Z), t(q), t(Bp), t(sk)
    out = kch.hca_core(Ct, Zt, qt, Bt, sink_logits=st, **kw)
    (out.double() * torch.tensor(W, device=dev)).sum().backward()
    torch.cuda.synchronize()
    for name, x in (("C", Ct), ("Z", Zt), ("q", qt), ("B_pos", Bt), ("sink_logits", st)):
        _check(name, x.grad.cpu().numpy(), ref[name], 1e-4)
