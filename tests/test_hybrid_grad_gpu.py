"""Gradients of the hybrid layers (needs a ROCm GPU).

The front-end backward kernels (``kch_layer_norm_bwd``, ``kch_short_conv_bwd``,
``kch_kda_gates_bwd``) and the KDA layer as a whole are compared with float64
torch statements of the reference's layer code (``ops_fused.py:42-60``,
``480-609``), differentiated by autograd on the CPU: fp32 within 1e-4 of each
tensor's largest gradient, bf16 within 3e-2. The stack is checked against the
reference's own contract (``run_correctness.py:2710-2830``): every parameter,
the indexer's included, gets a finite, non-zero gradient.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _check(name, got, ref, tol=1e-4):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert torch.isfinite(got).all(), f"{name}: non-finite"
    scale = ref.abs().max().item() + 1e-30
    err = (got - ref).abs().max().item()
    assert err <= tol * scale, f"{name}: max err {err:.3e} of max {scale:.3e}"


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 3e-2)])
def test_layer_norm_grad(dev, dtype, tol):
    from kch.hybrid import _Fp32LayerNorm
    torch.manual_seed(0)
    d = 96
    ln = _Fp32LayerNorm(d).to(dev)
    with torch.no_grad():
        ln.weight.normal_()
        ln.bias.normal_()
    x = torch.randn(3, 17, d, device=dev).to(dtype).requires_grad_(True)
    G = torch.randn(3, 17, d)
    (ln(x).double().cpu() * G).sum().backward()
    xr = x.detach().double().cpu().requires_grad_(True)
    wr = ln.weight.detach().double().cpu().requires_grad_(True)
    br = ln.bias.detach().double().cpu().requires_grad_(True)
    (F.layer_norm(xr, (d,), wr, br, ln.eps) * G).sum().backward()
    _check("dx", x.grad, xr.grad, tol)
    _check("dw", ln.weight.grad, wr.grad, tol)
    _check("db", ln.bias.grad, br.grad, tol)


@pytest.mark.parametrize("lookback,T", [(False, 75), (True, 75), ("grad", 75), ("grad", 1),
                                         ("grad", 2)])
def test_short_conv_grad(dev, lookback, T):
    """``lookback="grad"``: a lookback that requires grad (the previous
    chunk's rows kept in its graph) gets its gradient, compared with autograd
    of ``F.conv1d`` over ``[lookback ; x]`` (the reference's depthwise conv,
    ``ops_fused.py:480-527``)."""
    from kch.hybrid import _ShortConvFn
    torch.manual_seed(1)
    B, d = 2, 40
    x = torch.randn(B, T, d, device=dev, requires_grad=True)
    w = torch.randn(d, 1, 3, device=dev, requires_grad=True)
    b = torch.randn(d, device=dev, requires_grad=True)
    lb = torch.randn(B, 2, d, device=dev) if lookback else None
    if lookback == "grad":
        lb.requires_grad_(True)
    G = torch.randn(B, T, d)
    (_ShortConvFn.apply(x, w, b, lb).double().cpu() * G).sum().backward()
    xr, wr, br = (t.detach().double().cpu().requires_grad_(True) for t in (x, w, b))
    pre = (lb.detach().double().cpu() if lookback
           else torch.zeros(B, 2, d, dtype=torch.float64)).requires_grad_(True)
    xp = torch.cat([pre, xr], 1)
    out = F.conv1d(xp.transpose(1, 2), wr, br, groups=d).transpose(1, 2)
    (out * G).sum().backward()
    _check("dx", x.grad, xr.grad)
    _check("dw", w.grad, wr.grad)
    _check("db", b.grad, br.grad)
    if lookback == "grad":
        _check("dlookback", lb.grad, pre.grad)
    elif lookback:
        assert lb.grad is None


def test_kda_cross_chunk_bptt(dev):
    """``run_correctness.py:1731-1833`` on the HIP layer (fp32): with
    ``detach_lookback=True`` chunk 2's output does not reach chunk 1's input;
    with ``detach_lookback=False`` it does, through the lookback only (the
    state is detached): the gradient is non-zero on chunk 1's last two rows
    and zero on the others. The lookback gradient itself is checked against
    ``F.conv1d`` in ``test_short_conv_grad``."""
    import kch
    torch.manual_seed(123)
    cfg = kch.HybridConfig(d_model=16, n_heads_qk=2, n_heads_v=2, head_dim_k=8, head_dim_v=8,
                           kda_chunk_size=0, n_kda=1, n_csa=0, n_hca=0)
    layer = kch.KDAHybridLayer(cfg).to(dev)
    x1 = torch.randn(1, 8, cfg.d_model, device=dev)
    x2 = torch.randn(1, 8, cfg.d_model, device=dev)
    grads = {}
    for detach in (True, False):
        xa = x1.clone().requires_grad_(True)
        _, st, lb = layer.forward_functional(xa, None, None, detach_lookback=detach)
        o2, _, _ = layer.forward_functional(x2.clone(), st.detach(), lb, detach_lookback=detach)
        o2.sum().backward()
        grads[detach] = xa.grad
    assert grads[True] is None or grads[True].abs().sum().item() < 1e-12
    g = grads[False]
    assert g is not None and torch.isfinite(g).all()
    assert g[:, -2:].abs().sum().item() > 0
    assert g[:, :-2].abs().sum().item() == 0


def _gates_ref(proj, gl, H, HV, K, V, decay):
    B, T = proj.shape[:2]
    HK = H * K
    q = F.normalize(F.silu(proj[..., :HK]).view(B, T, H, K), dim=-1)
    k = F.normalize(F.silu(proj[..., HK:2 * HK]).view(B, T, H, K), dim=-1)
    v = F.silu(proj[..., 2 * HK:2 * HK + HV * V]).view(B, T, HV, V)
    beta = torch.sigmoid(proj[..., 2 * HK + HV * V:2 * HK + HV * V + HV])
    g = -F.softplus(gl).view(B, T, HV, K) * decay
    return q, k, v, g, beta


def test_gates_grad(dev):
    from kch.hybrid import _KdaGatesFn
    torch.manual_seed(2)
    B, T, H, HV, K, V = 2, 9, 2, 4, 32, 24
    N = 2 * H * K + HV * V + HV + K
    proj = torch.randn(B, T, N, device=dev, requires_grad=True)
    gl = (torch.randn(B, T, HV * K, device=dev) * 8).requires_grad_(True)  # some above 20
    outs = _KdaGatesFn.apply(proj, gl, (H, HV, K, V, 0.1))
    Gs = [torch.randn(o.shape) for o in outs]
    sum((o.double().cpu() * G).sum() for o, G in zip(outs, Gs)).backward()
    pr, glr = (t.detach().double().cpu().requires_grad_(True) for t in (proj, gl))
    refs = _gates_ref(pr, glr, H, HV, K, V, 0.1)
    for o, r in zip(outs, refs):
        _check("fwd", o, r, 1e-5)
    sum((r * G).sum() for r, G in zip(refs, Gs)).backward()
    _check("dproj", proj.grad, pr.grad)
    _check("dgl", gl.grad, glr.grad)


def _kda_layer_ref(layer, x, state, scale):
    """KDAHybridLayer's forward (``ops_fused.py:480-609``) in float64 torch on the
    CPU: conv (no lookback), projections, activations, the per-token KDA
    recurrence (``ops_kda.py:175-267``), o_proj."""
    cfg = layer.cfg
    H, K, V, HV = cfg.n_heads_qk, cfg.head_dim_k, cfg.head_dim_v, cfg.n_heads_v
    P = {n: p.detach().double().cpu().requires_grad_(True) for n, p in layer.named_parameters()}
    B, T, d = x.shape
    w = P["short_conv.weight"]
    xp = torch.cat([torch.zeros(B, 2, d, dtype=torch.float64), x], 1)
    xc = P["short_conv.bias"] + w[:, 0, 0] * xp[:, :-2] + w[:, 0, 1] * xp[:, 1:-1] + w[:, 0, 2] * xp[:, 2:]
    proj = torch.cat([xc @ P[f"{n}.weight"].T for n in ("q_proj", "k_proj", "v_proj", "beta")]
                     + [xc @ P["g_down.weight"].T], -1)
    gl = (xc @ P["g_down.weight"].T) @ P["g_up.weight"].T
    q, k, v, g, beta = _gates_ref(proj, gl, H, HV, K, V, cfg.kda_decay_scale)
    g = g.clamp(min=-10.0)
    G = HV // H
    qh = q.repeat_interleave(G, 2) * scale
    kh = k.repeat_interleave(G, 2)
    S = state.clone()
    outs = []
    for t in range(T):
        S = S * g[:, t].exp()[..., None]
        S = S + torch.einsum('bhk,bhv->bhkv', beta[:, t][..., None] * kh[:, t],
                             v[:, t] - (kh[:, t][..., None] * S).sum(-2))
        outs.append(torch.einsum('bhk,bhkv->bhv', qh[:, t], S))
    o = torch.stack(outs, 1).reshape(B, T, HV * V)
    return o @ P["o_proj.weight"].T, S, P


@pytest.mark.parametrize("chunk", [0, 16])
def test_kda_layer_grad(dev, chunk):
    """The whole KDA sub-layer in fp32 (recurrent and chunked operator) against
    the float64 statement: every parameter, the input and the initial state."""
    import kch
    torch.manual_seed(3)
    cfg = kch.HybridConfig(d_model=32, n_heads_qk=2, n_heads_v=2, head_dim_k=16, head_dim_v=16,
                           kda_chunk_size=chunk)
    layer = kch.KDAHybridLayer(cfg).to(dev)
    B, T = 2, 40
    x = torch.randn(B, T, 32, device=dev, requires_grad=True)
    s0 = (torch.randn(B, 2, 16, 16, device=dev) * 0.1).requires_grad_(True)
    G = torch.randn(B, T, 32)
    Gs = torch.randn(B, 2, 16, 16)
    out, st, _ = layer.forward_functional(x, s0, None)
    ((out.double().cpu() * G).sum() + (st.double().cpu() * Gs).sum()).backward()
    xr = x.detach().double().cpu().requires_grad_(True)
    sr = s0.detach().double().cpu().requires_grad_(True)
    ref, S, P = _kda_layer_ref(layer, xr, sr, layer._scale_value())
    _check("out", out, ref, 1e-5)
    ((ref * G).sum() + (S * Gs).sum()).backward()
    _check("dx", x.grad, xr.grad)
    _check("ds0", s0.grad, sr.grad)
    for n, p in layer.named_parameters():
        _check(n, p.grad, P[n].grad)


def test_hybrid_backward_produces_grads(dev):
    """``run_correctness.py:2710-2830`` on the HIP stack: T=64, the reference's
    config; every parameter gets a finite gradient, non-zero for all of them
    (indexer included, through the STE)."""
    import kch
    torch.manual_seed(200)
    cfg = kch.HybridConfig(d_model=32, n_heads_qk=2, n_heads_v=2, head_dim_k=16, head_dim_v=16,
                           csa_m=8, csa_topk=4, csa_nh=2, csa_c=16, csa_dc=32, csa_nIh=2, csa_cI=8,
                           csa_sliding_window=8, hca_m2=8, hca_nh=2, hca_c=16, hca_dc=32,
                           hca_sliding_window=8, n_kda=3, n_csa=1, n_hca=1)
    model = kch.HybridKCHAttention(cfg, total_layers=5).to(dev)
    model.train()
    model.reset_state()
    x = torch.randn(2, 64, 32, device=dev)
    y = model(x)
    y.square().mean().backward()
    missing, bad, zero = [], [], []
    for n, p in model.named_parameters():
        if p.grad is None:
            missing.append(n)
        elif not torch.isfinite(p.grad).all():
            bad.append(n)
        elif p.grad.abs().sum() == 0:
            zero.append(n)
    assert not missing and not bad and not zero, (missing, bad, zero)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hybrid_training_reduces_loss(dev, dtype):
    """A few optimizer steps on one batch through the HIP stack (KDA, CSA with
    the STE, HCA, LayerNorms): the loss goes down and stays finite."""
    import kch
    torch.manual_seed(11)
    cfg = kch.HybridConfig(d_model=64, n_heads_qk=2, n_heads_v=2, head_dim_k=32, head_dim_v=32,
                           csa_m=4, csa_topk=8, csa_nh=2, csa_c=64, csa_dc=32, csa_nIh=2,
                           csa_cI=32, csa_sliding_window=8, hca_m2=8, hca_nh=2, hca_c=64,
                           hca_dc=32, hca_sliding_window=8, kda_chunk_size=64)
    model = kch.HybridKCHAttention(cfg, total_layers=5).to(dev, dtype).train()
    opt = torch.optim.AdamW(model.parameters(), lr=3e-3)
    x = torch.randn(2, 128, 64, device=dev).to(dtype)
    target = torch.randn(2, 128, 64, device=dev).to(dtype)
    losses = []
    for _ in range(6):
        opt.zero_grad(set_to_none=True)
        y, _, _ = model.forward_functional(x, None, [None] * model.n_kda_layers)
        loss = (y.float() - target.float()).square().mean()
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert all(np.isfinite(losses)), losses
    assert losses[-1] < losses[0], losses
