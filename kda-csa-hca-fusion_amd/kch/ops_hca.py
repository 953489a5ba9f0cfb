"""HCA operator on the HIP backend (drop-in twin of ``/root/reference/ops_hca.py:30-201``).

Same signature, validation (``ValueError`` / ``TypeError`` messages of
``ops_hca.py:73-115``) and padding contract. The projections are ``F.linear``
GEMMs on the GPU (W_KV, W_Z and W_DQ concatenated: one GEMM reads H once); the heavy compression (with L2-normalised bf16 key rows and
the per-token window keys) and the dense MQA over compressed blocks + window +
sink run in ``libkch.so``. Keys/values are bf16-rounded L2-normalised rows
(fp32 in the reference). float64 inputs and head dims c above 128 run on the
generic SIMT kernels (``kch.generic``; float64 computed in float64), forward
only. With gradients enabled the projections run through autograd and the
core's backward is ``kch_hca_attn_bwd`` (fp32).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib, generic
from .ops_csa import (_HEAD_DIMS, _MAX_HEADS, _aligned, _attn_bwd_qdtype, _cat_cached,
                      _check_gpu_dtype, _compress, _f32_cached, _head_groups, _kernel_size,
                      _linear_up, _pad_last, l2_normalize_rows)


def hca_core(C, Z, q, B_pos, *, m2, sliding_window=0, sink_logits=None, scale=1.0,
             C_local_raw=None):
    """HCA after the projections (``ops_hca.py:132-194``) on the HIP backend.

    ``C, Z`` ``[B,T,c]`` (rows may be strided views), ``q`` ``[B,T,nh,c]``, T a
    multiple of m2; the window keys are L2norm(C) or L2norm(``C_local_raw``).
    Returns ``[B,T,nh,c]`` in ``q.dtype``. Differentiable in C, Z, q, B_pos,
    the sink logits and ``C_local_raw`` (backward on ``kch_hca_attn_bwd``).
    """
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad
            for t in (C, Z, q, B_pos, sink_logits, C_local_raw)):
        if generic.needs_generic_csa(dtype_tensors=(C, Z, q, C_local_raw), c=C.shape[-1]):
            generic.grad_not_supported("hca_core", "float64 inputs or c > 128")
        return _HcaCoreFunction.apply(C, Z, q, B_pos, sink_logits, C_local_raw, m2,
                                      sliding_window, scale)
    return _hca_core_fwd(C, Z, q, B_pos, m2=m2, sliding_window=sliding_window,
                         sink_logits=sink_logits, scale=scale, C_local_raw=C_local_raw)


def hca_core_grad(C, Z, q, B_pos, d_out, *, m2, sliding_window=0, sink_logits=None, scale=1.0,
                  C_local_raw=None):
    """Gradients of ``hca_core`` for ``d_out = dL/dout`` on ``kch_hca_attn_bwd``
    (fp32 arithmetic). Returns a dict with ``C, Z, q, B_pos`` and, where given,
    ``sink_logits`` and ``C_local_raw``, each in its input's dtype. Channels are
    zero-padded to the kernel's size (a zero channel changes no norm, score or
    softmax); more than 16 heads run as groups whose C/Z gradients add."""
    fn = "hca_core_grad"
    B_, T, c = C.shape
    nh = q.shape[2]
    if T % m2:
        raise ValueError(f"{fn}: T={T} must be a multiple of m2={m2}")
    cp = _kernel_size(fn, "c", c, _HEAD_DIMS)
    dev = C.device
    f32 = torch.float32

    def prep(x, dt=f32):
        x = x.to(dt)
        return (_pad_last(x, cp) if cp != c else x).contiguous()

    # q, d_out and dq move in their storage dtype (the MFMA kernels, 16 heads a call)
    qdt = _attn_bwd_qdtype(q, d_out)
    Cf, Zf, Bp = (prep(x) for x in (C, Z, B_pos))
    qf, dof = _aligned(prep(q, qdt)), _aligned(prep(d_out, qdt))
    Clr = None if C_local_raw is None else prep(C_local_raw)
    nb = T // m2
    win = int(sliding_window)
    kc = torch.empty(B_, nb, cp, device=dev, dtype=f32)
    raw = _compress(fn, Cf, Zf, Bp, m2, out_raw=True, key=kc, normalize=True)
    lsrc = kl = None
    if win > 0:
        lsrc = Cf if Clr is None else Clr
        kl = l2_normalize_rows(lsrc, out_dtype=f32)
    sink = None if sink_logits is None else sink_logits.detach().to(device=dev, dtype=f32).contiguous()
    dq = torch.empty_like(qf)
    dC = torch.zeros(B_, T, cp, device=dev, dtype=f32)
    dZ = torch.zeros_like(dC)
    dB = torch.zeros(cp, device=dev, dtype=f32).new_zeros(m2, cp)
    dloc = None if Clr is None else torch.zeros_like(dC)
    dsink = None if sink is None else torch.zeros(nh, device=dev, dtype=f32)
    hmax = _MAX_HEADS
    for h0 in range(0, nh, hmax):
        h1 = min(nh, h0 + hmax)
        g = h1 - h0
        qg = qf if g == nh else qf[:, :, h0:h1].contiguous()
        dog = dof if g == nh else dof[:, :, h0:h1].contiguous()
        dqg = dq if g == nh else torch.empty_like(qg)
        dCg, dZg = torch.empty_like(dC), torch.empty_like(dZ)
        dBp = torch.empty(B_, nb, m2, cp, device=dev, dtype=f32)
        dlg = None if dloc is None else torch.empty_like(dloc)
        sp = None if sink is None else torch.empty(B_, T, g, device=dev, dtype=f32)
        nbytes = _lib.load().kch_hca_attn_bwd_ws_bytes(B_, T, g, cp, m2, win)
        ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
        _lib.call("kch_hca_attn_bwd", _lib.ptr(qg), _lib.ptr(dog), _lib.ptr(kc), _lib.ptr(raw),
                  _lib.ptr(kl), _lib.ptr(lsrc), _lib.ptr(Cf), _lib.ptr(Zf), _lib.ptr(Bp),
                  _lib.ptr(None if sink is None else sink[h0:h1].contiguous()), _lib.ptr(dqg),
                  _lib.ptr(dCg), _lib.ptr(dZg), _lib.ptr(dBp), _lib.ptr(dlg), _lib.ptr(sp),
                  B_, T, g, cp, m2, win, float(scale), _lib.dtype_code(fn, qdt), _lib.ptr(ws),
                  nbytes, _lib.stream_of(qg))
        if dqg is not dq:
            dq[:, :, h0:h1] = dqg
        dC += dCg
        dZ += dZg
        dB += dBp.sum(dim=(0, 1))
        if dlg is not None:
            dloc += dlg
        if sp is not None:
            dsink[h0:h1] = -sp.sum(dim=(0, 1))
    out = {"C": dC[..., :c].to(C.dtype), "Z": dZ[..., :c].to(Z.dtype),
           "q": dq[..., :c].to(q.dtype), "B_pos": dB[:, :c].to(B_pos.dtype)}
    if sink_logits is not None:
        out["sink_logits"] = dsink.to(sink_logits.dtype)
    if C_local_raw is not None:
        out["C_local_raw"] = dloc[..., :c].to(C_local_raw.dtype)
    return out


class _HcaCoreFunction(torch.autograd.Function):
    """``hca_core`` with gradients: the forward kernels, and
    ``kch_hca_attn_bwd`` for the backward."""

    @staticmethod
    def forward(ctx, C, Z, q, B_pos, sink_logits, C_local_raw, m2, sliding_window, scale):
        ctx.save_for_backward(C, Z, q, B_pos, sink_logits, C_local_raw)
        ctx.cfg = (m2, sliding_window, scale)
        return _hca_core_fwd(C, Z, q, B_pos, m2=m2, sliding_window=sliding_window,
                             sink_logits=sink_logits, scale=scale, C_local_raw=C_local_raw)

    @staticmethod
    def backward(ctx, d_out):
        C, Z, q, B_pos, sink, Clr = ctx.saved_tensors
        m2, win, scale = ctx.cfg
        g = hca_core_grad(C, Z, q, B_pos, d_out, m2=m2, sliding_window=win, sink_logits=sink,
                          scale=scale, C_local_raw=Clr)
        return (g["C"], g["Z"], g["q"], g["B_pos"], g.get("sink_logits"), g.get("C_local_raw"),
                None, None, None)


def _hca_core_fwd(C, Z, q, B_pos, *, m2, sliding_window=0, sink_logits=None, scale=1.0,
                  C_local_raw=None):
    fn = "hca_core"
    B_, T, c = C.shape
    nh = q.shape[2]
    if generic.needs_generic_csa(dtype_tensors=(C, Z, q, C_local_raw), c=c):
        _lib.require_gpu(fn, C, Z, q)
        return generic.hca_core(C, Z, q, B_pos, m2=m2, sliding_window=sliding_window,
                                sink_logits=sink_logits, scale=scale, C_local_raw=C_local_raw)
    cp = _kernel_size(fn, "c", c, _HEAD_DIMS)
    if cp != c:
        # zero channels compress to zero and add nothing to norms and scores
        C, Z, q = (_pad_last(x, cp) for x in (C, Z, q))
        out = _hca_core_fwd(C, Z, q, _pad_last(B_pos, cp), m2=m2, sliding_window=sliding_window,
                            sink_logits=sink_logits, scale=scale,
                            C_local_raw=None if C_local_raw is None else _pad_last(C_local_raw, cp))
        return out[..., :c]
    device = C.device
    n_blocks = T // m2
    kv = torch.empty(B_, n_blocks, c, device=device, dtype=torch.bfloat16)
    local = None
    if sliding_window > 0:
        if C_local_raw is None:
            local = torch.empty(B_, T, c, device=device, dtype=torch.bfloat16)
        else:
            local = l2_normalize_rows(C_local_raw, out_dtype=torch.bfloat16)
    _compress(fn, C, Z, B_pos, m2, out_raw=False, key=kv, normalize=True,
              local=local if C_local_raw is None else None)
    sink = None if sink_logits is None else _f32_cached(sink_logits, device)
    out = torch.empty(B_, T, nh, c, device=device, dtype=q.dtype)
    code = _lib.dtype_code(fn, q.dtype)
    for h0, h1 in _head_groups(nh):
        qc = _aligned(q if h1 - h0 == nh else q[:, :, h0:h1])
        og = out if h1 - h0 == nh else torch.empty(B_, T, h1 - h0, c, device=device,
                                                   dtype=q.dtype)
        _lib.call("kch_hca_attn", _lib.ptr(qc), _lib.ptr(kv), _lib.ptr(local),
                  _lib.ptr(None if sink is None else sink[h0:h1]), _lib.ptr(og), B_, T, n_blocks,
                  h1 - h0, c, m2, sliding_window, float(scale), 1, code, code,
                  _lib.stream_of(qc))
        if og is not out:
            out[:, :, h0:h1] = og
    return out


def naive_hca(H, W_KV, W_Z, B_pos, W_DQ, W_UQ, *, m2, nh, c, dc, scale=1.0, sliding_window=0,
              sink_logits=None, return_projections=False, W_KV_local=None):
    """HCA forward on the HIP backend; returns ``[B, T, nh*c]`` in ``H.dtype``."""
    fn = "naive_hca"
    B_, T, d = H.shape
    if m2 < 1:
        raise ValueError(f"heavy compression factor m2={m2} must be >= 1")
    if nh < 1:
        raise ValueError(f"nh={nh} must be >= 1")
    if c < 1:
        raise ValueError(f"c={c} must be >= 1")
    if dc < 1:
        raise ValueError(f"dc={dc} must be >= 1")
    if sliding_window < 0:
        raise ValueError(
            f"sliding_window={sliding_window} must be >= 0 (0 disables the branch)")
    if not torch.is_floating_point(H):
        raise TypeError(f"naive_hca: H must be a floating-point tensor, got dtype={H.dtype}")
    if W_KV.shape != (c, d):
        raise ValueError(
            f"naive_hca: W_KV.shape={tuple(W_KV.shape)} must equal (c, d)=({c}, {d})")
    if W_Z.shape != (c, d):
        raise ValueError(
            f"naive_hca: W_Z.shape={tuple(W_Z.shape)} must equal (c, d)=({c}, {d})")
    if W_DQ.shape != (dc, d):
        raise ValueError(
            f"naive_hca: W_DQ.shape={tuple(W_DQ.shape)} must equal (dc, d)=({dc}, {d})")
    if W_UQ.shape != (c * nh, dc):
        raise ValueError(
            f"naive_hca: W_UQ.shape={tuple(W_UQ.shape)} must equal (c*nh, dc)=({c*nh}, {dc})")
    if B_pos.shape != (m2, c):
        raise ValueError(
            f"naive_hca: B_pos.shape={tuple(B_pos.shape)} must equal (m2, c)=({m2}, {c})")
    if sink_logits is not None and sink_logits.shape != (nh,):
        raise ValueError(
            f"naive_hca: sink_logits.shape={tuple(sink_logits.shape)} must equal (nh,)=({nh},)")
    if W_KV_local is not None and W_KV_local.shape != (c, d):
        raise ValueError(
            f"naive_hca: W_KV_local.shape={tuple(W_KV_local.shape)} must equal (c, d)=({c}, {d})")
    device = H.device
    if T == 0:
        out_empty = torch.zeros(B_, 0, nh * c, dtype=H.dtype, device=device)
        if return_projections:
            z = torch.zeros(B_, 0, c, dtype=H.dtype, device=device)
            return out_empty, (z, z.clone())
        return out_empty
    _lib.require_gpu(fn, H)
    original_T = T
    pad = (-T) % m2
    if pad:
        H = F.pad(H, (0, 0, 0, pad))
        T = T + pad
    n_blocks = T // m2
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad
            for t in (H, W_KV, W_Z, B_pos, W_DQ, W_UQ, sink_logits, W_KV_local)):
        # training: the projections through autograd (library GEMMs), the core
        # through its HIP backward
        C, Z, cQ = F.linear(H, torch.cat([W_KV, W_Z, W_DQ])).split([c, c, dc], dim=-1)
        q = F.linear(cQ, W_UQ).view(B_, T, nh, c)
        C_local_raw = F.linear(H, W_KV_local) if (W_KV_local is not None and sliding_window > 0) \
            else None
        out = hca_core(C, Z, q, B_pos, m2=m2, sliding_window=sliding_window,
                       sink_logits=sink_logits, scale=scale, C_local_raw=C_local_raw)
        out_final = out.reshape(B_, T, nh * c)[:, :original_T]
        if return_projections:
            return out_final, (C[:, :original_T], Z[:, :original_T])
        return out_final
    with torch.no_grad():
        # the three projections of H in one GEMM: H is read from HBM once
        CZQ = F.linear(H, _cat_cached([W_KV, W_Z, W_DQ], pad_rows_to=8))
        C, Z, cQ = CZQ[..., :2 * c + dc].split([c, c, dc], dim=-1)
        q = _linear_up(cQ, W_UQ).view(B_, T, nh, c)
        C_local_raw = F.linear(H, W_KV_local) if (W_KV_local is not None and sliding_window > 0) \
            else None
        out = hca_core(C, Z, q, B_pos, m2=m2, sliding_window=sliding_window,
                       sink_logits=sink_logits, scale=scale, C_local_raw=C_local_raw)
    out_final = out.reshape(B_, T, nh * c)[:, :original_T]
    if return_projections:
        return out_final, (C[:, :original_T], Z[:, :original_T])
    return out_final


__all__ = ["hca_core", "hca_core_grad", "naive_hca"]
