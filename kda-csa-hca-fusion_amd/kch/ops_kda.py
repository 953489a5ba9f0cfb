"""KDA operators on the HIP backend (drop-in twins of the reference's ``ops_kda``).

``naive_chunk_kda``      <- ``/root/reference/ops_kda.py:464-494``
``naive_recurrent_kda``  <- ``/root/reference/ops_kda.py:175-267``

Same signatures, argument meaning, validation messages (``ValueError`` naming
the operator, ``ops_kda.py:29-122``) and dtype contract (output in ``v.dtype``,
state in ``state_dtype`` or fp32). Inputs must live on a ROCm GPU; the work runs
in ``kch_kda_chunk_fwd`` / ``kch_kda_recurrent_fwd`` of ``libkch.so`` on the
current stream. ``chunk_size`` is validated as in the reference; the result
does not depend on it (chunking is a reassociation of the same recurrence), and
the kernel uses its own chunk length.

float64 inputs compute in fp64 with an fp64 state, as in the reference
(``ops_kda.py:125-127``), on ``kch_kda_recurrent_fwd_f64`` for both operators
(the chunked form is the same function).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import _lib


def _validate_kda_inputs(q, k, v, g, beta, fn_name):
    """Rank / batch / device / dtype contract of ``ops_kda.py:29-83``."""
    for name, t, rank in [('q', q, 4), ('k', k, 4), ('v', v, 4), ('g', g, 4), ('beta', beta, 3)]:
        if t.dim() != rank:
            expect = ("[B, T, H, K]" if name in ('q', 'k') else "[B, T, HV, V]" if name == 'v'
                      else "[B, T, HV, K]" if name == 'g' else "[B, T, HV]")
            raise ValueError(
                f"{fn_name}: {name} must have rank {rank} but got rank {t.dim()} "
                f"(shape={tuple(t.shape)}). Expected shape: {expect}")
    Bq, Tq = q.shape[0], q.shape[1]
    for name, t in [('k', k), ('v', v), ('g', g), ('beta', beta)]:
        if t.shape[0] != Bq or t.shape[1] != Tq:
            raise ValueError(
                f"{fn_name}: {name}.shape[0:2]={tuple(t.shape[0:2])} does not match "
                f"q.shape[0:2]=({Bq}, {Tq}). All inputs must share the same batch (B) "
                f"and sequence (T) dimensions.")
    for name, t in [('k', k), ('v', v), ('g', g), ('beta', beta)]:
        if t.device != q.device:
            raise ValueError(
                f"{fn_name}: {name}.device={t.device} does not match q.device={q.device}. "
                f"All inputs must be on the same device.")
    for name, t in [('k', k), ('v', v), ('g', g), ('beta', beta)]:
        if t.dtype != q.dtype:
            raise ValueError(
                f"{fn_name}: {name}.dtype={t.dtype} does not match q.dtype={q.dtype}. "
                f"All inputs must share the same dtype (cast before calling if needed).")


def _validate_kda_shapes(q, k, v, g, beta, fn_name, chunk_size=None):
    """Dimension contract of ``ops_kda.py:86-122``."""
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]
    if H < 1:
        raise ValueError(f"{fn_name}: H={H} must be >= 1 (would cause ZeroDivisionError in HV // H)")
    if K < 1:
        raise ValueError(f"{fn_name}: K={K} must be >= 1")
    if V < 1:
        raise ValueError(f"{fn_name}: V={V} must be >= 1")
    if chunk_size is not None and chunk_size < 1:
        raise ValueError(
            f"{fn_name}: chunk_size={chunk_size} must be >= 1 (would cause ZeroDivisionError "
            f"in T // chunk_size and (-T) % chunk_size)")
    if HV % H != 0:
        raise ValueError(f"{fn_name}: HV={HV} must be divisible by H={H} (GVA factor)")
    if g.shape[2] != HV:
        raise ValueError(
            f"{fn_name}: g.shape[2]={g.shape[2]} must equal HV={HV} "
            f"(g must be [B, T, HV, K], got {tuple(g.shape)})")
    if g.shape[-1] != K:
        raise ValueError(
            f"{fn_name}: g.shape[-1]={g.shape[-1]} must equal K={K} "
            f"(g must be [B, T, HV, K], got {tuple(g.shape)})")
    if beta.shape[2] != HV:
        raise ValueError(
            f"{fn_name}: beta.shape[2]={beta.shape[2]} must equal HV={HV} "
            f"(beta must be [B, T, HV], got {tuple(beta.shape)})")


def _scale_value(scale, K):
    if scale is None:
        return K ** -0.5
    if isinstance(scale, torch.Tensor):
        return float(scale.detach().float().item())
    return float(scale)


def _clamp_value(g_clamp_min) -> float:
    v = float(g_clamp_min)
    return v if v > -math.inf else -math.inf


def _aligned(t):
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _kernel_kv(entry, K, V, dtype):
    """(entry, K, V) the kernels run for head dims K, V: the chunk kernels take
    K in {64, 128} and V a multiple of 64 (bf16 / fp16: V in {64, 128} for the
    two-kernel path, larger V on the fused kernel), the recurrent kernel K in
    {16, 32, 64, 128, 256}; other sizes are zero-padded up to the next one, and
    a chunk call with K > 128 runs the recurrence (the same function)."""
    if entry == "kch_kda_chunk_fwd" and K > 128:
        entry = "kch_kda_recurrent_fwd"
    if entry == "kch_kda_chunk_fwd":
        Kp = 64 if K <= 64 else 128
        Vp = -(-V // 64) * 64
    else:
        Kp = next((n for n in (16, 32, 64, 128, 256) if n >= K), None)
        if Kp is None:
            raise NotImplementedError(f"KDA: head dim K={K} > 256 is not supported by the HIP "
                                      f"kernels")
        Vp = V
    return entry, Kp, Vp


def _run_f64(fn_name, q, k, v, g, beta, scale, initial_state, output_final_state, g_clamp_min,
             state_dtype):
    """float64 inputs: the fp64 recurrence (fp64 arithmetic and state; the
    reference's compute dtype for them, ``ops_kda.py:125-127``). K is
    zero-padded to the kernel's next size as on the other paths."""
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]
    if scale is None:
        sc = K ** -0.5
    elif isinstance(scale, torch.Tensor):
        sc = float(scale.detach().double().item())
    else:
        sc = float(scale)
    Kp = next((n for n in (16, 32, 64, 128, 256) if n >= K), None)
    if Kp is None:
        raise NotImplementedError(f"{fn_name}: head dim K={K} > 256 is not supported by the HIP "
                                  f"kernels")
    target_state = state_dtype if state_dtype is not None else torch.float64
    if Kp != K:
        q, k, g = (F.pad(t, (0, Kp - K)) for t in (q, k, g))
    q, k, v, g, beta = (t.contiguous() for t in (q, k, v, g, beta))
    s0 = None
    if initial_state is not None:
        s0 = initial_state.to(device=q.device, dtype=torch.float64)
        if Kp != K:
            s0 = F.pad(s0, (0, 0, 0, Kp - K))
        s0 = s0.contiguous()
    o = torch.empty_like(v)
    s_out = torch.empty(B, HV, Kp, V, device=q.device, dtype=torch.float64) \
        if output_final_state else None
    _lib.call("kch_kda_recurrent_fwd_f64", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g),
              _lib.ptr(beta), _lib.ptr(s0), _lib.ptr(o), _lib.ptr(s_out), B, T, H, HV, Kp, V, sc,
              _clamp_value(g_clamp_min), _lib.stream_of(q))
    if s_out is not None:
        s_out = s_out[:, :, :K].to(target_state).contiguous()
    return o, s_out


def _run(entry, fn_name, q, k, v, g, beta, scale, initial_state, output_final_state,
         g_clamp_min, state_dtype, chunk_size=None):
    _validate_kda_inputs(q, k, v, g, beta, fn_name)
    _validate_kda_shapes(q, k, v, g, beta, fn_name, chunk_size=chunk_size)
    _lib.require_gpu(fn_name, q, initial_state)
    if v.dtype == torch.float64:
        return _run_f64(fn_name, q, k, v, g, beta, scale, initial_state, output_final_state,
                        g_clamp_min, state_dtype)
    code = _lib.dtype_code(fn_name, v.dtype)
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]
    sc = _scale_value(scale, K)
    entry, Kp, Vp = _kernel_kv(entry, K, V, v.dtype)
    if (Kp, Vp) != (K, V):
        # Zero channels of q, k and g (no decay), zero columns of v and of the
        # initial state: every padded row and column of the state stays zero and
        # adds nothing to the outputs, which are the leading K x V block.
        target_state = state_dtype if state_dtype is not None else torch.float32
        q, k, g = (F.pad(t, (0, Kp - K)) for t in (q, k, g))
        v = F.pad(v, (0, Vp - V))
        s0 = None
        if initial_state is not None:
            s0 = F.pad(initial_state.to(device=q.device, dtype=torch.float32),
                       (0, Vp - V, 0, Kp - K))
        o, s = _run(entry, fn_name, q, k, v, g, beta, sc, s0, output_final_state, g_clamp_min,
                    None)
        o = o[..., :V].contiguous()
        if s is not None:
            s = s[:, :, :K, :V].to(target_state).contiguous()
        return o, s
    target_state = state_dtype if state_dtype is not None else torch.float32
    # the kernels read 16-byte vectors: contiguous, 16-byte aligned storage
    q, k, v, g, beta = (_aligned(t.contiguous()) for t in (q, k, v, g, beta))
    s0 = None
    if initial_state is not None:
        s0 = initial_state.to(device=q.device, dtype=torch.float32).contiguous()
    o = torch.empty_like(v)
    s_out = torch.empty(B, HV, K, V, device=q.device, dtype=torch.float32) \
        if output_final_state else None
    if T == 0 or B == 0:
        if s_out is not None:
            s_out.copy_(s0) if s0 is not None else s_out.zero_()
        return o, (s_out.to(target_state) if s_out is not None else None)
    args = (_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta),
            _lib.ptr(s0), _lib.ptr(o), _lib.ptr(s_out), B, T, H, HV, K, V, sc,
            _clamp_value(g_clamp_min), code)
    if entry == "kch_kda_chunk_fwd":
        # the two-kernel path: per-chunk operands go through a device workspace
        nbytes = _lib.load().kch_kda_chunk_ws_bytes(B, T, H, HV, K, V, code)
        ws = torch.empty(max(nbytes, 1), device=q.device, dtype=torch.uint8)
        _lib.call("kch_kda_chunk_fwd_ws", *args, _lib.ptr(ws), nbytes, _lib.stream_of(q))
    else:
        _lib.call(entry, *args, _lib.stream_of(q))
    if s_out is not None and target_state != torch.float32:
        s_out = s_out.to(target_state)
    return o, s_out


def _bwd_scale(scale, K, f64):
    if scale is None:
        return K ** -0.5
    if isinstance(scale, torch.Tensor):
        return float(scale.detach().double().item()) if f64 else float(scale.detach().float().item())
    return float(scale)


def kda_recurrent_grad(q, k, v, g, beta, d_o, scale=None, initial_state=None, ds_final=None,
                       *, g_clamp_min: float = -10.0, chunked: bool = False):
    """Gradients of ``naive_recurrent_kda`` / ``naive_chunk_kda`` (the same
    function, ``ops_kda.py:175-267`` / ``:464-494``) for the cotangents
    ``d_o = dL/do`` and ``ds_final = dL/dS_T`` (or ``None``), on
    ``kch_kda_recurrent_bwd`` or, with ``chunked`` (the gradient of the chunk
    form with 64-token chunks, ``ops_kda.py:340-536``), on
    ``kch_kda_chunk_bwd`` where it covers the shape (fp32 / bf16 / fp16, K
    padded to 64 or 128, V in {64, 128}). Returns ``(dq, dk, dv, dg, dbeta,
    ds0)``: the first five in the input dtype, ``ds0`` in the state dtype
    (fp32, fp64 for fp64 inputs) or ``None`` without an initial state. K is
    zero-padded to the kernel's next size; padded channels carry no
    gradient."""
    fn = "kda_recurrent_grad"
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]
    f64 = v.dtype == torch.float64
    code = 3 if f64 else _lib.dtype_code(fn, v.dtype)
    st = torch.float64 if f64 else torch.float32
    dtype = v.dtype
    sc = _bwd_scale(scale, K, f64)
    if T == 0 or B == 0:
        ds0 = None
        if initial_state is not None:
            ds0 = (ds_final.to(st).clone() if ds_final is not None
                   else torch.zeros(B, HV, K, V, device=q.device, dtype=st))
        z = [torch.zeros_like(t) for t in (q, k, v, g, beta)]
        return (*z, ds0)
    Kp = next((n for n in (16, 32, 64, 128, 256) if n >= K), None)
    if Kp is None:
        raise NotImplementedError(f"{fn}: head dim K={K} > 256 is not supported by the HIP kernels")
    q, k, g = (F.pad(t.to(dtype), (0, Kp - K)) if Kp != K else t.to(dtype) for t in (q, k, g))
    q, k, v, g, beta, d_o = (t.to(dtype).contiguous() for t in (q, k, v, g, beta, d_o))
    s0 = None if initial_state is None else initial_state.to(device=q.device, dtype=st)
    dsf = None if ds_final is None else ds_final.to(device=q.device, dtype=st)
    if Kp != K:
        s0 = None if s0 is None else F.pad(s0, (0, 0, 0, Kp - K))
        dsf = None if dsf is None else F.pad(dsf, (0, 0, 0, Kp - K))
    s0 = None if s0 is None else s0.contiguous()
    dsf = None if dsf is None else dsf.contiguous()
    dq, dk, dg = (torch.empty_like(t) for t in (q, k, g))
    dv, dbeta = torch.empty_like(v), torch.empty_like(beta)
    ds0 = torch.empty(B, HV, Kp, V, device=q.device, dtype=st) if initial_state is not None \
        else None
    entry = "kch_kda_recurrent_bwd"
    if chunked and code != 3 and Kp in (64, 128) and V in (64, 128):
        entry = "kch_kda_chunk_bwd"
        q, k, v, g, beta, d_o = (_aligned(t) for t in (q, k, v, g, beta, d_o))
        nbytes = _lib.load().kch_kda_chunk_bwd_ws_bytes(B, T, H, HV, Kp, V, code)
    else:
        nbytes = _lib.load().kch_kda_recurrent_bwd_ws_bytes(B, T, HV, Kp, V, code)
    ws = torch.empty(max(nbytes, 1), device=q.device, dtype=torch.uint8)
    _lib.call(entry, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g),
              _lib.ptr(beta), _lib.ptr(s0), _lib.ptr(d_o), _lib.ptr(dsf), _lib.ptr(dq),
              _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dg), _lib.ptr(dbeta), _lib.ptr(ds0),
              B, T, H, HV, Kp, V, sc, _clamp_value(g_clamp_min), code, _lib.ptr(ws), nbytes,
              _lib.stream_of(q))
    if Kp != K:
        dq, dk, dg = (t[..., :K].contiguous() for t in (dq, dk, dg))
        ds0 = None if ds0 is None else ds0[:, :, :K].contiguous()
    return dq, dk, dv, dg, dbeta, ds0


class _KdaFunction(torch.autograd.Function):
    """The operators with gradients: forward on the operator's own kernels,
    backward on ``kch_kda_chunk_bwd`` for ``naive_chunk_kda`` with 64-token
    chunks and on ``kch_kda_recurrent_bwd`` otherwise (the reference
    differentiates its torch code with autograd, ``run_correctness.py:765-833,
    1032-1092``)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, s0, entry, fn_name, scale, g_clamp_min, state_dtype,
                chunk_size):
        ctx.set_materialize_grads(False)
        o, s = _run(entry, fn_name, q, k, v, g, beta, scale, s0, True, g_clamp_min,
                    state_dtype, chunk_size)
        ctx.save_for_backward(q, k, v, g, beta, s0)
        ctx.scale, ctx.g_clamp_min = scale, g_clamp_min
        ctx.chunked = entry == "kch_kda_chunk_fwd" and (chunk_size is None or chunk_size == 64)
        return o, s

    @staticmethod
    def backward(ctx, d_o, d_s):
        q, k, v, g, beta, s0 = ctx.saved_tensors
        if d_o is None:
            d_o = torch.zeros_like(v)
        dq, dk, dv, dg, dbeta, ds0 = kda_recurrent_grad(
            q, k, v, g, beta, d_o, ctx.scale, s0, d_s, g_clamp_min=ctx.g_clamp_min,
            chunked=ctx.chunked)
        if ds0 is not None:
            ds0 = ds0.to(s0.dtype)
        return dq, dk, dv, dg, dbeta, ds0, None, None, None, None, None, None


def _needs_grad(*ts):
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


def _run_op(entry, fn_name, q, k, v, g, beta, scale, initial_state, output_final_state,
            g_clamp_min, state_dtype, chunk_size=None):
    if not _needs_grad(q, k, v, g, beta, initial_state):
        return _run(entry, fn_name, q, k, v, g, beta, scale, initial_state, output_final_state,
                    g_clamp_min, state_dtype, chunk_size)
    o, s = _KdaFunction.apply(q, k, v, g, beta, initial_state, entry, fn_name, scale,
                              g_clamp_min, state_dtype, chunk_size)
    return o, (s if output_final_state else None)


def naive_chunk_kda(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
                    chunk_size: int = 64, *, g_clamp_min: float = -10.0, state_dtype=None):
    """Chunkwise-parallel KDA on the HIP backend (``ops_kda.py:464-494``).
    Differentiable in q, k, v, g, beta and the initial state."""
    return _run_op("kch_kda_chunk_fwd", "naive_chunk_kda", q, k, v, g, beta, scale,
                   initial_state, output_final_state, g_clamp_min, state_dtype, chunk_size)


def naive_recurrent_kda(q, k, v, g, beta, scale=None, initial_state=None,
                        output_final_state=False, *, g_clamp_min: float = -10.0,
                        state_dtype=None):
    """Per-token KDA recurrence on the HIP backend (``ops_kda.py:175-267``).
    Differentiable in q, k, v, g, beta and the initial state."""
    return _run_op("kch_kda_recurrent_fwd", "naive_recurrent_kda", q, k, v, g, beta, scale,
                   initial_state, output_final_state, g_clamp_min, state_dtype)


def kda_recurrent_into(q, k, v, g, beta, scale, state, state_out):
    """One recurrent pass with the final state written to ``state_out`` (fp32
    ``[B,HV,K,V]``, contiguous, 16-byte aligned), which may be ``state``
    itself (or ``state`` None: zero initial state); returns ``o``."""
    fn = "kda_recurrent_into"
    _validate_kda_inputs(q, k, v, g, beta, fn)
    _validate_kda_shapes(q, k, v, g, beta, fn)
    _lib.require_gpu(fn, q, state, state_out)
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]
    if (state_out.dtype != torch.float32 or tuple(state_out.shape) != (B, HV, K, V)
            or not state_out.is_contiguous()):
        raise ValueError(f"{fn}: state_out must be a contiguous fp32 [{B}, {HV}, {K}, {V}] tensor")
    code = _lib.dtype_code(fn, v.dtype)
    q, k, v, g, beta = (_aligned(t.contiguous()) for t in (q, k, v, g, beta))
    s0 = None
    if state is not None:
        s0 = state if state.data_ptr() == state_out.data_ptr() else \
            state.to(device=q.device, dtype=torch.float32).contiguous()
    if T == 0 or B == 0:
        if s0 is None:
            state_out.zero_()
        elif s0.data_ptr() != state_out.data_ptr():
            state_out.copy_(s0)
        return torch.empty_like(v)
    return _recurrent_launch(q, k, v, g, beta, _scale_value(scale, K), s0, state_out, code,
                             _lib.stream_of(q))


def _recurrent_launch(q, k, v, g, beta, scale: float, s0, state_out, code, stream):
    """``kch_kda_recurrent_fwd`` on inputs already checked or built consistent by
    the caller: q, k ``[B,T,H,K]``, v ``[B,T,HV,V]``, g ``[B,T,HV,K]``, beta
    ``[B,T,HV]``, all contiguous, 16-byte aligned, one dtype; ``s0`` None, or an
    fp32 ``[B,HV,K,V]`` state that may be ``state_out`` itself. Returns ``o``."""
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[-1]
    o = torch.empty_like(v)
    _lib.call("kch_kda_recurrent_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g),
              _lib.ptr(beta), _lib.ptr(s0), _lib.ptr(o), _lib.ptr(state_out), B, T, H, HV, K, V,
              scale, -10.0, code, stream)
    return o


chunk_kda = naive_chunk_kda
recurrent_kda = naive_recurrent_kda
