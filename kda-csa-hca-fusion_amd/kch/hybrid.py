"""Hybrid KDA / CSA / HCA stack on the HIP backend.

Drop-in twins of the reference's composition layer:

``HybridConfig``        <- ``/root/reference/ops_fused.py:65-313`` (``kda_backend="hip"``)
``_Fp32LayerNorm``      <- ``ops_fused.py:42-60``
``KDAHybridLayer``      <- ``ops_fused.py:316-609``
``CSAHybridLayer``      <- ``ops_fused.py:612-713``
``HCAHybridLayer``      <- ``ops_fused.py:716-739``
``HybridKCHAttention``  <- ``ops_fused.py:742-1131``
``HybridDecoding``      <- ``/root/reference/run_decoding.py:601-851``

Parameter and buffer names, shapes and the layout rule are the reference's, so
a reference ``state_dict`` loads unchanged. The forward passes run on a ROCm
GPU: projections are torch GEMMs (hipBLASLt); the KDA short convolution and
activations, KDA itself, CSA, HCA and the decode caches are ``libkch.so``
kernels. With gradients enabled the layers run their HIP backward kernels.

``HybridDecoding`` takes any ``HybridConfig`` (the reference hard-codes a tiny
geometry with ``kda_chunk_size=0``); prefill goes through the chunked KDA
kernel and the bulk cache population, decode through the T=1 recurrent step
and the cache decode kernels.
"""

from __future__ import annotations

import logging
import math
import os
import warnings
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.nn.modules import module as _nn_module

from . import _lib
from .decoding_cache import CSADecodingCache, HCADecodingCache
from . import ops_csa
from .ops_csa import naive_csa
from .ops_hca import naive_hca
from .ops_kda import _recurrent_launch, kda_recurrent_into, naive_chunk_kda, naive_recurrent_kda
from .ops_kda_backend import kda_forward, validate_kda_backend

logger = logging.getLogger(__name__)

_CONV_K = 3  # short-conv kernel size (ops_fused.py:333)


def _rows_ok(t: torch.Tensor) -> bool:
    return t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0


def _linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``F.linear(x, w)`` without bias. A decode step's few rows (at most 16)
    go to ``kch_linear_rows``, one HIP launch: a BLAS call costs more host time
    than its GEMM takes on the GPU at that size. Larger inputs use ``F.linear``."""
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    if not (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and w.dtype == x.dtype
            and 0 < rows <= 16 and K % 32 == 0 and w.dim() == 2 and w.shape[1] == K):
        return F.linear(x, w)
    if x.is_contiguous() and x.data_ptr() % 16 == 0:
        xr = x  # rows of K elements, K % 32 == 0
    else:
        xr = x.reshape(rows, K)
        if not _rows_ok(xr):
            # fresh storage: a contiguous view that starts off a 16-byte
            # boundary (a column slice of one row) stays misaligned under
            # .contiguous(), which returns the view itself
            xr = xr.clone(memory_format=torch.contiguous_format)
    if w.is_contiguous() and w.data_ptr() % 16 == 0:
        ldw = K  # a contiguous [N, K] weight (its stride(0) is arbitrary when N == 1)
    else:
        if not _rows_ok(w):
            w = w.clone(memory_format=torch.contiguous_format)
        ldw = w.stride(0)
    N = w.shape[0]
    y = torch.empty(*x.shape[:-1], N, device=x.device, dtype=x.dtype)
    _lib.call("kch_linear_rows", _lib.ptr(xr), K if xr is x else xr.stride(0), _lib.ptr(w), ldw,
              _lib.ptr(y), N, rows, N, K, _lib.dtype_code("kch_linear_rows", x.dtype),
              _lib.stream_of(x))
    return y


def _linear_residual(x: torch.Tensor, w: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
    """``residual + F.linear(x, w)`` with the add in the GEMM's epilogue: one
    ``addmm`` (C = the residual stream, beta = 1) reads the residual and writes
    the new stream, so no separate add kernel reads both back. The sum is
    rounded once to the stream's dtype (the reference rounds the projection,
    then the sum: at most one unit in the last place apart). A decode step's
    few rows keep ``_linear`` and the add."""
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    if (rows <= 16 or not x.is_cuda or x.dtype != residual.dtype or w.dtype != x.dtype
            or residual.shape[:-1] != x.shape[:-1]):
        return residual + _linear(x, w)
    out = torch.addmm(residual.reshape(rows, residual.shape[-1]), x.reshape(rows, K), w.t())
    return out.view(residual.shape)


def _grad_wanted(*ts) -> bool:
    return torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in ts)


class _LayerNormFn(torch.autograd.Function):
    """``_Fp32LayerNorm`` with gradients: ``kch_layer_norm`` forward,
    ``kch_layer_norm_bwd`` backward (dx in x's dtype; dw, db accumulated in
    fp32, returned in the parameters' dtype)."""

    @staticmethod
    def forward(ctx, x, w, b, module):
        ctx.save_for_backward(x, w, b)
        ctx.eps = float(module.eps)
        with torch.no_grad():
            return module._forward_kernel(x)

    @staticmethod
    def backward(ctx, dy):
        x, w, b = ctx.saved_tensors
        d = w.shape[-1]
        xc = x.contiguous()
        dyc = dy.to(x.dtype).contiguous()
        wc = w.detach().contiguous()
        dx = torch.empty_like(xc)
        dw = torch.zeros(d, device=x.device, dtype=torch.float32)
        db = torch.zeros_like(dw) if b is not None else None
        fn = "_Fp32LayerNorm"
        _lib.call("kch_layer_norm_bwd", _lib.ptr(xc), _lib.ptr(wc), _lib.ptr(dyc), _lib.ptr(dx),
                  _lib.ptr(dw), _lib.ptr(db), xc.numel() // d, d, ctx.eps,
                  _lib.dtype_code(fn, xc.dtype), _lib.dtype_code(fn, wc.dtype),
                  _lib.stream_of(xc))
        return dx, dw.to(w.dtype), None if db is None else db.to(b.dtype), None


class _Fp32LayerNorm(nn.LayerNorm):
    """LayerNorm computed in fp32, returned in the input dtype (``ops_fused.py:42-60``),
    as one kernel (``kch_layer_norm``; backward ``kch_layer_norm_bwd``)."""

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if _grad_wanted(x, self.weight, self.bias) and x.numel():
            return _LayerNormFn.apply(x, self.weight, self.bias, self)
        return self._forward_kernel(x)

    def _forward_kernel(self, x: torch.Tensor) -> torch.Tensor:
        if x.numel() == 0:
            return torch.empty_like(x)
        if not x.is_cuda:
            _lib.require_gpu("_Fp32LayerNorm", x)
        ns, w, b = self.normalized_shape, self.weight, self.bias
        d = ns[-1]
        if len(ns) != 1 or x.shape[-1] != d or w is None:
            raise ValueError("_Fp32LayerNorm: expects an affine LayerNorm over the last dim")
        xc = x.contiguous()
        out = torch.empty_like(xc)
        fn = "_Fp32LayerNorm"
        # the kernel reads the parameters through raw pointers: no autograd use
        w = w.contiguous()
        if b is not None and (b.dtype != w.dtype or not b.is_contiguous()):
            b = b.detach().to(w.dtype).contiguous()
        _lib.call("kch_layer_norm", _lib.ptr(xc), _lib.ptr(w), _lib.ptr(b),
                  _lib.ptr(out), xc.numel() // d, d, float(self.eps),
                  _lib.dtype_code(fn, xc.dtype), _lib.dtype_code(fn, w.dtype),
                  _lib.stream_of(xc))
        return out


def _is_int(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


@dataclass
class HybridConfig:
    """Fields, defaults and validation of ``ops_fused.py:65-313``.

    ``kda_backend`` defaults to ``"hip"``, the backend this package provides.
    """

    d_model: int = 256
    n_heads_qk: int = 4
    n_heads_v: int = 4
    head_dim_k: int = 64
    head_dim_v: int = 64
    kda_chunk_size: int = 64
    kda_backend: str = "hip"
    csa_m: int = 16
    csa_topk: int = 8
    csa_nh: int = 4
    csa_c: int = 64
    csa_dc: int = 128
    csa_nIh: int = 2
    csa_cI: int = 32
    csa_sliding_window: int = 16
    hca_m2: int = 64
    hca_nh: int = 4
    hca_c: int = 64
    hca_dc: int = 128
    hca_sliding_window: int = 16
    n_kda: int = 3
    n_csa: int = 1
    n_hca: int = 1
    kda_decay_scale: float = 0.1
    init_std: float = 0.02
    dropout: float = 0.0

    def __post_init__(self):
        # dropout: type, finiteness and range first, then "not implemented"
        # for a valid non-zero rate (ops_fused.py:121-150)
        if not isinstance(self.dropout, (int, float)):
            raise TypeError(f"HybridConfig.dropout={self.dropout!r} must be a float, "
                            f"got {type(self.dropout).__name__}.")
        if isinstance(self.dropout, bool):
            raise TypeError(f"HybridConfig.dropout={self.dropout!r} must be a float, got bool.")
        if math.isnan(self.dropout) or math.isinf(self.dropout):
            raise ValueError(f"HybridConfig.dropout={self.dropout} must be finite (not NaN or Inf).")
        if self.dropout < 0.0 or self.dropout > 1.0:
            raise ValueError(f"HybridConfig.dropout={self.dropout} must be in [0.0, 1.0].")
        if self.dropout != 0.0:
            raise NotImplementedError(
                f"HybridConfig.dropout={self.dropout} is not yet implemented: the KDA/CSA/HCA "
                f"sub-layers apply no dropout. Set dropout=0.0.")
        validate_kda_backend(self.kda_backend)
        # head counts and the GVA factor (ops_fused.py:157-175)
        if not _is_int(self.n_heads_qk) or self.n_heads_qk < 1:
            raise ValueError(f"n_heads_qk={self.n_heads_qk!r} must be a positive int")
        if not _is_int(self.n_heads_v) or self.n_heads_v < 1:
            raise ValueError(f"n_heads_v={self.n_heads_v!r} must be a positive int")
        if self.n_heads_v % self.n_heads_qk != 0:
            raise ValueError(
                f"n_heads_v={self.n_heads_v} must be divisible by n_heads_qk={self.n_heads_qk} "
                f"(KDA GVA factor G = HV // H must be an integer).")
        # strictly positive dimensions (ops_fused.py:176-203)
        for name in ("d_model", "head_dim_k", "head_dim_v", "csa_m", "csa_c", "csa_dc", "csa_cI",
                     "csa_nIh", "hca_m2", "hca_c", "hca_dc"):
            val = getattr(self, name)
            if not _is_int(val):
                raise ValueError(f"HybridConfig.{name}={val!r} must be a positive int.")
            if val < 1:
                raise ValueError(f"HybridConfig.{name}={val} must be >= 1.")
        if not isinstance(self.kda_chunk_size, int):
            raise ValueError(
                f"kda_chunk_size={self.kda_chunk_size!r} must be an int (>= 1 enables the chunk "
                f"path; <= 0 forces the recurrent path; default 64).")
        # layer counts (ops_fused.py:237-262)
        for name in ("n_kda", "n_csa", "n_hca"):
            val = getattr(self, name)
            if not _is_int(val):
                raise ValueError(f"HybridConfig.{name}={val!r} must be an int.")
            if val < 0:
                raise ValueError(f"HybridConfig.{name}={val} must be >= 0.")
        if self.n_kda + self.n_csa + self.n_hca == 0:
            raise ValueError("HybridConfig has n_kda=n_csa=n_hca=0; the model would have no "
                             "attention layers at all.")
        # CSA / HCA branch parameters (ops_fused.py:263-296)
        if not _is_int(self.csa_topk) or self.csa_topk < 0:
            raise ValueError(f"csa_topk={self.csa_topk!r} must be a non-negative int "
                             f"(0 disables sparse selection).")
        if not _is_int(self.csa_nh) or self.csa_nh < 1:
            raise ValueError(f"csa_nh={self.csa_nh!r} must be a positive int (head count).")
        if not _is_int(self.csa_sliding_window) or self.csa_sliding_window < 0:
            raise ValueError(f"csa_sliding_window={self.csa_sliding_window!r} must be a "
                             f"non-negative int (0 disables the branch).")
        if not _is_int(self.hca_nh) or self.hca_nh < 1:
            raise ValueError(f"hca_nh={self.hca_nh!r} must be a positive int (head count).")
        if not _is_int(self.hca_sliding_window) or self.hca_sliding_window < 0:
            raise ValueError(f"hca_sliding_window={self.hca_sliding_window!r} must be a "
                             f"non-negative int (0 disables the branch).")
        # KDA decay scale (ops_fused.py:297-313)
        if not isinstance(self.kda_decay_scale, (int, float)):
            raise ValueError(f"kda_decay_scale={self.kda_decay_scale!r} must be a number.")
        if not math.isfinite(self.kda_decay_scale):
            raise ValueError(f"kda_decay_scale={self.kda_decay_scale} must be finite.")
        if self.kda_decay_scale < 0:
            raise ValueError(f"kda_decay_scale={self.kda_decay_scale} must be >= 0.")


class _FusedWeight:
    """Row-concatenation of several weight matrices, rebuilt only when one of
    them changes (storage, in-place version, dtype or device).

    Writes through ``param.data`` (``p.data.copy_(...)``, EMA or weight-swap
    code) change neither the storage nor the autograd version counter: after
    such a write call the owning layer's ``invalidate_weight_cache()``.
    ``load_state_dict`` and ``.to()`` / ``.half()`` invalidate by themselves."""

    def __init__(self):
        self._key = None
        self._w = None

    def invalidate(self):
        self._key = None
        self._w = None

    def get(self, params, dtype, device, build=None):
        """The row-concatenation of ``params`` in ``dtype`` on ``device``, or
        ``build()``'s result (anything derived from ``params``) when given."""
        key = tuple((0, 0) if p is None else (p.data_ptr(), p._version)
                    for p in params) + (dtype, device)
        if key != self._key:
            self._w = (torch.cat([p.detach() for p in params], 0).to(device=device, dtype=dtype)
                       if build is None else build())
            self._key = key
        return self._w


def _invalidate_after_load(module, incompatible_keys):
    module.invalidate_weight_cache()


class _FusedWeightLayer(nn.Module):
    """Base of the sub-layers that keep fused copies of their weights: the
    copies are dropped by ``load_state_dict``, by ``.to()`` / ``.half()`` /
    ``.cuda()`` (``_apply``) and by ``invalidate_weight_cache()``."""

    def __init__(self):
        super().__init__()
        self._fused = _FusedWeight()
        self._fused_step = _FusedWeight()  # the decode step's operands
        self.register_load_state_dict_post_hook(_invalidate_after_load)

    def invalidate_weight_cache(self) -> None:
        """Drop the fused weight copies (call after writing parameters through ``.data``)."""
        self._fused.invalidate()
        self._fused_step.invalidate()

    def _apply(self, fn, *args, **kwargs):
        self._fused.invalidate()
        self._fused_step.invalidate()
        return super()._apply(fn, *args, **kwargs)


class _ShortConvFn(torch.autograd.Function):
    """The KDA layer's causal depthwise conv with gradients: ``kch_short_conv``
    forward, ``kch_short_conv_bwd`` backward. A lookback that requires grad
    (the previous chunk's last two rows kept in its graph,
    ``detach_lookback=False``, ``ops_fused.py:480-527``) gets its gradient
    too: ``d lb[0] = w0 dy[0]``, ``d lb[1] = w1 dy[0] + w0 dy[1]``."""

    @staticmethod
    def forward(ctx, x, weight, bias, lookback):
        B, T, d = x.shape
        w = weight.detach().reshape(d, _CONV_K).to(x.dtype).contiguous()
        b = None if bias is None else bias.detach().to(x.dtype).contiguous()
        xc = x.contiguous()
        if xc.data_ptr() % 16:
            xc = xc.clone()
        lb = None if lookback is None else lookback.detach().to(x.dtype).contiguous()
        if lb is not None and lb.data_ptr() % 16:
            lb = lb.clone()
        out = torch.empty_like(xc)
        code = _lib.dtype_code("KDAHybridLayer", x.dtype)
        _lib.call("kch_short_conv", _lib.ptr(xc), _lib.ptr(lb), _lib.ptr(w), _lib.ptr(b),
                  _lib.ptr(out), B, T, d, code, _lib.stream_of(xc))
        ctx.save_for_backward(xc, w, lb)
        ctx.meta = (weight.shape, weight.dtype, None if bias is None else bias.dtype,
                    None if lookback is None else lookback.dtype)
        return out

    @staticmethod
    def backward(ctx, dy):
        xc, w, lb = ctx.saved_tensors
        wshape, wdt, bdt, lbdt = ctx.meta
        B, T, d = xc.shape
        dyc = dy.to(xc.dtype).contiguous()
        dx = torch.empty_like(xc)
        dw = torch.zeros(d * _CONV_K, device=xc.device, dtype=torch.float32)
        db = None if bdt is None else torch.zeros(d, device=xc.device, dtype=torch.float32)
        dlb = None
        if ctx.needs_input_grad[3]:
            dlb = (torch.empty(B, _CONV_K - 1, d, device=xc.device, dtype=xc.dtype) if T
                   else torch.zeros(B, _CONV_K - 1, d, device=xc.device, dtype=xc.dtype))
        _lib.call("kch_short_conv_bwd", _lib.ptr(xc), _lib.ptr(lb), _lib.ptr(w), _lib.ptr(dyc),
                  _lib.ptr(dx), _lib.ptr(dw), _lib.ptr(db), _lib.ptr(dlb), B, T, d,
                  _lib.dtype_code("KDAHybridLayer", xc.dtype), _lib.stream_of(xc))
        return (dx, dw.view(wshape).to(wdt), None if db is None else db.to(bdt),
                None if dlb is None else dlb.to(lbdt))


class _KdaGatesFn(torch.autograd.Function):
    """The KDA layer's q/k/v/g/beta activations with gradients:
    ``kch_kda_gates`` forward, ``kch_kda_gates_bwd`` backward
    (``ops_fused.py:559-581``)."""

    @staticmethod
    def forward(ctx, proj, gl, dims):
        H, HV, K, V, decay = dims
        B, T = proj.shape[:2]
        dev, dt = proj.device, proj.dtype
        q = torch.empty(B, T, H, K, device=dev, dtype=dt)
        k = torch.empty_like(q)
        v = torch.empty(B, T, HV, V, device=dev, dtype=dt)
        g = torch.empty(B, T, HV, K, device=dev, dtype=dt)
        beta = torch.empty(B, T, HV, device=dev, dtype=dt)
        code = _lib.dtype_code("KDAHybridLayer", dt)
        _lib.call("kch_kda_gates", _lib.ptr(proj), proj.stride(1), _lib.ptr(gl), gl.stride(1),
                  _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta),
                  B, T, H, HV, K, V, float(decay), code, _lib.stream_of(proj))
        ctx.save_for_backward(proj, gl)
        ctx.dims = dims
        return q, k, v, g, beta

    @staticmethod
    def backward(ctx, dq, dk, dv, dg, dbeta):
        proj, gl = ctx.saved_tensors
        H, HV, K, V, decay = ctx.dims
        B, T = proj.shape[:2]
        dt = proj.dtype

        def grad_or_zero(t, shape):
            return torch.zeros(shape, device=proj.device, dtype=dt) if t is None \
                else t.to(dt).contiguous()

        dq = grad_or_zero(dq, (B, T, H, K))
        dk = grad_or_zero(dk, (B, T, H, K))
        dv = grad_or_zero(dv, (B, T, HV, V))
        dg = grad_or_zero(dg, (B, T, HV, K))
        dbeta = grad_or_zero(dbeta, (B, T, HV))
        dproj = torch.zeros_like(proj)
        dgl = torch.zeros_like(gl)
        _lib.call("kch_kda_gates_bwd", _lib.ptr(proj), proj.stride(1), _lib.ptr(gl), gl.stride(1),
                  _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(dg), _lib.ptr(dbeta),
                  _lib.ptr(dproj), _lib.ptr(dgl), B, T, H, HV, K, V, float(decay),
                  _lib.dtype_code("KDAHybridLayer", dt), _lib.stream_of(proj))
        return dproj, dgl, None


class KDAHybridLayer(_FusedWeightLayer):
    """KDA sub-layer (``ops_fused.py:316-609``).

    The short convolution and the q/k/v/g/beta activations run in
    ``kch_short_conv`` / ``kch_kda_gates``; q, k, v, beta and the gate's
    down-projection are one GEMM against the concatenated weights.
    """

    def __init__(self, cfg: HybridConfig):
        super().__init__()
        self.cfg = cfg
        d, H, K, V = cfg.d_model, cfg.n_heads_qk, cfg.head_dim_k, cfg.head_dim_v
        self.q_proj = nn.Linear(d, H * K, bias=False)
        self.k_proj = nn.Linear(d, H * K, bias=False)
        self.v_proj = nn.Linear(d, cfg.n_heads_v * V, bias=False)
        self.g_down = nn.Linear(d, K, bias=False)
        self.g_up = nn.Linear(K, cfg.n_heads_v * K, bias=False)
        self.beta = nn.Linear(d, cfg.n_heads_v, bias=False)
        self.o_proj = nn.Linear(cfg.n_heads_v * V, d, bias=False)
        self.short_conv = nn.Conv1d(d, d, kernel_size=_CONV_K, padding=0, groups=d, bias=True)
        # a buffer so that .bfloat16() rounds it like the reference's (ops_fused.py:342-344)
        self.register_buffer('scale', torch.tensor(K ** -0.5), persistent=False)
        self.register_buffer('_conv_lookback', None, persistent=False)
        self._scale_cache = None

    def reset_conv_state(self) -> None:
        self._conv_lookback = None

    def _scale_value(self) -> float:
        # K^-0.5 rounded to the buffer's dtype, computed on the host (no device
        # sync) once per dtype
        dt = self.scale.dtype
        if self._scale_cache is None or self._scale_cache[0] != dt:
            self._scale_cache = (dt, float(torch.tensor(self.cfg.head_dim_k ** -0.5).to(dt)))
        return self._scale_cache[1]

    def _weights(self, dtype, device):
        """(fused q/k/v/beta/g_down weight, conv weight [d, 3], conv bias, g_up
        weight) in ``dtype``, rebuilt only when a parameter changes."""
        conv, bias = self.short_conv.weight, self.short_conv.bias
        fused = [self.q_proj.weight, self.k_proj.weight, self.v_proj.weight,
                 self.beta.weight, self.g_down.weight]
        g_up = self.g_up.weight

        def build():
            W = torch.cat([p.detach() for p in fused], 0).to(device=device, dtype=dtype)
            w = conv.detach().to(device=device, dtype=dtype).reshape(conv.shape[0], _CONV_K)
            b = None if bias is None else bias.detach().to(device=device, dtype=dtype)
            return W, w.contiguous(), None if b is None else b.contiguous(), \
                g_up.detach().to(device=device, dtype=dtype)
        return self._fused.get(fused + [conv, bias, g_up], dtype, device, build)

    def forward(self, x: torch.Tensor, state: torch.Tensor | None = None, *,
                state_out: torch.Tensor | None = None, residual: torch.Tensor | None = None):
        """Stateful forward: reads and writes ``self._conv_lookback`` (``ops_fused.py:365-389``).

        ``state_out`` (fp32 ``[B,HV,K,V]``, contiguous; may be ``state`` itself)
        receives the final state in place of a new tensor. With ``residual`` the
        output is ``residual + o_proj(...)`` (the add fused into the GEMM)."""
        o, new_state, new_lookback = self.forward_functional(x, state, self._conv_lookback,
                                                             state_out=state_out,
                                                             residual=residual)
        self._conv_lookback = new_lookback
        return o, new_state

    def forward_functional(self, x: torch.Tensor, state: torch.Tensor | None,
                           conv_lookback: torch.Tensor | None, *, detach_lookback: bool = True,
                           state_out: torch.Tensor | None = None,
                           residual: torch.Tensor | None = None):
        """Side-effect-free forward (``ops_fused.py:391-609``).

        Returns ``(output [B,T,d], new_state [B,HV,K,V] fp32, new_lookback [B,2,d] | None)``;
        with ``residual`` ``[B,T,d]`` the output is ``residual + o_proj(...)``.
        """
        B, T, d = x.shape
        cfg = self.cfg
        H, K, V, HV = cfg.n_heads_qk, cfg.head_dim_k, cfg.head_dim_v, cfg.n_heads_v
        if T == 0:  # ops_fused.py:468-479
            if state is not None and state.shape[0] == B:
                new_state = state.to(device=x.device, dtype=torch.float32)
            else:
                new_state = torch.zeros(B, HV, K, V, device=x.device, dtype=torch.float32)
            lb = conv_lookback
            if lb is not None:
                lb = None if lb.shape[0] != B else lb.to(device=x.device, dtype=x.dtype).clone()
            return (x.new_zeros(B, 0, d) if residual is None else residual.clone()), new_state, lb
        _lib.require_gpu("KDAHybridLayer", x)
        lookback = conv_lookback
        if lookback is not None:  # batch / device / dtype guards (ops_fused.py:500-518)
            if lookback.shape[0] != B:
                lookback = None
            else:
                lookback = lookback.to(device=x.device, dtype=x.dtype)
        if _grad_wanted(x, state, lookback, residual, *self.parameters()):
            out, new_state, new_lookback = self._forward_grad(x, state, lookback, detach_lookback)
            return (out if residual is None else residual + out), new_state, new_lookback
        with torch.no_grad():
            xc = x.contiguous()
            if xc.data_ptr() % 16:
                xc = xc.clone()
            lb = None
            if lookback is not None:
                lb = lookback.contiguous()
                if lb.data_ptr() % 16:
                    lb = lb.clone()
            # new lookback: the last two rows of [lookback ; x] (zeros if shorter)
            if T >= _CONV_K - 1:
                new_lookback = x[:, -(_CONV_K - 1):].clone()
            elif lookback is not None:
                new_lookback = torch.cat([lookback[:, T:], x], dim=1)  # the last K - 1 rows
            else:
                new_lookback = torch.cat([x.new_zeros(B, _CONV_K - 1 - T, d), x], dim=1)
            code = _lib.dtype_code("KDAHybridLayer", x.dtype)
            stream = _lib.stream_of(xc)
            W, w, bias, g_up = self._weights(x.dtype, x.device)
            x_conv = torch.empty_like(xc)
            _lib.call("kch_short_conv", _lib.ptr(xc), _lib.ptr(lb), _lib.ptr(w), _lib.ptr(bias),
                      _lib.ptr(x_conv), B, T, d, code, stream)
            proj = _linear(x_conv, W)  # [B, T, 2HK + HV*V + HV + K]
            off_gd = 2 * H * K + HV * V + HV
            gl = _linear(proj[..., off_gd:off_gd + K], g_up)
            q = torch.empty(B, T, H, K, device=x.device, dtype=x.dtype)
            k = torch.empty_like(q)
            v = torch.empty(B, T, HV, V, device=x.device, dtype=x.dtype)
            g = torch.empty(B, T, HV, K, device=x.device, dtype=x.dtype)
            beta = torch.empty(B, T, HV, device=x.device, dtype=x.dtype)
            _lib.call("kch_kda_gates", _lib.ptr(proj), proj.stride(1), _lib.ptr(gl), gl.stride(1),
                      _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta),
                      B, T, H, HV, K, V, float(cfg.kda_decay_scale), code, stream)
            use_chunk = cfg.kda_chunk_size >= 1 and T >= cfg.kda_chunk_size
            if state_out is not None and not use_chunk:
                # the recurrent kernel reads and writes each state element in the
                # same thread, so the state may be updated in place
                if T > 0 and B > 0 and (state is None or state.data_ptr() == state_out.data_ptr()) \
                        and state_out.dtype == torch.float32 and state_out.is_contiguous() \
                        and state_out.shape == (B, HV, K, V) and state_out.device == x.device:
                    # q, k, v, g, beta are this layer's own kch_kda_gates outputs
                    o = _recurrent_launch(q, k, v, g, beta, self._scale_value(), state,
                                          state_out, code, stream)
                else:
                    o = kda_recurrent_into(q, k, v, g, beta, self._scale_value(), state,
                                           state_out)
                new_state = state_out
            else:
                o, new_state = kda_forward(
                    q, k, v, g, beta, scale=self._scale_value(), initial_state=state,
                    output_final_state=True, chunk_size=max(cfg.kda_chunk_size, 1),
                    use_chunk=use_chunk, backend=cfg.kda_backend)
                if state_out is not None:
                    state_out.copy_(new_state)
                    new_state = state_out
            o2 = o.reshape(B, T, HV * V)
            out = (_linear(o2, self.o_proj.weight) if residual is None
                   else _linear_residual(o2, self.o_proj.weight, residual))
        return out, new_state, new_lookback

    def _forward_grad(self, x, state, lookback, detach_lookback):
        """The same layer with gradients: the conv and the activations through
        their HIP backward kernels, the projections through autograd (library
        GEMMs), the KDA operator through ``kch_kda_recurrent_bwd``."""
        B, T, d = x.shape
        cfg = self.cfg
        H, K, V, HV = cfg.n_heads_qk, cfg.head_dim_k, cfg.head_dim_v, cfg.n_heads_v
        if T >= _CONV_K - 1:
            new_lookback = x[:, -(_CONV_K - 1):]
        elif lookback is not None:
            new_lookback = torch.cat([lookback[:, T:], x], dim=1)
        else:
            new_lookback = torch.cat([x.new_zeros(B, _CONV_K - 1 - T, d), x], dim=1)
        if detach_lookback:
            new_lookback = new_lookback.detach()
        new_lookback = new_lookback.clone()
        x_conv = _ShortConvFn.apply(x, self.short_conv.weight, self.short_conv.bias, lookback)
        W = torch.cat([self.q_proj.weight, self.k_proj.weight, self.v_proj.weight,
                       self.beta.weight, self.g_down.weight], 0).to(x.dtype)
        proj = F.linear(x_conv, W)
        off_gd = 2 * H * K + HV * V + HV
        gl = F.linear(proj[..., off_gd:off_gd + K], self.g_up.weight.to(x.dtype))
        q, k, v, g, beta = _KdaGatesFn.apply(proj, gl, (H, HV, K, V, float(cfg.kda_decay_scale)))
        use_chunk = cfg.kda_chunk_size >= 1 and T >= cfg.kda_chunk_size
        st = None if state is None else state.to(device=x.device, dtype=torch.float32)
        if use_chunk:
            o, new_state = naive_chunk_kda(q, k, v, g, beta, scale=self._scale_value(),
                                           initial_state=st, output_final_state=True,
                                           chunk_size=cfg.kda_chunk_size)
        else:
            o, new_state = naive_recurrent_kda(q, k, v, g, beta, scale=self._scale_value(),
                                               initial_state=st, output_final_state=True)
        out = F.linear(o.reshape(B, T, HV * V), self.o_proj.weight.to(x.dtype))
        return out, new_state, new_lookback


def _out_proj(o_proj: nn.Linear, o: torch.Tensor, residual: torch.Tensor | None):
    """``o_proj(o)``, or ``residual + o_proj(o)``: fused into one GEMM when no
    gradient is taken."""
    if residual is None:
        return o_proj(o)
    if _grad_wanted(o, residual, o_proj.weight):
        return residual + o_proj(o)
    return _linear_residual(o, o_proj.weight, residual)


class CSAHybridLayer(_FusedWeightLayer):
    """CSA sub-layer (``ops_fused.py:612-713``): ``naive_csa`` then ``o_proj``."""

    _indexer_warned = False

    def __init__(self, cfg: HybridConfig):
        super().__init__()
        self.cfg = cfg
        d, c = cfg.d_model, cfg.csa_c
        self.W_aKV = nn.Linear(d, c, bias=False)
        self.W_bKV = nn.Linear(d, c, bias=False)
        self.W_aZ = nn.Linear(d, c, bias=False)
        self.W_bZ = nn.Linear(d, c, bias=False)
        self.Ba = nn.Parameter(torch.randn(cfg.csa_m, c) * cfg.init_std)
        self.Bb = nn.Parameter(torch.randn(cfg.csa_m, c) * cfg.init_std)
        self.W_DQ = nn.Linear(d, cfg.csa_dc, bias=False)
        self.W_UQ = nn.Linear(cfg.csa_dc, c * cfg.csa_nh, bias=False)
        self.W_IUQ = nn.Linear(cfg.csa_dc, cfg.csa_cI * cfg.csa_nIh, bias=False)
        self.W_w = nn.Linear(d, cfg.csa_nIh, bias=False)
        self.W_KV_idx = nn.Linear(d, cfg.csa_cI, bias=False)
        self.W_Z_idx = nn.Linear(d, cfg.csa_cI, bias=False)
        self.B_idx = nn.Parameter(torch.randn(cfg.csa_m, cfg.csa_cI) * cfg.init_std)
        self.sink = nn.Parameter(torch.zeros(cfg.csa_nh))
        self.o_proj = nn.Linear(c * cfg.csa_nh, d, bias=False)
        self.indexer_is_trained = True
        self.use_ste = True

    @classmethod
    def reset_warned(cls):
        cls._indexer_warned = False

    def _step_weights(self, dtype, device):
        """Operands of the device-driven decode step: the projection weight
        [W_aKV; W_bKV; W_aZ; W_bZ; W_KV_idx; W_Z_idx; W_DQ; W_w], the query
        up-projection [W_UQ; W_IUQ], and fp32 Ba, Bb, B_idx and sink."""
        proj = [self.W_aKV.weight, self.W_bKV.weight, self.W_aZ.weight, self.W_bZ.weight,
                self.W_KV_idx.weight, self.W_Z_idx.weight, self.W_DQ.weight, self.W_w.weight]
        up = [self.W_UQ.weight, self.W_IUQ.weight]
        small = [self.Ba, self.Bb, self.B_idx, self.sink]

        def build():
            cat = lambda ps: torch.cat([p.detach() for p in ps], 0).to(device=device, dtype=dtype)  # noqa: E731
            return (cat(proj), cat(up)) + tuple(
                p.detach().to(device=device, dtype=torch.float32).contiguous() for p in small)
        return self._fused_step.get(proj + up + small, dtype, device, build)

    def _maybe_warn_indexer(self):
        # only with STE explicitly disabled (ops_fused.py:678-692)
        if not self.indexer_is_trained and not CSAHybridLayer._indexer_warned:
            warnings.warn(
                "CSAHybridLayer: STE is disabled (use_ste=False), so the lightning indexer "
                "parameters (W_IUQ, W_w, W_KV_idx, W_Z_idx, B_idx) will NOT be trained.",
                stacklevel=3)
            CSAHybridLayer._indexer_warned = True

    def forward(self, x: torch.Tensor, state: torch.Tensor | None = None, *,
                residual: torch.Tensor | None = None):
        """``(o_proj(naive_csa(x)), None)``; with ``residual`` the first item is
        ``residual + o_proj(...)`` (the add fused into the GEMM without gradients)."""
        cfg = self.cfg
        if self.training and not self.use_ste:
            self._maybe_warn_indexer()
        # the operator takes its gradient path when autograd asks for one
        with torch.set_grad_enabled(torch.is_grad_enabled()):
            o = naive_csa(
                x, self.W_aKV.weight, self.W_bKV.weight, self.W_aZ.weight, self.W_bZ.weight,
                self.Ba, self.Bb, self.W_DQ.weight, self.W_UQ.weight, self.W_IUQ.weight,
                self.W_w.weight, self.W_KV_idx.weight, self.W_Z_idx.weight, self.B_idx,
                m=cfg.csa_m, topk=cfg.csa_topk, nh=cfg.csa_nh, nIh=cfg.csa_nIh, c=cfg.csa_c,
                c_I=cfg.csa_cI, dc=cfg.csa_dc, sliding_window=cfg.csa_sliding_window,
                sink_logits=self.sink, use_ste=self.use_ste, normalize_qk=True)
            return _out_proj(self.o_proj, o, residual), None


class HCAHybridLayer(_FusedWeightLayer):
    """HCA sub-layer (``ops_fused.py:716-739``): ``naive_hca`` then ``o_proj``."""

    def __init__(self, cfg: HybridConfig):
        super().__init__()
        self.cfg = cfg
        d, c = cfg.d_model, cfg.hca_c
        self.W_KV = nn.Linear(d, c, bias=False)
        self.W_Z = nn.Linear(d, c, bias=False)
        self.B_pos = nn.Parameter(torch.randn(cfg.hca_m2, c) * cfg.init_std)
        self.W_DQ = nn.Linear(d, cfg.hca_dc, bias=False)
        self.W_UQ = nn.Linear(cfg.hca_dc, c * cfg.hca_nh, bias=False)
        self.sink = nn.Parameter(torch.zeros(cfg.hca_nh))
        self.o_proj = nn.Linear(c * cfg.hca_nh, d, bias=False)

    def _step_weights(self, dtype, device):
        """Operands of the device-driven decode step: [W_KV; W_Z; W_DQ], W_UQ,
        and fp32 B_pos and sink."""
        proj = [self.W_KV.weight, self.W_Z.weight, self.W_DQ.weight]
        small = [self.B_pos, self.sink]

        def build():
            W = torch.cat([p.detach() for p in proj], 0).to(device=device, dtype=dtype)
            return (W, self.W_UQ.weight.detach().to(device=device, dtype=dtype).contiguous()) + \
                tuple(p.detach().to(device=device, dtype=torch.float32).contiguous() for p in small)
        return self._fused_step.get(proj + [self.W_UQ.weight] + small, dtype, device, build)

    def forward(self, x: torch.Tensor, state: torch.Tensor | None = None, *,
                residual: torch.Tensor | None = None):
        """``(o_proj(naive_hca(x)), None)``; with ``residual`` the first item is
        ``residual + o_proj(...)`` (the add fused into the GEMM without gradients)."""
        cfg = self.cfg
        with torch.set_grad_enabled(torch.is_grad_enabled()):
            o = naive_hca(x, self.W_KV.weight, self.W_Z.weight, self.B_pos, self.W_DQ.weight,
                          self.W_UQ.weight, m2=cfg.hca_m2, nh=cfg.hca_nh, c=cfg.hca_c,
                          dc=cfg.hca_dc, sliding_window=cfg.hca_sliding_window,
                          sink_logits=self.sink)
            return _out_proj(self.o_proj, o, residual), None


class HybridKCHAttention(nn.Module):
    """Stack of KDA / CSA / HCA sub-layers (``ops_fused.py:742-1131``).

    Layout ``[KDA * n_kda, CSA * n_csa, HCA * n_hca]`` repeated and cut to
    ``total_layers``; every sub-layer is ``x + layer(LayerNorm_fp32(x))``;
    one recurrent state and one conv lookback per KDA layer.
    """

    LAYER_TYPES = ('kda', 'csa', 'hca')
    _stateful_warned = False

    def __init__(self, cfg: HybridConfig, total_layers: int = 5):
        super().__init__()
        self.cfg = cfg
        if not isinstance(total_layers, int) or total_layers < 0:
            raise ValueError(f"total_layers={total_layers!r} must be a non-negative int "
                             f"(0 produces an empty no-op model).")
        self.total_layers = total_layers
        if total_layers > 0 and cfg.n_kda == 0 and cfg.n_csa == 0 and cfg.n_hca == 0:
            raise ValueError(
                "HybridKCHAttention requires at least one non-zero layer count (n_kda, n_csa, "
                f"n_hca); got ({cfg.n_kda}, {cfg.n_csa}, {cfg.n_hca}) with "
                f"total_layers={total_layers}.")
        self.layout = self._build_layout()
        kinds = {'kda': KDAHybridLayer, 'csa': CSAHybridLayer, 'hca': HCAHybridLayer}
        self.layers = nn.ModuleList([kinds[k](cfg) for k in self.layout])
        self.norms = nn.ModuleList([_Fp32LayerNorm(cfg.d_model) for _ in self.layout])
        self.n_kda_layers = sum(1 for k in self.layout if k == 'kda')
        self.register_buffer('_kda_state', None, persistent=False)

    def _build_layout(self) -> list[str]:
        unit = (['kda'] * self.cfg.n_kda + ['csa'] * self.cfg.n_csa + ['hca'] * self.cfg.n_hca)
        if not unit and self.total_layers > 0:
            raise ValueError("_build_layout: cannot build a non-empty layout from an empty "
                             "repeating unit (n_kda=n_csa=n_hca=0).")
        layout: list[str] = []
        while len(layout) < self.total_layers:
            layout.extend(unit)
        return layout[:self.total_layers]

    def layout_str(self) -> str:
        return '-'.join(s.upper() for s in self.layout)

    def reset_state(self) -> None:
        """Clear the KDA states and every KDA layer's conv lookback (``ops_fused.py:856-885``)."""
        self._kda_state = None
        for layer in self.layers:
            if isinstance(layer, KDAHybridLayer):
                layer.reset_conv_state()
        HybridKCHAttention._stateful_warned = False

    def _kda_layers(self):
        return [layer for layer in self.layers if isinstance(layer, KDAHybridLayer)]

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Stateful forward: reads and writes the KDA states and conv lookbacks."""
        if self.training and not HybridKCHAttention._stateful_warned:
            warnings.warn(
                "HybridKCHAttention.forward() mutates self._kda_state and per-layer "
                "_conv_lookback buffers; use forward_functional() for code that must not "
                "share module state.", stacklevel=2)
            HybridKCHAttention._stateful_warned = True
        kda = self._kda_layers()
        o, new_state, new_lbs = self.forward_functional(
            x, self._kda_state, [layer._conv_lookback for layer in kda])
        self._kda_state = new_state
        for layer, lb in zip(kda, new_lbs):
            layer._conv_lookback = lb
        return o

    def _unstack_states(self, kda_state, B, device, detach_state=True):
        stacked = kda_state
        if stacked is not None:
            if stacked.shape[1] != B:
                logger.debug("HybridKCHAttention: dropping KDA state (batch %d -> %d)",
                             stacked.shape[1], B)
                stacked = None
            else:
                stacked = stacked.to(device=device)
                if detach_state:
                    stacked = stacked.detach()
        if stacked is None:
            return [None] * self.n_kda_layers
        if stacked.shape[0] != self.n_kda_layers:
            raise ValueError(
                f"HybridKCHAttention.forward_functional: stacked KDA state has "
                f"{stacked.shape[0]} layers but the model has {self.n_kda_layers} KDA layers.")
        return list(stacked.unbind(0))

    def _stack_states(self, states):
        if self.n_kda_layers == 0:
            return None
        if any(s is None for s in states):
            raise RuntimeError("HybridKCHAttention: a KDA layer returned new_state=None.")
        ref = tuple(states[0].shape)
        for i, s in enumerate(states):
            if tuple(s.shape) != ref:
                raise RuntimeError(f"HybridKCHAttention: KDA layer {i} returned new_state with "
                                   f"shape {tuple(s.shape)}, layer 0 returned {ref}.")
        return torch.stack(states, dim=0)

    def forward_functional(self, x: torch.Tensor, kda_state: torch.Tensor | None,
                           conv_lookbacks: list, *, detach_state: bool = True,
                           detach_lookback: bool = True):
        """Pure forward (``ops_fused.py:956-1128``).

        Returns ``(output [B,T,d], new_kda_state [n_kda,B,HV,K,V] | None, new_conv_lookbacks)``.
        """
        states = self._unstack_states(kda_state, x.shape[0], x.device, detach_state)
        lookbacks = list(conv_lookbacks)
        if len(lookbacks) != self.n_kda_layers:
            raise ValueError(
                f"HybridKCHAttention.forward_functional: conv_lookbacks has length "
                f"{len(lookbacks)} but the model has {self.n_kda_layers} KDA layers.")
        kda_idx = 0
        new_lookbacks = []
        grad = _grad_wanted(x, *lookbacks, *self.parameters())
        with torch.set_grad_enabled(grad):
            for layer, norm, kind in zip(self.layers, self.norms, self.layout):
                # without gradients each sub-layer's output projection adds the
                # residual stream in its GEMM
                residual = None if grad else x
                h = norm(x)
                if kind == 'kda':
                    o, st, lb = layer.forward_functional(h, states[kda_idx], lookbacks[kda_idx],
                                                         detach_lookback=detach_lookback,
                                                         residual=residual)
                    states[kda_idx] = st
                    new_lookbacks.append(lb)
                    kda_idx += 1
                else:
                    o, _ = layer(h, None, residual=residual)
                x = o if residual is not None else x + o
            return x, self._stack_states(states), new_lookbacks


def _pad8(n: int) -> int:
    return (n + 7) & ~7


class _StepGraph:
    """A captured device-driven decode step, the buffers it replays on, and
    what a later step checks before replaying it: the input's shape, the
    tensors and caches it was captured on, every parameter's storage and
    in-place version, the fused weight copies, the modules whose hooks would
    send the step elsewhere, and the caches' block capacities."""

    def __init__(self, key, graph, xin, xout, idx_bufs):
        self.key, self.graph, self.xin, self.xout, self.idx_bufs = key, graph, xin, xout, idx_bufs
        self.stacked = None
        self.model = None
        self.watch = ()       # (param, data_ptr, _version)
        self.fused = ()       # (_FusedWeight, the copy it held at capture)
        self.lookbacks = ()   # (layer, lookback tensor)
        self.caches = ()      # (cache, its buffers, block capacity)
        self.hook_modules = ()


class HybridDecoding(nn.Module):
    """Hybrid stack with one decode cache per CSA / HCA sub-layer
    (``run_decoding.py:601-851``), for any ``HybridConfig``.

    ``forward(x)`` with T > 1 is a prefill: the full operators produce the
    output and their projections populate the caches in bulk; T == 1 is a
    decode step through the caches and the KDA recurrent state.

    Without ``cfg``: the reference's own decode geometry
    (``run_decoding.py:642-656``: 2 x 16 KDA heads on the recurrent path, CSA
    and HCA with 2 heads of 8, c_I = 4, one indexer head, m = m' = 4, windows
    of 4) with the backend from ``KDA_BACKEND`` (default ``"hip"``). Its head
    dims run zero-padded to the kernels' sizes.

    Decode steps on bf16 models whose sizes the step kernels take run the
    device-driven step: per sub-layer a norm-fused projection, the KDA
    front end and fused activation + recurrence kernels, the one-token cache
    append and the cache attention, and an output projection fused with the
    residual add, every per-step count (blocks, window, slots) read from one
    device counter of cached tokens. ``use_graphs`` (default on) captures that
    step once in a HIP graph and replays it on every later step; the graph is
    captured again when the batch, a parameter (address or in-place version),
    a fused weight copy, the KDA state or lookback buffers, or a cache buffer
    (which grows by doubling) change. Results are the eager step's, launch for
    launch. ``fused_decode = False`` keeps every step on the per-operator path
    of ``_forward_csa_layer`` / ``_forward_hca_layer``, as do models with
    forward hooks on the modules that path calls (the norms, the KDA layers).
    """

    def __init__(self, d_model: int = 64, total_layers: int = 5, csa_topk: int = 2, *,
                 cfg: HybridConfig | None = None, use_graphs: bool = True):
        super().__init__()
        self.use_graphs = use_graphs
        self.fused_decode = True
        self._graph = None
        self._n_dev = None        # device int32 [1]: tokens the caches held before the step
        self._n_dev_host = None   # the value it holds, None when unknown
        self._trace = None        # list: per call, the stream entering each sub-layer
        self._device_steps = 0    # decode steps run on the device-driven kernels
        self._graph_captures = 0
        if cfg is None:
            cfg = HybridConfig(
                d_model=d_model, n_heads_qk=2, n_heads_v=2, head_dim_k=16, head_dim_v=16,
                kda_chunk_size=0,
                kda_backend=validate_kda_backend(os.environ.get('KDA_BACKEND', 'hip')),
                csa_m=4, csa_topk=csa_topk, csa_nh=2, csa_c=8, csa_dc=8, csa_nIh=1, csa_cI=4,
                csa_sliding_window=4, hca_m2=4, hca_nh=2, hca_c=8, hca_dc=8,
                hca_sliding_window=4, n_kda=3, n_csa=1, n_hca=1)
        self.cfg = cfg
        self.model = HybridKCHAttention(cfg, total_layers=total_layers)
        self._csa_caches: list = [None for k in self.model.layout if k == 'csa']
        self._hca_caches: list = [None for k in self.model.layout if k == 'hca']

    def reset(self):
        self.model.reset_state()
        self._csa_caches = [None for _ in self._csa_caches]
        self._hca_caches = [None for _ in self._hca_caches]
        self._graph = None
        self._n_dev_host = None

    def _apply(self, fn, *args, **kwargs):
        self._graph = None
        self._n_dev = None
        self._n_dev_host = None
        return super()._apply(fn, *args, **kwargs)

    # ---------------- device-driven decode step ----------------
    def _called_modules(self):
        """The modules the per-operator decode step calls as modules (the norms
        and the KDA layers; the CSA / HCA layers' weights are used directly)."""
        model = self.model
        return list(model.norms) + [l for l, k in zip(model.layers, model.layout) if k == 'kda']

    def _caches(self):
        return self._csa_caches + self._hca_caches

    def _device_step_ok(self, x: torch.Tensor, stacked) -> bool:
        """Whether this decode step can run on the device-driven kernels."""
        if not (self.fused_decode and x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 3
                and x.shape[1] == 1 and 1 <= x.shape[0] <= 16):
            return False
        if _nn_module._global_forward_hooks or _nn_module._global_forward_pre_hooks \
                or any(m._forward_hooks or m._forward_pre_hooks for m in self._called_modules()):
            return False
        cfg, model = self.cfg, self.model
        B, d = x.shape[0], cfg.d_model
        if d % 32 or d > 4096 or B * d > 32768:
            return False
        for n in model.norms:
            if n.weight is None or len(n.normalized_shape) != 1 or \
                    (n.bias is not None and n.bias.dtype != n.weight.dtype):
                return False
        if model.n_kda_layers:
            H, HV, K, V = cfg.n_heads_qk, cfg.n_heads_v, cfg.head_dim_k, cfg.head_dim_v
            if stacked is None or tuple(stacked.shape) != (model.n_kda_layers, B, HV, K, V) \
                    or stacked.dtype != torch.float32 or not stacked.is_contiguous() \
                    or stacked.device != x.device:
                return False
            if K not in (16, 32, 64, 128, 256) or V % 32 or HV % H:
                return False
            for layer, kind in zip(model.layers, model.layout):
                if kind != 'kda':
                    continue
                lb = layer._conv_lookback
                if lb is None or tuple(lb.shape) != (B, 2, d) or lb.dtype != x.dtype \
                        or lb.device != x.device or not lb.is_contiguous() or lb.data_ptr() % 16:
                    return False
        if 'csa' in model.layout:
            c, cI, nIh, nh = cfg.csa_c, cfg.csa_cI, cfg.csa_nIh, cfg.csa_nh
            if c not in (64, 128) or cI not in (32, 64, 128) or nIh not in (1, 2, 4, 8, 16) \
                    or nh > 16 or cfg.csa_topk < 1 or cfg.csa_dc % 32 or c + cI > 256:
                return False
        if 'hca' in model.layout:
            if cfg.hca_c not in (64, 128) or cfg.hca_nh > 16 or cfg.hca_dc % 32:
                return False
        for cache in self._caches():
            if cache is None or cache.B != B or cache.device != x.device \
                    or not cache._device_ready(x.dtype):
                return False
        return True

    def _sync_counter(self, device) -> bool:
        """The device token counter holds the caches' common token count."""
        caches = self._caches()
        if not caches:
            return True
        n = caches[0].n_tokens_seen
        if any(c.n_tokens_seen != n for c in caches):
            return False
        if self._n_dev is None or self._n_dev.device != device:
            self._n_dev = torch.zeros(1, device=device, dtype=torch.int32)
            self._n_dev_host = 0
        if self._n_dev_host != n:
            self._n_dev.fill_(n)
            self._n_dev_host = n
        return True

    def _step_operands(self, dtype, device):
        """Every operand of the step that is not a parameter itself, built (or
        taken from the layers' caches) outside any capture."""
        ops = []
        for layer, kind in zip(self.model.layers, self.model.layout):
            ops.append(layer._weights(dtype, device) if kind == 'kda'
                       else layer._step_weights(dtype, device))
        return ops

    def _step_key(self, x, stacked, caps, ops):
        def ptrs(ts):
            return tuple(0 if t is None else t.data_ptr() for t in ts)
        model = self.model
        key = [tuple(x.shape), x.dtype, x.device, ptrs([stacked, self._n_dev]), tuple(caps)]
        key += [ptrs(op) for op in ops]
        key += [(p.data_ptr(), p._version) for p in model.parameters()]
        key += [ptrs([layer._conv_lookback]) for layer, k in zip(model.layers, model.layout)
                if k == 'kda']
        for cache in self._caches():
            key.append(ptrs(self._cache_bufs(cache)))
        return tuple(key)

    def _prepare_caches(self):
        """Room for the block this token may complete, in every cache; returns
        the block capacities (the CSA stores share one)."""
        caps = []
        for cache in self._caches():
            cap = cache._device_buffers()
            if isinstance(cache, CSADecodingCache):
                # the append kernel addresses both stores with one block stride
                cap = max(cache._C.rows.shape[1], cache._K.rows.shape[1])
                cache._C.ensure(cache.n_blocks, cap)
                cache._K.ensure(cache.n_blocks, cap)
            caps.append(cap)
        return caps

    def _device_step(self, x: torch.Tensor, stacked, caps, ops):
        """One token (``x`` ``[B, 1, d]``) through every sub-layer on the
        device-driven kernels. Returns the output ``[B, 1, d]`` and the CSA
        selections ``[B, topk]``; records the sub-layers' inputs when tracing."""
        model, cfg = self.model, self.cfg
        B, _, d = x.shape
        dt, dev = x.dtype, x.device
        code = _lib.dtype_code("HybridDecoding", dt)
        stream = _lib.stream_of(x)
        lib = _lib.load()
        x_cur = x.reshape(B, d)
        if x_cur.stride(1) != 1 or x_cur.stride(0) % 8 or x_cur.data_ptr() % 16:
            x_cur = x_cur.contiguous()
        n_dev = self._n_dev if self._caches() else None
        trace = [] if self._trace is not None else None
        idx_bufs = []
        csa_i = hca_i = kda_i = 0
        n_layers = len(model.layers)

        def linear(xin, ldx, w, y, ldy, *, norm=None, res=None, counter=None):
            ln_w = ln_b = None
            eps, wcode = 0.0, 0
            if norm is not None:
                ln_w, ln_b, eps = norm.weight, norm.bias, float(norm.eps)
                wcode = _lib.dtype_code("HybridDecoding", ln_w.dtype)
            N, K = w.shape
            _lib.call("kch_linear_rows_fused", _lib.ptr(xin), ldx, _lib.ptr(w), K, _lib.ptr(y),
                      ldy, B, N, K, _lib.ptr(ln_w), _lib.ptr(ln_b), eps, wcode, _lib.ptr(res),
                      0 if res is None else res.stride(0), _lib.ptr(counter), code, stream)
            return y

        for li, (layer, norm, kind) in enumerate(zip(model.layers, model.norms, model.layout)):
            if trace is not None:
                trace.append(x_cur.view(B, 1, d).clone())
            counter = n_dev if li == n_layers - 1 else None
            op = ops[li]
            if kind == 'kda':
                H, HV, K, V = cfg.n_heads_qk, cfg.n_heads_v, cfg.head_dim_k, cfg.head_dim_v
                W, w_conv, b_conv, g_up = op
                ln_w, ln_b = norm.weight, norm.bias
                NP = _pad8(W.shape[0])
                # the front (LayerNorm + conv over [lookback ; h]) in the
                # projection's prologue; the step kernel then advances the
                # lookback from h
                h = torch.empty(B, d, device=dev, dtype=dt)
                proj = torch.empty(B, NP, device=dev, dtype=dt)
                _lib.call("kch_kda_front_rows", _lib.ptr(x_cur), x_cur.stride(0), _lib.ptr(ln_w),
                          _lib.ptr(ln_b), float(norm.eps),
                          _lib.dtype_code("HybridDecoding", ln_w.dtype),
                          _lib.ptr(layer._conv_lookback), _lib.ptr(w_conv), _lib.ptr(b_conv),
                          _lib.ptr(h), _lib.ptr(W), W.shape[1], _lib.ptr(proj), NP, B,
                          W.shape[0], d, code, stream)
                o = torch.empty(B, HV * V, device=dev, dtype=dt)
                _lib.call("kch_kda_decode_step_shift", _lib.ptr(proj), NP, _lib.ptr(g_up),
                          _lib.ptr(stacked[kda_i]), _lib.ptr(o), B, H, HV, K, V,
                          layer._scale_value(), float(cfg.kda_decay_scale), -10.0,
                          _lib.ptr(layer._conv_lookback), _lib.ptr(h), d, code, stream)
                kda_i += 1
            else:
                csa = kind == 'csa'
                if csa:
                    cache = self._csa_caches[csa_i]
                    cap = caps[csa_i]
                    c, nh, dc = cfg.csa_c, cfg.csa_nh, cfg.csa_dc
                    Wp, Wq, Ba, Bb, Bk, sink = op
                else:
                    cache = self._hca_caches[hca_i]
                    cap = caps[len(self._csa_caches) + hca_i]
                    c, nh, dc = cfg.hca_c, cfg.hca_nh, cfg.hca_dc
                    Wp, Wq, Bpos, sink = op
                NP, NQ = _pad8(Wp.shape[0]), _pad8(Wq.shape[0])
                P = linear(x_cur, x_cur.stride(0), Wp, torch.empty(B, NP, device=dev, dtype=dt),
                           NP, norm=norm)
                off_cq = 4 * c + 2 * cfg.csa_cI if csa else 2 * c
                # the query up-projection Q = P[:, cq] Wq^T runs in the cache
                # append's launch (both read only P)
                Q = torch.empty(B, NQ, device=dev, dtype=dt)
                NW, KW = Wq.shape
                q_rows = (_lib.ptr(P[:, off_cq:]), NP, _lib.ptr(Wq), KW, _lib.ptr(Q), NQ, NW, KW)
                sw = cache._sw
                ring = None if sw is None else sw._buf
                win = 0 if sw is None else sw.win
                normalize = int(bool(cache._C.key_norm))
                out = torch.empty(B, nh * c, device=dev, dtype=dt)
                if csa:
                    cI, nIh, topk, m = cfg.csa_cI, cfg.csa_nIh, cfg.csa_topk, cfg.csa_m
                    _lib.call("kch_csa_cache_append_rows", _lib.ptr(P), NP,
                              _lib.ptr(cache._acc_buf), _lib.ptr(cache._prev_buf), _lib.ptr(Ba),
                              _lib.ptr(Bb), _lib.ptr(Bk), _lib.ptr(ring), _lib.ptr(cache._C.rows),
                              _lib.ptr(cache._C.keys), _lib.ptr(cache._K.rows),
                              _lib.ptr(cache._K.inv), _lib.ptr(n_dev), B, c, cI, m, win, cap,
                              normalize, *q_rows, code, stream)
                    nbytes = lib.kch_decode_dyn_ws_bytes(B, cap, nh, c, topk, win, 1)
                    ws = torch.empty(max(nbytes, 256), device=dev, dtype=torch.uint8)
                    idx = torch.empty(B, topk, device=dev, dtype=torch.int32)
                    _lib.call("kch_csa_decode_dyn", _lib.ptr(Q), NQ, _lib.ptr(Q[:, nh * c:]), NQ,
                              _lib.ptr(P[:, off_cq + dc:]), NP, _lib.ptr(cache._C.keys), cap * c,
                              _lib.ptr(cache._K.rows), cap * cI, _lib.ptr(cache._K.inv), cap,
                              _lib.ptr(ring), win * c, _lib.ptr(n_dev), m, win, cap,
                              _lib.ptr(sink), _lib.ptr(out), _lib.ptr(idx), B, nh, c, nIh, cI,
                              topk, 1.0, 1.0, 1, 1, code, code, code, _lib.ptr(ws), ws.numel(),
                              stream)
                    idx_bufs.append(idx)
                    csa_i += 1
                else:
                    m2 = cfg.hca_m2
                    _lib.call("kch_hca_cache_append_rows", _lib.ptr(P), NP,
                              _lib.ptr(cache._acc_buf), _lib.ptr(Bpos), _lib.ptr(ring),
                              _lib.ptr(cache._C.rows), _lib.ptr(cache._C.keys), _lib.ptr(n_dev),
                              B, c, m2, win, cap, normalize, *q_rows, code, stream)
                    nbytes = lib.kch_decode_dyn_ws_bytes(B, cap, nh, c, 0, win, 0)
                    ws = torch.empty(max(nbytes, 256), device=dev, dtype=torch.uint8)
                    _lib.call("kch_hca_decode_dyn", _lib.ptr(Q), NQ, _lib.ptr(cache._C.keys),
                              cap * c, _lib.ptr(ring), win * c, _lib.ptr(n_dev), m2, win, cap,
                              _lib.ptr(sink), _lib.ptr(out), B, nh, c, 1.0, 1, code, code,
                              _lib.ptr(ws), ws.numel(), stream)
                    hca_i += 1
                o = out
            x_cur = linear(o, o.stride(0), layer.o_proj.weight,
                           torch.empty(B, d, device=dev, dtype=dt), d, res=x_cur,
                           counter=counter)
        return x_cur.view(B, 1, d), idx_bufs, trace

    def _after_device_step(self, idx_bufs, B) -> None:
        """Host bookkeeping of a device step: the caches' counters, the
        selections for ``record_selections``."""
        self._device_steps += 1
        for cache in self._caches():
            cache._device_advance()
        if self._caches():
            self._n_dev_host += 1
        for cache, idx in zip(self._csa_caches, idx_bufs):
            cache._last_indices = idx
            if ops_csa._selection_log is not None:
                ops_csa._log_selection(idx.clone().view(B, 1, -1))

    @staticmethod
    def _cache_bufs(cache):
        K = getattr(cache, '_K', None)
        return (None if cache._sw is None else cache._sw._buf, cache._acc_buf,
                getattr(cache, '_prev_buf', None), cache._C.rows, cache._C.keys,
                None if K is None else K.rows, None if K is None else K.inv)

    def _graph_still_valid(self, g: _StepGraph, x: torch.Tensor, stacked) -> bool:
        """Whether the captured step replays correctly for this step (cheap
        checks of everything it was captured on); otherwise the full path
        re-checks, re-synchronises and captures again."""
        if not (self.use_graphs and self.fused_decode and self._trace is None
                and ops_csa._selection_log is None):
            return False
        if x.shape != g.xin.shape or x.dtype != g.xin.dtype or x.device != g.xin.device \
                or stacked is not g.stacked or self.model is not g.model:
            return False
        if _nn_module._global_forward_hooks or _nn_module._global_forward_pre_hooks:
            return False
        for m in g.hook_modules:
            if m._forward_hooks or m._forward_pre_hooks:
                return False
        for p, ptr, ver in g.watch:
            if p._version != ver or p.data_ptr() != ptr:
                return False
        for fw, w in g.fused:
            if fw._w is not w:
                return False
        for layer, lb in g.lookbacks:
            if layer._conv_lookback is not lb:
                return False
        caches = self._caches()
        if len(caches) != len(g.caches):
            return False
        n = self._n_dev_host
        for cache, (c0, bufs, cap) in zip(caches, g.caches):
            if cache is not c0 or cache.n_tokens_seen != n:
                return False
            m = cache.m if isinstance(cache, CSADecodingCache) else cache.m2
            if n // m >= cap:
                return False  # the block this token completes needs more room
            for a, b in zip(self._cache_bufs(cache), bufs):
                if a is not b:
                    return False
        return True

    def _forward_device(self, x: torch.Tensor, stacked) -> torch.Tensor | None:
        """The decode step on the device-driven kernels (from the captured graph
        when allowed), or None when the step does not qualify."""
        g = self._graph
        if g is not None and self._graph_still_valid(g, x, stacked):
            with torch.no_grad():
                g.xin.copy_(x)
                g.graph.replay()
                y = g.xout.clone()
            self._after_device_step(g.idx_bufs, x.shape[0])
            return y
        if not self._device_step_ok(x, stacked) or not self._sync_counter(x.device):
            return None
        caps = self._prepare_caches()
        ops = self._step_operands(x.dtype, x.device)
        B = x.shape[0]
        with torch.no_grad():
            if self.use_graphs and self._trace is None and ops_csa._selection_log is None:
                key = self._step_key(x, stacked, caps, ops)
                g = self._graph
                if g is None or g.key != key:
                    self._graph = None
                    xin = x.contiguous().clone()
                    torch.cuda.synchronize(x.device)
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph):
                        y, idx_bufs, _ = self._device_step(xin, stacked, caps, ops)
                    g = self._graph = _StepGraph(key, graph, xin, y, idx_bufs)
                    self._graph_captures += 1
                    model = self.model
                    g.stacked = stacked
                    g.model = model
                    g.watch = tuple((p, p.data_ptr(), p._version) for p in model.parameters())
                    g.fused = tuple((layer._fused if k == 'kda' else layer._fused_step,
                                     ops[i]) for i, (layer, k) in
                                    enumerate(zip(model.layers, model.layout)))
                    g.lookbacks = tuple((layer, layer._conv_lookback) for layer, k in
                                        zip(model.layers, model.layout) if k == 'kda')
                    g.caches = tuple((cache, self._cache_bufs(cache), cap)
                                     for cache, cap in zip(self._caches(), caps))
                    g.hook_modules = tuple(self._called_modules())
                g.xin.copy_(x)
                g.graph.replay()
                y, idx_bufs = g.xout.clone(), g.idx_bufs
            else:
                y, idx_bufs, trace = self._device_step(x, stacked, caps, ops)
                if trace is not None:
                    self._trace.append(trace)
        self._after_device_step(idx_bufs, B)
        return y

    def _ensure_csa_cache(self, idx: int, layer: CSAHybridLayer, h: torch.Tensor):
        cfg = layer.cfg
        cache = self._csa_caches[idx]
        if cache is None or cache.B != h.shape[0] or cache.device != h.device \
                or cache.dtype != h.dtype:
            cache = CSADecodingCache(h.shape[0], cfg.csa_c, cfg.csa_cI, cfg.csa_m,
                                     cfg.csa_sliding_window, h.device, h.dtype)
            self._csa_caches[idx] = cache
        return cache

    def _ensure_hca_cache(self, idx: int, layer: HCAHybridLayer, h: torch.Tensor):
        cfg = layer.cfg
        cache = self._hca_caches[idx]
        if cache is None or cache.B != h.shape[0] or cache.device != h.device \
                or cache.dtype != h.dtype:
            cache = HCADecodingCache(h.shape[0], cfg.hca_c, cfg.hca_m2, cfg.hca_sliding_window,
                                     h.device, h.dtype)
            self._hca_caches[idx] = cache
        return cache

    @staticmethod
    def _project_csa(layer: CSAHybridLayer, h: torch.Tensor):
        """The decode-step projections (``run_decoding.py:710-730``) as two GEMMs."""
        cfg = layer.cfg
        B, T, _ = h.shape
        c, cI, nh, nIh, dc = cfg.csa_c, cfg.csa_cI, cfg.csa_nh, cfg.csa_nIh, cfg.csa_dc
        W = layer._fused.get([layer.W_aKV.weight, layer.W_bKV.weight, layer.W_aZ.weight,
                              layer.W_bZ.weight, layer.W_KV_idx.weight, layer.W_Z_idx.weight,
                              layer.W_DQ.weight, layer.W_w.weight], h.dtype, h.device)
        out = _linear(h, W)
        Ca, Cb, Za, Zb, K_idx, Z_idx, cQ, w_idx = out.split([c, c, c, c, cI, cI, dc, nIh], -1)
        q = _linear(cQ, layer.W_UQ.weight).view(B, T, nh, c)
        q_idx = _linear(cQ, layer.W_IUQ.weight).view(B, T, nIh, cI)
        return Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx

    @staticmethod
    def _project_hca(layer: HCAHybridLayer, h: torch.Tensor):
        cfg = layer.cfg
        B, T, _ = h.shape
        W = layer._fused.get([layer.W_KV.weight, layer.W_Z.weight, layer.W_DQ.weight],
                             h.dtype, h.device)
        C, Z, cQ = _linear(h, W).split([cfg.hca_c, cfg.hca_c, cfg.hca_dc], -1)
        q = _linear(cQ, layer.W_UQ.weight).view(B, T, cfg.hca_nh, cfg.hca_c)
        return C, Z, q

    def _forward_csa_layer(self, layer: CSAHybridLayer, h: torch.Tensor, idx: int,
                           residual: torch.Tensor):
        """``residual + o_proj(CSA(h))`` with the cache updated."""
        cfg = layer.cfg
        B, T_new, _ = h.shape
        if T_new == 0:
            return residual.clone()
        cache = self._ensure_csa_cache(idx, layer, h)
        if T_new > 1:
            o_core, (Ca, Cb, Za, Zb, K_idx, Z_idx) = naive_csa(
                h, layer.W_aKV.weight, layer.W_bKV.weight, layer.W_aZ.weight, layer.W_bZ.weight,
                layer.Ba, layer.Bb, layer.W_DQ.weight, layer.W_UQ.weight, layer.W_IUQ.weight,
                layer.W_w.weight, layer.W_KV_idx.weight, layer.W_Z_idx.weight, layer.B_idx,
                m=cfg.csa_m, topk=cfg.csa_topk, nh=cfg.csa_nh, nIh=cfg.csa_nIh, c=cfg.csa_c,
                c_I=cfg.csa_cI, dc=cfg.csa_dc, sliding_window=cfg.csa_sliding_window,
                sink_logits=layer.sink, use_ste=False, normalize_qk=True,
                return_projections=True)
            cache.append_step(Ca, Cb, Za, Zb, K_idx, Z_idx, layer.Ba, layer.Bb, layer.B_idx)
        else:
            Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx = self._project_csa(layer, h)
            cache.append_step(Ca, Cb, Za, Zb, K_idx, Z_idx, layer.Ba, layer.Bb, layer.B_idx)
            # q is L2-normalised in the kernel (F.normalize(q.float()) of the reference)
            o = cache.forward_step(q, q_idx, w_idx, topk=cfg.csa_topk, nh=cfg.csa_nh,
                                   nIh=cfg.csa_nIh, scale=1.0, sink_logits=layer.sink,
                                   use_ste=False, normalize_qk=True, _normalize_q=True,
                                   _out_dtype=h.dtype)
            o_core = o.reshape(B, T_new, cfg.csa_nh * cfg.csa_c)
        return _linear_residual(o_core, layer.o_proj.weight, residual)

    def _forward_hca_layer(self, layer: HCAHybridLayer, h: torch.Tensor, idx: int,
                           residual: torch.Tensor):
        """``residual + o_proj(HCA(h))`` with the cache updated."""
        cfg = layer.cfg
        B, T_new, _ = h.shape
        if T_new == 0:
            return residual.clone()
        cache = self._ensure_hca_cache(idx, layer, h)
        if T_new > 1:
            o_core, (C, Z) = naive_hca(
                h, layer.W_KV.weight, layer.W_Z.weight, layer.B_pos, layer.W_DQ.weight,
                layer.W_UQ.weight, m2=cfg.hca_m2, nh=cfg.hca_nh, c=cfg.hca_c, dc=cfg.hca_dc,
                sliding_window=cfg.hca_sliding_window, sink_logits=layer.sink,
                return_projections=True)
            cache.append_step(C, Z, layer.B_pos)
        else:
            C, Z, q = self._project_hca(layer, h)
            cache.append_step(C, Z, layer.B_pos)
            # q is L2-normalised in the kernel (F.normalize(q.float()) of the reference)
            o = cache.forward_step(q, nh=cfg.hca_nh, scale=1.0, sink_logits=layer.sink,
                                   _normalize_q=True, _out_dtype=h.dtype)
            o_core = o.reshape(B, T_new, cfg.hca_nh * cfg.hca_c)
        return _linear_residual(o_core, layer.o_proj.weight, residual)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B = x.shape[0]
        model = self.model
        stacked = model._kda_state
        fresh = stacked is None or stacked.shape[1] != B
        if not fresh and (stacked.dtype != torch.float32 or stacked.device != x.device
                          or not stacked.is_contiguous()):
            stacked = stacked.to(device=x.device, dtype=torch.float32).contiguous()
        if not fresh and x.shape[1] == 1:
            model._kda_state = stacked
            y = self._forward_device(x, stacked)
            if y is not None:
                return y
        if model.n_kda_layers > 0 and fresh:
            cfg = model.cfg
            # one persistent [L, B, HV, K, V] fp32 state, updated in place by the layers
            stacked = torch.zeros(model.n_kda_layers, B, cfg.n_heads_v, cfg.head_dim_k,
                                  cfg.head_dim_v, device=x.device, dtype=torch.float32)
        kda_idx = csa_idx = hca_idx = 0
        trace = [] if self._trace is not None else None
        with torch.no_grad():
            for layer, norm, kind in zip(model.layers, model.norms, model.layout):
                if trace is not None:
                    trace.append(x.clone())
                h = norm(x)
                # each sub-layer's output projection adds the residual stream x
                if kind == 'kda':
                    st = stacked[kda_idx]
                    x, _ = layer(h, None if fresh else st, state_out=st, residual=x)
                    kda_idx += 1
                elif kind == 'csa':
                    x = self._forward_csa_layer(layer, h, csa_idx, x)
                    csa_idx += 1
                else:
                    x = self._forward_hca_layer(layer, h, hca_idx, x)
                    hca_idx += 1
            model._kda_state = stacked if model.n_kda_layers > 0 else None
        if trace is not None:
            self._trace.append(trace)
        return x


__all__ = ["HybridConfig", "KDAHybridLayer", "CSAHybridLayer", "HCAHybridLayer",
           "HybridKCHAttention", "HybridDecoding"]
