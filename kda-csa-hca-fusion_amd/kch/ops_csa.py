"""CSA operators on the HIP backend (drop-in twins of the reference's ``ops_csa``).

``csa_compress_kv``             <- ``/root/reference/ops_csa.py:198-234``
``csa_compress_kv_overlapped``  <- ``/root/reference/ops_csa.py:237-305``
``csa_lightning_indexer``       <- ``/root/reference/ops_csa.py:330-573`` (forward, soft weights)
``naive_csa``                   <- ``/root/reference/ops_csa.py:576-1184`` (forward and gradients)

Same signatures, argument meaning and validation messages as the reference.
The projections are plain ``F.linear`` GEMMs on the GPU (the reference's own
fused 6-way weight concatenation, ``ops_csa.py:837-850``, extended by
``W_DQ`` and ``W_w`` so that one GEMM reads H once); compression, the
indexer with top-k selection and the joint sparse + window + sink attention
run in ``libkch.so``.

Differences, all documented:

* Gradients: with autograd on and an input that requires grad, ``naive_csa``
  / ``csa_core`` run the projections through autograd (library GEMMs), the
  attention's backward on ``kch_csa_attn_bwd`` with the selection held fixed,
  and with ``use_ste`` the straight-through surrogate of
  ``ops_csa.py:1033-1099`` for the indexer inputs on ``kch_csa_ste_bwd``:
  ``ste_mode='topk_columns'`` and ``'full_softmax'`` (whose dense
  zero-in-forward term adds ``gsum C_comp_n^T`` to the soft weights'
  cotangent and ``soft^T gsum`` to the compressed rows'). ``'aux_contrastive'``
  raises ``NotImplementedError``, as the reference's indexer does. The
  forward value is the hard top-k path either way (the surrogate adds zero).
* Indexer logits are fp32-level: split-operand MFMA products (two fp16
  parts of unit rows, stored chunk-major for the indexer's loads, or three
  bf16 parts of raw rows).
* Exactly-equal indexer logits are ordered by ascending block index (the
  reference's ``torch.topk`` leaves that order unspecified).
* Attention keys/values are the L2-normalised compressed rows rounded to
  bfloat16 (the reference keeps them in fp32); scores and the softmax are fp32.
* float64 inputs, head dims ``c`` or ``c_I`` above 128, more than 16 indexer
  heads and non-standard ``causal_block_mask`` run on the generic SIMT
  kernels (``kch.generic``; float64 computed in float64), forward only:
  gradients through them raise ``NotImplementedError``.
"""

from __future__ import annotations

import contextlib

import torch
import torch.nn.functional as F

from . import _lib, generic

# the top-k selections made while ``record_selections()`` is active, else None
_selection_log = None


@contextlib.contextmanager
def record_selections():
    """Collect the int32 top-k selection (``[B, T, topk]``, -1 = empty slot,
    in no particular order) of every CSA attention computed inside the block:
    ``naive_csa`` / ``csa_core`` and ``CSADecodingCache.forward_step`` (one
    ``[B, 1, topk]`` entry per step), in call order. For tests that check the
    rest of a composed model on the selection this backend made."""
    global _selection_log
    prev, _selection_log = _selection_log, []
    try:
        yield _selection_log
    finally:
        _selection_log = prev


def _log_selection(idx):
    if _selection_log is not None:
        _selection_log.append(idx)


def _check_gpu_dtype(fn, *ts):
    _lib.require_gpu(fn, *ts)
    for t in ts:
        if t is not None and t.dtype == torch.float64:
            raise NotImplementedError(f"{fn}: float64 inputs are not supported by the HIP kernels")


def _rows(x):
    """(tensor, row stride) for a [B, T, c] tensor whose rows may be strided."""
    if (x.dim() == 3 and x.stride(-1) == 1 and x.stride(0) == x.shape[1] * x.stride(1)
            and x.data_ptr() % 16 == 0):
        return x, x.stride(1)
    x = x.contiguous()
    return x, x.shape[-1]


def _aligned(t):
    """Contiguous, 16-byte aligned storage (the kernels read 16-byte vectors)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _f32(t, device):
    return t.detach().to(device=device, dtype=torch.float32).contiguous()


class _DerivedCache:
    """Tensors derived from parameters (a row concatenation, an fp32 copy),
    kept across calls of the functional operators: an entry holds its source
    tensors (so that their storage cannot be reused while it lives) and is
    valid while each is the same object at the same in-place version."""

    def __init__(self, size=16):
        self.size = size
        self.entries = {}  # key -> (sources, versions, value)

    def get(self, key, sources, build):
        versions = tuple(t._version for t in sources)
        hit = self.entries.get(key)
        if hit is not None and hit[1] == versions and all(a is b for a, b in zip(hit[0], sources)):
            return hit[2]
        if len(self.entries) >= self.size:
            self.entries.pop(next(iter(self.entries)))
        value = build()
        self.entries[key] = (tuple(sources), versions, value)
        return value


_derived = _DerivedCache()


def _cat_cached(ws, pad_rows_to=1):
    """``torch.cat(ws, 0)`` (zero rows appended up to a multiple of
    ``pad_rows_to``), built once per set of weights."""
    key = ("cat", pad_rows_to) + tuple(id(w) for w in ws)

    def build():
        W = torch.cat([w.detach() for w in ws], 0)
        extra = (-W.shape[0]) % pad_rows_to
        return F.pad(W, (0, 0, 0, extra)) if extra else W
    return _derived.get(key, ws, build)


def _f32_cached(t, device):
    if t.dtype == torch.float32 and t.is_contiguous() and t.device == device:
        return t.detach()
    return _derived.get(("f32", id(t), device), (t,), lambda: _f32(t, device))


def _linear_up(x, w):
    """``F.linear(x, w)`` of a prefill's query latent x ``[..., K]`` (rows may be
    strided): ``kch_linear_up`` when it applies (bf16 / fp16, K in {32, 64,
    128, 256}, 16-byte aligned rows, at least 512 output columns), else
    ``F.linear``. At M = 131072, K = 128 on MI355X: N = 2048 126 us against
    183 us for ``F.linear``; N = 256 28 us against 27 us."""
    K = x.shape[-1]
    N = w.shape[0]
    x2 = x.reshape(-1, K) if x.dim() != 2 else x
    if not (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and w.dtype == x.dtype
            and K in (32, 64, 128, 256) and w.dim() == 2 and w.shape[1] == K and N >= 512
            and x2.stride(-1) == 1 and x2.stride(0) % 8 == 0 and x2.data_ptr() % 16 == 0):
        return F.linear(x, w)
    wc = w if (w.is_contiguous() and w.data_ptr() % 16 == 0) else w.clone(
        memory_format=torch.contiguous_format)
    y = torch.empty(*x.shape[:-1], N, device=x.device, dtype=x.dtype)
    _lib.call("kch_linear_up", _lib.ptr(x2), x2.stride(0), _lib.ptr(wc), K, _lib.ptr(y), N,
              x2.shape[0], N, K, _lib.dtype_code("linear_up", x.dtype), _lib.stream_of(x))
    return y


# Sizes the kernels take: attention head dim, indexer key dim, indexer heads,
# heads per attention launch. Other sizes up to the largest are zero-padded up
# to the next one: zero channels add nothing to a dot product or an L2 norm,
# a zero-weight indexer head adds nothing to a logit, and attention heads are
# independent, so more than 16 run as groups of 16.
_HEAD_DIMS = (64, 128)
_IDX_DIMS = (32, 64, 128)
_IDX_HEADS = (1, 2, 4, 8, 16)
_MAX_HEADS = 16


def _kernel_size(fn, what, n, sizes):
    for k in sizes:
        if n <= k:
            return k
    raise NotImplementedError(f"{fn}: {what}={n} exceeds the largest size the HIP kernels "
                              f"cover ({sizes[-1]})")


def _pad_last(x, n):
    """``x`` zero-padded along its last axis to ``n`` (``x`` itself when it has ``n``)."""
    k = x.shape[-1]
    return x if k == n else F.pad(x, (0, n - k))


def _head_groups(nh):
    return [(h0, min(nh, h0 + _MAX_HEADS)) for h0 in range(0, nh, _MAX_HEADS)]


def _attn_bwd_qdtype(q, d_out, normalize=True):
    """Storage dtype of q, d_out and dq in the attention backward: theirs when
    both are bf16 or both fp16 and the queries are normalised (the MFMA
    kernels read and write them directly), else float32."""
    if normalize and q.dtype == d_out.dtype and q.dtype in (torch.bfloat16, torch.float16):
        return q.dtype
    return torch.float32


def _compress(fn, C, Z, B_pos, m, *, out_raw=True, key=None, normalize=False, local=None,
              key_split=0):
    """``key_split``: 0 keys as ``key``'s dtype (bf16 / fp32); 1 bf16 three-part
    rows ``[B,nb,3c]``; 2 fp16 two-part rows of 256 x ``[B,nb,2c]`` (normalize
    only); 3 the parts of 2 chunk-major, ``[B, ceil(nb/16)*16, 2c]`` (normalize
    only, c a multiple of 32): the indexer's operands."""
    B_, T, c = C.shape
    if m < 1:
        raise ValueError(f"compression factor m={m} must be >= 1")
    if T % m != 0:
        raise ValueError(f"T={T} must be divisible by m={m}")
    if key is None and local is None and generic.compute_dtype(C, Z, B_pos) == torch.float64:
        _lib.require_gpu(fn, C, Z, B_pos)
        return generic.compress(C, Z, B_pos, m)
    _check_gpu_dtype(fn, C, Z)
    nb = T // m
    C, ldc = _rows(C)
    Z, ldz = _rows(Z)
    bpos = _f32_cached(B_pos, C.device)
    raw = torch.empty(B_, nb, c, device=C.device, dtype=torch.float32) if out_raw else None
    key_f32 = {1: 2, 2: 3, 3: 4}.get(int(key_split),
                               1 if (key is not None and key.dtype == torch.float32) else 0)
    _lib.call("kch_compress", _lib.ptr(C), ldc, _lib.ptr(Z), ldz, _lib.ptr(bpos), _lib.ptr(raw),
              _lib.ptr(key), key_f32, int(normalize), _lib.ptr(local), B_, T, m, c,
              _lib.dtype_code(fn, C.dtype), _lib.stream_of(C))
    return raw


def _compress_overlapped(fn, Ca, Cb, Za, Zb, Ba, Bb, m, *, out_raw=True, key=None,
                         normalize=False, local=None):
    B_, T, c = Ca.shape
    if m < 1:
        raise ValueError(f"compression factor m={m} must be >= 1")
    if T % m != 0:
        raise ValueError(f"T={T} must be divisible by m={m}")
    if T == 0:
        return Ca.new_zeros(B_, 0, c)
    if key is None and local is None and \
            generic.compute_dtype(Ca, Cb, Za, Zb, Ba, Bb) == torch.float64:
        _lib.require_gpu(fn, Ca, Cb, Za, Zb, Ba, Bb)
        return generic.compress(Ca, Za, Ba, m, Cb, Zb, Bb)
    _check_gpu_dtype(fn, Ca, Cb, Za, Zb)
    nb = T // m
    (Ca, lca), (Cb, lcb), (Za, lza), (Zb, lzb) = (_rows(x) for x in (Ca, Cb, Za, Zb))
    ba, bb = _f32_cached(Ba, Ca.device), _f32_cached(Bb, Ca.device)
    raw = torch.empty(B_, nb, c, device=Ca.device, dtype=torch.float32) if out_raw else None
    key_f32 = 1 if (key is not None and key.dtype == torch.float32) else 0
    _lib.call("kch_compress_overlapped", _lib.ptr(Ca), lca, _lib.ptr(Cb), lcb, _lib.ptr(Za), lza,
              _lib.ptr(Zb), lzb, _lib.ptr(ba), _lib.ptr(bb), _lib.ptr(raw), _lib.ptr(key),
              key_f32, int(normalize), _lib.ptr(local), B_, T, m, c,
              _lib.dtype_code(fn, Ca.dtype), _lib.stream_of(Ca))
    return raw


def csa_compress_kv(C, Z, B_pos, m):
    """Single-branch compression ``[B, T, c] -> [B, T//m, c]`` in fp32 (``ops_csa.py:198-234``)."""
    return _compress("csa_compress_kv", C, Z, B_pos, m)


def csa_compress_kv_overlapped(Ca, Cb, Za, Zb, Ba, Bb, m):
    """Two-branch overlapped compression in fp32 (``ops_csa.py:237-305``)."""
    return _compress_overlapped("csa_compress_kv_overlapped", Ca, Cb, Za, Zb, Ba, Bb, m)


def l2_normalize_rows(x, *, out_dtype=torch.float32, normalize=True):
    """``F.normalize(x, dim=-1)`` over the last axis on the GPU (or a dtype copy)."""
    shape = x.shape
    c = shape[-1]
    x2 = x.reshape(-1, c)
    if x2.stride(-1) != 1 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    out = torch.empty(x2.shape[0], c, device=x.device, dtype=out_dtype)
    _lib.call("kch_l2norm_rows", _lib.ptr(x2), x2.stride(0), _lib.ptr(out),
              1 if out_dtype == torch.float32 else 0, x2.shape[0], c, int(normalize),
              _lib.dtype_code("l2_normalize_rows", x.dtype), _lib.stream_of(x))
    return out.view(*shape)


def _standard_block_mask_m(mask, T, n_blocks):
    """Return m when ``mask`` equals ``(t + 1) // m > b`` (``ops_csa.py:179-195``), else None."""
    if mask.shape != (T, n_blocks):
        return None
    counts = mask.sum(-1)
    nz = torch.nonzero(counts)
    if nz.numel() == 0:
        return 0  # nothing visible anywhere
    m = int(nz[0, 0].item()) + 1
    t = torch.arange(T, device=mask.device)
    b = torch.arange(n_blocks, device=mask.device)
    expect = (t[:, None] + 1) // m > b[None, :]
    return m if bool(torch.equal(expect, mask.to(torch.bool))) else None


def _indexer(fn, q_idx, k_norm, w_idx, topk, scale, m, *, dense, pos0=0, normalize_q,
             idx64=True, want_logits=False, sorted_=True, key_split=0, nb=None):
    B_, T, HI, DI = q_idx.shape
    if nb is None:
        nb = k_norm.shape[1]
    q_idx = _aligned(q_idx)
    if w_idx is not None:
        w_idx = w_idx.to(q_idx.dtype).contiguous()
    idx = torch.empty(B_, T, topk, device=q_idx.device,
                      dtype=torch.int64 if idx64 else torch.int32)
    logits = (torch.empty(B_, T, nb, device=q_idx.device, dtype=torch.float32)
              if want_logits else None)
    _lib.call("kch_csa_indexer_topk", _lib.ptr(q_idx), _lib.ptr(k_norm), _lib.ptr(w_idx),
              _lib.ptr(idx), 1 if idx64 else 0, _lib.ptr(logits), B_, T, nb, HI, DI, topk,
              max(int(m), 1), pos0, int(dense), int(normalize_q), float(scale),
              int(sorted_), int(key_split), _lib.dtype_code(fn, q_idx.dtype),
              _lib.stream_of(q_idx))
    return idx, logits


def _nan_safe_softmax(logits, dim=-1):
    all_masked = logits.isinf().all(dim=dim, keepdim=True)
    soft = torch.softmax(logits.masked_fill(all_masked, 0.0), dim=dim)
    return soft.masked_fill(all_masked, 0.0)


def csa_lightning_indexer(q_idx, k_idx, w_idx, topk, scale=None, causal_block_mask=None,
                          return_soft_weights=False, *, ste_mode='topk_columns',
                          normalize_qk=False):
    """Top-k selection over compressed indexer keys (``ops_csa.py:330-573``).

    Returns int64 indices ``[B, T, topk]`` (descending logit, ties by ascending
    block index, -1 for masked blocks and padding); with
    ``return_soft_weights`` also the NaN-safe softmax of the logits.
    Any ``causal_block_mask`` broadcastable to ``[B, T, n_blocks]``: the
    standard block-causal one runs on the MFMA indexer, others (and float64,
    c_I > 128, nIh > 16) on the generic kernels.
    """
    fn = "csa_lightning_indexer"
    if topk < 0:
        raise ValueError(f"topk={topk} must be >= 0 (0 selects zero blocks)")
    if q_idx.shape[-1] < 1:
        raise ValueError(
            f"q_idx.shape[-1]={q_idx.shape[-1]} must be >= 1 "
            f"(indexer key dimension c_I must be positive)")
    if ste_mode not in ('topk_columns', 'full_softmax', 'aux_contrastive'):
        raise ValueError(
            f"ste_mode={ste_mode!r} must be one of 'topk_columns', "
            f"'full_softmax', or 'aux_contrastive'.")
    if ste_mode == 'aux_contrastive':
        raise NotImplementedError(
            "ste_mode='aux_contrastive' is reserved for a future implementation of "
            "DeepSeek-V4's contrastive auxiliary loss on the indexer selection logits.")
    _lib.require_gpu(fn, q_idx, k_idx, w_idx)
    if scale is None:
        scale = 1.0 if normalize_qk else q_idx.shape[-1] ** -0.5
    B_, T, HI, DI = q_idx.shape
    n_blocks = k_idx.shape[1]
    std_m = None
    if causal_block_mask is not None:
        std_m = _standard_block_mask_m(causal_block_mask.to(q_idx.device), T, n_blocks)
    if (generic.needs_generic_csa(dtype_tensors=(q_idx, k_idx, w_idx), c_I=DI, nIh=HI)
            or (causal_block_mask is not None and std_m is None)):
        # float64, wide heads or a mask other than the block-causal one
        kn = generic.l2norm(k_idx, normalize_qk, dt=generic.compute_dtype(q_idx, k_idx, w_idx))
        idx, logits = generic.indexer(q_idx, kn, w_idx, topk, scale, mask=causal_block_mask,
                                      normalize_q=normalize_qk, want_logits=return_soft_weights)
        if return_soft_weights:
            return idx, _nan_safe_softmax(logits, dim=-1)
        return idx
    _check_gpu_dtype(fn, q_idx, k_idx, w_idx)
    DIp = _kernel_size(fn, "c_I", DI, _IDX_DIMS)
    HIp = _kernel_size(fn, "nIh", HI, _IDX_HEADS)
    if (DIp, HIp) != (DI, HI):
        q_idx = F.pad(q_idx, (0, DIp - DI, 0, HIp - HI))
        k_idx = _pad_last(k_idx, DIp)
        w_idx = None if w_idx is None else _pad_last(w_idx, HIp)
        if w_idx is None and HIp != HI:
            # the reference's w_idx=None weighs every head 1: padded heads weigh 0
            w_idx = torch.cat([q_idx.new_ones(B_, T, HI), q_idx.new_zeros(B_, T, HIp - HI)], -1)
        B_, T, HI, DI = q_idx.shape
    n_blocks = k_idx.shape[1]
    dense, m = True, 1
    if causal_block_mask is not None:
        m = std_m
        dense = False
    k_norm = l2_normalize_rows(k_idx, normalize=normalize_qk)
    q_idx = _aligned(q_idx)
    if m == 0:  # mask with no visible block
        idx = torch.full((B_, T, topk), -1, dtype=torch.int64, device=q_idx.device)
        logits = torch.full((B_, T, n_blocks), float('-inf'), device=q_idx.device)
    elif topk == 0:
        idx = torch.zeros(B_, T, 0, dtype=torch.long, device=q_idx.device)
        logits = None
        if return_soft_weights:
            _, logits = _indexer(fn, q_idx, k_norm, w_idx, 1, scale, m, dense=dense,
                                 normalize_q=normalize_qk, want_logits=True)
    else:
        idx, logits = _indexer(fn, q_idx, k_norm, w_idx, topk, scale, m, dense=dense,
                               normalize_q=normalize_qk, want_logits=return_soft_weights)
    if return_soft_weights:
        return idx, _nan_safe_softmax(logits, dim=-1)
    return idx


def csa_core(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, *, m, topk,
             sliding_window=0, sink_logits=None, normalize_qk=True, scale=None,
             return_indices=False, use_ste=False, ste_mode='topk_columns'):
    """CSA after the projections (``ops_csa.py:869-1155``) on the HIP backend.

    ``Ca..Zb`` ``[B,T,c]``, ``K_idx, Z_idx`` ``[B,T,c_I]``, ``q`` ``[B,T,nh,c]``,
    ``q_idx`` ``[B,T,nIh,c_I]``, ``w_idx`` ``[B,T,nIh]`` (rows may be strided
    views of one fused projection), T a multiple of m. Returns ``[B,T,nh,c]``
    in ``q.dtype`` (and the int32 selection ``[B,T,topk]`` when asked).

    Differentiable (with gradients enabled) in Ca, Cb, Za, Zb, q, Ba, Bb and the
    sink logits through ``kch_csa_attn_bwd``, the selection held fixed; with
    ``use_ste`` also in the indexer inputs through the straight-through
    surrogate of ``ops_csa.py:1033-1099``: ``ste_mode='topk_columns'`` (the
    selected columns of the soft weights) or ``'full_softmax'`` (plus the
    dense zero-in-forward term that reaches every causal block and, through
    the expected row ``soft @ C_comp_n``, every compressed row).
    """
    if ste_mode not in ('topk_columns', 'full_softmax'):
        raise ValueError(f"csa_core: ste_mode={ste_mode!r} must be 'topk_columns' or "
                         f"'full_softmax'")
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad
            for t in (Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, sink_logits)):
        if generic.needs_generic_csa(dtype_tensors=(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx),
                                     c=Ca.shape[-1], c_I=K_idx.shape[-1], nIh=q_idx.shape[2]):
            generic.grad_not_supported("csa_core", "float64 inputs or c, c_I > 128, nIh > 16")
        out, idx = _CsaCoreFunction.apply(
            Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, sink_logits,
            dict(m=m, topk=topk, sliding_window=sliding_window, normalize_qk=normalize_qk,
                 scale=scale, use_ste=use_ste, ste_mode=ste_mode))
        return (out, idx) if return_indices else out
    return _csa_core(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, m=m, topk=topk,
                     sliding_window=sliding_window, sink_logits=sink_logits,
                     normalize_qk=normalize_qk, scale=scale, return_indices=return_indices)


def _csa_core(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, *, m, topk,
              sliding_window, sink_logits, normalize_qk, scale, return_indices, idx_scale=None):
    fn = "csa_core"
    B_, T, c = Ca.shape
    nh, c_I, nIh = q.shape[2], K_idx.shape[-1], q_idx.shape[2]
    if scale is None:
        scale = 1.0 if normalize_qk else c ** -0.5
    if idx_scale is None:
        idx_scale = 1.0 if normalize_qk else c_I ** -0.5
    if generic.needs_generic_csa(dtype_tensors=(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx),
                                 c=c, c_I=c_I, nIh=nIh):
        _lib.require_gpu(fn, Ca, q, q_idx)
        res = generic.csa_core(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, m=m,
                               topk=topk, sliding_window=sliding_window, sink_logits=sink_logits,
                               normalize_qk=normalize_qk, scale=scale, idx_scale=idx_scale,
                               return_indices=True)
        if topk > 0:
            _log_selection(res[1])
        return res if return_indices else res[0]
    cp = _kernel_size(fn, "c", c, _HEAD_DIMS)
    cIp = _kernel_size(fn, "c_I", c_I, _IDX_DIMS)
    nIp = _kernel_size(fn, "nIh", nIh, _IDX_HEADS)
    if (cp, cIp, nIp) != (c, c_I, nIh):
        # padded channels compress to zero (zero values under any softmax weights)
        Ca, Cb, Za, Zb, q = (_pad_last(x, cp) for x in (Ca, Cb, Za, Zb, q))
        Ba, Bb = _pad_last(Ba, cp), _pad_last(Bb, cp)
        K_idx, Z_idx, B_idx = (_pad_last(x, cIp) for x in (K_idx, Z_idx, B_idx))
        q_idx = F.pad(q_idx, (0, cIp - c_I, 0, nIp - nIh))
        w_idx = _pad_last(w_idx, nIp)
        res = _csa_core(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, m=m,
                        topk=topk, sliding_window=sliding_window, sink_logits=sink_logits,
                        normalize_qk=normalize_qk, scale=scale, return_indices=return_indices,
                        idx_scale=idx_scale)
        if return_indices:
            return res[0][..., :c], res[1]
        return res[..., :c]
    device = Ca.device
    n_blocks = T // m
    kv = torch.empty(B_, n_blocks, c, device=device, dtype=torch.bfloat16)
    local = (torch.empty(B_, T, c, device=device, dtype=torch.bfloat16)
             if sliding_window > 0 else None)
    _compress_overlapped(fn, Ca, Cb, Za, Zb, Ba, Bb, m, out_raw=False, key=kv,
                         normalize=normalize_qk, local=local)
    # indexer keys as the indexer's split MFMA operands: unit rows as the fp16
    # high and low parts of 256 x, chunk-major (whole 16-row chunks in the
    # indexer's load order), raw rows as bf16 high, middle and low parts
    if normalize_qk:
        ksplit = 3
        k_norm = torch.empty(B_, (n_blocks + 15) // 16 * 16, 2 * c_I, device=device,
                             dtype=torch.float16)
    else:
        ksplit = 1
        k_norm = torch.empty(B_, n_blocks, 3 * c_I, device=device, dtype=torch.bfloat16)
    _compress(fn, K_idx, Z_idx, B_idx, m, out_raw=False, key=k_norm, normalize=normalize_qk,
              key_split=ksplit)
    idx = None
    if topk > 0:
        # the attention takes the selected set in any order: sort only for a caller
        idx, _ = _indexer(fn, q_idx, k_norm, w_idx, topk, idx_scale, m, dense=False,
                          normalize_q=normalize_qk, idx64=False, sorted_=bool(return_indices),
                          key_split=ksplit, nb=n_blocks)
        _log_selection(idx)
    sink = None if sink_logits is None else _f32_cached(sink_logits, device)
    out = torch.empty(B_, T, nh, c, device=device, dtype=q.dtype)
    code = _lib.dtype_code(fn, q.dtype)
    for h0, h1 in _head_groups(nh):
        qc = _aligned(q if h1 - h0 == nh else q[:, :, h0:h1])
        og = out if h1 - h0 == nh else torch.empty(B_, T, h1 - h0, c, device=device,
                                                   dtype=q.dtype)
        _lib.call("kch_csa_sparse_attn", _lib.ptr(qc), _lib.ptr(kv), _lib.ptr(idx),
                  _lib.ptr(local), _lib.ptr(None if sink is None else sink[h0:h1]), _lib.ptr(og),
                  B_, T, n_blocks, h1 - h0, c, topk, sliding_window, float(scale),
                  int(normalize_qk), code, code, _lib.stream_of(qc))
        if og is not out:
            out[:, :, h0:h1] = og
    if return_indices:
        return out, idx
    return out


def csa_attn_grad(Ca, Cb, Za, Zb, q, Ba, Bb, idx, d_out, *, m, sliding_window=0,
                  sink_logits=None, normalize_qk=True, scale=None, want_gsum=False):
    """Gradients of the CSA attention (``ops_csa.py:869-1155``) with the selection
    ``idx`` ``[B,T,topk]`` (int32, -1 = unused) held fixed, on
    ``kch_csa_attn_bwd`` (fp32 arithmetic). Returns a dict with ``Ca, Cb, Za, Zb, q, Ba,
    Bb`` (input dtypes), ``sink_logits`` where given, and ``slot`` ``[B,T,topk]``
    (fp32): each selected row's gradient dotted with the row; with
    ``want_gsum`` also ``gsum`` ``[B,T,c]`` (fp32): the sum of the selected
    rows' gradients over the slots. Channels are zero-padded to the kernel's
    size; more than 16 heads run as groups."""
    fn = "csa_attn_grad"
    B_, T, c = Ca.shape
    nh = q.shape[2]
    if T % m:
        raise ValueError(f"{fn}: T={T} must be a multiple of m={m}")
    topk = 0 if idx is None else idx.shape[-1]
    if scale is None:
        scale = 1.0 if normalize_qk else c ** -0.5
    cp = _kernel_size(fn, "c", c, _HEAD_DIMS)
    dev = Ca.device
    f32 = torch.float32

    def prep(x, dt=f32):
        x = x.to(device=dev, dtype=dt)
        return (_pad_last(x, cp) if cp != c else x).contiguous()

    # q, d_out and dq move in their storage dtype where the MFMA kernels run
    qdt = _attn_bwd_qdtype(q, d_out, normalize_qk)
    Caf, Cbf, Zaf, Zbf, Baf, Bbf = (prep(x) for x in (Ca, Cb, Za, Zb, Ba, Bb))
    qf, dof = _aligned(prep(q, qdt)), _aligned(prep(d_out, qdt))
    nb = T // m
    kc = torch.empty(B_, nb, cp, device=dev, dtype=f32)
    raw = _compress_overlapped(fn, Caf, Cbf, Zaf, Zbf, Baf, Bbf, m, out_raw=True, key=kc,
                               normalize=bool(normalize_qk))
    if not normalize_qk:
        kc = raw
    win = int(sliding_window)
    kl = lsrc = None
    if win > 0:
        lsrc = Caf
        kl = l2_normalize_rows(Caf, out_dtype=f32) if normalize_qk else Caf
    idx32 = None if topk == 0 else idx.to(device=dev, dtype=torch.int32).contiguous()
    sink = None if sink_logits is None else sink_logits.detach().to(device=dev, dtype=f32).contiguous()
    dq = torch.empty_like(qf)
    dCa = torch.zeros(B_, T, cp, device=dev, dtype=f32)
    dCb, dZa, dZb = torch.zeros_like(dCa), torch.zeros_like(dCa), torch.zeros_like(dCa)
    dBa = torch.zeros(m, cp, device=dev, dtype=f32)
    dBb = torch.zeros_like(dBa)
    slot = torch.zeros(B_, T, topk, device=dev, dtype=f32)
    gsum = torch.zeros(B_, T, cp, device=dev, dtype=f32) if want_gsum else None
    dsink = None if sink is None else torch.zeros(nh, device=dev, dtype=f32)
    # 16 heads a call on the MFMA kernels (normalised rows), else as many as
    # one SIMT workgroup holds
    hmax = _MAX_HEADS if normalize_qk else 256 // (cp // 8)
    for h0 in range(0, nh, hmax):
        h1 = min(nh, h0 + hmax)
        g = h1 - h0
        qg = qf if g == nh else qf[:, :, h0:h1].contiguous()
        dog = dof if g == nh else dof[:, :, h0:h1].contiguous()
        dqg = dq if g == nh else torch.empty_like(qg)
        oa, ob = torch.empty_like(dCa), torch.zeros_like(dCa)
        za, zb = torch.empty_like(dCa), torch.zeros_like(dCa)
        bap = torch.empty(B_, nb, m, cp, device=dev, dtype=f32)
        bbp = torch.empty_like(bap)
        sp = None if sink is None else torch.empty(B_, T, g, device=dev, dtype=f32)
        gs = None if gsum is None else (gsum if g == nh else torch.empty_like(gsum))
        nbytes = _lib.load().kch_csa_attn_bwd_ws_bytes(B_, T, g, cp, m, win, topk)
        ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
        _lib.call("kch_csa_attn_bwd", _lib.ptr(qg), _lib.ptr(dog), _lib.ptr(kc), _lib.ptr(raw),
                  _lib.ptr(kl), _lib.ptr(lsrc), _lib.ptr(idx32), _lib.ptr(Caf), _lib.ptr(Cbf),
                  _lib.ptr(Zaf), _lib.ptr(Zbf), _lib.ptr(Baf), _lib.ptr(Bbf),
                  _lib.ptr(None if sink is None else sink[h0:h1].contiguous()), _lib.ptr(dqg),
                  _lib.ptr(oa), _lib.ptr(ob), _lib.ptr(za), _lib.ptr(zb), _lib.ptr(bap),
                  _lib.ptr(bbp), _lib.ptr(sp), _lib.ptr(slot if topk else None), _lib.ptr(gs),
                  B_, T, g, cp, m, topk, win, float(scale), int(bool(normalize_qk)),
                  _lib.dtype_code(fn, qdt), _lib.ptr(ws), nbytes, _lib.stream_of(qg))
        if dqg is not dq:
            dq[:, :, h0:h1] = dqg
        if gs is not None and gs is not gsum:
            gsum += gs
        dCa += oa
        dCb += ob
        dZa += za
        dZb += zb
        dBa += bap.sum(dim=(0, 1))
        dBb += bbp.sum(dim=(0, 1))
        if sp is not None:
            dsink[h0:h1] = -sp.sum(dim=(0, 1))
    out = {"Ca": dCa[..., :c].to(Ca.dtype), "Cb": dCb[..., :c].to(Cb.dtype),
           "Za": dZa[..., :c].to(Za.dtype), "Zb": dZb[..., :c].to(Zb.dtype),
           "q": dq[..., :c].to(q.dtype), "Ba": dBa[:, :c].to(Ba.dtype),
           "Bb": dBb[:, :c].to(Bb.dtype), "slot": slot}
    if gsum is not None:
        out["gsum"] = gsum[..., :c]
    if sink_logits is not None:
        out["sink_logits"] = dsink.to(sink_logits.dtype)
    return out


def _ste_indexer_grads(K_idx, Z_idx, q_idx, w_idx, B_idx, idx, slot, *, m, normalize_qk,
                       dsel_extra=None):
    """The straight-through surrogate's gradients for the indexer inputs
    (``ops_csa.py:1033-1099``): the selected columns of the soft weights
    (``softmax`` over every causal block of the indexer logits,
    ``ops_csa.py:545-572``) receive ``slot`` (``topk_columns``), and with
    ``dsel_extra`` ``[B,T,nb]`` every column receives that too (the dense term
    of ``full_softmax``), carried through the logits (``ops_csa.py:503-536``)
    and the key compression (``ops_csa.py:198-234``). On ``kch_csa_ste_bwd``
    when the padded ``nIh * c_I <= 512`` (a wave per query); beyond that,
    ``_ste_indexer_grads_dense``."""
    B_, T, cI = K_idx.shape
    nIh = q_idx.shape[2]
    cIp = 64 if cI <= 64 else 128
    nIp = next((n for n in (1, 2, 4, 8) if n >= nIh), None)
    if cI > 128 or nIp is None or nIp * cIp > 512:
        return _ste_indexer_grads_dense(K_idx, Z_idx, q_idx, w_idx, B_idx, idx, slot, m=m,
                                        normalize_qk=normalize_qk, dsel_extra=dsel_extra)
    fn = "csa_ste_grad"
    dev = K_idx.device
    f32 = torch.float32
    nb = T // m

    def prep(x, n):
        x = x.detach().to(device=dev, dtype=f32)
        return (_pad_last(x, n) if x.shape[-1] != n else x).contiguous()

    Kf, Zf = prep(K_idx, cIp), prep(Z_idx, cIp)
    Bf = prep(B_idx, cIp)
    qf = F.pad(q_idx.detach().to(f32), (0, cIp - cI, 0, nIp - nIh)).contiguous()
    wf = prep(w_idx, nIp)
    kc = torch.empty(B_, nb, cIp, device=dev, dtype=f32)
    raw = _compress(fn, Kf, Zf, Bf, m, out_raw=True, key=kc, normalize=bool(normalize_qk))
    if not normalize_qk:
        kc = raw
    idx64 = idx.long()
    dsel = (torch.zeros(B_, T, nb, device=dev, dtype=f32) if dsel_extra is None
            else dsel_extra.to(f32).clone()).scatter_add_(
        -1, idx64.clamp(min=0), slot.to(f32) * (idx64 >= 0).to(f32))
    scale = 1.0 if normalize_qk else cI ** -0.5
    dq = torch.empty_like(qf)
    dw = torch.empty_like(wf)
    dK = torch.zeros(B_, T, cIp, device=dev, dtype=f32)
    dZ = torch.zeros_like(dK)
    dBp = torch.empty(B_, nb, m, cIp, device=dev, dtype=f32)
    nbytes = _lib.load().kch_csa_ste_bwd_ws_bytes(B_, T, nIp, cIp, m)
    ws = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
    _lib.call("kch_csa_ste_bwd", _lib.ptr(qf), _lib.ptr(wf), _lib.ptr(kc), _lib.ptr(raw),
              _lib.ptr(Kf), _lib.ptr(Zf), _lib.ptr(Bf), _lib.ptr(dsel), _lib.ptr(dq), _lib.ptr(dw),
              _lib.ptr(dK), _lib.ptr(dZ), _lib.ptr(dBp), B_, T, m, nIp, cIp, float(scale),
              int(bool(normalize_qk)), _lib.ptr(ws), nbytes, _lib.stream_of(qf))
    return [dK[..., :cI].to(K_idx.dtype), dZ[..., :cI].to(Z_idx.dtype),
            dq[:, :, :nIh, :cI].to(q_idx.dtype), dw[..., :nIh].to(w_idx.dtype),
            dBp.sum(dim=(0, 1))[:, :cI].to(B_idx.dtype)]


def _ste_indexer_grads_dense(K_idx, Z_idx, q_idx, w_idx, B_idx, idx, slot, *, m, normalize_qk,
                             dsel_extra=None):
    """The same gradients for indexers wider than one wave per query
    (``nIh * c_I > 512`` after padding), dense over the blocks with torch
    operations."""
    leaves = [x.detach().requires_grad_(True) if x is not None else None
              for x in (K_idx, Z_idx, q_idx, w_idx, B_idx)]
    Kl, Zl, ql, wl, Bl = leaves
    B_, T, cI = Kl.shape
    nb = T // m
    with torch.enable_grad():
        f32 = torch.float32
        lg = Zl.to(f32).reshape(B_, nb, m, cI) + Bl.to(f32)
        kcmp = (torch.softmax(lg, dim=2) * Kl.to(f32).reshape(B_, nb, m, cI)).sum(2)
        qi = ql.to(f32)
        if normalize_qk:
            qi = F.normalize(qi, dim=-1)
            kcmp = F.normalize(kcmp, dim=-1)
        sc = 1.0 if normalize_qk else cI ** -0.5
        score = torch.relu(torch.einsum('bthd,bnd->bhtn', qi, kcmp) * sc)
        logits = torch.einsum('bhtn,bth->btn', score, wl.to(f32))
        t = torch.arange(T, device=Kl.device)
        n = torch.arange(nb, device=Kl.device)
        logits = logits.masked_fill(~((t[:, None] + 1) // m > n[None, :]), float('-inf'))
        soft = _nan_safe_softmax(logits, dim=-1)
        idx64 = idx.long()
        sel = torch.gather(soft, -1, idx64.clamp(min=0)) * (idx64 >= 0).to(f32)
        outs, gouts = [sel], [slot]
        if dsel_extra is not None:
            outs.append(soft)
            gouts.append(dsel_extra.to(f32))
        grads = torch.autograd.grad(outs, [x for x in leaves], grad_outputs=gouts,
                                    allow_unused=True)
    return [None if g is None else g.to(x.dtype) for g, x in zip(grads, (K_idx, Z_idx, q_idx, w_idx,
                                                                        B_idx))]


def _compress_overlapped_torch(Ca, Cb, Za, Zb, Ba, Bb, m):
    """``csa_compress_kv_overlapped`` (``ops_csa.py:237-305``) as differentiable
    fp32 torch operations: block i mixes Ca of its own m tokens with Cb of
    block i-1's under one softmax over the 2m logits ``Za + Ba``, ``Zb + Bb``
    (block 0: the second branch's logits -inf, its values zero)."""
    f32 = torch.float32
    B_, T, c = Ca.shape
    nb = T // m

    def blk(x):
        return x.to(f32).reshape(B_, nb, m, c)
    za, zb = blk(Za) + Ba.to(f32), blk(Zb) + Bb.to(f32)
    zb_prev = torch.cat([torch.full_like(zb[:, :1], float('-inf')), zb[:, :-1]], 1)
    cb = blk(Cb)
    cb_prev = torch.cat([torch.zeros_like(cb[:, :1]), cb[:, :-1]], 1)
    w = torch.softmax(torch.cat([za, zb_prev], 2), 2)
    return (w * torch.cat([blk(Ca), cb_prev], 2)).sum(2)


def _soft_weights(K_idx, Z_idx, q_idx, w_idx, B_idx, *, m, normalize_qk):
    """The indexer's soft weights ``[B,T,nb]`` fp32 (``ops_csa.py:545-572``):
    the NaN-safe softmax over the causal blocks of the HIP indexer's logits
    (fp32-level, ``kch_csa_indexer_topk`` with the logits written out)."""
    fn = "csa_soft_weights"
    B_, T, cI = K_idx.shape
    nIh = q_idx.shape[2]
    nb = T // m
    cIp = _kernel_size(fn, "c_I", cI, _IDX_DIMS)
    nIp = _kernel_size(fn, "nIh", nIh, _IDX_HEADS)
    f32 = torch.float32
    Kf, Zf, Bf = (_pad_last(x.detach().to(f32), cIp).contiguous() for x in (K_idx, Z_idx, B_idx))
    k_rows = torch.empty(B_, nb, cIp, device=K_idx.device, dtype=f32)
    _compress(fn, Kf, Zf, Bf, m, out_raw=False, key=k_rows, normalize=bool(normalize_qk))
    qf = F.pad(q_idx.detach().to(f32), (0, cIp - cI, 0, nIp - nIh)).contiguous()
    wf = _pad_last(w_idx.detach().to(f32), nIp).contiguous()
    scale = 1.0 if normalize_qk else cI ** -0.5
    _, logits = _indexer(fn, qf, k_rows, wf, 1, scale, m, dense=False,
                         normalize_q=bool(normalize_qk), idx64=False, want_logits=True,
                         sorted_=False)
    return _nan_safe_softmax(logits)


def _full_softmax_grads(Ca, Cb, Za, Zb, Ba, Bb, K_idx, Z_idx, q_idx, w_idx, B_idx, gsum, *, m,
                        normalize_qk):
    """The dense term of ``ste_mode='full_softmax'`` (``ops_csa.py:1050-1071``):
    ``soft_full = soft @ C_comp_n`` enters every selected slot as a zero in
    the forward, so its cotangent is ``gsum`` (the selected rows' gradients
    summed over the slots). Returns ``(dsel_extra [B,T,nb], grads of Ca, Cb,
    Za, Zb, Ba, Bb)``: the soft weights' cotangent ``gsum C_comp_n^T`` (carried
    on by the surrogate's indexer backward) and ``C_comp_n``'s,
    ``soft^T gsum``, through the L2 norm and the overlapped compression."""
    with torch.enable_grad():
        leaves = [x.detach().to(torch.float32).requires_grad_(True)
                  for x in (Ca, Cb, Za, Zb, Ba, Bb)]
        cc = _compress_overlapped_torch(*leaves, m)
        cn = F.normalize(cc, dim=-1) if normalize_qk else cc
    soft = _soft_weights(K_idx, Z_idx, q_idx, w_idx, B_idx, m=m, normalize_qk=normalize_qk)
    g = gsum.to(torch.float32)
    dsel_extra = torch.bmm(g, cn.detach().transpose(1, 2))
    dcn = torch.bmm(soft.transpose(1, 2), g)
    return dsel_extra, torch.autograd.grad(cn, leaves, dcn)


class _CsaCoreFunction(torch.autograd.Function):
    """``csa_core`` with gradients: the forward kernels (selection included),
    ``kch_csa_attn_bwd`` for the attention's backward, and the STE surrogate
    for the indexer inputs when asked."""

    @staticmethod
    def forward(ctx, Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, sink_logits, cfg):
        out, idx = _csa_core(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx,
                             m=cfg["m"], topk=cfg["topk"], sliding_window=cfg["sliding_window"],
                             sink_logits=sink_logits, normalize_qk=cfg["normalize_qk"],
                             scale=cfg["scale"], return_indices=True)
        if idx is None:
            idx = torch.zeros(Ca.shape[0], Ca.shape[1], 0, device=Ca.device, dtype=torch.int32)
        ctx.save_for_backward(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx,
                              sink_logits, idx)
        ctx.cfg = cfg
        ctx.mark_non_differentiable(idx)
        return out, idx

    @staticmethod
    def backward(ctx, d_out, _d_idx):
        Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, sink, idx = ctx.saved_tensors
        cfg = ctx.cfg
        full = cfg["use_ste"] and cfg["ste_mode"] == "full_softmax" and idx.shape[-1] > 0
        g = csa_attn_grad(Ca, Cb, Za, Zb, q, Ba, Bb, idx if idx.shape[-1] else None, d_out,
                          m=cfg["m"], sliding_window=cfg["sliding_window"], sink_logits=sink,
                          normalize_qk=cfg["normalize_qk"], scale=cfg["scale"], want_gsum=full)
        dsel_extra = None
        if full:
            dsel_extra, extra = _full_softmax_grads(
                Ca, Cb, Za, Zb, Ba, Bb, K_idx, Z_idx, q_idx, w_idx, B_idx, g["gsum"],
                m=cfg["m"], normalize_qk=cfg["normalize_qk"])
            for name, x, e in zip(("Ca", "Cb", "Za", "Zb", "Ba", "Bb"), (Ca, Cb, Za, Zb, Ba, Bb),
                                  extra):
                g[name] = (g[name].to(torch.float32) + e).to(x.dtype)
        ig = [None] * 5
        if cfg["use_ste"] and idx.shape[-1] and any(
                x.requires_grad for x in (K_idx, Z_idx, q_idx, w_idx, B_idx)):
            ig = _ste_indexer_grads(K_idx, Z_idx, q_idx, w_idx, B_idx, idx, g["slot"],
                                    m=cfg["m"], normalize_qk=cfg["normalize_qk"],
                                    dsel_extra=dsel_extra)
        return (g["Ca"], g["Cb"], g["Za"], g["Zb"], ig[0], ig[1], g["q"], ig[2], ig[3], g["Ba"],
                g["Bb"], ig[4], g.get("sink_logits"), None)


def naive_csa(H, W_aKV, W_bKV, W_aZ, W_bZ, Ba, Bb, W_DQ, W_UQ, W_IUQ, W_w, W_KV_idx, W_Z_idx,
              B_idx, *, m, topk, nh, nIh, c, c_I, dc, scale=None, sliding_window=0,
              sink_logits=None, use_ste=True, ste_mode='topk_columns', normalize_qk=False,
              fuse_projections=True, return_projections=False):
    """CSA forward on the HIP backend (``ops_csa.py:576-1184``); returns ``[B, T, nh*c]``."""
    fn = "naive_csa"
    B_, T, d = H.shape
    if m < 1:
        raise ValueError(f"compression factor m={m} must be >= 1")
    if topk < 0:
        raise ValueError(f"topk={topk} must be >= 0 (0 disables sparse selection)")
    if nh < 1:
        raise ValueError(f"nh={nh} must be >= 1")
    if c < 1:
        raise ValueError(f"c={c} must be >= 1")
    if dc < 1:
        raise ValueError(f"dc={dc} must be >= 1")
    if c_I < 1:
        raise ValueError(f"c_I={c_I} must be >= 1 (indexer key dim)")
    if nIh < 1:
        raise ValueError(f"nIh={nIh} must be >= 1 (indexer head count)")
    if sliding_window < 0:
        raise ValueError(
            f"sliding_window={sliding_window} must be >= 0 (0 disables the branch)")
    if ste_mode not in ('topk_columns', 'full_softmax', 'aux_contrastive'):
        raise ValueError(
            f"ste_mode={ste_mode!r} must be one of 'topk_columns', "
            f"'full_softmax', or 'aux_contrastive'.")
    device = H.device
    if T == 0:
        out_empty = torch.zeros(B_, 0, nh * c, dtype=H.dtype, device=device)
        if return_projections:
            z = lambda w: torch.zeros(B_, 0, w, dtype=H.dtype, device=device)  # noqa: E731
            return out_empty, (z(c), z(c), z(c), z(c), z(c_I), z(c_I))
        return out_empty
    for _w_name, _w in [('W_aKV', W_aKV), ('W_bKV', W_bKV), ('W_aZ', W_aZ), ('W_bZ', W_bZ),
                        ('W_KV_idx', W_KV_idx), ('W_Z_idx', W_Z_idx)]:
        if _w.device != H.device:
            raise ValueError(
                f"naive_csa: {_w_name}.device={_w.device} does not match "
                f"H.device={H.device}. All weights must be on the same "
                f"device as the input.")
        if _w.dtype != H.dtype:
            raise ValueError(
                f"naive_csa: {_w_name}.dtype={_w.dtype} does not match "
                f"H.dtype={H.dtype}. All weights must share the input's "
                f"dtype (cast before calling if needed).")
        if _w.shape[1] != d:
            raise ValueError(
                f"naive_csa: {_w_name}.shape={tuple(_w.shape)} — second dim "
                f"(in_features) must equal d={d} (H.shape[-1]).")
    if ste_mode == 'aux_contrastive':
        # raised by the reference's indexer call (ops_csa.py:486-491), which
        # every non-empty input reaches
        raise NotImplementedError(
            "ste_mode='aux_contrastive' is reserved for a future implementation of "
            "DeepSeek-V4's contrastive auxiliary loss on the indexer selection logits. "
            "Use 'topk_columns' (the default, simplified STE) or 'full_softmax' (dense STE) "
            "for now.")
    _lib.require_gpu(fn, H)
    original_T = T
    pad = (-T) % m
    if pad:
        H = F.pad(H, (0, 0, 0, pad))
        T = T + pad
    n_blocks = T // m
    if torch.is_grad_enabled() and any(
            t.requires_grad for t in (H, W_aKV, W_bKV, W_aZ, W_bZ, Ba, Bb, W_DQ, W_UQ, W_IUQ, W_w,
                                      W_KV_idx, W_Z_idx, B_idx)
            if t is not None) or (sink_logits is not None and sink_logits.requires_grad
                                  and torch.is_grad_enabled()):
        # training: the projections through autograd (library GEMMs), the core
        # through its HIP backward and, with use_ste, the STE surrogate
        Ca, Cb, Za, Zb, K_idx_raw, Z_idx, cQ, w_idx = F.linear(
            H, torch.cat([W_aKV, W_bKV, W_aZ, W_bZ, W_KV_idx, W_Z_idx, W_DQ, W_w])).split(
            [c, c, c, c, c_I, c_I, dc, nIh], dim=-1)
        q_idx = F.linear(cQ, W_IUQ).view(B_, T, nIh, c_I)
        q = F.linear(cQ, W_UQ).view(B_, T, nh, c)
        out = csa_core(Ca, Cb, Za, Zb, K_idx_raw, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, m=m,
                       topk=topk, sliding_window=sliding_window, sink_logits=sink_logits,
                       normalize_qk=normalize_qk, scale=scale, use_ste=use_ste,
                       ste_mode=ste_mode)
        out_final = out.reshape(B_, T, nh * c)[:, :original_T]
        if return_projections:
            return out_final, tuple(x[:, :original_T] for x in (Ca, Cb, Za, Zb, K_idx_raw, Z_idx))
        return out_final
    with torch.no_grad():
        if fuse_projections:
            # every projection of H in one GEMM: H is read from HBM once (rows
            # padded to a multiple of 8 columns, so that the latent's rows stay
            # 16-byte aligned for the up-projection)
            comb = F.linear(H, _cat_cached([W_aKV, W_bKV, W_aZ, W_bZ, W_KV_idx, W_Z_idx, W_DQ,
                                            W_w], pad_rows_to=8))
            Ca, Cb, Za, Zb, K_idx_raw, Z_idx, cQ, w_idx = comb[..., :4 * c + 2 * c_I + dc + nIh].split(
                [c, c, c, c, c_I, c_I, dc, nIh], dim=-1)
        else:
            Ca, Cb, Za, Zb = (F.linear(H, w) for w in (W_aKV, W_bKV, W_aZ, W_bZ))
            K_idx_raw, Z_idx = F.linear(H, W_KV_idx), F.linear(H, W_Z_idx)
            cQ = F.linear(H, W_DQ)
            w_idx = F.linear(H, W_w)
        q_idx = _linear_up(cQ, W_IUQ).view(B_, T, nIh, c_I)
        q = _linear_up(cQ, W_UQ).view(B_, T, nh, c)
        out = csa_core(Ca, Cb, Za, Zb, K_idx_raw, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, m=m,
                       topk=topk, sliding_window=sliding_window, sink_logits=sink_logits,
                       normalize_qk=normalize_qk, scale=scale)
    out_final = out.reshape(B_, T, nh * c)[:, :original_T]
    if return_projections:
        projections = tuple(x[:, :original_T] for x in (Ca, Cb, Za, Zb, K_idx_raw, Z_idx))
        return out_final, projections
    return out_final


__all__ = ["csa_attn_grad", "csa_compress_kv", "csa_compress_kv_overlapped", "csa_core",
           "csa_lightning_indexer", "naive_csa", "l2_normalize_rows", "record_selections"]
