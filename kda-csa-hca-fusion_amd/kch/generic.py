"""Generic CSA / HCA forward on ``kch_gen_*``: the inputs the MFMA kernels do
not take.

* float64 inputs, computed in float64 as the reference does for them
  (``/root/reference/ops_csa.py:229,263,510,922``; ``ops_hca.py:138``);
* head dims ``c`` or ``c_I`` above 128 and more than 16 indexer heads
  (computed in float32, the reference's compute dtype for fp32 / bf16 / fp16);
* indexer masks other than the standard block-causal one
  (``csa_lightning_indexer``'s ``causal_block_mask``, ``ops_csa.py:535-536``).

Forward only: gradients through these inputs raise ``NotImplementedError``.
The compression, row norms, indexer with its top-k sort and the joint-softmax
attention are SIMT HIP kernels (``csrc/csa_hca_generic.hip``); PyTorch only
allocates and converts.
"""

from __future__ import annotations

import torch

from . import _lib

_MAX_FAST_C = 128
_MAX_FAST_CI = 128
_MAX_FAST_NIH = 16


def compute_dtype(*ts):
    """float64 when any tensor is float64, else float32."""
    return torch.float64 if any(t is not None and t.dtype == torch.float64 for t in ts) \
        else torch.float32


def _code(dt):
    return 3 if dt == torch.float64 else 0


def _prep(x, dt):
    return None if x is None else x.to(dt).contiguous()


def needs_generic_csa(*, dtype_tensors, c=0, c_I=0, nIh=0):
    return (any(t is not None and t.dtype == torch.float64 for t in dtype_tensors)
            or c > _MAX_FAST_C or c_I > _MAX_FAST_CI or nIh > _MAX_FAST_NIH)


def grad_not_supported(fn, what):
    raise NotImplementedError(
        f"{fn}: gradients are not provided for {what} (the HIP backward kernels take "
        f"float32 / bfloat16 / float16 with c, c_I <= 128 and nIh <= 16)")


def compress(C, Z, B_pos, m, Cb=None, Zb=None, Bb=None, dt=None):
    """``csa_compress_kv`` (``Cb = Zb = Bb = None``) or the overlapped two-branch
    form, ``[B, T, c] -> [B, T // m, c]`` in ``dt``."""
    dt = dt or compute_dtype(C, Z, B_pos, Cb, Zb, Bb)
    B_, T, c = C.shape
    C, Z, B_pos, Cb, Zb, Bb = (_prep(x, dt) for x in (C, Z, B_pos, Cb, Zb, Bb))
    out = torch.empty(B_, T // m, c, device=C.device, dtype=dt)
    _lib.call("kch_gen_compress", _lib.ptr(C), _lib.ptr(Cb), _lib.ptr(Z), _lib.ptr(Zb),
              _lib.ptr(B_pos), _lib.ptr(Bb), _lib.ptr(out), B_, T, m, c, _code(dt),
              _lib.stream_of(C))
    return out


def l2norm(x, normalize=True, dt=None):
    """``F.normalize(x, dim=-1)`` (or a copy) in ``dt``."""
    dt = dt or compute_dtype(x)
    x = _prep(x, dt)
    y = torch.empty_like(x)
    c = x.shape[-1]
    _lib.call("kch_gen_l2norm", _lib.ptr(x), _lib.ptr(y), x.numel() // max(c, 1), c,
              int(normalize), _code(dt), _lib.stream_of(x))
    return y


def indexer(q_idx, k_rows, w_idx, topk, scale, *, mask=None, causal_m=0, normalize_q,
            want_logits=False, dt=None):
    """Top-k block selection (``ops_csa.py:503-554``): int64 ``[B, T, topk]``,
    descending logit, ties by ascending block index, -1 for masked blocks and
    padding; and the logits ``[B, T, n_blocks]`` when asked. ``mask`` is a
    boolean tensor broadcastable to ``[B, T, n_blocks]`` (True = visible), or
    None with the block-causal rule of ``causal_m`` (0: every block)."""
    dt = dt or compute_dtype(q_idx, k_rows, w_idx)
    B_, T, HI, DI = q_idx.shape
    nb = k_rows.shape[1]
    q_idx, k_rows, w_idx = (_prep(x, dt) for x in (q_idx, k_rows, w_idx))
    sb = st = 0
    mk = None
    if mask is not None:
        mk = mask.to(device=q_idx.device, dtype=torch.uint8)
        while mk.dim() < 3:
            mk = mk.unsqueeze(0)
        mk = mk.expand(B_, T, nb)
        if mk.stride(-1) != 1:
            mk = mk.contiguous()
        sb, st = mk.stride(0), mk.stride(1)
    idx = torch.empty(B_, T, topk, device=q_idx.device, dtype=torch.int64)
    logits = torch.empty(B_, T, nb, device=q_idx.device, dtype=dt) if want_logits else None
    _lib.call("kch_gen_indexer", _lib.ptr(q_idx), _lib.ptr(k_rows), _lib.ptr(w_idx), _lib.ptr(mk),
              sb, st, _lib.ptr(logits), _lib.ptr(idx), B_, T, nb, HI, DI, topk, int(causal_m),
              float(scale), int(normalize_q), _code(dt), _lib.stream_of(q_idx))
    return idx, logits


def attn(q, kv_rows, idx, local, sink, *, m, win, scale, normalize_q, hca, dt=None):
    """Joint sparse (``idx`` given, CSA) or dense causal (``idx`` None, HCA)
    attention with the window rows ``local`` and the sink: ``[B, T, nh, c]``."""
    dt = dt or compute_dtype(q, kv_rows)
    B_, T, nh, c = q.shape
    nb = kv_rows.shape[1]
    topk = 0 if idx is None else idx.shape[-1]
    q, kv_rows, local, sink = (_prep(x, dt) for x in (q, kv_rows, local, sink))
    idx = None if idx is None else idx.to(torch.int64).contiguous()
    out = torch.empty(B_, T, nh, c, device=q.device, dtype=dt)
    lib = _lib.load()
    nbytes = lib.kch_gen_attn_ws_bytes(B_, T, nh, nb, topk, win, int(idx is not None), _code(dt))
    ws = torch.empty(max(nbytes, 1), device=q.device, dtype=torch.uint8)
    _lib.call("kch_gen_attn", _lib.ptr(q), _lib.ptr(kv_rows), _lib.ptr(idx), _lib.ptr(local),
              _lib.ptr(sink), _lib.ptr(out), B_, T, nb, nh, c, topk, win, m, float(scale),
              int(normalize_q), int(hca), _code(dt), _lib.ptr(ws), nbytes, _lib.stream_of(q))
    return out


def csa_core(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, *, m, topk,
             sliding_window, sink_logits, normalize_qk, scale, idx_scale, return_indices):
    """``naive_csa`` after the projections (``ops_csa.py:869-1155``), T a
    multiple of m; output in ``q.dtype`` (computed in float64 for float64
    inputs, else float32)."""
    dt = compute_dtype(Ca, q, q_idx)
    C_comp = compress(Ca, Za, Ba, m, Cb, Zb, Bb, dt=dt)
    K_IComp = compress(K_idx, Z_idx, B_idx, m, dt=dt)
    kv = l2norm(C_comp, normalize_qk, dt=dt)
    kn = l2norm(K_IComp, normalize_qk, dt=dt)
    if topk > 0:
        idx, _ = indexer(q_idx, kn, w_idx, topk, idx_scale, causal_m=m, normalize_q=normalize_qk,
                         dt=dt)
    else:
        idx = torch.zeros(q.shape[0], q.shape[1], 0, dtype=torch.int64, device=q.device)
    local = l2norm(Ca, normalize_qk, dt=dt) if sliding_window > 0 else None
    out = attn(q, kv, idx, local, sink_logits, m=m, win=sliding_window, scale=scale,
               normalize_q=normalize_qk, hca=False, dt=dt).to(q.dtype)
    if return_indices:
        return out, idx.to(torch.int32)
    return out


def hca_core(C, Z, q, B_pos, *, m2, sliding_window, sink_logits, scale, C_local_raw):
    """``naive_hca`` after the projections (``ops_hca.py:132-194``); output in
    ``q.dtype``."""
    dt = compute_dtype(C, q)
    kv = l2norm(compress(C, Z, B_pos, m2, dt=dt), dt=dt)
    local = None
    if sliding_window > 0:
        local = l2norm(C if C_local_raw is None else C_local_raw, dt=dt)
    return attn(q, kv, None, local, sink_logits, m=m2, win=sliding_window, scale=scale,
                normalize_q=True, hca=True, dt=dt).to(q.dtype)
