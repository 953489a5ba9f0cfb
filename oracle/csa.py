"""CSA / HCA oracle: numpy restatement of the reference (test infrastructure only).

Functions and the reference lines each restates:

``compress_kv``              ``csa_compress_kv``            ``ops_csa.py:198-234``
``compress_kv_overlapped``   ``csa_compress_kv_overlapped`` ``ops_csa.py:237-305``
``causal_block_mask``        ``_causal_block_mask``         ``ops_csa.py:179-195``
``lightning_indexer``        ``csa_lightning_indexer``      ``ops_csa.py:330-573``
                             (forward only; the STE soft weights are training-only)
``window_scores``            ``_sliding_window_scores``     ``ops_csa.py:151-176``
``joint_softmax_csa``        joint softmax + sink           ``ops_csa.py:1126-1149``
``joint_softmax_hca``        joint softmax + sink           ``ops_hca.py:166-186``
``csa_core``                 ``naive_csa`` after the projections, ``ops_csa.py:869-1165``
``naive_csa``                ``naive_csa`` incl. bf16 projections, ``ops_csa.py:576-1184``
``hca_core``                 ``naive_hca`` after the projections, ``ops_hca.py:132-194``
``naive_hca``                ``naive_hca`` incl. bf16 projections, ``ops_hca.py:30-201``
``hca_core_grad``            ``naive_hca``'s autograd backward, ``ops_hca.py:132-194``
``csa_attn_grad``            ``naive_csa``'s attention backward, ``ops_csa.py:869-1155``
``csa_ste_grad``             the STE surrogate's backward, ``ops_csa.py:1033-1099``
                             (``topk_columns``, ``full_softmax``); pinned by the
                             reference's gradients (``tests/golden/csa_ste_fp32.npz``)

Tie rule: ``torch.topk`` (``ops_csa.py:550``) does not document its order on
exactly-equal logits (the reference notes it depends on the tensor size,
``ops_decoding_cache.py:62-87``). The oracle fixes it as "descending logit,
then ascending block index" (a stable descending sort), the same rule the HIP
kernels implement; the order on exact ties is therefore "parity unpinned"
against torch itself, and the tests compare such indices tie-aware.
"""

from __future__ import annotations

import numpy as np

from .common import bf16_round, l2_normalize, round_to

NEG_INF = -np.inf


def compress_kv(C, Z, B_pos, m, compute=np.float32):
    """Single-branch softmax-gated compression ``[B,T,c] -> [B,T//m,c]``."""
    C = np.asarray(C, compute)
    Z = np.asarray(Z, compute)
    Bn, T, c = C.shape
    if m < 1:
        raise ValueError("m must be >= 1")
    if T % m:
        raise ValueError("T must be divisible by m")
    nb = T // m
    C = C.reshape(Bn, nb, m, c)
    logits = Z.reshape(Bn, nb, m, c) + np.asarray(B_pos, compute)[None, None]
    mx = logits.max(axis=2, keepdims=True)
    e = np.exp(logits - mx)
    S = e / e.sum(axis=2, keepdims=True)
    return (S * C).sum(axis=2)


def compress_kv_overlapped(Ca, Cb, Za, Zb, Ba, Bb, m, compute=np.float32):
    """Two-branch overlapped compression: block i mixes Ca_i with Cb_{i-1}."""
    Ca, Cb, Za, Zb = (np.asarray(x, compute) for x in (Ca, Cb, Za, Zb))
    Bn, T, c = Ca.shape
    if m < 1:
        raise ValueError("m must be >= 1")
    if T % m:
        raise ValueError("T must be divisible by m")
    if T == 0:
        return np.zeros((Bn, 0, c), compute)
    nb = T // m
    Ca, Cb, Za, Zb = (x.reshape(Bn, nb, m, c) for x in (Ca, Cb, Za, Zb))
    a_log = Za + np.asarray(Ba, compute)[None, None]
    zb_prev = np.concatenate([np.full((Bn, 1, m, c), -np.inf, compute), Zb[:, :-1]], axis=1)
    b_log = zb_prev + np.asarray(Bb, compute)[None, None]
    allg = np.concatenate([a_log, b_log], axis=2)
    mx = allg.max(axis=2, keepdims=True)
    e = np.exp(allg - mx)
    S = e / e.sum(axis=2, keepdims=True)
    cb_prev = np.concatenate([np.zeros((Bn, 1, m, c), compute), Cb[:, :-1]], axis=1)
    return (S[:, :, :m] * Ca).sum(2) + (S[:, :, m:] * cb_prev).sum(2)


def causal_block_mask(T, n_blocks, m):
    """``mask[t, b] = (t + 1) // m > b``."""
    t = np.arange(T)[:, None]
    b = np.arange(n_blocks)[None, :]
    return (t + 1) // m > b


def topk_desc_lowest_index(logits, topk):
    """Top-k along the last axis: descending value, ties by ascending index.

    Entries whose value is +-inf become -1, and the result is padded with -1
    up to ``topk`` (``ops_csa.py:550-554``).
    """
    nb = logits.shape[-1]
    S = min(topk, nb)
    order = np.argsort(-logits, axis=-1, kind='stable')[..., :S]
    vals = np.take_along_axis(logits, order, axis=-1)
    idx = np.where(np.isinf(vals), -1, order).astype(np.int64)
    if topk > S:
        pad = np.full(idx.shape[:-1] + (topk - S,), -1, np.int64)
        idx = np.concatenate([idx, pad], axis=-1)
    return idx


def indexer_logits(q_idx, k_idx, w_idx, scale=None, causal_block_mask=None,
                   normalize_qk=False, compute=np.float32):
    """Head-weighted ReLU scores ``[B, T, n_blocks]`` (``ops_csa.py:503-536``)."""
    q = np.asarray(q_idx, compute)
    k = np.asarray(k_idx, compute)
    DI = q.shape[-1]
    if scale is None:
        scale = 1.0 if normalize_qk else DI ** -0.5
    if normalize_qk:
        q = l2_normalize(q)
        k = l2_normalize(k)
    score = np.maximum(np.einsum('bthd,bnd->bhtn', q, k) * compute(scale), compute(0))
    if w_idx is None:
        logits = score.sum(1)
    else:
        logits = np.einsum('bhtn,bth->btn', score, np.asarray(w_idx, compute))
    if causal_block_mask is not None:
        logits = np.where(causal_block_mask, logits, compute(-np.inf))
    return logits.astype(compute)


def lightning_indexer(q_idx, k_idx, w_idx, topk, scale=None, causal_block_mask=None,
                      normalize_qk=False, compute=np.float32, return_logits=False):
    if topk < 0:
        raise ValueError("topk must be >= 0")
    logits = indexer_logits(q_idx, k_idx, w_idx, scale, causal_block_mask,
                            normalize_qk, compute)
    Bn, T = logits.shape[:2]
    if topk == 0:
        idx = np.zeros((Bn, T, 0), np.int64)
    else:
        idx = topk_desc_lowest_index(logits, topk)
    return (idx, logits) if return_logits else idx


def window_scores(q, C_local, win, scale):
    """Per-query causal window scores ``[B,T,nh,win]`` and keys ``[B,T,win,c]``.

    Window slot ``j`` of query ``t`` holds position ``t - win + 1 + j``; slots
    before position 0 are ``-inf`` (``ops_csa.py:151-176``).
    """
    Bn, T, nh, c = q.shape
    Cp = np.concatenate([np.zeros((Bn, win - 1, c), C_local.dtype), C_local], axis=1)
    idx = np.arange(T)[:, None] + np.arange(win)[None, :]
    Cw = Cp[:, idx]                                    # [B, T, win, c]
    valid = np.arange(win)[None, :] >= (win - 1 - np.arange(T)[:, None])
    s = np.einsum('bthd,btwd->bthw', q, Cw) * q.dtype.type(scale)
    s = np.where(valid[None, :, None, :], s, -np.inf)
    return s, Cw, valid


def _logaddexp(a, b):
    return np.logaddexp(a, b)


def _logsumexp(x, axis=-1):
    mx = np.max(x, axis=axis, keepdims=True)
    mx_safe = np.where(np.isfinite(mx), mx, 0)
    with np.errstate(divide='ignore'):
        return np.log(np.exp(x - mx_safe).sum(axis=axis, keepdims=True)) + mx_safe


def joint_softmax_csa(cat, cat_valid, sink):
    """CSA / decode-cache joint softmax: ``row_max = max(0, max s)``."""
    all_invalid = ~cat_valid.any(-1, keepdims=True)
    if sink is not None:
        row_max = np.maximum(cat.max(-1, keepdims=True), 0)
        shifted = cat - row_max
        s_sink = sink - row_max
        lse = _logsumexp(shifted)
        log_denom = _logaddexp(lse, s_sink)
        with np.errstate(invalid='ignore'):
            p = np.exp(shifted - log_denom) * cat_valid
    else:
        safe = np.where(all_invalid, 0, cat)
        mx = safe.max(-1, keepdims=True)
        e = np.exp(safe - mx)
        p = e / e.sum(-1, keepdims=True)
    return np.where(all_invalid, 0, p).astype(cat.dtype)


def joint_softmax_hca(cat, sink):
    """naive_hca joint softmax: ``row_max = max s`` (0 if all masked)."""
    all_masked = np.isneginf(cat).all(-1, keepdims=True)
    if sink is not None:
        row_max = cat.max(-1, keepdims=True)
        row_max = np.where(np.isneginf(row_max), 0, row_max)
        shifted = cat - row_max
        lse = _logsumexp(shifted)
        log_denom = _logaddexp(lse, sink - row_max)
        p = np.exp(shifted - log_denom)
    else:
        safe = np.where(all_masked, 0, cat)
        mx = safe.max(-1, keepdims=True)
        e = np.exp(safe - mx)
        p = e / e.sum(-1, keepdims=True)
    return np.where(all_masked, 0, p).astype(cat.dtype)


def _pad_time(x, pad):
    if not pad:
        return x
    w = [(0, 0)] * x.ndim
    w[1] = (0, pad)
    return np.pad(x, w)


def csa_core(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, *,
             m, topk, sliding_window=0, sink_logits=None, normalize_qk=True,
             scale=None, compute=np.float32, return_indices=False, indices=None):
    """CSA forward from the projections: ``[B,T,nh,c]`` in ``compute``.

    Inputs are the bf16 projection values (as float arrays): ``Ca..Zb``
    ``[B,T,c]``, ``K_idx, Z_idx`` ``[B,T,cI]``, ``q`` ``[B,T,nh,c]``,
    ``q_idx`` ``[B,T,nIh,cI]``, ``w_idx`` ``[B,T,nIh]``. ``indices``
    (``[B,T,topk]``, -1 = unused) replaces the indexer's selection, so the
    attention can be checked on a given selection.
    """
    Bn, T, c = np.shape(Ca)
    nh = np.shape(q)[2]
    pad = (-T) % m
    Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx = (
        _pad_time(np.asarray(x, compute), pad)
        for x in (Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx))
    Tp = T + pad
    nb = Tp // m
    C_comp = compress_kv_overlapped(Ca, Cb, Za, Zb, Ba, Bb, m, compute)
    K_IComp = compress_kv(K_idx, Z_idx, B_idx, m, compute)
    cbm = causal_block_mask(Tp, nb, m)
    if indices is None:
        idx = lightning_indexer(q_idx, K_IComp, w_idx, topk, None, cbm, normalize_qk, compute)
    else:
        idx = np.asarray(indices, np.int64)
        if idx.shape[1] < Tp:
            idx = np.concatenate([idx, np.full((Bn, Tp - idx.shape[1], idx.shape[2]), -1,
                                               np.int64)], axis=1)
    if normalize_qk:
        qn = l2_normalize(q)
        Cn = l2_normalize(C_comp)
    else:
        qn, Cn = q, C_comp
    if scale is None:
        scale = 1.0 if normalize_qk else c ** -0.5
    if idx.shape[-1] == 0:
        scores = np.zeros((Bn, Tp, nh, 0), compute)
        valid = np.zeros((Bn, Tp, 0), bool)
        kv = np.zeros((Bn, Tp, 0, c), compute)
    else:
        valid = idx >= 0
        kv = Cn[np.arange(Bn)[:, None, None], np.maximum(idx, 0)]
        scores = np.einsum('bthd,btkd->bthk', qn, kv) * compute(scale)
        scores = np.where(valid[:, :, None, :], scores, -np.inf)
    if sliding_window > 0:
        C_local = l2_normalize(Ca) if normalize_qk else Ca
        sw, Cw, wvalid = window_scores(qn, C_local, sliding_window, scale)
    else:
        sw = np.zeros((Bn, Tp, nh, 0), compute)
        Cw = np.zeros((Bn, Tp, 0, c), compute)
        wvalid = np.zeros((Tp, 0), bool)
    cat = np.concatenate([scores, sw], axis=-1).astype(compute)
    cat_valid = np.concatenate(
        [valid[:, :, None, :],
         np.broadcast_to(wvalid[None, :, None, :], (Bn, Tp, 1, wvalid.shape[-1]))], axis=-1)
    if cat.shape[-1] == 0:
        out = np.zeros((Bn, Tp, nh, c), compute)
    else:
        sink = None if sink_logits is None else np.asarray(sink_logits, compute).reshape(1, 1, nh, 1)
        p = joint_softmax_csa(cat, cat_valid, sink)
        k_ = scores.shape[-1]
        out = (np.einsum('bthk,btkd->bthd', p[..., :k_], kv)
               + np.einsum('bthw,btwd->bthd', p[..., k_:], Cw))
    out = out[:, :T].astype(compute)
    if return_indices:
        return out, idx[:, :T]
    return out


def csa_core_at(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, *, m, topk,
                queries, sliding_window=0, sink_logits=None, normalize_qk=True, scale=None,
                compute=np.float32, indices=None, logits_compute=None, C_comp=None,
                K_IComp=None):
    """``csa_core`` evaluated at the query positions ``queries`` only.

    The same arithmetic per query row as ``csa_core`` (``ops_csa.py:959-1155``),
    for sequences whose full ``[B,T,topk,c]`` gather would not fit: T must be
    a multiple of m. ``indices`` (``[B,len(queries),topk]``) replaces the
    indexer's selection. Returns ``(out [B,Q,nh,c], idx [B,Q,topk],
    logits [B,Q,n_blocks])``; the logits are computed in ``logits_compute``
    (default ``compute``). ``C_comp`` / ``K_IComp`` (the two compressions of
    the sequence) may be passed in when they are already known.
    """
    Bn, T, c = np.shape(Ca)
    if T % m:
        raise ValueError("csa_core_at: T must be a multiple of m")
    Q = np.asarray(queries, np.int64)
    nh = np.shape(q)[2]
    nb = T // m
    Ca = np.asarray(Ca, compute)
    if C_comp is None:
        C_comp = compress_kv_overlapped(Ca, Cb, Za, Zb, Ba, Bb, m, compute)
    if K_IComp is None:
        K_IComp = compress_kv(np.asarray(K_idx, compute), np.asarray(Z_idx, compute), B_idx, m,
                              compute)
    cbm = causal_block_mask(T, nb, m)[Q]
    lc = compute if logits_compute is None else logits_compute
    logits = indexer_logits(np.asarray(q_idx)[:, Q], K_IComp, np.asarray(w_idx)[:, Q], None, cbm,
                            normalize_qk, lc)
    if indices is None:
        idx = topk_desc_lowest_index(logits, topk) if topk else np.zeros((Bn, len(Q), 0), np.int64)
    else:
        idx = np.asarray(indices, np.int64)
    qq = np.asarray(q, compute)[:, Q]
    if normalize_qk:
        qn = l2_normalize(qq)
        Cn = l2_normalize(C_comp)
    else:
        qn, Cn = qq, C_comp
    if scale is None:
        scale = 1.0 if normalize_qk else c ** -0.5
    valid = idx >= 0
    kv = Cn[np.arange(Bn)[:, None, None], np.maximum(idx, 0)]
    scores = np.einsum('bthd,btkd->bthk', qn, kv) * compute(scale)
    scores = np.where(valid[:, :, None, :], scores, -np.inf)
    win = sliding_window
    if win > 0:
        C_local = l2_normalize(Ca) if normalize_qk else Ca
        pos = Q[:, None] - win + 1 + np.arange(win)[None, :]          # [Q, win]
        wvalid = pos >= 0
        Cw = C_local[:, np.maximum(pos, 0)]                            # [B, Q, win, c]
        sw = np.einsum('bthd,btwd->bthw', qn, Cw) * compute(scale)
        sw = np.where(wvalid[None, :, None, :], sw, -np.inf)
    else:
        wvalid = np.zeros((len(Q), 0), bool)
        Cw = np.zeros((Bn, len(Q), 0, c), compute)
        sw = np.zeros((Bn, len(Q), nh, 0), compute)
    cat = np.concatenate([scores, sw], axis=-1).astype(compute)
    cat_valid = np.concatenate(
        [valid[:, :, None, :],
         np.broadcast_to(wvalid[None, :, None, :], (Bn, len(Q), 1, wvalid.shape[-1]))], axis=-1)
    sink = None if sink_logits is None else np.asarray(sink_logits, compute).reshape(1, 1, nh, 1)
    p = joint_softmax_csa(cat, cat_valid, sink)
    k_ = scores.shape[-1]
    out = (np.einsum('bthk,btkd->bthd', p[..., :k_], kv)
           + np.einsum('bthw,btwd->bthd', p[..., k_:], Cw)).astype(compute)
    return out, idx, logits


def hca_core(C, Z, q, B_pos, *, m2, sliding_window=0, sink_logits=None,
             scale=1.0, C_local_raw=None, compute=np.float32):
    """HCA forward from the projections: ``[B,T,nh,c]`` in ``compute``."""
    Bn, T, c = np.shape(C)
    nh = np.shape(q)[2]
    pad = (-T) % m2
    C, Z, q = (_pad_time(np.asarray(x, compute), pad) for x in (C, Z, q))
    if C_local_raw is not None:
        C_local_raw = _pad_time(np.asarray(C_local_raw, compute), pad)
    Tp = T + pad
    nb = Tp // m2
    Cn = l2_normalize(compress_kv(C, Z, B_pos, m2, compute))
    qn = l2_normalize(q)
    cbm = causal_block_mask(Tp, nb, m2)
    scores = np.einsum('bthd,bnd->bhtn', qn, Cn) * compute(scale)
    scores = np.where(cbm[None, None], scores, -np.inf)
    if sliding_window > 0:
        C_local = l2_normalize(C if C_local_raw is None else C_local_raw)
        sw, Cw, _ = window_scores(qn, C_local, sliding_window, scale)
        sw = sw.transpose(0, 2, 1, 3)
    else:
        sw = np.zeros((Bn, nh, Tp, 0), compute)
        Cw = np.zeros((Bn, Tp, 0, c), compute)
    cat = np.concatenate([scores, sw], axis=-1).astype(compute)
    if cat.shape[-1] == 0:
        out = np.zeros((Bn, Tp, nh, c), compute)
    else:
        sink = None if sink_logits is None else np.asarray(sink_logits, compute).reshape(1, nh, 1, 1)
        p = joint_softmax_hca(cat, sink)
        out = (np.einsum('bhtn,bnd->bthd', p[..., :nb], Cn)
               + np.einsum('bhtw,btwd->bthd', p[..., nb:], Cw))
    return out[:, :T].astype(compute)


def hca_core_at(C, Z, q, B_pos, *, m2, queries, sliding_window=0, sink_logits=None,
                scale=1.0, compute=np.float32, C_comp=None):
    """``hca_core`` evaluated at the query positions ``queries`` only: the same
    arithmetic per query row (``ops_hca.py:132-194``); T a multiple of m2.
    ``C_comp`` (the compressed blocks, ``compress_kv(C, Z, B_pos, m2)``) may be
    passed in when it is already known. Returns ``[B, len(queries), nh, c]``."""
    Bn, T, c = np.shape(C)
    if T % m2:
        raise ValueError("hca_core_at: T must be a multiple of m2")
    Q = np.asarray(queries, np.int64)
    nh = np.shape(q)[2]
    nb = T // m2
    C = np.asarray(C, compute)
    if C_comp is None:
        C_comp = compress_kv(C, np.asarray(Z, compute), B_pos, m2, compute)
    Cn = l2_normalize(np.asarray(C_comp, compute))
    qn = l2_normalize(np.asarray(q, compute)[:, Q])
    cbm = causal_block_mask(T, nb, m2)[Q]                                 # [Q, nb]
    scores = np.einsum('bthd,bnd->bhtn', qn, Cn) * compute(scale)
    scores = np.where(cbm[None, None], scores, -np.inf)
    win = sliding_window
    if win > 0:
        C_local = l2_normalize(C)
        pos = Q[:, None] - win + 1 + np.arange(win)[None, :]
        Cw = C_local[:, np.maximum(pos, 0)]                                # [B, Q, win, c]
        sw = np.einsum('bthd,btwd->bhtw', qn, Cw) * compute(scale)
        sw = np.where((pos >= 0)[None, None], sw, -np.inf)
    else:
        Cw = np.zeros((Bn, len(Q), 0, c), compute)
        sw = np.zeros((Bn, nh, len(Q), 0), compute)
    cat = np.concatenate([scores, sw], axis=-1).astype(compute)
    sink = None if sink_logits is None else np.asarray(sink_logits, compute).reshape(1, nh, 1, 1)
    p = joint_softmax_hca(cat, sink)
    out = (np.einsum('bhtn,bnd->bthd', p[..., :nb], Cn)
           + np.einsum('bhtw,btwd->bthd', p[..., nb:], Cw))
    return out.astype(compute)


def linear_lowp(x, W, dtype='bf16'):
    """``F.linear`` on low-precision tensors: fp32 accumulate, rounded output."""
    y = np.asarray(x, np.float32) @ np.asarray(W, np.float32).T
    return round_to(y, dtype)


def csa_projections(H, W, dtype='bf16', *, c, cI, nh, nIh):
    """The fused 6-way projection plus cQ/q/q_idx/w_idx (``ops_csa.py:841-878,923``)."""
    Bn, T, _ = H.shape
    Ca = linear_lowp(H, W['W_aKV'], dtype)
    Cb = linear_lowp(H, W['W_bKV'], dtype)
    Za = linear_lowp(H, W['W_aZ'], dtype)
    Zb = linear_lowp(H, W['W_bZ'], dtype)
    K_idx = linear_lowp(H, W['W_KV_idx'], dtype)
    Z_idx = linear_lowp(H, W['W_Z_idx'], dtype)
    cQ = linear_lowp(H, W['W_DQ'], dtype)
    q_idx = linear_lowp(cQ, W['W_IUQ'], dtype).reshape(Bn, T, nIh, cI)
    w_idx = linear_lowp(H, W['W_w'], dtype)
    q = linear_lowp(cQ, W['W_UQ'], dtype).reshape(Bn, T, nh, c)
    return Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx


def naive_csa(H, W, *, m, topk, nh, nIh, c, c_I, sliding_window=0, sink=None,
              dtype='bf16', normalize_qk=True, indices=None):
    """Full CSA forward incl. projections; returns ``[B,T,nh*c]`` rounded to dtype.

    ``indices`` (``[B,T,topk]``) replaces the indexer's selection (see ``csa_core``)."""
    Bn, T, _ = H.shape
    proj = csa_projections(H, W, dtype, c=c, cI=c_I, nh=nh, nIh=nIh)
    out = csa_core(*proj, W['Ba'], W['Bb'], W['B_idx'], m=m, topk=topk,
                   sliding_window=sliding_window, sink_logits=sink,
                   normalize_qk=normalize_qk, indices=indices)
    return round_to(out.reshape(Bn, T, nh * c), dtype), proj


def naive_hca(H, W, *, m2, nh, c, sliding_window=0, sink=None, dtype='bf16'):
    Bn, T, _ = H.shape
    C = linear_lowp(H, W['W_KV'], dtype)
    Z = linear_lowp(H, W['W_Z'], dtype)
    cQ = linear_lowp(H, W['W_DQ'], dtype)
    q = linear_lowp(cQ, W['W_UQ'], dtype).reshape(Bn, T, nh, c)
    out = hca_core(C, Z, q, W['B_pos'], m2=m2, sliding_window=sliding_window,
                   sink_logits=sink)
    return round_to(out.reshape(Bn, T, nh * c), dtype), (C, Z, q)


def _l2n_grad(x, dy, eps=1e-12):
    """Backward of ``l2_normalize`` (``F.normalize``): for ``||x|| > eps``,
    ``dx = (dy - y (y . dy)) / ||x||`` with ``y = x / ||x||``."""
    n = np.sqrt((x * x).sum(-1, keepdims=True))
    big = n > eps
    nn = np.where(big, n, eps)
    y = x / nn
    return np.where(big, (dy - y * (y * dy).sum(-1, keepdims=True)) / nn, dy / nn)


def compress_kv_grad(C, Z, B_pos, m, d_out):
    """Backward of ``compress_kv`` (``ops_csa.py:198-234``) for ``d_out``
    ``[B, T//m, c]``. With ``w = softmax_j(Z + B)`` per channel over the m
    tokens of a block and ``r = sum_j w_j C_j``: ``dC_j = w_j dr``,
    ``dZ_j = w_j (C_j - r) dr``, ``dB_j = sum over blocks of dZ_j``.
    Returns ``(dC, dZ, dB)``."""
    C = np.asarray(C, np.float64)
    Z = np.asarray(Z, np.float64)
    Bn, T, c = C.shape
    nb = T // m
    Cb = C.reshape(Bn, nb, m, c)
    lg = Z.reshape(Bn, nb, m, c) + np.asarray(B_pos, np.float64)[None, None]
    e = np.exp(lg - lg.max(axis=2, keepdims=True))
    w = e / e.sum(axis=2, keepdims=True)
    r = (w * Cb).sum(axis=2, keepdims=True)
    dr = np.asarray(d_out, np.float64)[:, :, None]
    dC = (w * dr).reshape(Bn, T, c)
    dlg = w * (Cb - r) * dr
    return dC, dlg.reshape(Bn, T, c), dlg.sum(axis=(0, 1))


def hca_core_grad(C, Z, q, B_pos, d_out, *, m2, sliding_window=0, sink_logits=None,
                  scale=1.0, C_local_raw=None):
    """Gradients of ``hca_core`` (``ops_hca.py:132-194``, differentiated by
    autograd in the reference) for ``d_out = dL/dout`` ``[B,T,nh,c]``, in fp64.

    With ``p`` the joint softmax over the causal blocks, the window and the
    sink, keys ``k_j`` (= values) the L2-normalised compressed rows and window
    rows, ``qn`` the L2-normalised queries: ``dp_j = dout . k_j``,
    ``D = sum_j p_j dp_j``, ``ds_j = p_j (dp_j - D)``, ``dqn = scale sum_j ds_j
    k_j``, ``dk_j += scale ds_j qn + p_j dout``, ``dsink = -sum p_sink D``;
    then the L2-norm and compression backwards. Returns a dict with ``C, Z,
    q, B_pos`` and ``sink_logits`` / ``C_local_raw`` where given."""
    f = np.float64
    C, Z, q, d_out = (np.asarray(x, f) for x in (C, Z, q, d_out))
    Bn, T, c = C.shape
    nh = q.shape[2]
    pad = (-T) % m2
    Cp, Zp, qp, dop = (_pad_time(x, pad) for x in (C, Z, q, d_out))
    Clr = None if C_local_raw is None else _pad_time(np.asarray(C_local_raw, f), pad)
    Tp = T + pad
    nb = Tp // m2
    raw = compress_kv(Cp, Zp, B_pos, m2, f)
    Cn = l2_normalize(raw)
    qn = l2_normalize(qp)
    cbm = causal_block_mask(Tp, nb, m2)
    sc = np.einsum('bthd,bnd->bhtn', qn, Cn) * scale
    sc = np.where(cbm[None, None], sc, -np.inf)
    w = sliding_window
    src_local = Cp if Clr is None else Clr
    if w > 0:
        Cl = l2_normalize(src_local)
        sw, Cw, valid = window_scores(qn, Cl, w, scale)
        sw = sw.transpose(0, 2, 1, 3)
    else:
        Cl = None
        sw = np.zeros((Bn, nh, Tp, 0))
        Cw = np.zeros((Bn, Tp, 0, c))
    cat = np.concatenate([sc, sw], axis=-1)
    sink = None if sink_logits is None else np.asarray(sink_logits, f).reshape(1, nh, 1, 1)
    grads = {}
    if cat.shape[-1] == 0:
        p = np.zeros((Bn, nh, Tp, 0))
    else:
        p = joint_softmax_hca(cat, sink)
    pb, pw = p[..., :nb], p[..., nb:]
    out = np.einsum('bhtn,bnd->bthd', pb, Cn) + np.einsum('bhtw,btwd->bthd', pw, Cw)
    dp_b = np.einsum('bthd,bnd->bhtn', dop, Cn)
    dp_w = np.einsum('bthd,btwd->bhtw', dop, Cw)
    D = np.einsum('bthd,bthd->bht', dop, out)[..., None]
    ds_b = pb * (dp_b - D)
    ds_w = pw * (dp_w - D)
    dqn = scale * (np.einsum('bhtn,bnd->bthd', ds_b, Cn) + np.einsum('bhtw,btwd->bthd', ds_w, Cw))
    dCn = (scale * np.einsum('bhtn,bthd->bnd', ds_b, qn)
           + np.einsum('bhtn,bthd->bnd', pb, dop))
    dC = np.zeros_like(Cp)
    dq = _l2n_grad(qp, dqn)
    draw = _l2n_grad(raw, dCn)
    dCc, dZ, dB = compress_kv_grad(Cp, Zp, B_pos, m2, draw)
    dC += dCc
    if w > 0:
        dCw = (scale * np.einsum('bhtw,bthd->btwd', ds_w, qn)
               + np.einsum('bhtw,bthd->btwd', pw, dop))      # [B, T, w, c]
        dCl = np.zeros_like(Cl)
        for i in range(w):
            # slot i of query t is position t - w + 1 + i
            src = np.arange(Tp) - w + 1 + i
            ok = src >= 0
            np.add.at(dCl, (slice(None), src[ok]), dCw[:, ok, i])
        dloc = _l2n_grad(src_local, dCl)
        if Clr is None:
            dC += dloc
        else:
            grads['C_local_raw'] = dloc[:, :T]
    if sink is not None:
        row_max = cat.max(-1, keepdims=True) if cat.shape[-1] else np.zeros((Bn, nh, Tp, 1))
        row_max = np.where(np.isneginf(row_max), 0, row_max)
        with np.errstate(divide='ignore'):
            lse = np.log(np.exp(cat - row_max).sum(-1, keepdims=True)) + row_max
        p_sink = np.exp(sink - np.logaddexp(lse, sink))
        grads['sink_logits'] = -(p_sink * D).sum(axis=(0, 2, 3))
    grads.update(C=dC[:, :T], Z=dZ[:, :T], q=dq[:, :T], B_pos=dB)
    return grads


def compress_kv_overlapped_grad(Ca, Cb, Za, Zb, Ba, Bb, m, d_out):
    """Backward of ``compress_kv_overlapped`` (``ops_csa.py:237-305``): block
    i's softmax runs over the 2m logits ``Za_i + Ba`` and ``Zb_{i-1} + Bb``
    (block 0: the second half is -inf, ``Cb_{-1} = 0``); with ``r`` the block's
    row and ``dr`` its cotangent, each weight ``w`` of value ``x`` gets
    ``dx = w dr`` and ``dlogit = w (x - r) dr``. Returns ``(dCa, dCb, dZa,
    dZb, dBa, dBb)``."""
    f = np.float64
    Ca, Cb, Za, Zb = (np.asarray(x, f) for x in (Ca, Cb, Za, Zb))
    Bn, T, c = Ca.shape
    nb = T // m
    Ca4, Cb4, Za4, Zb4 = (x.reshape(Bn, nb, m, c) for x in (Ca, Cb, Za, Zb))
    a_log = Za4 + np.asarray(Ba, f)[None, None]
    zb_prev = np.concatenate([np.full((Bn, 1, m, c), -np.inf), Zb4[:, :-1]], axis=1)
    b_log = zb_prev + np.asarray(Bb, f)[None, None]
    allg = np.concatenate([a_log, b_log], axis=2)
    e = np.exp(allg - allg.max(axis=2, keepdims=True))
    S = e / e.sum(axis=2, keepdims=True)
    cb_prev = np.concatenate([np.zeros((Bn, 1, m, c)), Cb4[:, :-1]], axis=1)
    vals = np.concatenate([Ca4, cb_prev], axis=2)
    r = (S * vals).sum(axis=2, keepdims=True)
    dr = np.asarray(d_out, f)[:, :, None]
    dv = S * dr
    dl = S * (vals - r) * dr
    dCa = dv[:, :, :m].reshape(Bn, T, c)
    dZa = dl[:, :, :m].reshape(Bn, T, c)
    dCb = np.zeros((Bn, nb, m, c))
    dZb = np.zeros((Bn, nb, m, c))
    dCb[:, :-1] = dv[:, 1:, m:]
    dZb[:, :-1] = dl[:, 1:, m:]
    return (dCa, dCb.reshape(Bn, T, c), dZa, dZb.reshape(Bn, T, c), dl[:, :, :m].sum((0, 1)),
            dl[:, 1:, m:].sum((0, 1)))


def csa_attn_grad(Ca, Cb, Za, Zb, q, Ba, Bb, idx, d_out, *, m, sliding_window=0,
                  sink_logits=None, normalize_qk=True, scale=None):
    """Gradients of ``csa_core``'s attention (``ops_csa.py:869-1155``) with the
    selection ``idx`` ``[B,T,topk]`` (-1 = unused) held fixed, in fp64; T a
    multiple of m. Same algebra as ``hca_core_grad`` over the selected rows,
    the window rows of ``Ca`` and the sink, then the overlapped compression
    backward. Also returns ``slot``: per selected slot, the gradient of the
    gathered row dotted with that row (``sum_h p ((dp - D) s + dp)``), the
    quantity the STE surrogate (``ops_csa.py:1033-1099``) turns into the
    indexer's gradient, and ``gsum`` ``[B,T,c]``: the gathered rows'
    gradients summed over the slots (the cotangent of ``full_softmax``'s
    zero-in-forward term, ``ops_csa.py:1050-1071``)."""
    f = np.float64
    Ca, Cb, Za, Zb, q, d_out = (np.asarray(x, f) for x in (Ca, Cb, Za, Zb, q, d_out))
    Bn, T, c = Ca.shape
    nh = q.shape[2]
    nb = T // m
    idx = np.asarray(idx, np.int64)
    if scale is None:
        scale = 1.0 if normalize_qk else c ** -0.5
    raw = compress_kv_overlapped(Ca, Cb, Za, Zb, Ba, Bb, m, f)
    Cn = l2_normalize(raw) if normalize_qk else raw
    qn = l2_normalize(q) if normalize_qk else q
    topk = idx.shape[-1]
    valid = idx >= 0
    kv = Cn[np.arange(Bn)[:, None, None], np.maximum(idx, 0)]            # [B,T,k,c]
    s_k = np.einsum('bthd,btkd->bthk', qn, kv) * scale
    s_k = np.where(valid[:, :, None, :], s_k, -np.inf)
    w = sliding_window
    if w > 0:
        Cl = l2_normalize(Ca) if normalize_qk else Ca
        s_w, Cw, wvalid = window_scores(qn, Cl, w, scale)
    else:
        s_w = np.zeros((Bn, T, nh, 0))
        Cw = np.zeros((Bn, T, 0, c))
        wvalid = np.zeros((T, 0), bool)
    cat = np.concatenate([s_k, s_w], axis=-1)
    cat_valid = np.concatenate(
        [np.broadcast_to(valid[:, :, None, :], (Bn, T, nh, topk)),
         np.broadcast_to(wvalid[None, :, None, :], (Bn, T, nh, wvalid.shape[-1]))], axis=-1)
    sink = None if sink_logits is None else np.asarray(sink_logits, f).reshape(1, 1, nh, 1)
    if cat.shape[-1]:
        p = joint_softmax_csa(cat, cat_valid, sink)
    else:
        p = np.zeros((Bn, T, nh, 0))
    pk, pw = p[..., :topk], p[..., topk:]
    out = np.einsum('bthk,btkd->bthd', pk, kv) + np.einsum('bthw,btwd->bthd', pw, Cw)
    dp_k = np.einsum('bthd,btkd->bthk', d_out, kv)
    dp_w = np.einsum('bthd,btwd->bthw', d_out, Cw)
    D = np.einsum('bthd,bthd->bth', d_out, out)[..., None]
    ds_k = pk * (dp_k - D)
    ds_w = pw * (dp_w - D)
    dqn = scale * (np.einsum('bthk,btkd->bthd', ds_k, kv) + np.einsum('bthw,btwd->bthd', ds_w, Cw))
    dkv = scale * np.einsum('bthk,bthd->btkd', ds_k, qn) + np.einsum('bthk,bthd->btkd', pk, d_out)
    slot = np.where(valid, (dkv * kv).sum(-1), 0.0)
    dCn = np.zeros((Bn, nb, c))
    bi = np.broadcast_to(np.arange(Bn)[:, None, None], idx.shape)
    np.add.at(dCn, (bi[valid], idx[valid]), dkv[valid])
    dq = _l2n_grad(q, dqn) if normalize_qk else dqn
    draw = _l2n_grad(raw, dCn) if normalize_qk else dCn
    dCa, dCb, dZa, dZb, dBa, dBb = compress_kv_overlapped_grad(Ca, Cb, Za, Zb, Ba, Bb, m, draw)
    if w > 0:
        dCw = scale * np.einsum('bthw,bthd->btwd', ds_w, qn) + np.einsum('bthw,bthd->btwd', pw, d_out)
        dCl = np.zeros((Bn, T, c))
        for i in range(w):
            src = np.arange(T) - w + 1 + i
            ok = src >= 0
            np.add.at(dCl, (slice(None), src[ok]), dCw[:, ok, i])
        dCa = dCa + (_l2n_grad(Ca, dCl) if normalize_qk else dCl)
    g = dict(Ca=dCa, Cb=dCb, Za=dZa, Zb=dZb, q=dq, Ba=dBa, Bb=dBb, slot=slot,
             gsum=dkv.sum(axis=2))
    if sink is not None:
        row_max = np.maximum(np.where(cat_valid, cat, -np.inf).max(-1, keepdims=True), 0) \
            if cat.shape[-1] else np.zeros((Bn, T, nh, 1))
        with np.errstate(divide='ignore', invalid='ignore'):
            lse = np.log(np.where(cat_valid, np.exp(cat - row_max), 0).sum(-1, keepdims=True)) + row_max
        p_sink = np.exp(sink - np.logaddexp(lse, sink))
        g['sink_logits'] = -(p_sink * D).sum(axis=(0, 1, 3))
    return g


def csa_ste_grad(Ca, Cb, Za, Zb, K_idx, Z_idx, q, q_idx, w_idx, Ba, Bb, B_idx, idx, d_out, *,
                 m, sliding_window=0, sink_logits=None, normalize_qk=True, scale=None,
                 ste_mode='topk_columns'):
    """Gradients of ``csa_core`` with the straight-through surrogate
    (``ops_csa.py:1033-1099``), the selection ``idx`` held fixed, in fp64; T a
    multiple of m.

    The forward value is the hard top-k path; the backward adds, through
    ``kv + (soft_kv - soft_kv.detach())`` with ``soft_kv = soft[idx] kv``:

    * the soft weights' cotangent: ``slot`` (``csa_attn_grad``) at the selected
      columns; with ``ste_mode='full_softmax'`` also ``gsum C_comp_n^T`` at
      every column, and ``C_comp_n`` receives ``soft^T gsum`` (the expected
      row ``soft @ C_comp_n``, broadcast over the slots, enters as
      ``aux - aux.detach()``, ``ops_csa.py:1050-1071``);
    * the softmax backward over the causal blocks (``ops_csa.py:545-572``),
      ``dl = soft (dsoft - sum soft dsoft)``;
    * the indexer logits ``lg = sum_h w_h relu(a_h)``,
      ``a_h = scale qn_h . kn`` (``ops_csa.py:503-536``): ``dw_h = sum_n dl
      relu(a_h)``, ``da_h = dl w_h [a_h > 0]``, then ``dqn``, ``dkn``;
    * the L2-norm backwards and the key compression's (``ops_csa.py:198-234``).

    Returns the dict of ``csa_attn_grad`` plus ``K_idx, Z_idx, q_idx, w_idx,
    B_idx``."""
    if ste_mode not in ('topk_columns', 'full_softmax'):
        raise ValueError(f"ste_mode={ste_mode!r}")
    f = np.float64
    g = csa_attn_grad(Ca, Cb, Za, Zb, q, Ba, Bb, idx, d_out, m=m, sliding_window=sliding_window,
                      sink_logits=sink_logits, normalize_qk=normalize_qk, scale=scale)
    Bn, T, c = np.shape(Ca)
    nb = T // m
    cI = np.shape(K_idx)[-1]
    kraw = compress_kv(np.asarray(K_idx, f), np.asarray(Z_idx, f), B_idx, m, f)
    kn = l2_normalize(kraw) if normalize_qk else kraw
    qi = np.asarray(q_idx, f)
    qin = l2_normalize(qi) if normalize_qk else qi
    iscale = 1.0 if normalize_qk else cI ** -0.5
    w = np.asarray(w_idx, f)
    a = np.einsum('bthd,bnd->bthn', qin, kn) * iscale
    relu = np.maximum(a, 0.0)
    lg = np.einsum('bthn,bth->btn', relu, w)
    lg = np.where(causal_block_mask(T, nb, m)[None], lg, -np.inf)
    finite = np.isfinite(lg)
    any_vis = finite.any(-1, keepdims=True)
    mx = np.where(any_vis, np.where(finite, lg, -np.inf).max(-1, keepdims=True), 0.0)
    e = np.where(finite, np.exp(np.where(finite, lg, 0.0) - mx), 0.0)
    soft = np.where(any_vis, e / np.where(any_vis, e.sum(-1, keepdims=True), 1.0), 0.0)
    idx = np.asarray(idx, np.int64)
    valid = idx >= 0
    dsoft = np.zeros((Bn, T, nb))
    bi, ti = np.broadcast_to(np.arange(Bn)[:, None, None], idx.shape), \
        np.broadcast_to(np.arange(T)[None, :, None], idx.shape)
    np.add.at(dsoft, (bi[valid], ti[valid], idx[valid]), g['slot'][valid])
    if ste_mode == 'full_softmax':
        raw = compress_kv_overlapped(np.asarray(Ca, f), Cb, Za, Zb, Ba, Bb, m, f)
        cn = l2_normalize(raw) if normalize_qk else raw
        dsoft = dsoft + np.einsum('btc,bnc->btn', g['gsum'], cn)
        dcn = np.einsum('btn,btc->bnc', soft, g['gsum'])
        draw = _l2n_grad(raw, dcn) if normalize_qk else dcn
        for name, x in zip(('Ca', 'Cb', 'Za', 'Zb', 'Ba', 'Bb'),
                           compress_kv_overlapped_grad(Ca, Cb, Za, Zb, Ba, Bb, m, draw)):
            g[name] = g[name] + x
    dl = soft * (dsoft - (soft * dsoft).sum(-1, keepdims=True))
    dw = np.einsum('btn,bthn->bth', dl, relu)
    da = dl[:, :, None, :] * w[..., None] * (a > 0)
    dqin = iscale * np.einsum('bthn,bnd->bthd', da, kn)
    dkn = iscale * np.einsum('bthn,bthd->bnd', da, qin)
    dqi = _l2n_grad(qi, dqin) if normalize_qk else dqin
    dkraw = _l2n_grad(kraw, dkn) if normalize_qk else dkn
    dK, dZ, dB = compress_kv_grad(K_idx, Z_idx, B_idx, m, dkraw)
    g.update(K_idx=dK, Z_idx=dZ, q_idx=dqi, w_idx=dw, B_idx=dB)
    return g
