"""Incremental CSA / HCA decode state on the HIP backend.

Drop-in twins of ``/root/reference/ops_decoding_cache.py``:

``SlidingWindowRingBuffer``  <- ``_SlidingWindowRingBuffer`` (``:251-400``)
``CSADecodingCache``         <- ``CSADecodingCache`` (``:407-1070``)
``HCADecodingCache``         <- ``HCADecodingCache`` (``:1077-1395``)

Same constructors, ``append_step`` / ``forward_step`` / ``reset`` / ``to``,
properties (``n_tokens_seen``, ``n_blocks``, ``accumulator_len``,
``C_comp``, ``K_IComp``, ``sw_buffer``) and the ``_normalize_qk`` attribute.

State lives in GPU tensors instead of Python lists:

* the partial-block accumulator is a ``[B, m, width]`` buffer per projection;
* completed blocks are compressed by ``kch_compress(_overlapped)`` in one
  launch per ``append_step`` (however many blocks it completes, so a prefill
  populates the cache in bulk), rounded to the cache dtype as the reference
  stores them (``:750-763``), with the previous block's ``Cb / Zb`` kept for
  the overlap;
* the L2-normalised bf16 attention rows and the indexer keys' inverse norms
  are produced once per new block, where the reference re-normalises every
  cached block on every step (``:919-924``); the indexer reads the stored
  rows (cache dtype) times their inverse norm;
* ``forward_step`` is one ``kch_csa_decode`` / ``kch_hca_decode`` call: the
  indexer, top-k and the joint sparse/window/sink softmax, each split across
  the cache so that a step streams it at memory bandwidth.

Forward only (``use_ste`` does not change the forward value); float64 caches
are not supported.
"""

from __future__ import annotations

import torch

from . import _lib, ops_csa
from .ops_csa import (_HEAD_DIMS, _IDX_DIMS, _IDX_HEADS, _aligned, _compress,
                      _compress_overlapped, _f32, _head_groups, _kernel_size, _pad_last,
                      l2_normalize_rows)


def _validate_cache_dtype(dtype) -> None:
    try:
        is_float = torch.empty((), dtype=dtype).is_floating_point()
    except (TypeError, RuntimeError) as exc:
        raise TypeError(f'cache dtype must be a floating torch.dtype, got {dtype!r}') from exc
    if not is_float:
        raise TypeError(f'cache dtype must be floating-point, got {dtype!r}')
    if dtype == torch.float64:
        raise NotImplementedError("float64 caches are not supported by the HIP kernels")


class SlidingWindowRingBuffer:
    """FIFO of the last ``win`` entries ``[B, c]``; the i-th entry ever written
    sits at row ``i % win`` (``ops_decoding_cache.py:321-357``)."""

    def __init__(self, B: int, win: int, c: int, device, dtype):
        if win < 1:
            raise ValueError(
                f"_SlidingWindowRingBuffer: win={win} must be >= 1 "
                f"(win=0 disables the SW branch and should bypass this class entirely).")
        self.B, self.win, self.c = B, win, c
        self.device, self.dtype = torch.device(device), dtype
        self._buf = torch.zeros(B, win, c, device=self.device, dtype=dtype)
        self._written = 0

    def reset(self) -> None:
        self._buf.zero_()
        self._written = 0

    def append(self, x: torch.Tensor) -> None:
        """Append ``x`` ``[B, T_new, c]`` (oldest first)."""
        if x.dim() != 3 or x.shape[0] != self.B or x.shape[-1] != self.c:
            raise ValueError(
                f"_SlidingWindowRingBuffer.append: expected [{self.B}, T_new, {self.c}], "
                f"got {tuple(x.shape)}.")
        x = x.to(device=self._buf.device, dtype=self._buf.dtype)
        T_new = x.shape[1]
        if T_new == 0:
            return
        keep = min(T_new, self.win)
        first = (self._written + T_new - keep) % self.win
        src = x[:, T_new - keep:]
        # ring positions first, first + 1, ... (mod win): at most two runs
        n1 = min(keep, self.win - first)
        self._buf[:, first:first + n1] = src[:, :n1]
        if keep > n1:
            self._buf[:, :keep - n1] = src[:, n1:]
        self._written += T_new

    @property
    def n_valid(self) -> int:
        return min(self._written, self.win)

    @property
    def _sw_len(self) -> int:
        return self.n_valid

    @property
    def _sw_head(self) -> int:
        return 0 if self._written < self.win else self._written % self.win

    def get(self) -> torch.Tensor:
        """Contents in causal order (oldest first), ``[B, n_valid, c]``."""
        n = self.n_valid
        if n < self.win:
            return self._buf[:, :n]
        h = self._sw_head
        return self._buf if h == 0 else torch.cat([self._buf[:, h:], self._buf[:, :h]], dim=1)

    def raw(self) -> torch.Tensor:
        """The storage ``[B, win, c]``; its first ``n_valid`` rows are the window."""
        return self._buf

    def to(self, device=None, dtype=None) -> 'SlidingWindowRingBuffer':
        if device is not None:
            self._buf = self._buf.to(device=torch.device(device))
            self.device = self._buf.device
        if dtype is not None and dtype != self._buf.dtype:
            self._buf = self._buf.to(dtype=dtype)
            self.dtype = dtype
        return self


class _BlockStore:
    """Geometric-capacity rows ``[B, cap, width]`` in the cache dtype plus, per
    row, either the attention copy (``key_dtype``: bf16 or fp32, optionally
    L2-normalised) or, with ``key_dtype=None``, the fp32 ``1 / max(||row||,
    1e-12)`` of the stored row (``inv``)."""

    def __init__(self, B, width, device, dtype, key_dtype):
        self.B, self.width, self.device, self.dtype, self.key_dtype = B, width, device, dtype, key_dtype
        self.rows = None
        self.keys = None
        self.inv = None
        self.key_norm = None

    def ensure(self, n_valid, required):
        if self.rows is not None and required <= self.rows.shape[1]:
            return
        old = 0 if self.rows is None else self.rows.shape[1]
        cap = max(required, max(1, old * 2))
        rows = torch.empty(self.B, cap, self.width, device=self.device, dtype=self.dtype)
        if self.key_dtype is not None:
            keys = torch.empty(self.B, cap, self.width, device=self.device, dtype=self.key_dtype)
        else:
            keys = None
            inv = torch.empty(self.B, cap, device=self.device, dtype=torch.float32)
        if n_valid:
            rows[:, :n_valid] = self.rows[:, :n_valid]
            if keys is not None:
                keys[:, :n_valid] = self.keys[:, :n_valid]
            else:
                inv[:, :n_valid] = self.inv[:, :n_valid]
        self.rows, self.keys = rows, keys
        if keys is None:
            self.inv = inv

    def _inv_of(self, rows):
        return rows.float().norm(dim=-1).clamp_min(1e-12).reciprocal()

    def push(self, n_valid, new_rows, normalize):
        k = new_rows.shape[1]
        self.ensure(n_valid, n_valid + k)
        self.rows[:, n_valid:n_valid + k] = new_rows.to(self.dtype)
        if self.key_dtype is None:
            self.inv[:, n_valid:n_valid + k] = self._inv_of(self.rows[:, n_valid:n_valid + k])
            return
        if self.key_norm is None:
            self.key_norm = normalize
        self.keys[:, n_valid:n_valid + k] = l2_normalize_rows(
            self.rows[:, n_valid:n_valid + k], out_dtype=self.key_dtype,
            normalize=self.key_norm)

    def keys_for(self, n_valid, normalize):
        """Attention rows normalised as asked (rebuilt if the flag changed)."""
        if self.rows is not None and n_valid and self.key_norm != normalize:
            self.keys[:, :n_valid] = l2_normalize_rows(self.rows[:, :n_valid],
                                                       out_dtype=self.key_dtype,
                                                       normalize=normalize)
            self.key_norm = normalize
        return self.keys

    def to(self, device, dtype, n_valid):
        self.device, self.dtype = device, dtype
        if self.rows is not None:
            self.rows = self.rows.to(device=device, dtype=dtype)
            if self.key_dtype is None:
                self.inv = self.inv.to(device=device)
                if n_valid:
                    self.inv[:, :n_valid] = self._inv_of(self.rows[:, :n_valid])
                return
            self.keys = self.keys.to(device=device)
            if n_valid:
                self.keys[:, :n_valid] = l2_normalize_rows(
                    self.rows[:, :n_valid], out_dtype=self.key_dtype,
                    normalize=bool(self.key_norm))


def _device(device):
    d = torch.device(device)
    if d.type == 'cuda' and d.index is None and torch.cuda.is_available():
        d = torch.device('cuda', torch.cuda.current_device())
    return d


def _ring_bf16(sw):
    buf = sw.raw()
    return buf if buf.dtype == torch.bfloat16 else buf.to(torch.bfloat16)


def _alloc_acc(new, B, m):
    """Accumulators for the projections of a block still being filled: one
    ``[B, m, sum of widths]`` buffer split into per-input views when the inputs
    share a dtype (so that one copy can fill them all), else separate buffers."""
    widths = [x.shape[-1] for x in new]
    dt, dev = new[0].dtype, new[0].device
    if all(x.dtype == dt for x in new):
        buf = torch.empty(B, m, sum(widths), device=dev, dtype=dt)
        return buf, list(buf.split(widths, -1))
    return None, [torch.empty(B, m, w, device=dev, dtype=x.dtype) for w, x in zip(widths, new)]


def _column_group(ts):
    """One ``[..., sum of widths]`` view over ``ts`` when they are adjacent column
    ranges of one tensor (the slices of one projection output), else None."""
    t0 = ts[0]
    st = t0.stride()
    if st[-1] != 1:
        return None
    lead, dt, es = t0.shape[:-1], t0.dtype, t0.element_size()
    p, w = t0.data_ptr(), 0
    for t in ts:
        if t.dtype != dt or t.stride() != st or t.shape[:-1] != lead or t.data_ptr() != p + w * es:
            return None
        w += t.shape[-1]
    return t0.as_strided((*lead, w), st)


def _ring_rows(x, dtype, normalize):
    """Sliding-window rows of ``x``: L2-normalised in fp32 and rounded to the
    cache dtype (the kernel writes bf16 itself, rounding the same fp32 value)."""
    if dtype == torch.bfloat16:
        return l2_normalize_rows(x, out_dtype=torch.bfloat16, normalize=normalize)
    return l2_normalize_rows(x, out_dtype=torch.float32, normalize=normalize).to(dtype)


class CSADecodingCache:
    """CSA incremental decode state (``ops_decoding_cache.py:407-1070``) on the HIP backend."""

    def __init__(self, B: int, c: int, c_I: int, m: int, win: int, device, dtype):
        if B < 1:
            raise ValueError(f"B={B} must be >= 1")
        if c < 1:
            raise ValueError(f"c={c} must be >= 1")
        if c_I < 1:
            raise ValueError(f"c_I={c_I} must be >= 1")
        if m < 1:
            raise ValueError(f"m={m} must be >= 1")
        if win < 0:
            raise ValueError(f"win={win} must be >= 0 (0 disables SW)")
        self.B, self.c, self.c_I, self.m, self.win = B, c, c_I, m, win
        _validate_cache_dtype(dtype)
        self.device, self.dtype = _device(device), dtype
        self._normalize_qk: bool = True
        self.reset()

    def reset(self) -> None:
        self._acc = None          # 6 buffers [B, m, width] (projection dtype)
        self._acc_buf = None      # the buffer they are views of, if one
        self._acc_len = 0
        self._prev = None         # (Cb, Zb) of the last completed block, [B, m, c]:
        self._prev_buf = None     # views of one [B, m, 2c] buffer at a fixed address
        self._C = _BlockStore(self.B, self.c, self.device, self.dtype, torch.bfloat16)
        # indexer keys: the stored rows and their inverse norms (no normalised copy)
        self._K = _BlockStore(self.B, self.c_I, self.device, self.dtype, None)
        self._sw = (SlidingWindowRingBuffer(self.B, self.win, self.c, self.device, self.dtype)
                    if self.win > 0 else None)
        self._n_tokens_seen = 0
        self._n_blocks = 0

    @property
    def n_tokens_seen(self) -> int:
        return self._n_tokens_seen

    @property
    def n_blocks(self) -> int:
        return self._n_blocks

    @property
    def accumulator_len(self) -> int:
        return self._acc_len

    @property
    def C_comp(self):
        return None if self._C.rows is None else self._C.rows[:, :self._n_blocks]

    @property
    def K_IComp(self):
        return None if self._K.rows is None else self._K.rows[:, :self._n_blocks]

    @property
    def sw_buffer(self):
        return self._sw

    def to(self, device=None, dtype=None) -> 'CSADecodingCache':
        if device is not None:
            self.device = torch.device(device)
        if dtype is not None:
            _validate_cache_dtype(dtype)
            self.dtype = dtype
        if self._acc_buf is not None:
            self._acc_buf = self._acc_buf.to(device=self.device)
            self._acc = list(self._acc_buf.split([a.shape[-1] for a in self._acc], -1))
        elif self._acc is not None:
            self._acc = [a.to(device=self.device) for a in self._acc]
        if self._prev_buf is not None:
            self._set_prev_buf(self._prev_buf.to(device=self.device))
        self._C.to(self.device, self.dtype, self._n_blocks)
        self._K.to(self.device, self.dtype, self._n_blocks)
        if self._sw is not None:
            self._sw.to(device=self.device, dtype=self.dtype)
        return self

    def append_step(self, Ca_new, Cb_new, Za_new, Zb_new, K_idx_new, Z_idx_new, Ba, Bb, B_idx):
        """Append ``T_new`` tokens' projections; returns the new block indices."""
        B, T_new, c = Ca_new.shape
        if B != self.B:
            raise ValueError(
                f"CSADecodingCache.append_step: batch size {B} does not match cache's "
                f"B={self.B}. Call reset() between sequences with different batch sizes.")
        if c != self.c:
            raise ValueError(
                f"CSADecodingCache.append_step: c={c} does not match cache's c={self.c}.")
        if K_idx_new.shape[-1] != self.c_I:
            raise ValueError(
                f"CSADecodingCache.append_step: c_I={K_idx_new.shape[-1]} does not match "
                f"cache's c_I={self.c_I}.")
        for _name, _t in [('Cb_new', Cb_new), ('Za_new', Za_new), ('Zb_new', Zb_new),
                          ('K_idx_new', K_idx_new), ('Z_idx_new', Z_idx_new)]:
            if _t.shape[1] != T_new:
                raise ValueError(
                    f"CSADecodingCache.append_step: {_name}.shape[1]={_t.shape[1]} does not "
                    f"match Ca_new.shape[1]={T_new}. All inputs must share the same T_new.")
        if T_new == 0:
            return []
        _lib.require_gpu("CSADecodingCache.append_step", Ca_new)
        new = [Ca_new, Cb_new, Za_new, Zb_new, K_idx_new, Z_idx_new]
        with torch.no_grad():
            if self._sw is not None:
                self._sw.append(_ring_rows(Ca_new, self.dtype, self._normalize_qk))
            if self._acc is None:
                self._acc_buf, self._acc = _alloc_acc(new, B, self.m)
            total = self._acc_len + T_new
            nfull = total // self.m
            rem = total - nfull * self.m
            out_idx = []
            if nfull:
                take = nfull * self.m - self._acc_len
                toks = [torch.cat([a[:, :self._acc_len], x[:, :take].to(a.dtype)], dim=1)
                        for a, x in zip(self._acc, new)]
                Ca, Cb, Za, Zb, Ki, Zi = toks
                if self._prev is not None:
                    z = torch.zeros_like(Ca[:, :self.m])
                    Ca_s, Za_s = torch.cat([z, Ca], 1), torch.cat([z, Za], 1)
                    Cb_s, Zb_s = torch.cat([self._prev[0], Cb], 1), torch.cat([self._prev[1], Zb], 1)
                    rows = _compress_overlapped("CSADecodingCache", Ca_s, Cb_s, Za_s, Zb_s, Ba, Bb,
                                                self.m)[:, 1:]
                else:
                    rows = _compress_overlapped("CSADecodingCache", Ca, Cb, Za, Zb, Ba, Bb, self.m)
                krows = _compress("CSADecodingCache", Ki, Zi, B_idx, self.m)
                self._C.push(self._n_blocks, rows, self._normalize_qk)
                self._K.push(self._n_blocks, krows, self._normalize_qk)
                out_idx = list(range(self._n_blocks, self._n_blocks + nfull))
                self._n_blocks += nfull
                if self._prev_buf is None or self._prev_buf.dtype != Cb.dtype:
                    self._set_prev_buf(torch.empty(B, self.m, 2 * c, device=Cb.device,
                                                   dtype=Cb.dtype))
                self._prev[0].copy_(Cb[:, -self.m:])
                self._prev[1].copy_(Zb[:, -self.m:])
                for a, x in zip(self._acc, new):
                    if rem:
                        a[:, :rem] = x[:, T_new - rem:].to(a.dtype)
            else:
                grp = None if self._acc_buf is None else _column_group(new)
                if grp is not None and grp.dtype == self._acc_buf.dtype:
                    self._acc_buf[:, self._acc_len:total] = grp
                else:
                    for a, x in zip(self._acc, new):
                        a[:, self._acc_len:total] = x.to(a.dtype)
            self._acc_len = rem
            self._n_tokens_seen += T_new
        return out_idx

    def _set_prev_buf(self, buf):
        self._prev_buf = buf
        self._prev = (buf[..., :self.c], buf[..., self.c:])

    # ---- device-driven steps (kch_csa_cache_append, kch_csa_decode_dyn) ----
    def _device_ready(self, dtype) -> bool:
        """Whether one-token device steps can continue this cache in place: the
        accumulator is one buffer of the step's dtype (or none yet), and so are
        the block stores."""
        if self.dtype != dtype:
            return False
        if self._acc is not None and (self._acc_buf is None or self._acc_buf.dtype != dtype):
            return False
        return self._prev_buf is None or self._prev_buf.dtype == dtype

    def _device_buffers(self, headroom: int = 1):
        """Allocate what a device step writes and return the block capacity:
        room for the block the next token may complete (``headroom`` blocks past
        the current ones, doubling the storage when it grows)."""
        B, m, c, cI = self.B, self.m, self.c, self.c_I
        if self._acc is None:
            self._acc_buf = torch.empty(B, m, 4 * c + 2 * cI, device=self.device, dtype=self.dtype)
            self._acc = list(self._acc_buf.split([c, c, c, c, cI, cI], -1))
        if self._prev_buf is None:
            self._set_prev_buf(torch.zeros(B, m, 2 * c, device=self.device, dtype=self.dtype))
        need = max(1, self._n_blocks + headroom)
        self._C.ensure(self._n_blocks, need)
        self._K.ensure(self._n_blocks, need)
        if self._C.key_norm is None:
            self._C.key_norm = self._normalize_qk
        return min(self._C.rows.shape[1], self._K.rows.shape[1])

    def _device_advance(self) -> None:
        """The host counters after one token appended on the device."""
        n = self._n_tokens_seen
        if self._sw is not None:
            self._sw._written += 1
        if n % self.m == self.m - 1:
            self._n_blocks += 1
        self._acc_len = (n + 1) % self.m
        self._n_tokens_seen = n + 1

    def forward_step(self, q, q_idx, w_idx, *, topk, nh, nIh, scale=None, sink_logits=None,
                     use_ste=True, ste_mode='topk_columns', normalize_qk=True,
                     _normalize_q=False, _out_dtype=None):
        """CSA output ``[B, 1, nh, c]`` (fp32) for the last appended token.

        ``_normalize_q`` (internal): L2-normalise ``q`` in the kernel (the
        caller passes the raw projection); ``_out_dtype``: output dtype."""
        B, T_new = q.shape[0], q.shape[1]
        if T_new != 1:
            raise ValueError(
                f"CSADecodingCache.forward_step: T_new={T_new} must be 1. For multi-token "
                f"chunks, call append_step + forward_step in a loop (or use naive_csa on the "
                f"full chunk and populate the cache via the prefill path).")
        if B != self.B:
            raise ValueError(
                f"CSADecodingCache.forward_step: batch size {B} does not match cache's B={self.B}.")
        if q.shape[2] != nh:
            raise ValueError(f"q.shape[2]={q.shape[2]} does not match nh={nh}.")
        if q_idx.shape[2] != nIh:
            raise ValueError(f"q_idx.shape[2]={q_idx.shape[2]} does not match nIh={nIh}.")
        if q.device != self.device:
            raise ValueError(
                f"CSADecodingCache.forward_step: q.device={q.device} does not match cache's "
                f"device={self.device}. Call cache.to(device=q.device) or move q to the cache's "
                f"device.")
        if ste_mode not in ('topk_columns', 'full_softmax', 'aux_contrastive'):
            raise ValueError(
                f"ste_mode={ste_mode!r} must be one of 'topk_columns', "
                f"'full_softmax', or 'aux_contrastive'.")
        _lib.require_gpu("CSADecodingCache.forward_step", q)
        core_scale = (1.0 if normalize_qk else self.c ** -0.5) if scale is None else scale
        nb = self._n_blocks
        n_win = self._sw.n_valid if self._sw is not None else 0
        odt = torch.float32 if _out_dtype is None else _out_dtype
        if nb == 0 and n_win == 0:
            return torch.zeros(B, 1, nh, self.c, device=q.device, dtype=odt)
        if q.dtype == torch.float64:
            raise NotImplementedError("float64 queries are not supported by the HIP kernels")
        fn = "CSADecodingCache.forward_step"
        c, cI = self.c, self.c_I
        cp = _kernel_size(fn, "c", c, _HEAD_DIMS)
        cIp = _kernel_size(fn, "c_I", cI, _IDX_DIMS)
        nIp = _kernel_size(fn, "nIh", nIh, _IDX_HEADS)
        out = torch.empty(B, 1, nh, cp, device=q.device, dtype=odt)
        with torch.no_grad():
            kv = self._C.keys_for(nb, normalize_qk) if nb else None
            krows = self._K.rows if nb else None
            kinv = self._K.inv if (nb and normalize_qk) else None
            ring = _ring_bf16(self._sw) if n_win else None
            qi = q_idx.to(q.dtype)
            wi = None if w_idx is None else w_idx.to(q.dtype)
            if (cp, cIp, nIp) != (c, cI, nIh):
                # sizes between the kernels' own: zero-padded copies of this
                # step's operands (zero channels and zero-weight indexer heads
                # change no score, norm or logit)
                kv = None if kv is None else _pad_last(kv[:, :nb], cp)
                krows = None if krows is None else _pad_last(krows[:, :nb], cIp)
                ring = None if ring is None else _pad_last(ring, cp)
                q = _pad_last(q, cp)
                qi = torch.nn.functional.pad(qi, (0, cIp - cI, 0, nIp - nIh))
                if wi is None and nIp != nIh:
                    wi = torch.cat([qi.new_ones(B, 1, nIh), qi.new_zeros(B, 1, nIp - nIh)], -1)
                elif wi is not None:
                    wi = _pad_last(wi, nIp)
            qi = _aligned(qi)
            wi = None if wi is None else wi.contiguous()
            idx = torch.empty(B, max(topk, 1), device=q.device, dtype=torch.int32)
            self._last_indices = idx
            sink = None if sink_logits is None else _f32(sink_logits, q.device)
            cap_c = kv.shape[1] if kv is not None else 0
            cap_k = krows.shape[1] if krows is not None else 0
            win_stride = (ring.shape[1] if ring is not None else self.win) * cp
            lib = _lib.load()
            for h0, h1 in _head_groups(nh):
                # (the indexer runs once per head group, with the same selection)
                qc = _aligned(q if h1 - h0 == nh else q[:, :, h0:h1])
                og = out if h1 - h0 == nh else torch.empty(B, 1, h1 - h0, cp, device=q.device,
                                                           dtype=odt)
                nbytes = lib.kch_decode_ws_bytes(B, nb, h1 - h0, cp, topk, n_win, 1)
                ws = torch.empty(max(nbytes, 1), device=q.device, dtype=torch.uint8)
                _lib.call("kch_csa_decode", _lib.ptr(qc), _lib.ptr(qi), _lib.ptr(wi),
                          _lib.ptr(kv), cap_c * cp, _lib.ptr(krows), cap_k * cIp,
                          _lib.ptr(kinv), cap_k, _lib.ptr(ring), win_stride, n_win,
                          _lib.ptr(None if sink is None else sink[h0:h1]), _lib.ptr(og),
                          _lib.ptr(idx) if topk else None, B, nb, h1 - h0, cp, nIp, cIp, topk,
                          float(core_scale), 1.0 if normalize_qk else cI ** -0.5,
                          int(_normalize_q), int(normalize_qk), _lib.dtype_code(fn, q.dtype),
                          _lib.dtype_code(fn, self.dtype), _lib.dtype_code(fn, odt),
                          _lib.ptr(ws), nbytes, _lib.stream_of(q))
                if og is not out:
                    out[:, :, h0:h1] = og
        if topk:
            ops_csa._log_selection(idx.view(B, 1, topk))
        return out if cp == c else out[..., :c]


class HCADecodingCache:
    """HCA incremental decode state (``ops_decoding_cache.py:1077-1395``) on the HIP backend."""

    def __init__(self, B: int, c: int, m2: int, win: int, device, dtype):
        if B < 1:
            raise ValueError(f"B={B} must be >= 1")
        if c < 1:
            raise ValueError(f"c={c} must be >= 1")
        if m2 < 1:
            raise ValueError(f"m2={m2} must be >= 1")
        if win < 0:
            raise ValueError(f"win={win} must be >= 0 (0 disables SW)")
        self.B, self.c, self.m2, self.win = B, c, m2, win
        _validate_cache_dtype(dtype)
        self.device, self.dtype = _device(device), dtype
        self._normalize_qk: bool = True
        self.reset()

    def reset(self) -> None:
        self._acc = None
        self._acc_buf = None
        self._acc_len = 0
        self._C = _BlockStore(self.B, self.c, self.device, self.dtype, torch.bfloat16)
        self._sw = (SlidingWindowRingBuffer(self.B, self.win, self.c, self.device, self.dtype)
                    if self.win > 0 else None)
        self._n_tokens_seen = 0
        self._n_blocks = 0

    @property
    def n_tokens_seen(self) -> int:
        return self._n_tokens_seen

    @property
    def n_blocks(self) -> int:
        return self._n_blocks

    @property
    def accumulator_len(self) -> int:
        return self._acc_len

    @property
    def C_comp(self):
        return None if self._C.rows is None else self._C.rows[:, :self._n_blocks]

    @property
    def sw_buffer(self):
        return self._sw

    def to(self, device=None, dtype=None) -> 'HCADecodingCache':
        if device is not None:
            self.device = torch.device(device)
        if dtype is not None:
            _validate_cache_dtype(dtype)
            self.dtype = dtype
        if self._acc_buf is not None:
            self._acc_buf = self._acc_buf.to(device=self.device)
            self._acc = list(self._acc_buf.split([a.shape[-1] for a in self._acc], -1))
        elif self._acc is not None:
            self._acc = [a.to(device=self.device) for a in self._acc]
        self._C.to(self.device, self.dtype, self._n_blocks)
        if self._sw is not None:
            self._sw.to(device=self.device, dtype=self.dtype)
        return self

    def append_step(self, C_new, Z_new, B_pos):
        """Append ``T_new`` tokens' projections; returns the new block indices."""
        B, T_new, c = C_new.shape
        if B != self.B:
            raise ValueError(
                f"HCADecodingCache.append_step: batch size {B} does not match cache's "
                f"B={self.B}. Call reset() between sequences with different batch sizes.")
        if c != self.c:
            raise ValueError(
                f"HCADecodingCache.append_step: c={c} does not match cache's c={self.c}.")
        if Z_new.shape[1] != T_new:
            raise ValueError(
                f"HCADecodingCache.append_step: Z_new.shape[1]={Z_new.shape[1]} does not "
                f"match C_new.shape[1]={T_new}.")
        if T_new == 0:
            return []
        _lib.require_gpu("HCADecodingCache.append_step", C_new)
        new = [C_new, Z_new]
        with torch.no_grad():
            if self._sw is not None:
                self._sw.append(_ring_rows(C_new, self.dtype, self._normalize_qk))
            if self._acc is None:
                self._acc_buf, self._acc = _alloc_acc(new, B, self.m2)
            total = self._acc_len + T_new
            nfull = total // self.m2
            rem = total - nfull * self.m2
            out_idx = []
            if nfull:
                take = nfull * self.m2 - self._acc_len
                Cc, Zc = (torch.cat([a[:, :self._acc_len], x[:, :take].to(a.dtype)], dim=1)
                          for a, x in zip(self._acc, new))
                rows = _compress("HCADecodingCache", Cc, Zc, B_pos, self.m2)
                self._C.push(self._n_blocks, rows, self._normalize_qk)
                out_idx = list(range(self._n_blocks, self._n_blocks + nfull))
                self._n_blocks += nfull
                for a, x in zip(self._acc, new):
                    if rem:
                        a[:, :rem] = x[:, T_new - rem:].to(a.dtype)
            else:
                grp = None if self._acc_buf is None else _column_group(new)
                if grp is not None and grp.dtype == self._acc_buf.dtype:
                    self._acc_buf[:, self._acc_len:total] = grp
                else:
                    for a, x in zip(self._acc, new):
                        a[:, self._acc_len:total] = x.to(a.dtype)
            self._acc_len = rem
            self._n_tokens_seen += T_new
        return out_idx

    # ---- device-driven steps (kch_hca_cache_append, kch_hca_decode_dyn) ----
    def _device_ready(self, dtype) -> bool:
        if self.dtype != dtype:
            return False
        return self._acc is None or (self._acc_buf is not None and self._acc_buf.dtype == dtype)

    def _device_buffers(self, headroom: int = 1):
        B, m2, c = self.B, self.m2, self.c
        if self._acc is None:
            self._acc_buf = torch.empty(B, m2, 2 * c, device=self.device, dtype=self.dtype)
            self._acc = list(self._acc_buf.split([c, c], -1))
        self._C.ensure(self._n_blocks, max(1, self._n_blocks + headroom))
        if self._C.key_norm is None:
            self._C.key_norm = self._normalize_qk
        return self._C.rows.shape[1]

    def _device_advance(self) -> None:
        n = self._n_tokens_seen
        if self._sw is not None:
            self._sw._written += 1
        if n % self.m2 == self.m2 - 1:
            self._n_blocks += 1
        self._acc_len = (n + 1) % self.m2
        self._n_tokens_seen = n + 1

    def forward_step(self, q, *, nh, scale=None, sink_logits=None, normalize_qk=True,
                     _normalize_q=False, _out_dtype=None):
        """HCA output ``[B, 1, nh, c]`` (fp32) for the last appended token.

        ``_normalize_q`` (internal): L2-normalise ``q`` in the kernel (the
        caller passes the raw projection); ``_out_dtype``: output dtype."""
        B, T_new = q.shape[0], q.shape[1]
        if T_new != 1:
            raise ValueError(f"HCADecodingCache.forward_step: T_new={T_new} must be 1.")
        if B != self.B:
            raise ValueError(
                f"HCADecodingCache.forward_step: batch size {B} does not match cache's B={self.B}.")
        if q.shape[2] != nh:
            raise ValueError(f"q.shape[2]={q.shape[2]} does not match nh={nh}.")
        if q.device != self.device:
            raise ValueError(
                f"HCADecodingCache.forward_step: q.device={q.device} does not match cache's "
                f"device={self.device}. Call cache.to(device=q.device) or move q to the cache's "
                f"device.")
        _lib.require_gpu("HCADecodingCache.forward_step", q)
        core_scale = (1.0 if normalize_qk else self.c ** -0.5) if scale is None else scale
        nb = self._n_blocks
        n_win = self._sw.n_valid if self._sw is not None else 0
        odt = torch.float32 if _out_dtype is None else _out_dtype
        if nb == 0 and n_win == 0:
            return torch.zeros(B, 1, nh, self.c, device=q.device, dtype=odt)
        if q.dtype == torch.float64:
            raise NotImplementedError("float64 queries are not supported by the HIP kernels")
        fn = "HCADecodingCache.forward_step"
        c = self.c
        cp = _kernel_size(fn, "c", c, _HEAD_DIMS)
        out = torch.empty(B, 1, nh, cp, device=q.device, dtype=odt)
        with torch.no_grad():
            kv = self._C.keys_for(nb, normalize_qk) if nb else None
            ring = _ring_bf16(self._sw) if n_win else None
            if cp != c:
                # a head dim between the kernels' own: zero-padded copies of this
                # step's operands (zero channels change no norm or score)
                kv = None if kv is None else _pad_last(kv[:, :nb], cp)
                ring = None if ring is None else _pad_last(ring, cp)
                q = _pad_last(q, cp)
            sink = None if sink_logits is None else _f32(sink_logits, q.device)
            cap = kv.shape[1] if kv is not None else 0
            win_stride = (ring.shape[1] if ring is not None else self.win) * cp
            for h0, h1 in _head_groups(nh):
                qc = _aligned(q if h1 - h0 == nh else q[:, :, h0:h1])
                og = out if h1 - h0 == nh else torch.empty(B, 1, h1 - h0, cp, device=q.device,
                                                           dtype=odt)
                nbytes = _lib.load().kch_decode_ws_bytes(B, nb, h1 - h0, cp, 0, n_win, 0)
                ws = torch.empty(max(nbytes, 1), device=q.device, dtype=torch.uint8)
                _lib.call("kch_hca_decode", _lib.ptr(qc), _lib.ptr(kv), cap * cp,
                          _lib.ptr(ring), win_stride, n_win,
                          _lib.ptr(None if sink is None else sink[h0:h1]), _lib.ptr(og), B,
                          nb, h1 - h0, cp, float(core_scale), int(_normalize_q),
                          _lib.dtype_code(fn, q.dtype), _lib.dtype_code(fn, odt),
                          _lib.ptr(ws), nbytes, _lib.stream_of(q))
                if og is not out:
                    out[:, :, h0:h1] = og
        return out if cp == c else out[..., :c]


_SlidingWindowRingBuffer = SlidingWindowRingBuffer

__all__ = ["CSADecodingCache", "HCADecodingCache", "SlidingWindowRingBuffer"]
