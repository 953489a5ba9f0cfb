"""Decode-cache oracle (test infrastructure only).

Restates the incremental CSA/HCA decode state of
``/root/reference/ops_decoding_cache.py``:

``CSACacheOracle``  ``CSADecodingCache`` (``:407-1070``): per-token accumulator
    of the six projections (``append_step`` ``:631-779``), compression of a
    completed block with the previous block's ``Cb/Zb`` (``:128-195``) and of
    the indexer keys (``:222-244``), rows stored rounded to the cache dtype
    (``:750-763``), a ring of ``L2norm(Ca)`` rounded to the cache dtype
    (``:713-730``), and ``forward_step`` (``:783-1070``).
``HCACacheOracle``  ``HCADecodingCache`` (``:1077-1395``).

The ring buffer is kept as an explicit FIFO list (oldest first), which is
what ``_SlidingWindowRingBuffer.get`` returns (``:372-391``).
"""

from __future__ import annotations

import numpy as np

from .common import l2_normalize, round_to
from .csa import joint_softmax_csa, lightning_indexer


def _softmax_axis1(x):
    mx = x.max(axis=1, keepdims=True)
    e = np.exp(x - mx)
    return e / e.sum(axis=1, keepdims=True)


class CSACacheOracle:
    def __init__(self, B, c, c_I, m, win, dtype='bf16'):
        self.B, self.c, self.c_I, self.m, self.win, self.dtype = B, c, c_I, m, win, dtype
        self.reset()

    def reset(self):
        self.acc = []            # list of 6-tuples of [B, width] arrays
        self.prev_Cb = None
        self.prev_Zb = None
        self.C_comp = np.zeros((self.B, 0, self.c), np.float32)
        self.K_IComp = np.zeros((self.B, 0, self.c_I), np.float32)
        self.ring = []           # oldest first, each [B, c]
        self.n_tokens_seen = 0

    @property
    def n_blocks(self):
        return self.C_comp.shape[1]

    def append_step(self, Ca, Cb, Za, Zb, K_idx, Z_idx, Ba, Bb, B_idx):
        rd = lambda x: round_to(np.asarray(x, np.float32), self.dtype)
        Ca, Cb, Za, Zb, K_idx, Z_idx = map(rd, (Ca, Cb, Za, Zb, K_idx, Z_idx))
        new = []
        for i in range(Ca.shape[1]):
            self.acc.append(tuple(x[:, i] for x in (Ca, Cb, Za, Zb, K_idx, Z_idx)))
            self.n_tokens_seen += 1
            if self.win > 0:
                self.ring.append(rd(l2_normalize(Ca[:, i].astype(np.float32))))
                if len(self.ring) > self.win:
                    self.ring.pop(0)
            if len(self.acc) == self.m:
                blk = [np.stack([a[j] for a in self.acc], axis=1) for j in range(6)]
                ca, cb, za, zb, ki, zi = blk
                a_log = za + np.asarray(Ba, np.float32)[None]
                if self.prev_Cb is None:
                    b_log = np.full_like(a_log, -np.inf)
                    cb_prev = np.zeros_like(cb)
                else:
                    b_log = self.prev_Zb + np.asarray(Bb, np.float32)[None]
                    cb_prev = self.prev_Cb
                S = _softmax_axis1(np.concatenate([a_log, b_log], axis=1))
                row = (S[:, :self.m] * ca).sum(1) + (S[:, self.m:] * cb_prev).sum(1)
                Si = _softmax_axis1(zi + np.asarray(B_idx, np.float32)[None])
                krow = (Si * ki).sum(1)
                self.C_comp = np.concatenate([self.C_comp, rd(row)[:, None]], axis=1)
                self.K_IComp = np.concatenate([self.K_IComp, rd(krow)[:, None]], axis=1)
                new.append(self.n_blocks - 1)
                self.prev_Cb, self.prev_Zb = cb, zb
                self.acc = []
        return new

    def forward_step(self, q, q_idx, w_idx, *, topk, scale=None, sink_logits=None,
                     normalize_qk=True, indices=None):
        """``q`` ``[B,1,nh,c]`` (already normalised), returns ``[B,1,nh,c]`` fp32.

        ``indices`` (``[B,1,topk]``, -1 = unused) replaces the indexer's selection.
        """
        q = np.asarray(q, np.float32)
        Bn, _, nh, c = q.shape
        t = self.n_tokens_seen - 1
        core_scale = (1.0 if normalize_qk else c ** -0.5) if scale is None else scale
        nb = self.n_blocks
        if nb == 0:
            scores = np.zeros((Bn, 1, nh, 0), np.float32)
            valid = np.zeros((Bn, 1, 0), bool)
            kv = np.zeros((Bn, 1, 0, c), np.float32)
        else:
            cbm = (np.arange(nb) < (t + 1) // self.m)[None, :]
            Cn = l2_normalize(self.C_comp) if normalize_qk else self.C_comp
            if indices is None:
                idx = lightning_indexer(np.asarray(q_idx, np.float32), self.K_IComp,
                                        np.asarray(w_idx, np.float32), topk, None, cbm,
                                        normalize_qk)
            else:
                idx = np.asarray(indices, np.int64).reshape(Bn, 1, -1)
            if idx.shape[-1] == 0:
                scores = np.zeros((Bn, 1, nh, 0), np.float32)
                valid = np.zeros((Bn, 1, 0), bool)
                kv = np.zeros((Bn, 1, 0, c), np.float32)
            else:
                valid = idx >= 0
                kv = Cn[np.arange(Bn)[:, None, None], np.maximum(idx, 0)]
                scores = np.einsum('bthd,btkd->bthk', q, kv) * np.float32(core_scale)
                scores = np.where(valid[:, :, None, :], scores, -np.inf)
        if self.win > 0 and self.ring:
            Cl = np.stack(self.ring, axis=1).astype(np.float32)
            sw = (np.einsum('bhd,bsd->bhs', q[:, 0], Cl) * np.float32(core_scale))[:, None]
        else:
            Cl = np.zeros((Bn, 0, c), np.float32)
            sw = np.zeros((Bn, 1, nh, 0), np.float32)
        cat = np.concatenate([scores, sw], axis=-1).astype(np.float32)
        if cat.shape[-1] == 0:
            return np.zeros((Bn, 1, nh, c), np.float32)
        cat_valid = np.concatenate(
            [valid[:, :, None, :], np.ones((Bn, 1, 1, sw.shape[-1]), bool)], axis=-1)
        sink = None if sink_logits is None else np.asarray(sink_logits, np.float32).reshape(1, 1, nh, 1)
        p = joint_softmax_csa(cat, cat_valid, sink)
        k_ = scores.shape[-1]
        return (np.einsum('bthk,btkd->bthd', p[..., :k_], kv)
                + np.einsum('bthw,bwd->bthd', p[..., k_:], Cl)).astype(np.float32)


class HCACacheOracle:
    def __init__(self, B, c, m2, win, dtype='bf16'):
        self.B, self.c, self.m2, self.win, self.dtype = B, c, m2, win, dtype
        self.reset()

    def reset(self):
        self.acc = []
        self.C_comp = np.zeros((self.B, 0, self.c), np.float32)
        self.ring = []
        self.n_tokens_seen = 0

    @property
    def n_blocks(self):
        return self.C_comp.shape[1]

    def append_step(self, C, Z, B_pos):
        rd = lambda x: round_to(np.asarray(x, np.float32), self.dtype)
        C, Z = rd(C), rd(Z)
        new = []
        for i in range(C.shape[1]):
            self.acc.append((C[:, i], Z[:, i]))
            self.n_tokens_seen += 1
            if self.win > 0:
                self.ring.append(rd(l2_normalize(C[:, i].astype(np.float32))))
                if len(self.ring) > self.win:
                    self.ring.pop(0)
            if len(self.acc) == self.m2:
                cb = np.stack([a[0] for a in self.acc], axis=1)
                zb = np.stack([a[1] for a in self.acc], axis=1)
                S = _softmax_axis1(zb + np.asarray(B_pos, np.float32)[None])
                self.C_comp = np.concatenate([self.C_comp, rd((S * cb).sum(1))[:, None]], axis=1)
                new.append(self.n_blocks - 1)
                self.acc = []
        return new

    def forward_step(self, q, *, scale=None, sink_logits=None, normalize_qk=True):
        q = np.asarray(q, np.float32)
        Bn, _, nh, c = q.shape
        core_scale = (1.0 if normalize_qk else c ** -0.5) if scale is None else scale
        t = self.n_tokens_seen - 1
        nb = self.n_blocks
        if nb == 0:
            scores = np.zeros((Bn, 1, nh, 0), np.float32)
            Cn = np.zeros((Bn, 0, c), np.float32)
        else:
            cbm = np.arange(nb) < (t + 1) // self.m2
            Cn = l2_normalize(self.C_comp) if normalize_qk else self.C_comp
            scores = np.einsum('bthd,bnd->bthn', q, Cn) * np.float32(core_scale)
            scores = np.where(cbm[None, None, None, :], scores, -np.inf)
        if self.win > 0 and self.ring:
            Cl = np.stack(self.ring, axis=1).astype(np.float32)
            sw = (np.einsum('bhd,bsd->bhs', q[:, 0], Cl) * np.float32(core_scale))[:, None]
        else:
            Cl = np.zeros((Bn, 0, c), np.float32)
            sw = np.zeros((Bn, 1, nh, 0), np.float32)
        cat = np.concatenate([scores, sw], axis=-1).astype(np.float32)
        if cat.shape[-1] == 0:
            return np.zeros((Bn, 1, nh, c), np.float32)
        valid = ~np.isinf(cat)
        sink = None if sink_logits is None else np.asarray(sink_logits, np.float32).reshape(1, 1, nh, 1)
        p = joint_softmax_csa(cat, valid, sink)
        return (np.einsum('bthn,bnd->bthd', p[..., :nb], Cn)
                + np.einsum('bthw,bwd->bthd', p[..., nb:], Cl)).astype(np.float32)
