"""Shared numerics for the oracle (test infrastructure only).

* ``bf16_round``: round-to-nearest-even of float32 values to bfloat16,
  returned as float32 (what ``tensor.to(torch.bfloat16).float()`` yields).
* ``l2_normalize``: ``F.normalize(x, dim=-1)`` semantics,
  ``x / max(||x||_2, 1e-12)`` (used by the reference at ``ops_kda`` callers,
  ``ops_csa.py:523-525,929,950,1110-1112`` and ``ops_hca.py:135,141,154``).
* ``softmax_lastdim``: numerically-stable softmax (``torch.softmax``).
"""

from __future__ import annotations

import numpy as np


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even)."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32)
    # u + 0x7FFF + lsb stays below 2^32 for every non-NaN pattern (the largest,
    # -inf = 0xFF800000, gains at most 0x8000); NaNs are restored afterwards
    r = (u >> 16) & np.uint32(1)
    r += np.uint32(0x7FFF)
    r += u
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.nan
    return out


def fp16_round(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x, dtype: str) -> np.ndarray:
    """Round float values to the storage dtype named by ``dtype``."""
    if dtype in ("bf16", "bfloat16"):
        return bf16_round(x)
    if dtype in ("fp16", "float16"):
        return fp16_round(x)
    if dtype in ("fp32", "float32"):
        return np.asarray(x, dtype=np.float32)
    if dtype in ("fp64", "float64"):
        return np.asarray(x, dtype=np.float64)
    raise ValueError(dtype)


def l2_normalize(x, eps: float = 1e-12):
    """``F.normalize(x, p=2, dim=-1)``: ``x / max(||x||, eps)``."""
    x = np.asarray(x)
    n = np.sqrt((x * x).sum(-1, keepdims=True))
    return x / np.maximum(n, np.asarray(eps, dtype=x.dtype))


def softmax_lastdim(x, axis: int = -1):
    x = np.asarray(x)
    m = x.max(axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(axis=axis, keepdims=True)


def logsigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    return -np.logaddexp(0.0, -x)


def sigmoid(x):
    x = np.asarray(x, dtype=np.float64)
    return 1.0 / (1.0 + np.exp(-x))
