"""``kda_forward`` with the ``"hip"`` backend (twin of ``ops_kda_backend.py``).

Mirrors ``/root/reference/ops_kda_backend.py:158-251``: the same signature,
the same ``g_clamp_min`` checks (``TypeError`` for a non-real, ``ValueError``
for NaN, ``:184-187``), the same dispatch on ``use_chunk`` (``:237-251``) and
the same dtype contract (output in ``v.dtype``, fp32 state, ``:139-155``).

Backends of this package: ``"hip"`` (the gfx950 kernels) and ``"auto"``
(= ``"hip"``; there is no other implementation here). The reference's own
``"reference"`` and ``"fla"`` backends belong to the reference package, which
reaches this one by adding ``"hip"`` to its backend set and dispatching here.
The gate clamp is applied inside the kernels (the same values as clamping
once on the host, without an extra pass over ``g``).
"""

from __future__ import annotations

import math

import torch

from .ops_kda import naive_chunk_kda, naive_recurrent_kda

_VALID_BACKENDS = {"hip", "auto"}


def validate_kda_backend(backend: str) -> str:
    """Validate and return a KDA backend name (``ops_kda_backend.py:29-35``)."""
    if backend not in _VALID_BACKENDS:
        raise ValueError(
            f"kda_backend={backend!r} must be one of {sorted(_VALID_BACKENDS)}.")
    return backend


def hip_available() -> bool:
    """Whether the native library loads and a ROCm device is visible."""
    try:
        from . import _lib
        _lib.load()
    except (ImportError, OSError):
        return False
    return torch.cuda.is_available()


def kda_forward(q, k, v, g, beta, *, scale=None, initial_state=None,
                output_final_state: bool = False, chunk_size: int = 64,
                use_chunk: bool = False, g_clamp_min: float = -10.0,
                backend: str = "hip"):
    """Run KDA on the HIP backend; returns ``(o, final_state | None)``."""
    validate_kda_backend(backend)
    if not isinstance(g_clamp_min, (int, float)) or isinstance(g_clamp_min, bool):
        raise TypeError(f"g_clamp_min must be a real number, got {g_clamp_min!r}")
    if math.isnan(float(g_clamp_min)):
        raise ValueError("g_clamp_min must not be NaN")
    if not q.is_cuda:
        raise RuntimeError(
            f"KDA backend {backend!r} requires tensors on a ROCm GPU device; "
            f"use the reference package for CPU experiments.")
    if use_chunk:
        return naive_chunk_kda(q, k, v, g, beta, scale=scale, initial_state=initial_state,
                               output_final_state=output_final_state, chunk_size=chunk_size,
                               g_clamp_min=g_clamp_min)
    return naive_recurrent_kda(q, k, v, g, beta, scale=scale, initial_state=initial_state,
                               output_final_state=output_final_state, g_clamp_min=g_clamp_min)


__all__ = ["hip_available", "kda_forward", "validate_kda_backend"]
