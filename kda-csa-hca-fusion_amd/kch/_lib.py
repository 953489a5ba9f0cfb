"""ctypes binding of ``libkch.so`` (the gfx950 kernels behind ``include/kch.h``).

The library is loaded lazily on first use. A missing library raises
``ImportError`` naming the path and the build command; there is no fallback
path of any kind: every operator in this package runs the HIP kernels.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# KCH_LIBRARY names another build of the same library (the host-sanitizer
# build of build_lib.py's ``asan`` target, for the CPU validation tests)
LIB_PATH = os.environ.get("KCH_LIBRARY") or os.path.join(_HERE, "libkch.so")

_lock = threading.Lock()
_lib = None

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_L = ctypes.c_longlong
_D = ctypes.c_double
_SZ = ctypes.c_size_t

# name -> argument types (all return int status)
_SIGNATURES = {
    "kch_kda_chunk_fwd": [_P] * 8 + [_I] * 6 + [_F, _F, _I, _P],
    "kch_kda_chunk_fwd_ws": [_P] * 8 + [_I] * 6 + [_F, _F, _I, _P, _SZ, _P],
    "kch_kda_recurrent_fwd": [_P] * 8 + [_I] * 6 + [_F, _F, _I, _P],
    "kch_kda_recurrent_fwd_f64": [_P] * 8 + [_I] * 6 + [_D, _D, _P],
    "kch_kda_recurrent_bwd": [_P] * 14 + [_I] * 6 + [_D, _D, _I, _P, _SZ, _P],
    "kch_kda_chunk_bwd": [_P] * 14 + [_I] * 6 + [_D, _D, _I, _P, _SZ, _P],
    "kch_gen_compress": [_P] * 7 + [_I] * 5 + [_P],
    "kch_gen_l2norm": [_P, _P, _L, _I, _I, _I, _P],
    "kch_gen_indexer": [_P] * 4 + [_L, _L, _P, _P] + [_I] * 7 + [_D, _I, _I, _P],
    "kch_gen_attn": [_P] * 6 + [_I] * 8 + [_D, _I, _I, _I, _P, _SZ, _P],
    "kch_hca_attn_bwd": [_P] * 16 + [_I] * 6 + [_F, _I, _P, _SZ, _P],
    "kch_csa_attn_bwd": [_P] * 24 + [_I] * 7 + [_F, _I, _I, _P, _SZ, _P],
    "kch_kda_gates_bwd": [_P, _L, _P, _L] + [_P] * 7 + [_I] * 6 + [_F, _I, _P],
    "kch_csa_ste_bwd": [_P] * 13 + [_I] * 5 + [_F, _I, _P, _SZ, _P],
    "kch_short_conv_bwd": [_P] * 8 + [_I] * 4 + [_P],
    "kch_layer_norm_bwd": [_P] * 6 + [_L, _I, _F, _I, _I, _P],
    "kch_compress": [_P, _L, _P, _L, _P, _P, _P, _I, _I, _P, _I, _I, _I, _I, _I, _P],
    "kch_compress_overlapped": [_P, _L, _P, _L, _P, _L, _P, _L, _P, _P, _P, _P, _I, _I, _P,
                                _I, _I, _I, _I, _I, _P],
    "kch_csa_indexer_topk": [_P] * 4 + [_I, _P] + [_I] * 10 + [_F, _I, _I, _I, _P],
    "kch_csa_sparse_attn": [_P] * 6 + [_I] * 7 + [_F, _I, _I, _I, _P],
    "kch_hca_attn": [_P] * 5 + [_I] * 7 + [_F, _I, _I, _I, _P],
    "kch_l2norm_rows": [_P, _L, _P, _I, _I, _I, _I, _I, _P],
    "kch_csa_decode_step": [_P, _P, _P, _P, _L, _P, _L, _P, _L, _I, _P, _P, _P] + [_I] * 7
                           + [_F, _F, _I, _I, _I, _I, _P],
    "kch_hca_decode_step": [_P, _P, _L, _P, _L, _I, _P, _P] + [_I] * 4 + [_F, _I, _I, _I, _P],
    "kch_short_conv": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "kch_csa_decode": [_P, _P, _P, _P, _L, _P, _L, _P, _L, _P, _L, _I, _P, _P, _P] + [_I] * 7
                      + [_F, _F] + [_I] * 5 + [_P, _SZ, _P],
    "kch_hca_decode": [_P, _P, _L, _P, _L, _I, _P, _P] + [_I] * 4 + [_F, _I, _I, _I, _P, _SZ, _P],
    "kch_csa_decode_noalloc": [_P, _P, _P, _P, _L, _P, _L, _P, _L, _P, _L, _I, _P, _P, _P]
                              + [_I] * 7 + [_F, _F] + [_I] * 5 + [_P],
    "kch_kda_gates": [_P, _L, _P, _L, _P, _P, _P, _P, _P] + [_I] * 6 + [_F, _I, _P],
    "kch_layer_norm": [_P, _P, _P, _P, _I, _I, _F, _I, _I, _P],
    "kch_linear_rows": [_P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _P],
    "kch_linear_up": [_P, _L, _P, _L, _P, _L, _L, _I, _I, _I, _P],
    "kch_linear_rows_fused": [_P, _L, _P, _L, _P, _L, _I, _I, _I, _P, _P, _F, _I, _P, _L, _P,
                              _I, _P],
    "kch_kda_decode_front": [_P, _L, _P, _P, _F, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "kch_kda_decode_step": [_P, _L, _P, _P, _P] + [_I] * 5 + [_F] * 3 + [_I, _P],
    "kch_kda_front_rows": [_P, _L, _P, _P, _F, _I, _P, _P, _P, _P, _P, _L, _P, _L, _I, _I, _I,
                           _I, _P],
    "kch_kda_decode_step_shift": [_P, _L, _P, _P, _P] + [_I] * 5 + [_F] * 3 + [_P, _P, _I, _I,
                                                                               _P],
    "kch_csa_cache_append": [_P, _L] + [_P] * 11 + [_I] * 8 + [_P],
    "kch_hca_cache_append": [_P, _L] + [_P] * 6 + [_I] * 7 + [_P],
    "kch_csa_cache_append_rows": [_P, _L] + [_P] * 11 + [_I] * 7 + [_P, _L, _P, _L, _P, _L, _I, _I,
                                                                    _I, _P],
    "kch_hca_cache_append_rows": [_P, _L] + [_P] * 6 + [_I] * 6 + [_P, _L, _P, _L, _P, _L, _I, _I,
                                                                   _I, _P],
    "kch_csa_decode_dyn": [_P, _L] * 7 + [_P, _I, _I, _I, _P, _P, _P] + [_I] * 6 + [_F, _F]
                          + [_I] * 5 + [_P, _SZ, _P],
    "kch_hca_decode_dyn": [_P, _L] * 3 + [_P, _I, _I, _I, _P, _P, _I, _I, _I, _F, _I, _I, _I,
                                          _P, _SZ, _P],
}

# name -> (return type, argument types) of the entry points that return a value
_QUERIES = {
    "kch_kda_chunk_ws_bytes": (_SZ, [_I] * 7),
    "kch_kda_recurrent_bwd_ws_bytes": (_SZ, [_I] * 6),
    "kch_kda_chunk_bwd_ws_bytes": (_SZ, [_I] * 7),
    "kch_gen_attn_ws_bytes": (_SZ, [_I] * 8),
    "kch_hca_attn_bwd_ws_bytes": (_SZ, [_I] * 6),
    "kch_csa_attn_bwd_ws_bytes": (_SZ, [_I] * 7),
    "kch_csa_ste_bwd_ws_bytes": (_SZ, [_I] * 5),
    "kch_decode_ws_bytes": (_SZ, [_I] * 7),
    "kch_decode_dyn_ws_bytes": (_SZ, [_I] * 7),
}

EXPORTED = ["kch_abi_version", "kch_last_error"] + sorted(_SIGNATURES) + sorted(_QUERIES)

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def load():
    """Load and type the shared library (thread-safe, once)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"kch: native library {LIB_PATH} is missing; build it with "
                f"`python -c 'import __graft_entry__ as g; g.build()'` from the repo root")
        lib = ctypes.CDLL(LIB_PATH)
        lib.kch_abi_version.restype = _I
        lib.kch_abi_version.argtypes = []
        lib.kch_last_error.restype = ctypes.c_char_p
        lib.kch_last_error.argtypes = []
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = _I
            fn.argtypes = args
        for name, (ret, args) in _QUERIES.items():
            fn = getattr(lib, name)
            fn.restype = ret
            fn.argtypes = args
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Invoke ``name`` and raise ``RuntimeError`` on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.kch_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (status {rc}): {msg}")


def ptr(t):
    """Device pointer of a tensor (or None for an absent optional tensor)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


# torch's raw current-stream query (one C call) where this torch provides it;
# torch.cuda.current_stream() costs about 2 us of host time per call, which a
# decode step pays some thirty times
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor):
    """The current HIP stream of ``t``'s device, as a ctypes pointer."""
    if _raw_stream is not None and t.is_cuda:
        return ctypes.c_void_p(_raw_stream(t.get_device()))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(fn: str, *tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"{fn}: the HIP backend requires tensors on a ROCm GPU device "
                f"(got {t.device}); this package has no CPU path.")


def dtype_code(fn: str, dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise NotImplementedError(
            f"{fn}: dtype {dtype} is not supported by the HIP kernels "
            f"(float32, bfloat16, float16)") from None
