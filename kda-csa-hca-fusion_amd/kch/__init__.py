"""kch: MI355X (gfx950) HIP backend for the KDA / CSA / HCA hybrid-attention forward path.

Drop-in twins of the reference operators (``/root/reference/ops_*.py``),
running hand-written HIP kernels from ``libkch.so`` through the C ABI declared
in ``include/kch.h``. Tensors must be on a ROCm GPU; there is no CPU path.
"""

from .decoding_cache import CSADecodingCache, HCADecodingCache, SlidingWindowRingBuffer
from .hybrid import (CSAHybridLayer, HCAHybridLayer, HybridConfig, HybridDecoding,
                     HybridKCHAttention, KDAHybridLayer)
from .ops_csa import (csa_compress_kv, csa_compress_kv_overlapped, csa_core, record_selections,
                      csa_lightning_indexer, l2_normalize_rows, naive_csa)
from .ops_hca import hca_core, naive_hca
from .ops_kda import kda_recurrent_grad, naive_chunk_kda, naive_recurrent_kda
from .ops_kda_backend import hip_available, kda_forward, validate_kda_backend

__all__ = [
    "CSAHybridLayer",
    "HCAHybridLayer",
    "HybridConfig",
    "HybridDecoding",
    "HybridKCHAttention",
    "KDAHybridLayer",
    "CSADecodingCache",
    "HCADecodingCache",
    "SlidingWindowRingBuffer",
    "csa_compress_kv",
    "csa_compress_kv_overlapped",
    "csa_core",
    "kda_recurrent_grad",
    "hca_core",
    "csa_lightning_indexer",
    "hip_available",
    "l2_normalize_rows",
    "naive_csa",
    "record_selections",
    "naive_hca",
    "kda_forward",
    "naive_chunk_kda",
    "naive_recurrent_kda",
    "validate_kda_backend",
]
