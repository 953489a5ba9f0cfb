"""C-ABI checks that need no GPU: the library loads and exports every symbol
that ``include/kch.h`` declares, with the declared version."""

from __future__ import annotations

import ctypes
import os
import re

from conftest import REPO

HEADER = os.path.join(REPO, "include", "kch.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(kch_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    names = _declared()
    assert "kch_abi_version" in names and "kch_last_error" in names
    assert "kch_kda_chunk_fwd" in names


def test_library_exports_every_declared_symbol():
    from kch import _lib
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), f"libkch.so does not export {name}"
    version = int(re.search(r"#define KCH_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert lib.kch_abi_version() == version


def test_python_binding_covers_header():
    from kch import _lib
    assert set(_declared()) == set(_lib.EXPORTED)


def test_invalid_arguments_report_errors_without_gpu():
    # argument validation happens before any HIP call
    from kch import _lib
    lib = _lib.load()
    rc = lib.kch_kda_chunk_fwd(None, None, None, None, None, None, None, None,
                               1, 8, 3, 4, 128, 128, ctypes.c_float(1.0),
                               ctypes.c_float(-10.0), 1, None)
    assert rc == 1
    assert b"divisible" in lib.kch_last_error()
    rc = lib.kch_kda_chunk_fwd(None, None, None, None, None, None, None, None,
                               1, 8, 2, 2, 96, 128, ctypes.c_float(1.0),
                               ctypes.c_float(-10.0), 1, None)
    assert rc == 2
    # kch_linear_rows: row count and K checked before any pointer or HIP call
    rc = lib.kch_linear_rows(None, 64, None, 64, None, 8, 17, 8, 64, 1, None)
    assert rc == 2 and b"M=17" in lib.kch_last_error()
    rc = lib.kch_linear_rows(None, 64, None, 64, None, 8, 2, 8, 48, 1, None)
    assert rc == 2 and b"multiple of 32" in lib.kch_last_error()
    # the prefill projections: sizes checked before any pointer or HIP call
    rc = lib.kch_linear_up(None, 48, None, 48, None, 8, 4, 8, 48, 1, None)
    assert rc == 2 and b"K=48" in lib.kch_last_error()
    rc = lib.kch_linear_up(None, 64, None, 64, None, 8, 4, 8, 64, 0, None)
    assert rc == 2 and b"bf16 or fp16" in lib.kch_last_error()
    rc = lib.kch_linear_up(None, 64, None, 64, None, 8, 4, 8, 64, 1, None)
    assert rc == 1 and b"null pointer" in lib.kch_last_error()
    assert lib.kch_linear_up(None, 64, None, 64, None, 8, 0, 8, 64, 1, None) == 0


def test_kda_backward_validation_and_workspace():
    """kch_kda_recurrent_bwd: sizes checked before any pointer or HIP call; the
    workspace is the checkpoints (one state slice per segment) plus one
    partial record (3K + 1 values) per (b, t, hv, 16-column slice)."""
    from kch import _lib
    lib = _lib.load()
    P = [None] * 14
    rc = lib.kch_kda_recurrent_bwd(*P, 1, 8, 2, 2, 48, 16, 0.25, -10.0, 0, None, 0, None)
    assert rc == 2 and b"K=48" in lib.kch_last_error()
    rc = lib.kch_kda_recurrent_bwd(*P, 1, 0, 2, 2, 64, 16, 0.25, -10.0, 0, None, 0, None)
    assert rc == 1 and b"T >= 1" in lib.kch_last_error()
    rc = lib.kch_kda_recurrent_bwd(*P, 1, 8, 2, 2, 64, 16, 0.25, -10.0, 7, None, 0, None)
    assert rc == 1 and b"dtype" in lib.kch_last_error()
    rc = lib.kch_kda_recurrent_bwd(*P, 1, 8, 2, 2, 64, 16, 0.25, -10.0, 3, None, 0, None)
    assert rc == 1 and b"null" in lib.kch_last_error()
    assert lib.kch_kda_recurrent_bwd_ws_bytes(1, 8, 2, 48, 16, 0) == 0
    pad = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # 16-column slices; K = 128: 8-token segments (fp32), 4 (fp64: LDS)
    B, T, HV, K, V = 2, 100, 3, 128, 40
    nvs = (V + 15) // 16
    for code, acc, seg in ((0, 4, 8), (1, 4, 8), (3, 8, 4)):
        ck = B * HV * nvs * (-(-T // seg)) * K * 16 * acc
        part = B * T * HV * nvs * (3 * K + 1) * acc
        assert lib.kch_kda_recurrent_bwd_ws_bytes(B, T, HV, K, V, code) == pad(ck) + pad(part)


def test_chunk_workspace_size_query():
    """kch_kda_chunk_ws_bytes: 0 where no workspace is used, else the sum of
    the six per-chunk records, each region padded to 256 bytes."""
    from kch import _lib
    lib = _lib.load()
    assert lib.kch_kda_chunk_ws_bytes(2, 100, 2, 2, 128, 128, 0) == 0    # fp32
    assert lib.kch_kda_chunk_ws_bytes(2, 100, 2, 2, 128, 192, 1) == 0    # V outside {64,128}
    assert lib.kch_kda_chunk_ws_bytes(2, 0, 2, 2, 128, 128, 1) == 0
    B, T, HV, K, V = 2, 100, 4, 128, 64
    R = B * HV * ((T + 63) // 64)
    pad = lambda x: (x + 255) // 256 * 256  # noqa: E731
    expect = (3 * pad(R * 64 * K * 2) + pad(R * 64 * 64 * 2) + pad(R * 64 * V * 2)
              + pad(R * K * 4))
    assert lib.kch_kda_chunk_ws_bytes(B, T, 2, HV, K, V, 1) == expect


def test_hybrid_decoding_default_geometry_is_the_references():
    """``HybridDecoding()`` builds the reference's decode model
    (``run_decoding.py:642-656``)."""
    import kch
    cfg = kch.HybridDecoding().cfg
    expect = dict(d_model=64, n_heads_qk=2, n_heads_v=2, head_dim_k=16, head_dim_v=16,
                  kda_chunk_size=0, csa_m=4, csa_topk=2, csa_nh=2, csa_c=8, csa_dc=8,
                  csa_nIh=1, csa_cI=4, csa_sliding_window=4, hca_m2=4, hca_nh=2, hca_c=8,
                  hca_dc=8, hca_sliding_window=4, n_kda=3, n_csa=1, n_hca=1)
    assert {k: getattr(cfg, k) for k in expect} == expect
