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
