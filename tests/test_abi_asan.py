"""The C-ABI layer under the host AddressSanitizer (CPU only).

``build_lib.py asan`` compiles ``csrc/abi.hip`` (argument validation,
workspace planning, error reporting) with ``-fsanitize=address`` for the host
pass and links it with the other objects; ``test_abi.py`` then runs in a child
process against that library (``KCH_LIBRARY``) with the clang ASan runtime
preloaded. Any heap or stack error in the validation paths aborts the child
with an AddressSanitizer report. Leak detection is off: the Python
interpreter itself holds allocations to exit.
"""

from __future__ import annotations

import importlib.util
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "kda-csa-hca-fusion_amd")


def _build_lib():
    spec = importlib.util.spec_from_file_location("kch_build_lib", os.path.join(PKG, "build_lib.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_abi_tests_pass_under_host_asan():
    bl = _build_lib()
    rt = bl.asan_runtime()
    if rt is None or not os.path.exists(bl.HIPCC):
        pytest.skip("no hipcc / clang ASan runtime in this image")
    lib = bl.build_asan(verbose=False)
    env = dict(os.environ)
    env["KCH_LIBRARY"] = lib
    env["LD_PRELOAD"] = rt + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0"
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                        os.path.join(REPO, "tests", "test_abi.py")],
                       cwd=REPO, env=env, capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
