"""Build ``kch/libkch.so`` from ``csrc/*.hip`` with hipcc for gfx950.

Usage: ``python kda-csa-hca-fusion_amd/build_lib.py`` (also called by
``__graft_entry__.build()``). Objects go to ``_build/`` next to this file; the
shared library is written in-tree so it travels with the source tree.

``python kda-csa-hca-fusion_amd/build_lib.py asan`` builds
``_build_asan/libkch_asan.so``: the same library with the C-ABI layer
(``csrc/abi.hip``: argument validation, workspace planning, error reporting)
compiled with the host AddressSanitizer (device code is unchanged), for the CPU
tests of that layer (``KCH_LIBRARY`` selects it; the process needs the clang
ASan runtime preloaded, ``asan_runtime()``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "kch", "libkch.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # packed-fp32 instructions are disabled for all device code on this pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources")
    return OUT


ASAN_DIR = os.path.join(HERE, "_build_asan")
ASAN_OUT = os.path.join(ASAN_DIR, "libkch_asan.so")


def asan_runtime():
    """Path of the clang ASan runtime shared library of this ROCm, or None."""
    root = os.path.join(os.path.dirname(HIPCC), "..", "llvm", "lib", "clang")
    if not os.path.isdir(root):
        return None
    for ver in sorted(os.listdir(root), reverse=True):
        rt = os.path.join(root, ver, "lib", "linux", "libclang_rt.asan-x86_64.so")
        if os.path.exists(rt):
            return os.path.abspath(rt)
    return None


def build_asan(verbose: bool = True) -> str:
    """libkch_asan.so: abi.hip with host ASan, linked with the other objects
    of the plain build (built first when missing)."""
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = [os.path.join(BUILD, f.replace(".hip", ".o")) for f in srcs if f != "abi.hip"]
    if not all(os.path.exists(o) for o in objs):
        build(verbose)
    os.makedirs(ASAN_DIR, exist_ok=True)
    abi_obj = os.path.join(ASAN_DIR, "abi.o")
    cmd = [HIPCC, *[f for f in FLAGS if f != "-O3"], "-O1", "-g",
           "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer",
           "-c", os.path.join(CSRC, "abi.hip"), "-o", abi_obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for abi.hip (asan):\n{r.stderr}")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-shared-libasan",
           "-Xarch_host", "-fsanitize=address", "-o", ASAN_OUT, abi_obj, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"asan link failed:\n{r.stderr}")
    if verbose:
        print(f"built {ASAN_OUT}")
    return ASAN_OUT


if __name__ == "__main__":
    if sys.argv[1:] == ["asan"]:
        build_asan()
    else:
        build()
    sys.exit(0)
