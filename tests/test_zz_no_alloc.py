"""``kch_csa_decode_noalloc`` against ``kch_csa_decode`` (needs a ROCm GPU).

The allocation-free entry point runs the same kernels on the same inputs with
its workspace in the library's static device array, so its outputs and
selected indices must equal the workspace entry point's bit for bit. Two calls
in a row, the second smaller, check that nothing of the first call's scratch
contents leaks into the second; a size beyond the array is refused on the host
with a clear error.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, B, nb, c, cI, nh, nIh, win, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    kr = torch.randn(B, nb, cI, device=dev, generator=g).to(torch.bfloat16)
    kinv = kr.float().norm(dim=-1).clamp_min(1e-12).reciprocal()
    kv = torch.nn.functional.normalize(torch.randn(B, nb, c, device=dev, generator=g),
                                       dim=-1).to(torch.bfloat16)
    ring = torch.nn.functional.normalize(torch.randn(B, win, c, device=dev, generator=g),
                                         dim=-1).to(torch.bfloat16)
    q = torch.randn(B, nh, c, device=dev, generator=g)
    qi = torch.randn(B, nIh, cI, device=dev, generator=g)
    wi = torch.randn(B, nIh, device=dev, generator=g)
    sink = torch.randn(nh, device=dev, generator=g)
    return kr, kinv, kv, ring, q, qi, wi, sink


def _run(name, dev, B, nb, c, cI, nh, nIh, win, topk, seed):
    from kch import _lib
    lib = _lib.load()
    kr, kinv, kv, ring, q, qi, wi, sink = _inputs(dev, B, nb, c, cI, nh, nIh, win, seed)
    outs, idxs = [], []
    for fn in ("kch_csa_decode", name):
        out = torch.full((B, nh, c), float("nan"), device=dev)
        idx = torch.full((B, topk), -7, device=dev, dtype=torch.int32)
        args = [_lib.ptr(q), _lib.ptr(qi), _lib.ptr(wi), _lib.ptr(kv), nb * c, _lib.ptr(kr),
                nb * cI, _lib.ptr(kinv), nb, _lib.ptr(ring), win * c, win, _lib.ptr(sink),
                _lib.ptr(out), _lib.ptr(idx), B, nb, nh, c, nIh, cI, topk, 1.0, 1.0, 1, 1,
                0, 1, 0]
        if fn == "kch_csa_decode":
            nbytes = lib.kch_decode_ws_bytes(B, nb, nh, c, topk, win, 1)
            ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
            args += [_lib.ptr(ws), nbytes]
        _lib.call(fn, *args, _lib.stream_of(q))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
        idxs.append(idx.cpu().numpy())
    return outs, idxs


def test_noalloc_matches_workspace_entry_point(dev):
    name = "kch_csa_decode_noalloc"
    # calls in a row: a large multi-range step, a smaller one, then a larger
    # batch again
    for (B, nb, c, cI, nh, nIh, win, topk, seed) in [(4, 20000, 128, 64, 16, 4, 128, 512, 1),
                                                      (2, 3000, 64, 32, 8, 2, 16, 64, 2),
                                                      (96, 2000, 128, 64, 16, 4, 128, 256, 3)]:
        print(f"{name}: B={B} nb={nb} topk={topk} win={win}", flush=True)
        (o_ws, o_na), (i_ws, i_na) = _run(name, dev, B, nb, c, cI, nh, nIh, win, topk, seed)
        assert np.isfinite(o_na).all()
        np.testing.assert_array_equal(i_na, i_ws)
        np.testing.assert_array_equal(o_na.view(np.uint32), o_ws.view(np.uint32))


def test_noalloc_refuses_sizes_beyond_its_scratch(dev):
    from kch import _lib
    lib = _lib.load()
    B, nb, c, cI, nh, nIh, win, topk = 256, 262144, 128, 64, 16, 4, 128, 512
    assert lib.kch_decode_ws_bytes(B, nb, nh, c, topk, win, 1) > 16 * 1024 * 1024
    q = torch.zeros(1, device=dev)
    # checked on the host before any pointer is used or any kernel launched
    with pytest.raises(RuntimeError, match="bytes of scratch"):
        _lib.call("kch_csa_decode_noalloc", None, None, None, None, nb * c, None, nb * cI, None,
                  nb, None, win * c, win, None, None, None, B, nb, nh, c, nIh, cI, topk, 1.0,
                  1.0, 1, 1, 0, 1, 0, _lib.stream_of(q))
