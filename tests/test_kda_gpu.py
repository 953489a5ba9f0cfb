"""HIP KDA kernels vs the CPU oracle (needs a ROCm GPU).

Tolerances (north star): fp32 inputs 1e-4 absolute on outputs/state;
bf16/fp16 inputs ``|hip - ref| <= 2e-3 + 2e-2 |ref|`` elementwise.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.common import bf16_round, l2_normalize, logsigmoid, sigmoid
from oracle.kda import chunk_kda as o_chunk, recurrent_kda as o_rec

pytestmark = pytest.mark.gpu

TD = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}


def make(seed, B, T, H, HV, K, V, dtype, s0_std=0.02, g_fn=None):
    rng = np.random.default_rng(seed)
    q = l2_normalize(rng.standard_normal((B, T, H, K)))
    k = l2_normalize(rng.standard_normal((B, T, H, K)))
    v = rng.standard_normal((B, T, HV, V))
    g = logsigmoid(rng.standard_normal((B, T, HV, K))) if g_fn is None else g_fn(rng, (B, T, HV, K))
    beta = sigmoid(rng.standard_normal((B, T, HV)))
    s0 = s0_std * rng.standard_normal((B, HV, K, V)) if s0_std else None
    ts = [torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(TD[dtype]) for x in (q, k, v, g, beta)]
    host = [t.float().numpy() for t in ts]          # exact values the kernel sees
    s0t = None if s0 is None else torch.from_numpy(s0.astype(np.float32))
    return ts, host, s0t


def check(name, got, ref, dtype):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite output"
    if dtype == "fp32":
        err = np.abs(got - ref).max()
        assert err < 1e-4, f"{name}: max abs err {err:.3e} (fp32 tol 1e-4)"
    else:
        bad = np.abs(got - ref) > 2e-3 + 2e-2 * np.abs(ref)
        frac = bad.mean()
        assert not bad.any(), (f"{name}: {bad.sum()} elements ({frac:.2e}) outside "
                               f"atol 2e-3 + rtol 2e-2; max abs err {np.abs(got - ref).max():.3e}")


def run_chunk(dev, ts, s0, **kw):
    import kch
    ts = [t.to(dev) for t in ts]
    o, s = kch.naive_chunk_kda(*ts, initial_state=None if s0 is None else s0.to(dev),
                               output_final_state=True, **kw)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), s.cpu().numpy()


def run_rec(dev, ts, s0, **kw):
    import kch
    ts = [t.to(dev) for t in ts]
    o, s = kch.naive_recurrent_kda(*ts, initial_state=None if s0 is None else s0.to(dev),
                                   output_final_state=True, **kw)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), s.cpu().numpy()


def ref_out(o, dtype):
    return o if dtype == "fp32" else (bf16_round(o) if dtype == "bf16" else
                                      o.astype(np.float16).astype(np.float32))


def test_config0_fp32_chunk_matches_oracle_and_recurrence(dev):
    # B1 T1024 H4 K=V=64 fp32, zero initial state
    ts, host, _ = make(0, 1, 1024, 4, 4, 64, 64, "fp32", s0_std=0)
    o, s = run_chunk(dev, ts, None)
    o_ref, s_ref = o_chunk(*host, chunk_size=64)
    check("o vs oracle chunk", o, o_ref, "fp32")
    check("state vs oracle chunk", s, s_ref, "fp32")
    o_r, s_r = o_rec(*host, compute=np.float64)
    check("o vs fp64 recurrence", o, o_r, "fp32")
    check("state vs fp64 recurrence", s, s_r, "fp32")


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("shape", [(2, 300, 2, 2, 128, 128), (1, 130, 2, 4, 128, 64),
                                   (2, 5, 1, 1, 64, 64), (1, 192, 4, 4, 64, 128)])
def test_chunk_lowp_matches_oracle(dev, dtype, shape):
    B, T, H, HV, K, V = shape
    ts, host, s0 = make(sum(shape), B, T, H, HV, K, V, dtype)
    o, s = run_chunk(dev, ts, s0)
    o_ref, s_ref = o_chunk(*host, initial_state=s0.numpy(), chunk_size=64)
    check("o", o, ref_out(o_ref, dtype), dtype)
    check("state", s, s_ref, dtype)


@pytest.mark.parametrize("shape", [(1, 100, 2, 2, 128, 128), (2, 77, 1, 2, 64, 64)])
def test_chunk_fp32_shapes(dev, shape):
    B, T, H, HV, K, V = shape
    ts, host, s0 = make(7 + T, B, T, H, HV, K, V, "fp32")
    o, s = run_chunk(dev, ts, s0, scale=0.3)
    o_ref, s_ref = o_chunk(*host, initial_state=s0.numpy(), scale=0.3, chunk_size=64)
    check("o", o, o_ref, "fp32")
    check("state", s, s_ref, "fp32")


def test_chunk_exact_path_strong_decay(dev):
    # per-token decay of 6 nats: |G_r - G_anchor| leaves the anchored range
    ts, host, s0 = make(11, 1, 256, 2, 2, 128, 128, "bf16",
                        g_fn=lambda rng, sh: -6.0 + 0.1 * rng.standard_normal(sh))
    o, s = run_chunk(dev, ts, s0)
    o_ref, s_ref = o_chunk(*host, initial_state=s0.numpy(), chunk_size=64)
    check("o", o, bf16_round(o_ref), "bf16")
    check("state", s, s_ref, "bf16")


def test_chunk_exact_path_mixed_sign_gate(dev):
    # a few positive gate entries with a wide decay range select the exact path
    def gfn(rng, sh):
        g = -1.0 + 0.2 * rng.standard_normal(sh)
        g[..., ::7, :, :3] = 0.05
        return g
    ts, host, s0 = make(12, 1, 200, 2, 2, 64, 64, "bf16", g_fn=gfn)
    o, s = run_chunk(dev, ts, s0)
    o_ref, s_ref = o_chunk(*host, initial_state=s0.numpy(), chunk_size=64)
    check("o", o, bf16_round(o_ref), "bf16")
    check("state", s, s_ref, "bf16")


def test_chunk_clamp_disabled(dev):
    ts, host, s0 = make(13, 1, 128, 2, 2, 64, 64, "fp32",
                        g_fn=lambda rng, sh: -0.5 * rng.random(sh) - 0.05)
    o, s = run_chunk(dev, ts, s0, g_clamp_min=-math.inf)
    o_ref, s_ref = o_chunk(*host, initial_state=s0.numpy(), g_clamp_min=-np.inf)
    check("o", o, o_ref, "fp32")
    check("state", s, s_ref, "fp32")


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("T", [1, 17])
def test_recurrent_matches_oracle(dev, dtype, T):
    ts, host, s0 = make(20 + T, 2, T, 2, 4, 128, 128, dtype)
    o, s = run_rec(dev, ts, s0)
    o_ref, s_ref = o_rec(*host, initial_state=s0.numpy(), compute=np.float64)
    check("o", o, ref_out(o_ref, dtype), dtype)
    check("state", s, s_ref, dtype)


def test_chunk_equals_recurrent_kernel(dev):
    ts, host, s0 = make(30, 1, 96, 2, 2, 64, 64, "fp32")
    o1, s1 = run_chunk(dev, ts, s0)
    o2, s2 = run_rec(dev, ts, s0)
    assert np.abs(o1 - o2).max() < 1e-4 and np.abs(s1 - s2).max() < 1e-4


def test_deterministic(dev):
    ts, _, s0 = make(31, 2, 200, 2, 2, 128, 128, "bf16")
    a = run_chunk(dev, ts, s0)
    b = run_chunk(dev, ts, s0)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_kda_forward_dispatch_and_errors(dev):
    import kch
    ts, host, s0 = make(32, 1, 70, 1, 1, 64, 64, "fp32")
    ts = [t.to(dev) for t in ts]
    o1, s1 = kch.kda_forward(*ts, initial_state=s0.to(dev), output_final_state=True,
                             use_chunk=True, backend="hip")
    o2, s2 = kch.kda_forward(*ts, initial_state=s0.to(dev), output_final_state=True,
                             use_chunk=False, backend="hip")
    assert (o1 - o2).abs().max().item() < 1e-4
    assert s1.dtype == torch.float32 and o1.dtype == ts[2].dtype
    with pytest.raises(TypeError):
        kch.kda_forward(*ts, g_clamp_min="x")
    with pytest.raises(TypeError):
        kch.kda_forward(*ts, g_clamp_min=True)
    with pytest.raises(ValueError):
        kch.kda_forward(*ts, g_clamp_min=float("nan"))
    with pytest.raises(ValueError):
        kch.kda_forward(*ts, backend="fla")
    with pytest.raises(ValueError, match="naive_chunk_kda"):
        kch.naive_chunk_kda(ts[0], ts[1], ts[2], ts[3][..., :32], ts[4])
    o3, s3 = kch.naive_chunk_kda(*[t[:, :0] for t in ts], initial_state=s0.to(dev),
                                 output_final_state=True)
    assert o3.shape == (1, 0, 1, 64) and torch.equal(s3.cpu(), s0)


def test_fused_entry_point_without_workspace(dev):
    """kch_kda_chunk_fwd (one fused kernel, no workspace) stays correct beside
    the two-kernel path of kch_kda_chunk_fwd_ws."""
    from kch import _lib
    B, T, H, HV, K, V = 2, 150, 2, 2, 128, 128
    ts, host, s0 = make(21, B, T, H, HV, K, V, "bf16")
    q, k, v, g, beta = [t.to(dev) for t in ts]
    s0d = s0.to(dev)
    o = torch.empty_like(v)
    s = torch.empty(B, HV, K, V, device=dev)
    _lib.call("kch_kda_chunk_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g),
              _lib.ptr(beta), _lib.ptr(s0d), _lib.ptr(o), _lib.ptr(s), B, T, H, HV, K, V,
              K ** -0.5, -10.0, 1, _lib.stream_of(q))
    torch.cuda.synchronize()
    o_ref, s_ref = o_chunk(*host, initial_state=s0.numpy(), chunk_size=64)
    check("o", o.float().cpu().numpy(), bf16_round(o_ref), "bf16")
    check("state", s.cpu().numpy(), s_ref, "bf16")


def test_workspace_too_small_is_an_error(dev):
    from kch import _lib
    B, T, H, HV, K, V = 1, 64, 1, 1, 64, 64
    ts, _, _ = make(22, B, T, H, HV, K, V, "bf16")
    q, k, v, g, beta = [t.to(dev) for t in ts]
    o = torch.empty_like(v)
    need = _lib.load().kch_kda_chunk_ws_bytes(B, T, H, HV, K, V, 1)
    ws = torch.empty(need, device=dev, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("kch_kda_chunk_fwd_ws", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g),
                  _lib.ptr(beta), None, _lib.ptr(o), None, B, T, H, HV, K, V, 0.125, -10.0, 1,
                  _lib.ptr(ws), need - 1, _lib.stream_of(q))


def test_chunk_exact_path_some_chunks_k128(dev):
    # strong decay only in the second and fourth chunk: exact and anchored chunks alternate
    def gfn(rng, sh):
        g = logsigmoid(rng.standard_normal(sh))
        g[:, 64:128] = -5.0 + 0.1 * rng.standard_normal(g[:, 64:128].shape)
        g[:, 192:240] = -4.0
        return g
    ts, host, s0 = make(23, 2, 250, 2, 4, 128, 64, "bf16", g_fn=gfn)
    o, s = run_chunk(dev, ts, s0)
    o_ref, s_ref = o_chunk(*host, initial_state=s0.numpy(), chunk_size=64)
    check("o", o, bf16_round(o_ref), "bf16")
    check("state", s, s_ref, "bf16")


def make64(seed, B, T, H, HV, K, V, s0_std=0.02):
    rng = np.random.default_rng(seed)
    q = l2_normalize(rng.standard_normal((B, T, H, K)))
    k = l2_normalize(rng.standard_normal((B, T, H, K)))
    v = rng.standard_normal((B, T, HV, V))
    g = logsigmoid(rng.standard_normal((B, T, HV, K)))
    beta = sigmoid(rng.standard_normal((B, T, HV)))
    s0 = s0_std * rng.standard_normal((B, HV, K, V)) if s0_std else None
    host = [np.ascontiguousarray(x, np.float64) for x in (q, k, v, g, beta)]
    return host, s0


@pytest.mark.parametrize("B,T,H,HV,K,V", [(2, 70, 2, 2, 64, 64), (1, 200, 2, 4, 128, 128),
                                          (2, 33, 1, 2, 40, 24), (1, 9, 1, 1, 16, 200)])
def test_fp64_matches_oracle(dev, B, T, H, HV, K, V):
    """float64 inputs: fp64 arithmetic and state, as the reference computes
    them; both operators against the fp64 oracle (recurrence and chunked WY
    form), to the accumulation-order level of fp64."""
    import kch
    host, s0 = make64(B * T + K, B, T, H, HV, K, V)
    ts = [torch.from_numpy(x).to(dev) for x in host]
    s0t = torch.from_numpy(s0).to(dev)
    o_r, s_r = kch.naive_recurrent_kda(*ts, initial_state=s0t, output_final_state=True)
    o_c, s_c = kch.naive_chunk_kda(*ts, initial_state=s0t, output_final_state=True)
    torch.cuda.synchronize()
    assert o_r.dtype == torch.float64 and s_r.dtype == torch.float64
    ref_o, ref_s = o_rec(*host, initial_state=s0, compute=np.float64)
    ch_o, ch_s = o_chunk(*host, initial_state=s0, chunk_size=64, compute=np.float64)
    for name, got, ref in (("o rec", o_r, ref_o), ("S rec", s_r, ref_s), ("o chunk", o_c, ch_o),
                           ("S chunk", s_c, ch_s)):
        err = float(np.abs(got.cpu().numpy() - ref).max())
        assert err < 1e-10, f"{name}: max abs err {err:.3e}"


def test_fp64_options(dev):
    """fp64: no initial state, the gate clamp off, a requested fp32 state, and
    T = 0 (the initial state passes through)."""
    import kch
    host, s0 = make64(5, 1, 21, 2, 2, 64, 32, s0_std=0)
    host[3] = host[3] * 30.0  # gates below the default clamp
    ts = [torch.from_numpy(x).to(dev) for x in host]
    o, s = kch.naive_recurrent_kda(*ts, output_final_state=True, g_clamp_min=float("-inf"),
                                   state_dtype=torch.float32)
    torch.cuda.synchronize()
    ref_o, ref_s = o_rec(*host, g_clamp_min=-np.inf, compute=np.float64)
    assert s.dtype == torch.float32
    assert float(np.abs(o.cpu().numpy() - ref_o).max()) < 1e-10
    assert float(np.abs(s.double().cpu().numpy() - ref_s).max()) < 1e-6
    z = [t[:, :0] for t in ts]
    s_init = torch.randn(1, 2, 64, 32, device=dev, dtype=torch.float64)
    o0, s0_out = kch.naive_chunk_kda(*z, initial_state=s_init, output_final_state=True)
    torch.cuda.synchronize()
    assert o0.shape == (1, 0, 2, 32) and torch.equal(s0_out, s_init)
