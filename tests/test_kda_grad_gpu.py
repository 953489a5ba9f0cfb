"""Gradients of the HIP KDA operators (needs a ROCm GPU).

The reference differentiates its torch code with autograd and checks the
result two ways (``run_correctness.py:765-833``: autograd vs central finite
differences, fp64, max relative error < 1e-6; ``:1032-1092``: chunk-form
gradients == recurrent gradients, fp64, < 1e-8). Both are repeated here on
``kch``'s operators, whose backward is ``kch_kda_recurrent_bwd``, and the
gradients are compared with ``oracle.kda.recurrent_kda_grad`` (itself pinned by
finite differences on the CPU):

* fp64 inputs: within 1e-10 of the oracle, relative to the tensor's largest
  gradient;
* fp32 inputs: 1e-4 of the largest gradient per tensor (fp32 sums over up to
  a few hundred tokens);
* bf16 inputs: ``|hip - ref| <= 2e-2 max|ref| + 2e-2 |ref|`` (bf16-rounded
  outputs and fp32 arithmetic, against fp64 on the same bf16 inputs).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.common import l2_normalize, logsigmoid, sigmoid
from oracle.kda import recurrent_kda, recurrent_kda_grad

pytestmark = pytest.mark.gpu


def _make(seed, B, T, H, HV, K, V, s0_std=0.05, clamp_frac=0.0):
    rng = np.random.default_rng(seed)
    q = l2_normalize(rng.standard_normal((B, T, H, K)))
    k = l2_normalize(rng.standard_normal((B, T, H, K)))
    v = rng.standard_normal((B, T, HV, V))
    g = logsigmoid(rng.standard_normal((B, T, HV, K)))
    if clamp_frac:
        g = np.where(rng.random(g.shape) < clamp_frac, -10.5 - rng.random(g.shape), g)
    beta = sigmoid(rng.standard_normal((B, T, HV)))
    s0 = s0_std * rng.standard_normal((B, HV, K, V)) if s0_std else None
    w_o = rng.standard_normal((B, T, HV, V))
    w_s = rng.standard_normal((B, HV, K, V))
    return [q, k, v, g, beta], s0, w_o, w_s


def _leaves(host, s0, dev, dtype, state_dtype):
    ts = [torch.tensor(x, dtype=dtype, device=dev, requires_grad=True) for x in host]
    s0t = None if s0 is None else torch.tensor(s0, dtype=state_dtype, device=dev,
                                               requires_grad=True)
    return ts, s0t


def _hip_grads(op, ts, s0t, w_o, w_s, **kw):
    """Gradients of L = sum(o * w_o) + sum(S_T * w_s) through ``op``."""
    o, s = op(*ts, initial_state=s0t, output_final_state=w_s is not None, **kw)
    dev = o.device
    loss = (o.double() * torch.tensor(w_o, device=dev)).sum()
    if w_s is not None:
        loss = loss + (s.double() * torch.tensor(w_s, device=dev)).sum()
    loss.backward()
    torch.cuda.synchronize()
    out = [t.grad.double().cpu().numpy() for t in ts]
    out.append(None if s0t is None else s0t.grad.double().cpu().numpy())
    return out


def _ref(host, s0, w_o, w_s, **kw):
    return recurrent_kda_grad(*host, w_o, initial_state=s0, ds_final=w_s, **kw)


NAMES = ["dq", "dk", "dv", "dg", "dbeta", "ds0"]


def _check(got, ref, rtol_max, rtol_elem=0.0, label=""):
    for name, a, b in zip(NAMES, got, ref):
        if b is None:
            assert a is None, name
            continue
        assert a.shape == b.shape, (label, name, a.shape, b.shape)
        assert np.isfinite(a).all(), f"{label} {name}: non-finite gradient"
        scale = np.abs(b).max() + 1e-30
        bad = np.abs(a - b) > rtol_max * scale + rtol_elem * np.abs(b)
        assert not bad.any(), (f"{label} {name}: {bad.sum()} of {bad.size} outside "
                               f"{rtol_max} max + {rtol_elem} rel; max err "
                               f"{np.abs(a - b).max():.3e} of max {scale:.3e}")


@pytest.mark.parametrize("B,T,H,HV,K,V", [(1, 16, 2, 2, 4, 4), (2, 37, 1, 2, 16, 24),
                                          (1, 70, 2, 4, 64, 40), (1, 45, 1, 1, 128, 128),
                                          (1, 9, 1, 1, 256, 32)])
def test_fp64_matches_oracle(dev, B, T, H, HV, K, V):
    """fp64: every gradient (q, k, v, g, beta, S0; loss on o and on S_T) within
    1e-10 of the oracle; covers GVA, K padding (4, 40 -> 16, 64), partial V
    slices and several checkpoint segments."""
    import kch
    host, s0, w_o, w_s = _make(B * T + K, B, T, H, HV, K, V, clamp_frac=0.1)
    ts, s0t = _leaves(host, s0, dev, torch.float64, torch.float64)
    got = _hip_grads(kch.naive_recurrent_kda, ts, s0t, w_o, w_s)
    _check(got, _ref(host, s0, w_o, w_s), 1e-10, label="fp64")


def test_fp64_finite_differences_reference_case(dev):
    """``run_correctness.py:765-833`` on the HIP operator: B=1, T=16, H=2,
    K=V=4, fp64, L = sum(o^2), 8 coordinates of each input. The bound is the
    reference's 1e-6, taken relative to |num| + |ana| + 1e-2 (central
    differences carry ~1e-10 of rounding noise)."""
    import kch
    torch.manual_seed(6)
    B, T, H, K, V = 1, 16, 2, 4, 4
    q = torch.randn(B, T, H, K, dtype=torch.float64, device=dev, requires_grad=True)
    k = torch.randn(B, T, H, K, dtype=torch.float64, device=dev, requires_grad=True)
    v = torch.randn(B, T, H, V, dtype=torch.float64, device=dev, requires_grad=True)
    g = (-torch.rand(B, T, H, K, dtype=torch.float64, device=dev) * 0.1).requires_grad_(True)
    beta = (torch.rand(B, T, H, dtype=torch.float64, device=dev) * 0.2).requires_grad_(True)

    def loss_fn(*xs):
        o, _ = kch.naive_recurrent_kda(*xs)
        return (o ** 2).sum()

    loss_fn(q, k, v, g, beta).backward()
    worst = 0.0
    for t in (q, k, v, g, beta):
        flat = t.detach().view(-1)
        ana = t.grad.view(-1)
        for idx in torch.randperm(flat.numel())[:8].tolist():
            orig = flat[idx].item()
            with torch.no_grad():
                flat[idx] = orig + 1e-6
                lp = loss_fn(q, k, v, g, beta).item()
                flat[idx] = orig - 1e-6
                lm = loss_fn(q, k, v, g, beta).item()
                flat[idx] = orig
            num = (lp - lm) / 2e-6
            a = ana[idx].item()
            worst = max(worst, abs(num - a) / (abs(num) + abs(a) + 1e-2))
    assert worst < 1e-6, worst


def test_fp64_chunk_grad_equals_recurrent_grad(dev):
    """``run_correctness.py:1032-1092``: B=1, T=64, H=2, K=V=8, chunk 16, fp64,
    L = sum(o^2): chunk-form gradients equal the recurrent ones to 1e-8."""
    import kch
    torch.manual_seed(7)
    B, T, H, K, V = 1, 64, 2, 8, 8
    base = [torch.randn(B, T, H, K, dtype=torch.float64), torch.randn(B, T, H, K, dtype=torch.float64),
            torch.randn(B, T, H, V, dtype=torch.float64) * 0.1,
            -torch.rand(B, T, H, K, dtype=torch.float64) * 0.05,
            torch.rand(B, T, H, dtype=torch.float64) * 0.2]
    grads = []
    for op, kw in ((kch.naive_recurrent_kda, {}), (kch.naive_chunk_kda, {"chunk_size": 16})):
        xs = [t.to(dev).requires_grad_(True) for t in base]
        o, _ = op(*xs, output_final_state=False, **kw)
        (o ** 2).sum().backward()
        grads.append([x.grad.cpu() for x in xs])
    for a, b in zip(*grads):
        assert (a - b).abs().max().item() < 1e-8
    # and both equal the oracle's gradients of the same loss
    host = [t.numpy() for t in base]
    o_ref, _ = recurrent_kda(*host, compute=np.float64)
    ref = recurrent_kda_grad(*host, 2 * o_ref)
    _check([g.numpy() for g in grads[0]] + [None], list(ref[:5]) + [None], 1e-10, label="fd-case")


@pytest.mark.parametrize("op", ["recurrent", "chunk"])
@pytest.mark.parametrize("B,T,H,HV,K,V", [(2, 203, 2, 4, 128, 128), (1, 130, 1, 1, 64, 64),
                                          (2, 50, 2, 2, 32, 48)])
def test_fp32_matches_oracle(dev, op, B, T, H, HV, K, V):
    import kch
    host, s0, w_o, w_s = _make(7 * T + K, B, T, H, HV, K, V)
    host = [np.asarray(x, np.float32).astype(np.float64) for x in host]
    s0 = s0.astype(np.float32).astype(np.float64)
    ts, s0t = _leaves(host, s0, dev, torch.float32, torch.float32)
    fn = kch.naive_recurrent_kda if op == "recurrent" else kch.naive_chunk_kda
    got = _hip_grads(fn, ts, s0t, w_o, w_s)
    _check(got, _ref(host, s0, w_o, w_s), 1e-4, label=f"fp32 {op}")


@pytest.mark.parametrize("B,T,H,HV,K,V", [(2, 300, 2, 2, 128, 128), (1, 100, 1, 2, 64, 64)])
def test_bf16_matches_oracle(dev, B, T, H, HV, K, V):
    """bf16 inputs through the chunk operator (the split kernels forward),
    gradients in bf16 against fp64 gradients of the same bf16 inputs."""
    import kch
    host, s0, w_o, w_s = _make(3 * T + K, B, T, H, HV, K, V)
    tb = [torch.tensor(x, dtype=torch.bfloat16) for x in host]
    host = [t.double().numpy() for t in tb]
    s0 = s0.astype(np.float32).astype(np.float64)
    ts, s0t = _leaves(host, s0, dev, torch.bfloat16, torch.float32)
    got = _hip_grads(kch.naive_chunk_kda, ts, s0t, w_o, w_s)
    _check(got, _ref(host, s0, w_o, w_s), 2e-2, 2e-2, label="bf16")


def test_grad_without_initial_state_or_final_state(dev):
    """Only o enters the loss and there is no initial state: ds_final is None
    inside the backward, ds0 is not produced."""
    import kch
    host, _, w_o, _ = _make(5, 1, 40, 1, 1, 32, 32, s0_std=0)
    ts, _ = _leaves(host, None, dev, torch.float32, torch.float32)
    got = _hip_grads(kch.naive_recurrent_kda, ts, None, w_o, None)
    ref = recurrent_kda_grad(*host, w_o)
    _check(got, list(ref[:5]) + [None], 1e-4, label="no-state")


def test_no_grad_path_unchanged(dev):
    """Without requires_grad the operators return exactly what they did before
    (no autograd node); with it, the forward values are identical."""
    import kch
    host, s0, _, _ = _make(9, 1, 70, 2, 2, 64, 64)
    xs = [torch.tensor(x, dtype=torch.bfloat16, device=dev) for x in host]
    o1, s1 = kch.naive_chunk_kda(*xs, initial_state=torch.tensor(s0, dtype=torch.float32, device=dev),
                                 output_final_state=True)
    assert o1.grad_fn is None
    ys = [x.clone().requires_grad_(True) for x in xs]
    o2, s2 = kch.naive_chunk_kda(*ys, initial_state=torch.tensor(s0, dtype=torch.float32, device=dev),
                                 output_final_state=True)
    assert o2.grad_fn is not None
    assert torch.equal(o1, o2.detach()) and torch.equal(s1, s2.detach())


@pytest.mark.parametrize("B,T,H,HV,K,V", [(1, 1, 1, 4, 32, 16), (2, 17, 2, 2, 16, 33)])
def test_fp64_edge_shapes(dev, B, T, H, HV, K, V):
    """One token; GVA with four value heads per key head; V not a multiple of
    the 32-column slice; T not a multiple of the checkpoint segment."""
    import kch
    host, s0, w_o, w_s = _make(B + T + HV, B, T, H, HV, K, V)
    ts, s0t = _leaves(host, s0, dev, torch.float64, torch.float64)
    got = _hip_grads(kch.naive_recurrent_kda, ts, s0t, w_o, w_s)
    _check(got, _ref(host, s0, w_o, w_s), 1e-10, label="edge")


def test_empty_sequence_grad(dev):
    """T = 0: zero gradients, and dS0 = dL/dS_T (the state passes through)."""
    import kch
    q = torch.zeros(1, 0, 1, 16, dtype=torch.float64, device=dev, requires_grad=True)
    k = torch.zeros_like(q, requires_grad=True)
    v = torch.zeros(1, 0, 1, 16, dtype=torch.float64, device=dev, requires_grad=True)
    g = torch.zeros_like(q, requires_grad=True)
    beta = torch.zeros(1, 0, 1, dtype=torch.float64, device=dev, requires_grad=True)
    s0 = torch.randn(1, 1, 16, 16, dtype=torch.float64, device=dev, requires_grad=True)
    o, s = kch.naive_recurrent_kda(q, k, v, g, beta, initial_state=s0, output_final_state=True)
    w = torch.randn_like(s)
    (s * w).sum().backward()
    assert torch.equal(s0.grad, w)


def test_fp32_wide_grid_matches_oracle(dev):
    """A grid with a workgroup for every CU (B * HV * V / 32 >= 256): the
    backward then runs 32-column slices (8 row phases per column) instead of
    16-column ones; same bar as the other fp32 cases."""
    import kch
    B, T, H, HV, K, V = 4, 40, 8, 16, 64, 128
    host, s0, w_o, w_s = _make(99, B, T, H, HV, K, V)
    host = [np.asarray(x, np.float32).astype(np.float64) for x in host]
    s0 = s0.astype(np.float32).astype(np.float64)
    ts, s0t = _leaves(host, s0, dev, torch.float32, torch.float32)
    got = _hip_grads(kch.naive_recurrent_kda, ts, s0t, w_o, w_s)
    _check(got, _ref(host, s0, w_o, w_s), 1e-4, label="fp32 wide")


@pytest.mark.parametrize("case", ["strong_decay", "mixed_sign", "gva_fp16"])
def test_chunk_bwd_exact_path_matches_oracle(dev, case):
    """``kch_kda_chunk_bwd`` where its decay products are formed exactly (one
    exponential per pair and channel): gates of -3 to -4 nats a token (in-chunk
    ranges far beyond 60 nats) and gates of both signs (no clamp reached), fp32
    against the recurrence oracle at 1e-4 of each tensor's largest gradient;
    fp16 with grouped value heads (per-head partials summed by the reduce
    kernel) at the bf16 bar."""
    import kch
    B, T, H, HV, K, V = {"strong_decay": (1, 150, 2, 2, 128, 64),
                         "mixed_sign": (2, 130, 1, 1, 64, 128),
                         "gva_fp16": (1, 97, 1, 2, 128, 128)}[case]
    host, s0, w_o, w_s = _make(11 * T + K, B, T, H, HV, K, V)
    rng = np.random.default_rng(T)
    if case == "strong_decay":
        host[3] = host[3] - 3.0
    elif case == "mixed_sign":
        host[3] = 0.3 * rng.standard_normal(host[3].shape)
    if case == "gva_fp16":
        tb = [torch.tensor(x, dtype=torch.float16) for x in host]
        host = [t.double().numpy() for t in tb]
        dtype, tol = torch.float16, (2e-2, 2e-2)
    else:
        host = [np.asarray(x, np.float32).astype(np.float64) for x in host]
        dtype, tol = torch.float32, (1e-4, 0.0)
    s0 = s0.astype(np.float32).astype(np.float64)
    ts, s0t = _leaves(host, s0, dev, dtype, torch.float32)
    got = _hip_grads(kch.naive_chunk_kda, ts, s0t, w_o, w_s)
    _check(got, _ref(host, s0, w_o, w_s), *tol, label=case)


def test_chunk_bwd_clamp_matches_chunk_form_autograd(dev):
    """Where ``clamp(max=50)`` of the in-chunk decay exponents
    (``ops_kda.py:414,516``) is reached, the chunk form's gradient is no longer
    the recurrence's: the clamped exponent has zero gradient. Channel 0 of
    every head runs a gate valley (-1.7 nats a token for 32 tokens, then +1.7),
    so ``G_i - G_j`` passes 50 for late rows against mid-chunk columns (in
    Aqk), with k of that channel scaled by 1e-23 so that ``k e^(G_l - G)``
    and the clamped ``q k e^50`` stay of order one. The HIP gradients (fp32) are compared with fp64 autograd of
    ``oracle.kda_torch.chunk_kda`` (the chunk form, clamp included) on the same
    inputs, at 1e-4 of each tensor's largest gradient."""
    import kch
    from oracle.kda_torch import chunk_kda as torch_chunk
    B, T, H, HV, K, V = 1, 64, 2, 2, 64, 64
    host, s0, w_o, w_s = _make(404, B, T, H, HV, K, V)
    q, k, v, g, beta = host
    k = k.copy()
    k[..., 0] *= 1e-23
    g = g.copy()
    g[:, :32, :, 0] = -1.7
    g[:, 32:, :, 0] = 1.7
    host = [np.asarray(x, np.float32).astype(np.float64) for x in (q, k, v, g, beta)]
    s0 = s0.astype(np.float32).astype(np.float64)
    ts, s0t = _leaves(host, s0, dev, torch.float32, torch.float32)
    got = _hip_grads(kch.naive_chunk_kda, ts, s0t, w_o, w_s)

    leaves = [torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in host]
    s0c = torch.tensor(s0, dtype=torch.float64, requires_grad=True)
    o, s = torch_chunk(*leaves, initial_state=s0c, dtype=torch.float64)
    loss = (o * torch.tensor(w_o)).sum() + (s * torch.tensor(w_s)).sum()
    loss.backward()
    ref = [t.grad.numpy() for t in leaves] + [s0c.grad.numpy()]
    # the clamp is reached: the recurrence's gradients of q and g differ visibly
    rec = _ref(host, s0, w_o, w_s)
    assert np.abs(rec[0] - ref[0]).max() > 0.5 * np.abs(ref[0]).max()
    assert np.abs(rec[3] - ref[3]).max() > 1e-2 * np.abs(ref[3]).max()
    _check(got, ref, 1e-4, label="clamp")
