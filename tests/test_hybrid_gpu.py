"""Hybrid composition on the HIP backend vs the CPU oracle (needs a ROCm GPU).

* ``kch_short_conv`` / ``kch_kda_gates`` (through the C-ABI) vs
  ``oracle.hybrid.short_conv`` and the activation formulas;
* ``KDAHybridLayer`` (chunk and recurrent paths, state + lookback threading),
  ``HybridKCHAttention`` and ``HybridDecoding`` vs ``oracle.hybrid``;
* ``HybridDecoding`` prefill + decode == ``HybridKCHAttention`` on the full
  sequence (the reference's ``run_correctness.py:5065-5115`` property);
* the padding regression of ``run_correctness.py:2158-2207``.

Tolerance: rtol 2e-2 + atol 2e-3 (the bf16 bar) on every element, also for
fp32 models, whose CSA / HCA keys are bf16 rows in the kernels. Where a CSA
layer selects top-k blocks, the oracle is given the selection the kernels
made (``kch.record_selections``), so a near-tie between two blocks cannot
turn into an output difference; the selections themselves are checked
against the oracle's in ``test_csa_hca_gpu.py`` and ``test_regimes_gpu.py``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from composed_check import LayerInputs, check_layers, close, decode_vs_oracle, end_to_end, host_sel
from oracle import hybrid as OH

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _forward_only():
    """These are forward-parity tests: the layers' parameters require grad, so
    with autograd on they would take their gradient path (and return tensors
    that require grad); that path is tested in test_hybrid_grad_gpu.py."""
    with torch.no_grad():
        yield


def small_cfg(**kw):
    import kch
    base = dict(d_model=128, n_heads_qk=2, n_heads_v=2, head_dim_k=64, head_dim_v=64,
                kda_chunk_size=64, csa_m=4, csa_topk=64, csa_nh=2, csa_c=64, csa_dc=32,
                csa_nIh=2, csa_cI=32, csa_sliding_window=8, hca_m2=16, hca_nh=2, hca_c=64,
                hca_dc=32, hca_sliding_window=8)
    base.update(kw)
    return kch.HybridConfig(**base)


def cfg_dict(cfg):
    return {k: getattr(cfg, k) for k in cfg.__dataclass_fields__}


def build(cfg, dev, dtype, total_layers=5, seed=0):
    import kch
    torch.manual_seed(seed)
    model = kch.HybridKCHAttention(cfg, total_layers=total_layers)
    with torch.no_grad():
        for layer in model.layers:
            if hasattr(layer, 'sink'):
                layer.sink.normal_()
            if hasattr(layer, 'short_conv'):
                layer.short_conv.weight.mul_(3.0)
        for n in model.norms:
            n.weight.normal_(1.0, 0.1)
            n.bias.normal_(0.0, 0.1)
    model = model.to(dev, dtype).eval()
    sd = {k: v.float().cpu().numpy() for k, v in model.state_dict().items()}
    return model, sd


DT = {torch.float32: 'fp32', torch.bfloat16: 'bf16'}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d,T,with_lb", [(128, 37, False), (128, 37, True), (40, 5, True),
                                         (2048, 1, True), (64, 1, False)])
def test_short_conv(dev, dtype, d, T, with_lb):
    from kch import _lib
    rng = np.random.default_rng(d + T)
    B = 3
    x = torch.from_numpy(rng.standard_normal((B, T, d)).astype(np.float32)).to(dev, dtype)
    lb = torch.from_numpy(rng.standard_normal((B, 2, d)).astype(np.float32)).to(dev, dtype) \
        if with_lb else None
    w = torch.from_numpy(rng.standard_normal((d, 3)).astype(np.float32)).to(dev, dtype)
    b = torch.from_numpy(rng.standard_normal(d).astype(np.float32)).to(dev, dtype)
    out = torch.empty_like(x)
    _lib.call("kch_short_conv", _lib.ptr(x), _lib.ptr(lb), _lib.ptr(w), _lib.ptr(b), _lib.ptr(out),
              B, T, d, _lib.dtype_code("t", dtype), _lib.stream_of(x))
    ref = OH.short_conv(x.float().cpu().numpy(), w.float().cpu().numpy(), b.float().cpu().numpy(),
                        None if lb is None else lb.float().cpu().numpy(), DT[dtype])
    tol = (1e-5, 1e-5) if dtype == torch.float32 else (2 ** -8, 1e-6)
    close("short_conv", out.float().cpu().numpy(), ref, *tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("H,HV,K,V", [(2, 2, 64, 64), (2, 4, 128, 64), (16, 16, 128, 128),
                                      (1, 1, 40, 24), (2, 2, 16, 16), (3, 5, 8, 8)])
@pytest.mark.parametrize("aligned", [False, True])
def test_kda_gates(dev, dtype, H, HV, K, V, aligned):
    """Odd row strides take the element-wise kernel; rows of whole 16-byte
    pieces (bf16, K / 8 a power of two) the wave-per-row kernel."""
    from kch import _lib
    rng = np.random.default_rng(H * K + V)
    B, T = 2, 9
    width = 2 * H * K + HV * V + HV + K  # plus the gate down-projection
    width += (8 + (-width) % 8) if aligned else 3  # and slack
    proj = torch.from_numpy((2 * rng.standard_normal((B, T, width))).astype(np.float32))
    proj = proj.to(dev, dtype)
    gl = torch.from_numpy((8 * rng.standard_normal((B, T, HV * K))).astype(np.float32)).to(dev, dtype)
    q = torch.empty(B, T, H, K, device=dev, dtype=dtype)
    k, v = torch.empty_like(q), torch.empty(B, T, HV, V, device=dev, dtype=dtype)
    g, beta = torch.empty(B, T, HV, K, device=dev, dtype=dtype), torch.empty(B, T, HV, device=dev,
                                                                             dtype=dtype)
    _lib.call("kch_kda_gates", _lib.ptr(proj), proj.stride(1), _lib.ptr(gl), gl.stride(1),
              _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta),
              B, T, H, HV, K, V, 0.1, _lib.dtype_code("t", dtype), _lib.stream_of(proj))
    P = proj.float().cpu().numpy()
    G = gl.float().cpu().numpy()
    o2 = 2 * H * K + HV * V
    refs = OH.kda_activations(P[..., :H * K], P[..., H * K:2 * H * K], P[..., 2 * H * K:o2], G,
                              P[..., o2:o2 + HV], H, HV, K, V, 0.1, DT[dtype])
    # the oracle's rounding chain is the reference's (pinned by tests/golden); the
    # kernel's exp / sqrt / division may round an intermediate by one ulp
    # differently from numpy: then that element is one ulp off
    tol = (1e-5, 1e-6) if dtype == torch.float32 else (2 ** -7, 1e-6)
    for name, got, ref in zip(("q", "k", "v", "g", "beta"), (q, k, v, g, beta), refs):
        gn = got.float().cpu().numpy()
        close(name, gn, ref, *tol)
        if dtype == torch.bfloat16:
            exact = np.mean(gn == ref)
            assert exact >= 0.99, f"{name}: only {exact:.4f} of the elements bit-identical"


def test_kda_gates_fast_activations_exhaustive(dev):
    """The wave-per-row kernel (rows of whole 16-byte pieces) takes bf16
    activations on the hardware exponential; the element-wise kernel (odd row
    strides) the library's expf / log1pf. On inputs that hold every finite
    bf16 value in every activation's position, the two give bit-identical
    q, k, v, g and beta."""
    from kch import _lib
    B, T, H, HV, K, V = 1, 16384, 1, 4, 128, 128
    width = 2 * H * K + HV * V + HV
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    finite = bits[torch.isfinite(bits.float())]
    gen = torch.Generator().manual_seed(0)

    def fill(n):  # n values cycling through every finite bf16 value, shuffled
        reps = -(-n // finite.numel())
        v = finite.repeat(reps)[:n]
        return v[torch.randperm(n, generator=gen)]

    cols = torch.cat([fill(T * 2 * H * K).view(T, -1), fill(T * HV * V).view(T, -1),
                      finite.repeat(-(-T * HV // finite.numel()))[:T * HV].view(T, HV)], dim=1)
    assert cols.shape[1] == width
    gl_vals = fill(T * HV * K).view(B, T, HV * K)
    outs = []
    for ld in (width + (-width) % 8, width + 1 - width % 2):  # aligned, then odd
        proj = torch.zeros(B, T, ld, dtype=torch.bfloat16)
        proj[0, :, :width] = cols
        proj = proj.to(dev)
        gl = gl_vals.to(dev)
        q = torch.empty(B, T, H, K, device=dev, dtype=torch.bfloat16)
        k = torch.empty_like(q)
        v = torch.empty(B, T, HV, V, device=dev, dtype=torch.bfloat16)
        g = torch.empty(B, T, HV, K, device=dev, dtype=torch.bfloat16)
        beta = torch.empty(B, T, HV, device=dev, dtype=torch.bfloat16)
        _lib.call("kch_kda_gates", _lib.ptr(proj), proj.stride(1), _lib.ptr(gl), gl.stride(1),
                  _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(g), _lib.ptr(beta),
                  B, T, H, HV, K, V, 0.1, _lib.dtype_code("t", torch.bfloat16),
                  _lib.stream_of(proj))
        torch.cuda.synchronize()
        outs.append([t.view(torch.int16).cpu() for t in (q, k, v, g, beta)])
    for name, a, b in zip(("q", "k", "v", "g", "beta"), *outs):
        diff = int((a != b).sum())
        assert diff == 0, f"{name}: {diff} of {a.numel()} elements differ"


@pytest.mark.parametrize("dtype,wdtype", [(torch.bfloat16, torch.float32),
                                          (torch.bfloat16, torch.bfloat16),
                                          (torch.float16, torch.float32)])
@pytest.mark.parametrize("rows,d", [(1, 64), (37, 2048), (5, 4096), (6, 1000), (3, 200)])
@pytest.mark.parametrize("bias", [True, False])
def test_layer_norm(dev, dtype, wdtype, rows, d, bias):
    """kch_layer_norm against torch's fp32 LayerNorm of the same inputs, rounded
    once to the output dtype: the two may differ by the fp32 summation order
    of the mean and variance, at most one output ulp."""
    from kch import _lib
    g = torch.Generator().manual_seed(rows * d)
    x = (3 * torch.randn(rows, d, generator=g) + 0.5).to(dev, dtype)
    w = (1 + 0.1 * torch.randn(d, generator=g)).to(dev, wdtype)
    b = (0.1 * torch.randn(d, generator=g)).to(dev, wdtype) if bias else None
    out = torch.empty_like(x)
    _lib.call("kch_layer_norm", _lib.ptr(x), _lib.ptr(w), _lib.ptr(b), _lib.ptr(out), rows, d, 1e-5,
              _lib.dtype_code("t", dtype), _lib.dtype_code("t", wdtype), _lib.stream_of(x))
    ref = torch.nn.functional.layer_norm(x.float(), (d,), w.float(), None if b is None else b.float(),
                                         1e-5)
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10  # one ulp, relative
    err = (out.float() - ref).abs()
    assert bool((err <= ulp * ref.abs() + 1e-5).all()), float((err / (ref.abs() + 1e-6)).max())
    assert float((out.float() == ref.to(dtype).float()).float().mean()) >= 0.99


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kda_layer_chunk_and_recurrent(dev, dtype):
    cfg = small_cfg()
    model, sd = build(cfg, dev, dtype, total_layers=1, seed=1)
    layer = model.layers[0]
    W = OH.layer_weights(sd, 0)
    c = cfg_dict(cfg)
    rng = np.random.default_rng(7)
    x = torch.from_numpy(rng.standard_normal((2, 150, cfg.d_model)).astype(np.float32)).to(dev, dtype)
    xn = x.float().cpu().numpy()
    # call 1: chunk path (T >= 64); calls 2, 3: recurrent path (T < 64), threading state + lookback
    st = lb = None
    sto = lbo = None
    for a, b in [(0, 130), (130, 131), (131, 150)]:
        y, st, lb = layer.forward_functional(x[:, a:b], st, lb)
        yo, sto, lbo = OH.kda_layer(xn[:, a:b], W, c, sto, lbo, DT[dtype])
        close(f"kda layer y[{a}:{b}]", y.float().cpu().numpy(), yo)
        close(f"kda layer state after {b}", st.cpu().numpy(), sto)
        np.testing.assert_array_equal(lb.float().cpu().numpy(), lbo)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [128, 100])
def test_hybrid_forward_vs_oracle(dev, dtype, T):
    cfg = small_cfg()
    model, sd = build(cfg, dev, dtype, seed=2)
    rng = np.random.default_rng(T)
    x = torch.from_numpy(rng.standard_normal((2, T, cfg.d_model)).astype(np.float32)).to(dev, dtype)
    import kch
    cap = LayerInputs(model)
    with kch.record_selections() as sel:
        y, states, lbs = model.forward_functional(x, None, [None] * 3)
    cap.remove()
    assert len(sel) == 1
    forced = {model.layout.index("csa"): host_sel(sel[0])}
    xn = x.float().cpu().numpy()
    outs, so, lo = OH.hybrid_forward(xn, sd, cfg_dict(cfg), model.layout, dtype=DT[dtype],
                                     csa_indices=forced, layer_inputs=cap.get())
    check_layers("hybrid", cap.get(), y, outs)
    for i in range(3):
        close(f"hybrid state {i}", states[i].cpu().numpy(), so[i])
        close(f"hybrid lookback {i}", lbs[i].float().cpu().numpy(), lo[i])
    yo, _, _ = OH.hybrid_forward(xn, sd, cfg_dict(cfg), model.layout, dtype=DT[dtype],
                                 csa_indices=forced)
    end_to_end("hybrid y", y.float().cpu().numpy(), yo, dtype)


@pytest.mark.parametrize("topk", [64, 5])
def test_hybrid_decoding_incremental_equals_full(dev, topk):
    """Prefill 128 tokens, then 12 single-token steps == the full 140-token
    forward at the last 12 positions (fp32 model; the property of
    ``run_correctness.py:5065-5115``). With topk < n_blocks the full forward and
    a decode step may select differently at a near-tie (their indexers read the
    keys in different precisions), so the decode steps whose selection equals
    the full forward's at that position are compared with it; every decode
    step is also checked against the oracle on its own selection."""
    import kch
    cfg = small_cfg(csa_topk=topk)
    dec = kch.HybridDecoding(cfg=cfg, total_layers=5)
    torch.manual_seed(3)
    with torch.no_grad():
        for layer in dec.model.layers:
            if hasattr(layer, 'sink'):
                layer.sink.normal_()
    dec = dec.to(dev).eval()
    x = torch.randn(2, 140, cfg.d_model, generator=torch.Generator().manual_seed(9)).to(dev)
    dec.reset()
    with kch.record_selections() as sel_full:
        y_full = dec.model(x)
    dec.reset()
    with kch.record_selections() as sel_dec:
        y_pre = dec(x[:, :128])
        ys = [dec(x[:, t:t + 1]) for t in range(128, 140)]
    torch.cuda.synchronize()
    close("prefill", y_pre.cpu().numpy(), y_full[:, :128].cpu().numpy(), 1e-4, 1e-4)
    full_sel = host_sel(sel_full[0])
    same = 0
    for s, t in enumerate(range(128, 140)):
        step_sel = host_sel(sel_dec[1 + s])[:, 0]
        for b in range(x.shape[0]):
            if set(step_sel[b].tolist()) == set(full_sel[b, t].tolist()):
                same += 1
                close(f"decode b{b} t{t}", ys[s][b].cpu().numpy(), y_full[b, t:t + 1].cpu().numpy())
    if topk >= 140 // cfg.csa_m:
        assert same == 12 * x.shape[0]
    assert same >= 12 * x.shape[0] // 2
    sd = {k: v.float().cpu().numpy() for k, v in dec.model.state_dict().items()}
    oracle = OH.HybridDecodingOracle(sd, cfg_dict(cfg), dec.model.layout, 'fp32')
    pos = dec.model.layout.index("csa")
    xn = x.cpu().numpy()
    oracle.step(xn[:, :128], csa_indices={pos: host_sel(sel_dec[0])})
    for s, t in enumerate(range(128, 140)):
        close(f"decode step {t} vs oracle", ys[s].cpu().numpy(),
              oracle.step(xn[:, t:t + 1], csa_indices={pos: host_sel(sel_dec[1 + s])}))
    assert dec._csa_caches[0].n_tokens_seen == 140
    assert dec._hca_caches[0].n_blocks == 140 // cfg.hca_m2


@pytest.mark.parametrize("dtype,fused", [(torch.float32, True), (torch.bfloat16, True),
                                         (torch.bfloat16, False)])
def test_hybrid_decoding_vs_oracle(dev, dtype, fused):
    """Decode steps across CSA (m=4) and HCA (m'=16, at t=79) block completions;
    bf16 steps run on the device-driven kernels unless ``fused_decode`` is off."""
    import kch
    cfg = small_cfg()
    model, sd = build(cfg, dev, dtype, seed=4)
    dec = kch.HybridDecoding(cfg=cfg, total_layers=5)
    dec.model = model
    dec.fused_decode = fused
    oracle = OH.HybridDecodingOracle(sd, cfg_dict(cfg), model.layout, DT[dtype])
    rng = np.random.default_rng(11)
    x = torch.from_numpy(rng.standard_normal((2, 82, cfg.d_model)).astype(np.float32)).to(dev, dtype)
    n_dev = decode_vs_oracle(dec, oracle, x, 67, DT[dtype])
    assert n_dev == (15 if fused and dtype == torch.bfloat16 else 0)


def test_hybrid_padding_no_crash(dev):
    cfg = small_cfg(csa_m=8, csa_topk=4, hca_m2=16)
    model, _ = build(cfg, dev, torch.float32, seed=5)
    for B in (1, 3, 8):
        for T in (10, 13, 20, 1):
            model.reset_state()
            x = 0.1 * torch.randn(B, T, cfg.d_model, device=dev)
            y = model(x)
            assert y.shape == x.shape and bool(torch.isfinite(y).all())


@pytest.mark.parametrize("hv,fused", [(2, False), (4, False), (2, True), (4, True)])
def test_hybrid_decoding_bf16_single_sequence(dev, hv, fused):
    """B=1 bf16 decode: the KDA gate input is a column slice of the fused
    projection that starts 2HK+HV*V+HV elements into the row; with one row and
    HV % 8 != 0 it is contiguous but not 16-byte aligned, so the few-row
    projection of the per-operator path must copy it into fresh storage (the
    device-driven step reads it in place)."""
    import kch
    cfg = small_cfg(n_heads_v=hv)
    model, sd = build(cfg, dev, torch.bfloat16, seed=6)
    dec = kch.HybridDecoding(cfg=cfg, total_layers=5)
    dec.model = model
    dec.fused_decode = fused
    oracle = OH.HybridDecodingOracle(sd, cfg_dict(cfg), model.layout, 'bf16')
    rng = np.random.default_rng(12 + hv)
    x = torch.from_numpy(rng.standard_normal((1, 40, cfg.d_model)).astype(np.float32)).to(
        dev, torch.bfloat16)
    assert decode_vs_oracle(dec, oracle, x, 34, "bf16 B1") == (6 if fused else 0)
