"""CPU pins of the hybrid-composition oracle and of the HIP package's host-side
config / module structure (no GPU needed).

* short conv == per-channel ``np.convolve`` (the textbook causal convolution),
  and splitting a sequence with the lookback rule reproduces the whole;
* LayerNorm against its closed form;
* KDA layer: state + lookback threading over two calls == one call;
* hybrid decode: prefill + single-token steps through the cache oracles ==
  the full-sequence forward (the reference's own property,
  ``run_correctness.py:5065-5115``, with ``topk >= n_blocks``);
* ``kch.HybridConfig`` validation, layout string and ``state_dict`` names
  (``ops_fused.py:65-313,742-900``).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import hybrid as H

CFG = dict(d_model=32, n_heads_qk=2, n_heads_v=2, head_dim_k=8, head_dim_v=8,
           kda_chunk_size=8, kda_decay_scale=0.1,
           csa_m=4, csa_topk=64, csa_nh=2, csa_c=8, csa_dc=16, csa_nIh=2, csa_cI=4,
           csa_sliding_window=4, hca_m2=8, hca_nh=2, hca_c=8, hca_dc=16, hca_sliding_window=4,
           n_kda=3, n_csa=1, n_hca=1)


def _weights(cfg, total_layers, seed=0):
    rng = np.random.default_rng(seed)
    d, Hh, K, V, HV = (cfg[k] for k in ('d_model', 'n_heads_qk', 'head_dim_k', 'head_dim_v',
                                        'n_heads_v'))
    layout = H.build_layout(cfg, total_layers)
    sd = {}

    def lin(name, o, i):
        sd[name] = (rng.standard_normal((o, i)) / np.sqrt(i)).astype(np.float32)

    for i, kind in enumerate(layout):
        p = f'layers.{i}.'
        sd[f'norms.{i}.weight'] = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
        sd[f'norms.{i}.bias'] = (0.1 * rng.standard_normal(d)).astype(np.float32)
        if kind == 'kda':
            lin(p + 'q_proj.weight', Hh * K, d)
            lin(p + 'k_proj.weight', Hh * K, d)
            lin(p + 'v_proj.weight', HV * V, d)
            lin(p + 'g_down.weight', K, d)
            lin(p + 'g_up.weight', HV * K, K)
            lin(p + 'beta.weight', HV, d)
            lin(p + 'o_proj.weight', d, HV * V)
            sd[p + 'short_conv.weight'] = (0.5 * rng.standard_normal((d, 1, 3))).astype(np.float32)
            sd[p + 'short_conv.bias'] = (0.1 * rng.standard_normal(d)).astype(np.float32)
        elif kind == 'csa':
            c, cI, nh, nIh, dc, m = (cfg[k] for k in ('csa_c', 'csa_cI', 'csa_nh', 'csa_nIh',
                                                      'csa_dc', 'csa_m'))
            for n in ('W_aKV', 'W_bKV', 'W_aZ', 'W_bZ'):
                lin(p + n + '.weight', c, d)
            lin(p + 'W_DQ.weight', dc, d)
            lin(p + 'W_UQ.weight', c * nh, dc)
            lin(p + 'W_IUQ.weight', cI * nIh, dc)
            lin(p + 'W_w.weight', nIh, d)
            lin(p + 'W_KV_idx.weight', cI, d)
            lin(p + 'W_Z_idx.weight', cI, d)
            lin(p + 'o_proj.weight', d, c * nh)
            for n, w in (('Ba', c), ('Bb', c), ('B_idx', cI)):
                sd[p + n] = (0.02 * rng.standard_normal((m, w))).astype(np.float32)
            sd[p + 'sink'] = rng.standard_normal(nh).astype(np.float32)
        else:
            c, nh, dc, m2 = (cfg[k] for k in ('hca_c', 'hca_nh', 'hca_dc', 'hca_m2'))
            lin(p + 'W_KV.weight', c, d)
            lin(p + 'W_Z.weight', c, d)
            lin(p + 'W_DQ.weight', dc, d)
            lin(p + 'W_UQ.weight', c * nh, dc)
            lin(p + 'o_proj.weight', d, c * nh)
            sd[p + 'B_pos'] = (0.02 * rng.standard_normal((m2, c))).astype(np.float32)
            sd[p + 'sink'] = rng.standard_normal(nh).astype(np.float32)
    return sd, layout


def test_short_conv_is_causal_convolution():
    rng = np.random.default_rng(1)
    B, T, d = 2, 11, 5
    x = rng.standard_normal((B, T, d)).astype(np.float32)
    w = rng.standard_normal((d, 1, 3)).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    out = H.short_conv(x, w, b)
    for bb in range(B):
        for c in range(d):
            # np.convolve flips the kernel: the tap on x[t] is w[c,0,2]
            ref = np.convolve(x[bb, :, c], w[c, 0, ::-1])[:T] + b[c]
            np.testing.assert_allclose(out[bb, :, c], ref, rtol=1e-5, atol=1e-5)
    # the lookback rule: conv(x) == [conv(x[:, :s]) ; conv(x[:, s:], lookback)]
    for s in (1, 2, 7):
        lb = H.new_lookback(x[:, :s], None)
        two = np.concatenate([H.short_conv(x[:, :s], w, b),
                              H.short_conv(x[:, s:], w, b, lookback=lb)], axis=1)
        np.testing.assert_allclose(two, out, rtol=1e-6, atol=1e-6)
    # three single-token calls thread the lookback through a length-1 chunk
    lb = None
    parts = []
    for t in range(3):
        parts.append(H.short_conv(x[:, t:t + 1], w, b, lookback=lb))
        lb = H.new_lookback(x[:, t:t + 1], lb)
    np.testing.assert_allclose(np.concatenate(parts, 1), out[:, :3], rtol=1e-6, atol=1e-6)


def test_layer_norm_closed_form():
    rng = np.random.default_rng(2)
    x = (3 + 2 * rng.standard_normal((4, 7, 16))).astype(np.float32)
    y = H.layer_norm(x, np.ones(16), np.zeros(16))
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-5)
    np.testing.assert_allclose(y.var(-1), 1, atol=1e-3)
    v = np.array([[1.0, 2.0, 3.0, 6.0]], np.float32)
    # mean 3, biased variance 3.5
    np.testing.assert_allclose(H.layer_norm(v, [2, 2, 2, 2], [1, 1, 1, 1], eps=0.0),
                               1 + 2 * (v - 3) / np.sqrt(3.5), rtol=1e-6)


def test_kda_layer_split_equals_whole():
    sd, layout = _weights(CFG, 1)
    W = H.layer_weights(sd, 0)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 21, CFG['d_model'])).astype(np.float32)
    y, S, lb = H.kda_layer(x, W, CFG)
    y1, S1, lb1 = H.kda_layer(x[:, :9], W, CFG)
    y2, S2, lb2 = H.kda_layer(x[:, 9:], W, CFG, S1, lb1)
    np.testing.assert_allclose(np.concatenate([y1, y2], 1), y, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(S2, S, rtol=1e-4, atol=1e-5)
    np.testing.assert_array_equal(lb2, lb)


def test_hybrid_decode_oracle_matches_full():
    sd, layout = _weights(CFG, 5, seed=4)
    assert layout == ['kda', 'kda', 'kda', 'csa', 'hca']
    rng = np.random.default_rng(5)
    T0, n = 17, 6
    x = (0.5 * rng.standard_normal((2, T0 + n, CFG['d_model']))).astype(np.float32)
    y_full, _, _ = H.hybrid_forward(x, sd, CFG, layout)
    dec = H.HybridDecodingOracle(sd, CFG, layout)
    y_pre = dec.step(x[:, :T0])
    np.testing.assert_allclose(y_pre, y_full[:, :T0], rtol=1e-4, atol=1e-5)
    for t in range(T0, T0 + n):
        y_t = dec.step(x[:, t:t + 1])
        np.testing.assert_allclose(y_t, y_full[:, t:t + 1], rtol=1e-4, atol=1e-5)


def test_hybrid_config_validation():
    import kch
    cfg = kch.HybridConfig()
    assert cfg.kda_backend == "hip"
    with pytest.raises(ValueError):
        kch.HybridConfig(kda_backend="triton")
    with pytest.raises(ValueError, match="divisible"):
        kch.HybridConfig(n_heads_qk=3, n_heads_v=4)
    with pytest.raises(NotImplementedError):
        kch.HybridConfig(dropout=0.1)
    with pytest.raises(TypeError):
        kch.HybridConfig(dropout="x")
    with pytest.raises(ValueError):
        kch.HybridConfig(dropout=float("nan"))
    with pytest.raises(ValueError):
        kch.HybridConfig(csa_topk=-1)
    with pytest.raises(ValueError):
        kch.HybridConfig(n_kda=0, n_csa=0, n_hca=0)
    with pytest.raises(ValueError):
        kch.HybridConfig(head_dim_k=0)
    with pytest.raises(ValueError):
        kch.HybridConfig(kda_decay_scale=-1.0)
    with pytest.raises(ValueError):
        kch.HybridKCHAttention(cfg, total_layers=-1)


def test_hybrid_layout_and_state_dict_names():
    import kch
    cfg = kch.HybridConfig(d_model=64, head_dim_k=64, head_dim_v=64, n_heads_qk=2, n_heads_v=2)
    model = kch.HybridKCHAttention(cfg, total_layers=5)
    assert model.layout_str() == 'KDA-KDA-KDA-CSA-HCA'
    assert kch.HybridKCHAttention(cfg, total_layers=7).layout_str() == \
        'KDA-KDA-KDA-CSA-HCA-KDA-KDA'
    sd = model.state_dict()
    kda = ['q_proj.weight', 'k_proj.weight', 'v_proj.weight', 'g_down.weight', 'g_up.weight',
           'beta.weight', 'o_proj.weight', 'short_conv.weight', 'short_conv.bias']
    csa = ['W_aKV.weight', 'W_bKV.weight', 'W_aZ.weight', 'W_bZ.weight', 'Ba', 'Bb',
           'W_DQ.weight', 'W_UQ.weight', 'W_IUQ.weight', 'W_w.weight', 'W_KV_idx.weight',
           'W_Z_idx.weight', 'B_idx', 'sink', 'o_proj.weight']
    hca = ['W_KV.weight', 'W_Z.weight', 'B_pos', 'W_DQ.weight', 'W_UQ.weight', 'sink',
           'o_proj.weight']
    expect = []
    for i, names in enumerate([kda, kda, kda, csa, hca]):
        expect += [f'layers.{i}.{n}' for n in names]
    expect += [f'norms.{i}.{n}' for i in range(5) for n in ('weight', 'bias')]
    assert sorted(sd) == sorted(expect)
    assert sd['layers.0.short_conv.weight'].shape == (64, 1, 3)
    assert sd['layers.3.B_idx'].shape == (cfg.csa_m, cfg.csa_cI)
    # the KDA scale buffer rounds with the module (ops_fused.py:342-344)
    layer = model.layers[0].to(torch.bfloat16)
    assert layer._scale_value() == float(torch.tensor(64 ** -0.5).bfloat16())


def test_hybrid_forward_needs_gpu():
    import kch
    cfg = kch.HybridConfig(d_model=64, head_dim_k=64, head_dim_v=64, n_heads_qk=2, n_heads_v=2)
    model = kch.HybridKCHAttention(cfg, total_layers=1)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        model(torch.zeros(1, 4, 64))
    # T == 0 needs no kernel
    y = model(torch.zeros(2, 0, 64))
    assert y.shape == (2, 0, 64)
