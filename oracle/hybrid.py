"""CPU restatement of the hybrid KDA / CSA / HCA composition (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline
use this module, as the checker.

Follows the reference's module code:

* ``layer_norm``        <- ``_Fp32LayerNorm`` (``ops_fused.py:42-60``)
* ``short_conv``        <- the causal depthwise conv with lookback (``ops_fused.py:480-527``)
* ``kda_layer``         <- ``KDAHybridLayer.forward_functional`` (``ops_fused.py:391-609``)
* ``csa_layer`` / ``hca_layer`` <- ``CSAHybridLayer.forward`` / ``HCAHybridLayer.forward``
  (``ops_fused.py:694-739``)
* ``hybrid_forward``    <- ``HybridKCHAttention.forward_functional`` (``ops_fused.py:956-1128``)
* ``HybridDecodingOracle`` <- ``HybridDecoding`` (``run_decoding.py:601-851``)

Weights come as a dict of numpy arrays named like the reference's
``state_dict`` (``layers.<i>.q_proj.weight`` ...). ``dtype`` names the model
dtype: every tensor the reference stores in it is rounded to it here (GEMM
outputs, activations, residual sums), arithmetic is fp32 otherwise.

Pinned by: the conv against ``np.convolve`` and the lookback split rule, the
LayerNorm against its closed form, the layer chain through
``oracle.kda`` / ``oracle.csa`` (pinned on their own), and the decode path
through the property "incremental == full" of the reference's test
``run_correctness.py:5065-5115`` (both checked in ``tests/test_oracle_hybrid.py``).
"""

from __future__ import annotations

import numpy as np

from .caches import CSACacheOracle, HCACacheOracle
from .common import l2_normalize, round_to
from .csa import csa_projections, linear_lowp, naive_csa, naive_hca
from .kda import chunk_kda, recurrent_kda


def layer_norm(x, w, b, eps=1e-5, dtype='fp32'):
    """LayerNorm over the last axis in fp32 (biased variance), rounded to ``dtype``."""
    x = np.asarray(x, np.float32)
    mu = x.mean(-1, keepdims=True, dtype=np.float64)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps) * np.asarray(w, np.float32) + np.asarray(b, np.float32)
    return round_to(y.astype(np.float32), dtype)


def short_conv(x, weight, bias, lookback=None, dtype='fp32'):
    """``out[t] = bias + w0 x[t-2] + w1 x[t-1] + w2 x[t]`` over ``[lookback ; x]``
    (zeros without a lookback); ``weight`` ``[d,1,3]`` or ``[d,3]``; fp32 sums."""
    x = np.asarray(x, np.float32)
    B, T, d = x.shape
    w = np.asarray(weight, np.float32).reshape(d, 3)
    left = np.zeros((B, 2, d), np.float32) if lookback is None else np.asarray(lookback, np.float32)
    xp = np.concatenate([left, x], axis=1)
    out = xp[:, 0:T] * w[:, 0] + xp[:, 1:T + 1] * w[:, 1] + xp[:, 2:T + 2] * w[:, 2]
    if bias is not None:
        out = out + np.asarray(bias, np.float32)
    return round_to(out, dtype)


def new_lookback(x, lookback):
    """The last two rows of ``[lookback ; x]`` (zero-padded on the left)."""
    B, T, d = x.shape
    if T >= 2:
        return np.array(x[:, -2:], np.float32)
    left = np.zeros((B, 2, d), np.float32) if lookback is None else np.asarray(lookback, np.float32)
    return np.concatenate([left, x], axis=1)[:, -2:]


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def _normalize_lowp(x, dtype):
    """``F.normalize`` on a tensor of ``dtype``: the norm and the quotient are
    each stored in ``dtype``."""
    n = round_to(np.sqrt((np.asarray(x, np.float64) ** 2).sum(-1, keepdims=True)), dtype)
    return round_to(x / np.maximum(n, 1e-12), dtype)


def kda_activations(pq, pk, pv, gl, pb, H, HV, K, V, decay_scale, dtype='fp32'):
    """The KDA layer's activations from its projections (``ops_fused.py:571-581``):
    ``q, k = F.normalize(F.silu(.))`` per head, ``v = F.silu(.)``,
    ``g = -F.softplus(.) * decay_scale``, ``beta = sigmoid(.)``, each torch
    operation's result stored in ``dtype``. Inputs ``[B, T, width]``."""
    B, T = pq.shape[:2]
    q = _normalize_lowp(round_to(_silu(pq), dtype).reshape(B, T, H, K), dtype)
    k = _normalize_lowp(round_to(_silu(pk), dtype).reshape(B, T, H, K), dtype)
    v = round_to(_silu(pv), dtype).reshape(B, T, HV, V)
    g = round_to(-round_to(_softplus(gl), dtype) * np.float32(decay_scale), dtype)
    g = g.reshape(B, T, HV, K)
    beta = round_to(1.0 / (1.0 + np.exp(-np.asarray(pb, np.float32))), dtype)
    return q, k, v, g, beta


def kda_layer(x, W, cfg, state=None, lookback=None, dtype='fp32'):
    """One KDA sub-layer; returns ``(out [B,T,d], new_state fp32, new_lookback)``."""
    B, T, d = x.shape
    H, K, V, HV = cfg['n_heads_qk'], cfg['head_dim_k'], cfg['head_dim_v'], cfg['n_heads_v']
    xc = short_conv(x, W['short_conv.weight'], W.get('short_conv.bias'), lookback, dtype)
    lb = new_lookback(x, lookback)
    gl = linear_lowp(linear_lowp(xc, W['g_down.weight'], dtype), W['g_up.weight'], dtype)
    q, k, v, g, beta = kda_activations(
        linear_lowp(xc, W['q_proj.weight'], dtype), linear_lowp(xc, W['k_proj.weight'], dtype),
        linear_lowp(xc, W['v_proj.weight'], dtype), gl, linear_lowp(xc, W['beta.weight'], dtype),
        H, HV, K, V, cfg['kda_decay_scale'], dtype)
    scale = float(round_to(np.float32(K ** -0.5), dtype).reshape(-1)[0])
    cs = cfg['kda_chunk_size']
    if cs >= 1 and T >= cs:
        o, S = chunk_kda(q, k, v, g, beta, scale=scale, initial_state=state, chunk_size=cs)
    else:
        o, S = recurrent_kda(q, k, v, g, beta, scale=scale, initial_state=state)
    o = round_to(o, dtype).reshape(B, T, HV * V)
    return linear_lowp(o, W['o_proj.weight'], dtype), S.astype(np.float32), lb


def _csa_w(W):
    names = ['W_aKV', 'W_bKV', 'W_aZ', 'W_bZ', 'W_DQ', 'W_UQ', 'W_IUQ', 'W_w', 'W_KV_idx',
             'W_Z_idx']
    out = {n: W[n + '.weight'] for n in names}
    out.update(Ba=W['Ba'], Bb=W['Bb'], B_idx=W['B_idx'])
    return out


def _hca_w(W):
    out = {n: W[n + '.weight'] for n in ['W_KV', 'W_Z', 'W_DQ', 'W_UQ']}
    out['B_pos'] = W['B_pos']
    return out


def csa_layer(x, W, cfg, dtype='fp32', indices=None):
    o, _ = naive_csa(x, _csa_w(W), m=cfg['csa_m'], topk=cfg['csa_topk'], nh=cfg['csa_nh'],
                     nIh=cfg['csa_nIh'], c=cfg['csa_c'], c_I=cfg['csa_cI'],
                     sliding_window=cfg['csa_sliding_window'], sink=W['sink'], dtype=dtype,
                     indices=indices)
    return linear_lowp(o, W['o_proj.weight'], dtype)


def hca_layer(x, W, cfg, dtype='fp32'):
    o, _ = naive_hca(x, _hca_w(W), m2=cfg['hca_m2'], nh=cfg['hca_nh'], c=cfg['hca_c'],
                     sliding_window=cfg['hca_sliding_window'], sink=W['sink'], dtype=dtype)
    return linear_lowp(o, W['o_proj.weight'], dtype)


def layer_weights(sd, i):
    """The weights of sub-layer ``i`` from a flat ``state_dict``-named dict."""
    pre = f'layers.{i}.'
    return {k[len(pre):]: v for k, v in sd.items() if k.startswith(pre)}


def build_layout(cfg, total_layers):
    unit = ['kda'] * cfg['n_kda'] + ['csa'] * cfg['n_csa'] + ['hca'] * cfg['n_hca']
    layout = []
    while len(layout) < total_layers:
        layout.extend(unit)
    return layout[:total_layers]


def hybrid_forward(x, sd, cfg, layout, states=None, lookbacks=None, dtype='fp32',
                   csa_indices=None, layer_inputs=None):
    """Returns ``(y, states, lookbacks)`` (one state / lookback per KDA layer).

    ``csa_indices`` maps a CSA layer's position in ``layout`` to a selection
    ``[B,T,topk]`` that replaces its indexer's (to check the rest of the stack
    on a given selection). ``layer_inputs`` (one ``[B,T,d]`` residual stream per
    layer) feeds layer i that stream instead of layer i-1's output, and the
    result is then ``(per-layer outputs, states, lookbacks)``: each layer
    checked on the input another implementation gave it."""
    x = round_to(x, dtype)
    n_kda = layout.count('kda')
    states = list(states) if states is not None else [None] * n_kda
    lookbacks = list(lookbacks) if lookbacks is not None else [None] * n_kda
    outs = []
    j = 0
    for i, kind in enumerate(layout):
        if layer_inputs is not None:
            x = round_to(layer_inputs[i], dtype)
        W = layer_weights(sd, i)
        h = layer_norm(x, sd[f'norms.{i}.weight'], sd[f'norms.{i}.bias'], dtype=dtype)
        if kind == 'kda':
            o, states[j], lookbacks[j] = kda_layer(h, W, cfg, states[j], lookbacks[j], dtype)
            j += 1
        elif kind == 'csa':
            o = csa_layer(h, W, cfg, dtype, None if csa_indices is None else csa_indices.get(i))
        else:
            o = hca_layer(h, W, cfg, dtype)
        x = round_to(x + o, dtype)
        outs.append(x)
    return (outs if layer_inputs is not None else x), states, lookbacks


class HybridDecodingOracle:
    """Prefill (T > 1, full operators + bulk cache population) and T == 1
    decode steps through the cache oracles (``run_decoding.py:676-851``)."""

    def __init__(self, sd, cfg, layout, dtype='fp32'):
        self.sd, self.cfg, self.layout, self.dtype = sd, cfg, layout, dtype
        self.reset()

    def reset(self):
        n_kda = self.layout.count('kda')
        self.states = [None] * n_kda
        self.lookbacks = [None] * n_kda
        self.caches = {}

    def _cache(self, i, kind, B):
        if i not in self.caches:
            cfg = self.cfg
            cd = 'fp32' if self.dtype == 'fp32' else self.dtype
            if kind == 'csa':
                self.caches[i] = CSACacheOracle(B, cfg['csa_c'], cfg['csa_cI'], cfg['csa_m'],
                                                cfg['csa_sliding_window'], cd)
            else:
                self.caches[i] = HCACacheOracle(B, cfg['hca_c'], cfg['hca_m2'],
                                                cfg['hca_sliding_window'], cd)
        return self.caches[i]

    def step(self, x, csa_indices=None, layer_inputs=None):
        """One call of ``HybridDecoding.forward``; ``csa_indices`` (layer position
        -> selection ``[B,T,topk]``) replaces a CSA layer's indexer output;
        ``layer_inputs`` feeds each layer a given residual stream and makes the
        result the list of per-layer outputs (as in ``hybrid_forward``)."""
        cfg, dtype = self.cfg, self.dtype
        x = round_to(x, dtype)
        B, T, _ = x.shape
        outs = []
        j = 0
        for i, kind in enumerate(self.layout):
            if layer_inputs is not None:
                x = round_to(layer_inputs[i], dtype)
            W = layer_weights(self.sd, i)
            h = layer_norm(x, self.sd[f'norms.{i}.weight'], self.sd[f'norms.{i}.bias'],
                           dtype=dtype)
            if kind == 'kda':
                o, self.states[j], self.lookbacks[j] = kda_layer(
                    h, W, cfg, self.states[j], self.lookbacks[j], dtype)
                j += 1
            elif kind == 'csa':
                cache = self._cache(i, 'csa', B)
                w = _csa_w(W)
                sel = None if csa_indices is None else csa_indices.get(i)
                if T > 1:
                    oc, proj = naive_csa(h, w, m=cfg['csa_m'], topk=cfg['csa_topk'],
                                         nh=cfg['csa_nh'], nIh=cfg['csa_nIh'], c=cfg['csa_c'],
                                         c_I=cfg['csa_cI'],
                                         sliding_window=cfg['csa_sliding_window'],
                                         sink=W['sink'], dtype=dtype, indices=sel)
                    cache.append_step(*proj[:6], w['Ba'], w['Bb'], w['B_idx'])
                else:
                    Ca, Cb, Za, Zb, Ki, Zi, q, qi, wi = csa_projections(
                        h, w, dtype, c=cfg['csa_c'], cI=cfg['csa_cI'], nh=cfg['csa_nh'],
                        nIh=cfg['csa_nIh'])
                    cache.append_step(Ca, Cb, Za, Zb, Ki, Zi, w['Ba'], w['Bb'], w['B_idx'])
                    oc = cache.forward_step(l2_normalize(q), qi, wi, topk=cfg['csa_topk'],
                                            scale=1.0, sink_logits=W['sink'], normalize_qk=True,
                                            indices=sel)
                    oc = round_to(oc.reshape(B, T, -1), dtype)
                o = linear_lowp(oc, W['o_proj.weight'], dtype)
            else:
                cache = self._cache(i, 'hca', B)
                w = _hca_w(W)
                if T > 1:
                    oc, (C, Z, _q) = naive_hca(h, w, m2=cfg['hca_m2'], nh=cfg['hca_nh'],
                                               c=cfg['hca_c'],
                                               sliding_window=cfg['hca_sliding_window'],
                                               sink=W['sink'], dtype=dtype)
                    cache.append_step(C, Z, w['B_pos'])
                else:
                    C = linear_lowp(h, w['W_KV'], dtype)
                    Z = linear_lowp(h, w['W_Z'], dtype)
                    q = linear_lowp(linear_lowp(h, w['W_DQ'], dtype), w['W_UQ'], dtype)
                    q = q.reshape(B, T, cfg['hca_nh'], cfg['hca_c'])
                    cache.append_step(C, Z, w['B_pos'])
                    oc = cache.forward_step(l2_normalize(q), scale=1.0, sink_logits=W['sink'])
                    oc = round_to(oc.reshape(B, T, -1), dtype)
                o = linear_lowp(oc, W['o_proj.weight'], dtype)
            x = round_to(x + o, dtype)
            outs.append(x)
        return outs if layer_inputs is not None else x
