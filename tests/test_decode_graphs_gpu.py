"""The device-driven decode step, graphed and eager (needs a ROCm GPU).

``HybridDecoding`` runs a bf16 decode step on kernels that read every
per-step count (blocks, window length, accumulator and ring slots) from one
device counter of cached tokens, and replays that step from one captured HIP
graph. Two copies of one model, one replaying the graph and one launching the
same kernels eagerly (``use_graphs=False``), are stepped side by side through
prefill and decode steps that cross CSA and HCA block completions and the
doubling of the caches' block storage (each a re-capture), with a device
synchronisation and the eager copy's own work between the graphed steps: every
output and every CSA selection must be bit-identical. The graph must be
captured again after weight changes (``load_state_dict``, an in-place update,
a write through ``.data`` followed by ``invalidate_weight_cache()``); steps on
the per-operator path in between (``fused_decode=False``, or a forward hook)
must leave the device counter consistent. Agreement with the oracle is
checked by the decode tests of ``test_hybrid_gpu.py`` and
``test_regimes_gpu.py``, which run on this path.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from composed_check import check_layers, host_sel
from oracle import hybrid as OH

pytestmark = pytest.mark.gpu


def _cfg():
    import kch
    return kch.HybridConfig(d_model=128, n_heads_qk=2, n_heads_v=2, head_dim_k=64, head_dim_v=64,
                            kda_chunk_size=64, csa_m=4, csa_topk=8, csa_nh=2, csa_c=64, csa_dc=32,
                            csa_nIh=2, csa_cI=32, csa_sliding_window=8, hca_m2=16, hca_nh=2,
                            hca_c=64, hca_dc=32, hca_sliding_window=8)


def _pair(dev, seed):
    import kch
    torch.manual_seed(seed)
    dg = kch.HybridDecoding(cfg=_cfg(), total_layers=5)
    with torch.no_grad():
        for layer in dg.model.layers:
            if hasattr(layer, 'sink'):
                layer.sink.normal_()
        for n in dg.model.norms:
            n.weight.normal_(1.0, 0.1)
            n.bias.normal_(0.0, 0.1)
    dg = dg.to(dev, torch.bfloat16).eval()
    de = copy.deepcopy(dg)
    de.use_graphs = False
    return dg, de


def _x(seed, T):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.standard_normal((2, T, 128)).astype(np.float32)).to(
        "cuda", torch.bfloat16)


def _steps(dg, de, x, t0, t1):
    for t in range(t0, t1):
        yg = dg(x[:, t:t + 1])
        torch.cuda.synchronize()
        ye = de(x[:, t:t + 1])
        torch.cuda.synchronize()
        assert torch.equal(yg, ye), f"step {t}: graphed and eager outputs differ"
        assert torch.equal(dg._csa_caches[0]._last_indices, de._csa_caches[0]._last_indices), \
            f"step {t}: selections differ"


def test_graphed_step_matches_eager(dev):
    dg, de = _pair(dev, 5)
    x = _x(6, 90)
    assert torch.equal(dg(x[:, :37]), de(x[:, :37]))
    _steps(dg, de, x, 37, 90)   # 13 CSA blocks (m=4), 3 HCA blocks (m'=16), storage doubling
    assert dg._graph is not None and de._graph is None
    assert dg._device_steps == de._device_steps == 53
    c = dg._csa_caches[0]
    assert c.n_tokens_seen == 90 and c.n_blocks == 22 and dg._hca_caches[0].n_blocks == 5
    for a, b in zip(dg._caches(), de._caches()):
        assert torch.equal(a._C.keys[:, :a.n_blocks], b._C.keys[:, :b.n_blocks])
        assert torch.equal(a._sw._buf, b._sw._buf)


def test_graphs_follow_weight_changes(dev):
    dg, de = _pair(dev, 7)
    x = _x(8, 60)
    dg(x[:, :20])
    de(x[:, :20])
    _steps(dg, de, x, 20, 26)
    first = dg._graph
    # new contents through load_state_dict (same storage, version bumps)
    sd = {k: v + 0.01 * torch.randn_like(v) if v.is_floating_point() else v
          for k, v in de.model.state_dict().items()}
    dg.model.load_state_dict(sd)
    de.model.load_state_dict(sd)
    _steps(dg, de, x, 26, 34)
    assert dg._graph is not first
    second = dg._graph
    # an in-place update of a norm weight (read by the graph directly)
    with torch.no_grad():
        dg.model.norms[1].weight.mul_(1.5)
        de.model.norms[1].weight.mul_(1.5)
    _steps(dg, de, x, 34, 40)
    assert dg._graph is not second
    # a write through .data (no version bump) announced to the layer
    for d in (dg, de):
        layer = d.model.layers[d.model.layout.index('csa')]
        layer.W_aKV.weight.data.mul_(1.25)
        layer.invalidate_weight_cache()
    _steps(dg, de, x, 40, 46)


def test_per_operator_steps_in_between(dev):
    """Steps on the per-operator path (a forward hook; ``fused_decode=False``)
    between device steps: each sub-layer against the teacher-forced oracle."""
    import kch
    dg, _ = _pair(dev, 9)
    x = _x(10, 70)
    sd = {k: v.float().cpu().numpy() for k, v in dg.model.state_dict().items()}
    cfg = dg.cfg
    oracle = OH.HybridDecodingOracle(sd, {k: getattr(cfg, k) for k in cfg.__dataclass_fields__},
                                     dg.model.layout, 'bf16')
    pos = dg.model.layout.index("csa")
    xn = x.float().cpu().numpy()
    seen = []
    hook = None
    dg._trace = []
    try:
        for a, b in [(0, 30)] + [(t, t + 1) for t in range(30, 70)]:
            if a == 38:
                hook = dg.model.norms[2].register_forward_hook(lambda m, i, o: seen.append(1))
            if a == 42:
                hook.remove()
            dg.fused_decode = not (50 <= a < 55)
            before = dg._device_steps
            with kch.record_selections() as sel:
                y = dg(x[:, a:b])
            device = dg._device_steps > before
            assert device == (a >= 30 and not 38 <= a < 42 and not 50 <= a < 55), a
            layer_in = [t.float().cpu().numpy() for t in dg._trace.pop()]
            outs = oracle.step(xn[:, a:b], csa_indices={pos: host_sel(sel[0])},
                               layer_inputs=layer_in)
            check_layers(f"step [{a}:{b}]", layer_in, y, outs)
    finally:
        dg._trace = None
    assert len(seen) == 4
    assert dg._csa_caches[0].n_tokens_seen == 70


def test_graph_replays_with_eager_work_between(dev):
    """Graph replays interleaved with the eager copy's steps and a device
    synchronisation each time; then the graphed copy alone for several steps
    and one final comparison of the caches."""
    dg, de = _pair(dev, 11)
    x = _x(12, 64)
    dg(x[:, :33])
    de(x[:, :33])
    _steps(dg, de, x, 33, 45)
    for t in range(45, 64):
        yg = dg(x[:, t:t + 1])
        ye = de(x[:, t:t + 1])
        assert torch.equal(yg, ye), t
    torch.cuda.synchronize()
    for a, b in zip(dg._caches(), de._caches()):
        assert torch.equal(a._C.rows[:, :a.n_blocks], b._C.rows[:, :b.n_blocks])
    assert torch.equal(dg.model._kda_state, de.model._kda_state)
