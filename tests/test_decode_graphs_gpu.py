"""Graphed decode steps against eager ones (needs a ROCm GPU).

``HybridDecoding`` replays HIP graphs of a decode step's static parts (norms,
KDA layers with in-place lookback and state, projections, residual adds) with
the cache updates and decode attention run eagerly between them. Two copies
of one model, one with graphs and one without, are stepped side by side
through prefill and decode steps that cross CSA and HCA block boundaries
(compressions fire between the replays), with a device synchronisation and
the eager copy's own work between the graphed steps: every output must be
bit-identical (the same kernels on the same values). The graphs must be
captured again after the weights change: by ``load_state_dict`` (new
contents, same storage) and by an in-place update of one parameter.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

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
    dg = dg.to(dev, torch.bfloat16).eval()
    de = copy.deepcopy(dg)
    de.use_graphs = False
    return dg, de


def _steps(dg, de, x, t0, t1):
    for t in range(t0, t1):
        yg = dg(x[:, t:t + 1])
        torch.cuda.synchronize()
        ye = de(x[:, t:t + 1])
        torch.cuda.synchronize()
        assert torch.equal(yg, ye), f"step {t}: graphed and eager outputs differ"


def test_graphed_decode_matches_eager(dev):
    dg, de = _pair(dev, 5)
    rng = np.random.default_rng(6)
    x = torch.from_numpy(rng.standard_normal((2, 70, 128)).astype(np.float32)).to(
        dev, torch.bfloat16)
    assert torch.equal(dg(x[:, :37]), de(x[:, :37]))
    _steps(dg, de, x, 37, 70)   # crosses 8 CSA blocks (m=4) and 2 HCA blocks (m'=16)
    assert dg._graphs is not None and de._graphs is None


def test_graphs_follow_weight_changes(dev):
    dg, de = _pair(dev, 7)
    rng = np.random.default_rng(8)
    x = torch.from_numpy(rng.standard_normal((2, 60, 128)).astype(np.float32)).to(
        dev, torch.bfloat16)
    dg(x[:, :20])
    de(x[:, :20])
    _steps(dg, de, x, 20, 26)
    first = dg._graphs
    # new contents through load_state_dict (same storage; fused copies rebuilt)
    sd = {k: v + 0.01 * torch.randn_like(v) if v.is_floating_point() else v
          for k, v in de.model.state_dict().items()}
    dg.model.load_state_dict(sd)
    de.model.load_state_dict(sd)
    _steps(dg, de, x, 26, 34)
    assert dg._graphs is not first
    second = dg._graphs
    # an in-place update of one parameter (version bump)
    with torch.no_grad():
        dg.model.norms[1].weight.mul_(1.5)
        de.model.norms[1].weight.mul_(1.5)
    _steps(dg, de, x, 34, 40)
    assert dg._graphs is not second


def test_forward_hooks_keep_the_eager_step(dev):
    """A forward hook must see every step's values: a hooked model is not graphed."""
    dg, de = _pair(dev, 9)
    rng = np.random.default_rng(10)
    x = torch.from_numpy(rng.standard_normal((2, 30, 128)).astype(np.float32)).to(
        dev, torch.bfloat16)
    seen = []
    hook = dg.model.norms[2].register_forward_hook(lambda m, i, o: seen.append(o.float().cpu()))
    try:
        dg(x[:, :24])
        de(x[:, :24])
        _steps(dg, de, x, 24, 30)
    finally:
        hook.remove()
    assert dg._graphs is None and len(seen) == 7
    assert not torch.equal(seen[-1], seen[-2])
    _steps(dg, de, x.flip(1), 0, 3)   # hook removed: the next steps are graphed
    assert dg._graphs is not None
