"""HIP decode caches vs the cache oracle (needs a ROCm GPU).

A bulk prefill ``append_step`` followed by single-token ``append_step`` +
``forward_step`` steps, fed identically to ``kch.CSADecodingCache`` /
``kch.HCADecodingCache`` and to ``oracle.caches``. Checked each step: block
counts, accumulator length, ring contents (cache dtype, 1 bf16 ulp), cached
compressed rows (1 bf16 ulp) and the outputs (atol 2e-3 + rtol 2e-2; with
topk < n_blocks the oracle uses the HIP selection, which is checked against
the oracle's own to be tie-consistent).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.caches import CSACacheOracle, HCACacheOracle
from oracle.common import l2_normalize
from oracle.csa import causal_block_mask, lightning_indexer
from selection_check import check_selection, logit_eps

pytestmark = pytest.mark.gpu


def close(name, got, ref, rtol=2e-2, atol=2e-3):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    bad = np.abs(got - ref) > atol + rtol * np.abs(ref)
    assert not bad.any(), f"{name}: {bad.sum()} bad, max abs err {np.abs(got - ref).max():.3e}"


def ulp_close(name, got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    tol = 2.0 ** -7 * np.maximum(np.abs(ref), 1e-30) + 1e-30
    assert np.all(np.abs(got - ref) <= tol), f"{name}: beyond one bf16 ulp"


def bf(rng, shape, dev):
    t = torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dev, torch.bfloat16)
    return t, t.float().cpu().numpy()


@pytest.mark.parametrize("topk", [64, 6])
def test_csa_cache_prefill_then_decode(dev, topk):
    import kch
    rng = np.random.default_rng(topk)
    B, c, cI, m, win, nh, nIh = 2, 128, 64, 4, 16, 16, 4
    Ba = (0.02 * rng.standard_normal((m, c))).astype(np.float32)
    Bb = (0.02 * rng.standard_normal((m, c))).astype(np.float32)
    Bi = (0.02 * rng.standard_normal((m, cI))).astype(np.float32)
    sink = rng.standard_normal(nh).astype(np.float32)
    tb = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    hip = kch.CSADecodingCache(B, c, cI, m, win, dev, torch.bfloat16)
    ora = CSACacheOracle(B, c, cI, m, win, 'bf16')

    def feed(T):
        d = [bf(rng, (B, T, w), dev) for w in (c, c, c, c, cI, cI)]
        new_h = hip.append_step(*[x[0] for x in d], tb(Ba), tb(Bb), tb(Bi))
        new_o = ora.append_step(*[x[1] for x in d], Ba, Bb, Bi)
        assert new_h == new_o
        assert hip.n_blocks == ora.n_blocks and hip.accumulator_len == len(ora.acc)
        assert hip.n_tokens_seen == ora.n_tokens_seen

    feed(37)
    for step in range(20):
        feed(1)
        q = l2_normalize(rng.standard_normal((B, 1, nh, c))).astype(np.float32)
        qi, qi_h = bf(rng, (B, 1, nIh, cI), dev)
        wi, wi_h = bf(rng, (B, 1, nIh), dev)
        out = hip.forward_step(tb(q), qi, wi, topk=topk, nh=nh, nIh=nIh,
                               sink_logits=tb(sink), normalize_qk=True)
        torch.cuda.synchronize()
        assert out.dtype == torch.float32 and out.shape == (B, 1, nh, c)
        idx = None
        nb = hip.n_blocks
        if topk < nb:
            idx = hip._last_indices.cpu().numpy()[:, None, :].astype(np.int64)
            cbm = (np.arange(nb) < (ora.n_tokens_seen) // m)[None, :]
            # the exact logits of the key rows this cache holds (their parity with
            # the oracle's rows is checked below, within one rounding of bf16)
            k_rows = hip.K_IComp.float().cpu().numpy()
            ref_idx, lg = lightning_indexer(qi_h, k_rows, wi_h, topk, None, cbm, True,
                                            compute=np.float64, return_logits=True)
            # only a near-tie of the k-th logit, within the kernels' error bound, may differ
            check_selection(f"csa step {step}", idx, ref_idx, lg, logit_eps(wi_h, nIh))
        ref = ora.forward_step(q, qi_h, wi_h, topk=topk, sink_logits=sink, normalize_qk=True,
                               indices=idx)
        close(f"csa step {step}", out.cpu().numpy(), ref)
    ulp_close("C_comp", hip.C_comp.float().cpu().numpy(), ora.C_comp)
    ulp_close("K_IComp", hip.K_IComp.float().cpu().numpy(), ora.K_IComp)
    ring = hip.sw_buffer.get().float().cpu().numpy()
    ulp_close("ring", ring, np.stack(ora.ring, axis=1))
    hip.reset()
    assert hip.n_blocks == 0 and hip.n_tokens_seen == 0 and hip.sw_buffer.n_valid == 0


def test_hca_cache_prefill_then_decode(dev):
    import kch
    rng = np.random.default_rng(11)
    B, c, m2, win, nh = 2, 128, 16, 32, 16
    bpos = (0.02 * rng.standard_normal((m2, c))).astype(np.float32)
    sink = rng.standard_normal(nh).astype(np.float32)
    tb = lambda x: torch.from_numpy(x).to(dev)  # noqa: E731
    hip = kch.HCADecodingCache(B, c, m2, win, dev, torch.bfloat16)
    ora = HCACacheOracle(B, c, m2, win, 'bf16')

    def feed(T):
        (C, Ch), (Z, Zh) = bf(rng, (B, T, c), dev), bf(rng, (B, T, c), dev)
        assert hip.append_step(C, Z, tb(bpos)) == ora.append_step(Ch, Zh, bpos)
        assert hip.n_blocks == ora.n_blocks and hip.accumulator_len == len(ora.acc)

    feed(70)
    for step in range(40):
        feed(1)
        q = l2_normalize(rng.standard_normal((B, 1, nh, c))).astype(np.float32)
        out = hip.forward_step(tb(q), nh=nh, sink_logits=tb(sink))
        torch.cuda.synchronize()
        ref = ora.forward_step(q, sink_logits=sink)
        close(f"hca step {step}", out.cpu().numpy(), ref)
    ulp_close("C_comp", hip.C_comp.float().cpu().numpy(), ora.C_comp)


def test_cache_validation_and_empty(dev):
    import kch
    with pytest.raises(ValueError):
        kch.CSADecodingCache(0, 128, 64, 4, 8, dev, torch.bfloat16)
    with pytest.raises(TypeError):
        kch.HCADecodingCache(1, 128, 8, 8, dev, torch.int32)
    h = kch.HCADecodingCache(1, 128, 8, 8, dev, torch.bfloat16)
    q = torch.zeros(1, 1, 4, 128, device=dev)
    assert torch.equal(h.forward_step(q, nh=4), torch.zeros(1, 1, 4, 128, device=dev))
    with pytest.raises(ValueError, match="T_new"):
        h.forward_step(torch.zeros(1, 2, 4, 128, device=dev), nh=4)
