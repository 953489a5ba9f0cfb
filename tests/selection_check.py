"""Index parity of the HIP top-k selections against the oracle's (test helper).

The kernels form indexer logits from split MFMA products of fp32 rows, every
product exact in fp32 and accumulated in fp32: L2-normalised rows as the two
fp16 parts of ``256 x`` (``hi*hi + hi*lo + lo*hi``: 22 significant bits per
element, the dropped ``lo*lo`` at ``2^-22`` relative), other rows as three
bf16 parts (``x = hi + mid + lo``, the six cross products down to ``2^-16``,
terms of ``2^-24`` dropped). The logits thus carry the error of an fp32
computation (a few units of ``2^-24`` per element), as the reference's fp32
einsum (``ops_csa.py:529-534``) does, against ``2^-16`` for a two-part bf16
split. Against the exact (fp64) logit of the same bf16 projections, the rest
of the error is the fp32 rounding of the compressed key, of the two L2
normalisations and of the 64- or 128-term dot product. The bound used,
``eps = 1e-6 * sum_h |w_h| + 1e-7`` (4 units of ``2^-22`` per unit of head
weight, the worst case of the fp16 split being 3), is asserted on the
kernels' own logits wherever a test can read them (``check_logits``), so the
selection rule below rests on a checked bound, not an assumed one.

A HIP selection may differ from the oracle's (fp64 logits, ties by ascending
block index) only where the k-th and (k+1)-th exact logits lie within
``2 eps``, and then only by blocks whose logits lie within ``2 eps`` of the
k-th. Exactly equal logits (duplicated rows, ReLU zeros) tie in both and
follow the same lowest-index rule, so they never differ.
"""

from __future__ import annotations

import numpy as np


EPS_PER_WEIGHT = 1e-6


def logit_eps(w_idx, nIh):
    """Per-row logit error bound; ``w_idx`` ``[..., nIh]`` or None (all ones)."""
    if w_idx is None:
        return np.float64(EPS_PER_WEIGHT * nIh + 1e-7)
    return EPS_PER_WEIGHT * np.abs(np.asarray(w_idx, np.float64)).sum(-1) + 1e-7


def check_logits(name, got, exact, eps):
    """Every finite kernel logit within ``eps`` (row-wise) of the exact one, and
    the same masked (-inf) positions. Returns the largest error in units of
    ``eps``."""
    got = np.asarray(got, np.float64)
    exact = np.asarray(exact, np.float64)
    assert got.shape == exact.shape, (name, got.shape, exact.shape)
    fin = np.isfinite(exact)
    assert np.array_equal(fin, np.isfinite(got)), f"{name}: masked positions differ"
    eps = np.broadcast_to(np.asarray(eps, np.float64)[..., None], got.shape)
    err = np.where(fin, np.abs(got - np.where(fin, exact, 0.0)), 0.0)
    worst = float((err / eps).max()) if err.size else 0.0
    assert worst <= 1.0, f"{name}: a logit is off by {worst:.2f} eps"
    return worst


def check_selection(name, got, ref, logits, eps, sorted_=False):
    """Compare ``got`` with ``ref`` (``[..., topk]``, -1 = empty) under the rule
    above; ``logits`` ``[..., n_blocks]`` (exact, -inf = masked), ``eps``
    broadcastable to the row shape. With ``sorted_`` the HIP rows must also
    be in descending logit order (within ``2 eps``).

    Returns ``(rows, rows_that_differ, rows_with_a_near_tie_at_the_boundary)``."""
    got = np.asarray(got, np.int64)
    ref = np.asarray(ref, np.int64)
    lg = np.asarray(logits, np.float64)
    topk = got.shape[-1]
    rows_shape = got.shape[:-1]
    eps = np.broadcast_to(np.asarray(eps, np.float64), rows_shape)
    got2 = got.reshape(-1, topk)
    ref2 = ref.reshape(-1, topk)
    lg2 = lg.reshape(got2.shape[0], -1)
    eps2 = eps.reshape(-1)
    differ = near = 0
    for r in range(got2.shape[0]):
        a, b, e = got2[r], ref2[r], 2 * eps2[r]
        ka, kb = np.count_nonzero(a >= 0), np.count_nonzero(b >= 0)
        assert ka == kb, f"{name}: row {r} has {ka} selected blocks, the oracle {kb}"
        assert np.all(a[:ka] >= 0) and np.all(a[ka:] == -1), f"{name}: row {r} -1 slots"
        assert len(set(a[:ka].tolist())) == ka, f"{name}: row {r} repeats a block"
        vis = np.sort(lg2[r][np.isfinite(lg2[r])])[::-1]
        tie = False
        if 0 < kb < vis.size:
            kth = vis[kb - 1]
            tie = (kth - vis[kb]) <= e
        near += int(tie)
        if sorted_ and ka > 1:
            va = lg2[r, a[:ka]]
            assert np.all(va[:-1] >= va[1:] - e), f"{name}: row {r} not in descending order"
        sa, sb = set(a[:ka].tolist()), set(b[:kb].tolist())
        if sa == sb:
            continue
        differ += 1
        assert tie, f"{name}: row {r} differs without a near-tie at the boundary"
        diff = np.array(sorted(sa ^ sb))
        assert np.all(np.abs(lg2[r, diff] - kth) <= e), \
            f"{name}: row {r} differs by a block beyond the error bound"
    return got2.shape[0], differ, near
