"""The oracle's STE gradients against the reference's (CPU).

``oracle.csa.csa_ste_grad`` (the straight-through surrogate of
``ops_csa.py:1033-1099`` on top of ``csa_attn_grad``) is held to the
gradients the reference's own ``naive_csa`` produced in fp32 under autograd
(``tests/golden/csa_ste_fp32.npz``), for ``ste_mode`` ``topk_columns`` and
``full_softmax`` with and without ``normalize_qk``, on the reference's own
selection: every gradient (H, every weight, the sink) within 1e-5 of its
largest entry (fp32 against fp64). A planted mistake fails the same check:
the other ``ste_mode``'s gradients, and ``full_softmax`` without its term on
the compressed rows.
"""

from __future__ import annotations

import numpy as np
import pytest

import ste_fixture as SF
from oracle import csa as OC


def _oracle(z, meta, W, norm, mode, drop_rows_term=False):
    P, cQ = SF.projections(z["H"], W, meta)
    idx = z[f"{SF.tag(norm, mode)}.idx"]
    G = np.asarray(z["G"], np.float64).reshape(meta["B"], meta["T"], meta["nh"], meta["c"])
    args = [P[k] for k in ("Ca", "Cb", "Za", "Zb", "K_idx", "Z_idx", "q", "q_idx", "w_idx")]
    g = OC.csa_ste_grad(*args, W["Ba"], W["Bb"], W["B_idx"], idx, G, m=meta["m"],
                        sliding_window=meta["win"], sink_logits=z["sink"], normalize_qk=norm,
                        ste_mode=mode)
    if drop_rows_term:
        # the planted mistake: full_softmax's indexer term kept, its term on the
        # compressed rows dropped
        gt = OC.csa_attn_grad(*args[:4], P["q"], W["Ba"], W["Bb"], idx, G, m=meta["m"],
                              sliding_window=meta["win"], sink_logits=z["sink"],
                              normalize_qk=norm)
        for k in ("Ca", "Cb", "Za", "Zb", "Ba", "Bb"):
            g[k] = gt[k]
    return SF.weight_grads(g, z["H"], W, cQ, meta)


@pytest.mark.parametrize("norm,mode", SF.CASES)
def test_oracle_ste_grads_match_reference(norm, mode):
    z, meta, W = SF.load()
    err = SF.worst_rel(_oracle(z, meta, W, norm, mode), z, SF.tag(norm, mode))
    assert len(err) == len(SF.NAMES) + 2   # every weight, H and the sink
    bad = {k: v for k, v in err.items() if v > 1e-5}
    assert not bad, bad


@pytest.mark.parametrize("norm", [True, False])
def test_planted_ste_mistakes_fail(norm):
    z, meta, W = SF.load()
    t = SF.tag(norm, "full_softmax")
    # the other mode's gradients differ from full_softmax's fixture
    other = SF.worst_rel(_oracle(z, meta, W, norm, "topk_columns"), z, t)
    assert max(other[k] for k in ("dW_KV_idx", "dW_aKV")) > 1e-3, other
    # dropping the dense term on the compressed rows is caught
    dropped = SF.worst_rel(_oracle(z, meta, W, norm, "full_softmax", drop_rows_term=True), z, t)
    assert dropped["dW_aKV"] > 1e-3, dropped
    # the two modes' forward values are the same (the surrogate adds zero)
    np.testing.assert_array_equal(z[f"{SF.tag(norm, 'topk_columns')}.out"], z[f"{t}.out"])
