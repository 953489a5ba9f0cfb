"""CPU oracle for the hybrid-attention forward path (TEST INFRASTRUCTURE ONLY).

This package is a from-scratch numpy restatement of the reference algorithms
(``/root/reference/ops_kda.py``, ``ops_csa.py``, ``ops_hca.py``,
``ops_decoding_cache.py``). It exists to *check* the HIP product path and to
time a CPU baseline. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package
(``kda-csa-hca-fusion_amd/kch``) never does, and it has no CPU fallback.

Every public function cites the reference lines it restates. How each one is
pinned (independent formulas, invariants, brute force) is listed in
``tests/test_oracle_*.py``; a function without such a check would be marked
"parity unpinned" in its docstring (none currently are, except the tie order
of ``torch.topk`` on exactly-equal logits, which the oracle replaces by the
documented rule "descending value, then ascending block index").
"""
