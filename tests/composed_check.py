"""Checks of composed HIP models against the oracle (test helper, GPU tests).

* ``close``: every element within atol 2e-3 + rtol 2e-2 (the bf16 bar of
  ``north_star``), no element allowance.
* Teacher-forced per-layer checks: forward hooks on the model's LayerNorms
  record the residual stream entering each sub-layer; the oracle's sub-layer
  i is fed that same stream (``layer_inputs``), keeping its own KDA states and
  decode caches from those inputs, and its output is compared with the
  stream the HIP sub-layer i passed on. Each layer is then held to the bar on
  its own; one-ulp bf16 roundings of early layers cannot compound.
* ``end_to_end``: the free-running stack, strict in fp32 and a relative
  Frobenius bound of 1e-2 in bf16 (where the oracle and the reference
  themselves differ by ~1e-3, ``tests/golden``).
* CSA layers run on the selection the kernels made (``kch.record_selections``);
  the selections themselves are checked in ``test_csa_hca_gpu.py`` and
  ``test_regimes_gpu.py``.
"""

from __future__ import annotations

import numpy as np
import torch

RTOL, ATOL = 2e-2, 2e-3


def close(name, got, ref, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite output"
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    w = np.unravel_index(np.argmax(err - rtol * np.abs(ref)), err.shape)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert not bad.any(), (f"{name}: {bad.sum()} of {bad.size} beyond tolerance, "
                           f"max abs err {err.max():.3e}, worst {w}: got {got[w]:.6g} "
                           f"ref {ref[w]:.6g}, |ref|max {np.abs(ref).max():.3g}, "
                           f"rel fro {rel:.2e}")


def host_sel(t):
    return t.cpu().numpy().astype(np.int64)


class LayerInputs:
    """Forward hooks on a model's LayerNorms: after each call, ``get()`` is the
    residual stream that entered each sub-layer (the norm's input)."""

    def __init__(self, model):
        self.store = {}
        self.hooks = [n.register_forward_hook(
            lambda mod, inp, out, i=i: self.store.__setitem__(i, inp[0].float().cpu().numpy()))
            for i, n in enumerate(model.norms)]

    def get(self):
        return [self.store[i] for i in range(len(self.store))]

    def remove(self):
        for h in self.hooks:
            h.remove()


def check_layers(name, layer_in, y, outs):
    """Teacher-forced check: the oracle's sub-layer i, fed the stream that entered
    the HIP sub-layer i, against the stream the HIP sub-layer i passed on."""
    hip_out = layer_in[1:] + [y.float().cpu().numpy()]
    for i, (got, ref) in enumerate(zip(hip_out, outs)):
        close(f"{name} layer {i}", got, ref)


def end_to_end(name, got, ref, dtype):
    """The whole stack, free-running: strict in fp32; in bf16 the one-ulp
    roundings of early layers pass through later ones (as they do between the
    reference and the oracle, tests/golden), so a relative Frobenius bound."""
    if dtype != torch.bfloat16:
        close(name, got, ref)
        return
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    rel = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert rel <= 1e-2, f"{name}: relative Frobenius error {rel:.2e}"


def decode_vs_oracle(dec, oracle, x, T0, dtype_name):
    """Prefill ``x[:, :T0]`` then one token at a time; at every call each HIP
    sub-layer is checked against the teacher-forced oracle (fed the same
    residual stream, keeping its own KDA states and caches from those inputs,
    with the CSA layer on the HIP selection), every element at the bar. The
    stream entering each sub-layer comes from the decoder's own trace
    (``dec._trace``), so each step runs on the path it takes without the
    check: the device-driven step kernels wherever they apply. Returns the
    number of decode steps that ran on them."""
    import kch
    xn = x.float().cpu().numpy()
    pos = dec.model.layout.index("csa")
    dec._trace = []
    steps0 = dec._device_steps
    try:
        for a, b in [(0, T0)] + [(t, t + 1) for t in range(T0, x.shape[1])]:
            with kch.record_selections() as sel:
                y = dec(x[:, a:b])
            assert len(sel) == 1
            assert len(dec._trace) == 1
            layer_in = [t.float().cpu().numpy() for t in dec._trace.pop()]
            outs = oracle.step(xn[:, a:b], csa_indices={pos: host_sel(sel[0])},
                               layer_inputs=layer_in)
            check_layers(f"{dtype_name} [{a}:{b}]", layer_in, y, outs)
    finally:
        dec._trace = None
    return dec._device_steps - steps0
