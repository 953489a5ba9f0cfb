"""The reference's STE gradients (``tests/golden/csa_ste_fp32.npz``, written by
``make_golden.py`` from ``naive_csa``, ``ops_csa.py:576-1184`` with
``ops_csa.py:1033-1099``) and the chain rule through ``naive_csa``'s
projections (test helper).

``projections`` forms ``Ca .. w_idx`` from H and the weights in fp64;
``weight_grads`` turns the gradients of those projections (an
``oracle.csa.csa_ste_grad`` result) into the gradients of H and of every
weight, the loss being ``sum(out * G)``."""

from __future__ import annotations

import os

import numpy as np

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "csa_ste_fp32.npz")
NAMES = ("W_aKV", "W_bKV", "W_aZ", "W_bZ", "Ba", "Bb", "W_DQ", "W_UQ", "W_IUQ", "W_w",
         "W_KV_idx", "W_Z_idx", "B_idx")
CASES = [(norm, mode) for norm in (True, False) for mode in ("topk_columns", "full_softmax")]


def load():
    z = np.load(PATH)
    B, T, d, c, nh, dc, nIh, cI, m, win, topk = (int(x) for x in z["meta"])
    meta = dict(B=B, T=T, d=d, c=c, nh=nh, dc=dc, nIh=nIh, cI=cI, m=m, win=win, topk=topk)
    W = {n: z[f"w.{n}"] for n in NAMES}
    return z, meta, W


def tag(norm, mode):
    return f"{'norm' if norm else 'raw'}.{mode}"


def projections(H, W, meta):
    f = np.float64
    H = np.asarray(H, f)
    Wf = {k: np.asarray(v, f) for k, v in W.items()}
    B, T, nh, c, nIh, cI = (meta[k] for k in ("B", "T", "nh", "c", "nIh", "cI"))
    P = {n: H @ Wf[w].T for n, w in (("Ca", "W_aKV"), ("Cb", "W_bKV"), ("Za", "W_aZ"),
                                     ("Zb", "W_bZ"), ("K_idx", "W_KV_idx"), ("Z_idx", "W_Z_idx"),
                                     ("w_idx", "W_w"))}
    cQ = H @ Wf["W_DQ"].T
    P["q"] = (cQ @ Wf["W_UQ"].T).reshape(B, T, nh, c)
    P["q_idx"] = (cQ @ Wf["W_IUQ"].T).reshape(B, T, nIh, cI)
    return P, cQ


def weight_grads(g, H, W, cQ, meta):
    """dL/dH and dL/dW for every weight from the projections' gradients ``g``."""
    f = np.float64
    H = np.asarray(H, f)
    Wf = {k: np.asarray(v, f) for k, v in W.items()}
    B, T = meta["B"], meta["T"]
    dq = g["q"].reshape(B, T, -1)
    dqi = g["q_idx"].reshape(B, T, -1)
    dcQ = dq @ Wf["W_UQ"] + dqi @ Wf["W_IUQ"]
    lin = {"W_aKV": g["Ca"], "W_bKV": g["Cb"], "W_aZ": g["Za"], "W_bZ": g["Zb"],
           "W_KV_idx": g["K_idx"], "W_Z_idx": g["Z_idx"], "W_w": g["w_idx"]}
    out = {f"d{n}": np.einsum("bto,btd->od", dp, H) for n, dp in lin.items()}
    out["dW_UQ"] = np.einsum("bto,btd->od", dq, cQ)
    out["dW_IUQ"] = np.einsum("bto,btd->od", dqi, cQ)
    out["dW_DQ"] = np.einsum("bto,btd->od", dcQ, H)
    out.update(dBa=g["Ba"], dBb=g["Bb"], dB_idx=g["B_idx"])
    out["dH"] = sum(dp @ Wf[n] for n, dp in lin.items()) + dcQ @ Wf["W_DQ"]
    if "sink_logits" in g:
        out["dsink"] = g["sink_logits"]
    return out


def worst_rel(got, z, t):
    """Largest error of each gradient relative to the fixture's largest entry."""
    res = {}
    for k, v in got.items():
        r = np.asarray(z[f"{t}.{k}"], np.float64)
        res[k] = float(np.abs(np.asarray(v, np.float64) - r).max() / max(np.abs(r).max(), 1e-30))
    return res
