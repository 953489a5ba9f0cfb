"""Benchmark of the MI355X hybrid-attention forward path (one JSON line on stdout).

Headline workload: KDA chunked prefill, bf16 inputs
with fp32 state, B=8 T=4096 H=16 K=V=128, q/k L2-normalised N(0,1), v N(0,1),
g = logsigmoid(N(0,1)) per channel, beta = sigmoid(N(0,1)), S0 ~ 0.02 N(0,1).
A step is one ``kch.naive_chunk_kda`` call over that batch (inputs resident in
HBM). ``value`` is B*T tokens per second of step time, measured with HIP events
on the stream the kernel runs on (the torch current stream).

``roofline``: algorithmic HBM bytes of the step (q,k,v,g,o bf16 + beta bf16 +
S0 read and S write fp32) over the measured step time, against 8 TB/s. The step
is two kernels (a parallel per-chunk kernel and the state-carrying kernel);
``traffic`` is their measured HBM bytes per step (rocprofv3 FETCH_SIZE +
WRITE_SIZE, scaled by the same counters on a copy of known size), including the
per-chunk workspace that passes between them.
``cpu_baseline``: the oracle (from-scratch CPU restatements of the reference
algorithm) on bounded samples of configs[1]-[3]: configs[1] on the torch-CPU
restatement (``oracle.kda_torch``, one of the 8 sequences with all 16 heads)
under ``torch.set_num_threads(N)``, N the process's cores, and under one
thread, as the reference's own torch CPU path runs; configs[2] / [3] on the
numpy restatement (one sequence, query subsets); one warm-up and the median
of three runs, and the CPU model. The configs[2] sample also checks the GPU
indexer's selection at its queries against the oracle's fp64 logits
(``selection_vs_oracle``: rows that differ, rows with a near-tie).

``extra`` (skipped with ``--headline-only``): the other prefill workloads of
the metric, each at its configuration, with the same timing protocol:
  * ``kda_T8K``: KDA chunk at B=4 T=8192 (same generators);
  * ``csa_C2``: ``naive_csa`` at configs[2] (B4 T8192 d2048, 16 heads of 128,
    m=4 overlapped, indexer 4x64 top-512, window 128 + sink) and its core
    (compression + indexer + sparse attention, projections excluded);
  * ``hca_C3`` / ``hca_T8K``: ``naive_hca`` at configs[3] (B4 T32768 d2048,
    16 heads of 128, m'=128, window 128 + sink) and at T=8192, plus its core;
  * ``decode_bw``: one CSA and one HCA decode step on long caches (B=64 /
    B=128 at a 1M-token context), HBM bandwidth against 8 TB/s;
  * ``hybrid_C4``: ``HybridDecoding`` (5 layers, 3:1:1, d2048, the configs
    1-3 head shapes) prefill of B=2 T=16384, then 256 single-token steps.
Weights are N(0, 1/fan_in) random (no checkpoints), inputs N(0,1).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--headline-only]
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "kda-csa-hca-fusion_amd"), REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

METRIC = "prefill tokens/s (KDA chunk, CSA, HCA) at T=8K; % of MFMA/HBM roofline"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3

# Measured HBM bytes per headline step (both kernels): rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE (KiB per dispatch) on `bench.py --headline-only`, each scaled by the
# counter's reading on a device copy of known size (profiles/kda_split_C1.md).
HEADLINE_TRAFFIC_BYTES = int(((263994 + 301219) * 2.0 + (594634 + 139264) * 1.0) * 1024)


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def kda_inputs(B, T, H, K, V, seed=1, dev="cuda"):
    g = torch.Generator().manual_seed(seed)
    q = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    k = torch.nn.functional.normalize(torch.randn(B, T, H, K, generator=g), dim=-1)
    v = torch.randn(B, T, H, V, generator=g)
    gt = torch.nn.functional.logsigmoid(torch.randn(B, T, H, K, generator=g))
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    s0 = 0.02 * torch.randn(B, H, K, V, generator=g)
    xs = [x.to(torch.bfloat16) for x in (q, k, v, gt, beta)]
    return [x.to(dev) for x in xs], s0.to(dev), [x.float().numpy() for x in xs], s0.numpy()


def kda_algorithmic(B, T, H, K, V, C=64):
    tok_heads = B * T * H
    flops = tok_heads * (2 * (3 * K * V + C * (3 * K + 2 * V)) + C * C / 3.0)
    bytes_ = tok_heads * (2 * (3 * K + 2 * V) + 2) + 2 * B * H * K * V * 4
    return flops, bytes_


SETTLE_S = 0.3   # minimum wall time of untimed work before timing (GPU clock ramp)
SETTLE_STEPS = {}


def time_steps(fn, steps, warmup, per_step=False):
    """Mean ms per step over ``steps`` back-to-back steps, bracketed by one pair of
    HIP events on the current stream with a synchronize on both sides (no event
    packets between the steps). With ``per_step`` a second, separate pass records
    an event pair around every step for the median.

    After the ``warmup`` steps, further untimed steps run until ``SETTLE_S``
    seconds of warm-up have passed: a few steps of well under a millisecond
    finish before the GPU clocks have ramped, and the first timed steps would
    then measure the ramp. Their count is kept in ``SETTLE_STEPS``."""
    t0 = time.perf_counter()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    extra = 0
    while time.perf_counter() - t0 < SETTLE_S:
        for _ in range(8):
            fn()
        extra += 8
        torch.cuda.synchronize()
    SETTLE_STEPS[getattr(fn, "__name__", "step")] = extra
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    mean = e0.elapsed_time(e1) / steps
    med = mean
    if per_step:
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
        for a, b in ev:
            a.record(stream)
            fn()
            b.record(stream)
        torch.cuda.synchronize()
        med = float(np.median([a.elapsed_time(b) for a, b in ev]))
    return float(mean), med, wall


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _cpu_timed(fn, threads):
    """One warm-up, then the median of three runs (the CPU protocol of the
    reference's ``run_benchmark._measure``, run_benchmark.py:169-198), with the
    BLAS thread pool limited to ``threads``."""
    from threadpoolctl import threadpool_limits
    with threadpool_limits(threads):
        fn()
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def _cpu_timed_torch(fn, threads):
    """The same protocol on torch's intra-op thread pool (``torch.set_num_threads``)."""
    old = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        fn()
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(old)
    return float(np.median(ts))


def _selection_vs_oracle(proj, par, Q, m, topk, win, sink):
    """The GPU indexer's selection (``kch.csa_core``) at the queries ``Q``
    against the oracle's (fp64 logits, ties by ascending index): rows whose
    sets differ, and rows whose k-th and (k+1)-th exact logits lie within
    2 eps (eps = 1e-6 sum_h |w_h| + 1e-7, the kernels' fp32-level bound)."""
    import kch
    from oracle.csa import compress_kv, indexer_logits, topk_desc_lowest_index, causal_block_mask
    dev = torch.device("cuda:0")
    Ca, Cb, Za, Zb, Ki, Zi, qq, qi, wi = proj
    Ba, Bb, Bi = par
    td = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
    with torch.no_grad():
        _, idx = kch.csa_core(*(td(x) for x in proj), *(td(x) for x in par), m=m, topk=topk,
                              sliding_window=win, sink_logits=td(sink), normalize_qk=True,
                              return_indices=True)
    got = idx.cpu().numpy()[0, Q].astype(np.int64)
    T = Ca.shape[1]
    kc = compress_kv(Ki.astype(np.float64), Zi.astype(np.float64), Bi, m, np.float64)
    lg = indexer_logits(qi[:, Q], kc, wi[:, Q], None, causal_block_mask(T, T // m, m)[Q], True,
                        np.float64)[0]
    ref = topk_desc_lowest_index(lg[None], topk)[0]
    eps = 1e-6 * np.abs(wi[0, Q].astype(np.float64)).sum(-1) + 1e-7
    differ = near = 0
    for r in range(len(Q)):
        vis = np.sort(lg[r][np.isfinite(lg[r])])[::-1]
        kb = int((ref[r] >= 0).sum())
        if 0 < kb < vis.size and vis[kb - 1] - vis[kb] <= 2 * eps[r]:
            near += 1
        if set(got[r][got[r] >= 0].tolist()) != set(ref[r][ref[r] >= 0].tolist()):
            differ += 1
    return {"rows": int(len(Q)), "differ": differ, "near_ties": near,
            "rule": "sets compared; a differing row is allowed only at a near-tie (tests)"}


def cpu_baselines(host, s0):
    """The oracle (from-scratch CPU restatements of the reference algorithm) on
    bounded samples of configs[1], [2] and [3], with all the process's cores
    and with one thread; tokens/s of the whole workload."""
    from oracle.csa import compress_kv, compress_kv_overlapped, csa_core_at, hca_core_at
    from oracle.kda_torch import chunk_kda as chunk_kda_torch
    n_aff = len(os.sched_getaffinity(0))
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    N = min(n_aff, omp) if omp > 0 else n_aff
    rng = np.random.default_rng(0)
    res = {}

    # one of the 8 sequences with all 16 heads, T=4096 (all 64
    # chunks), on the torch-CPU restatement
    q, k, v, g, beta = (torch.from_numpy(np.ascontiguousarray(x[:1])) for x in host[:5])
    S0 = torch.from_numpy(np.ascontiguousarray(s0[:1]))
    T = q.shape[1]
    fn = lambda: chunk_kda_torch(q, k, v, g, beta, initial_state=S0, chunk_size=64)  # noqa: E731
    t = {th: _cpu_timed_torch(fn, th) for th in (N, 1)}
    res["C1_kda_chunk"] = {th: T / t[th] for th in t}
    samples = ["C1: chunk_kda (torch-CPU restatement, torch.set_num_threads) on 1 of 8 "
               "sequences with all 16 heads, T=4096"]

    # the CSA core of one sequence (T=8192): its two compressions,
    # then the sparse + window attention at 256 evenly spaced queries
    T, c, cI, nh, nIh, m, topk, win = 8192, 128, 64, 16, 4, 4, 512, 128
    r = lambda *sh: rng.standard_normal(sh).astype(np.float32)  # noqa: E731
    Ca, Cb, Za, Zb, Ki, Zi = r(1, T, c), r(1, T, c), r(1, T, c), r(1, T, c), r(1, T, cI), r(1, T, cI)
    Ba, Bb, Bi = 0.02 * r(m, c), 0.02 * r(m, c), 0.02 * r(m, cI)
    Q = np.linspace(0, T - 1, 256).astype(np.int64)
    qq, qi, wi = np.zeros((1, T, nh, c), np.float32), np.zeros((1, T, nIh, cI), np.float32), \
        np.zeros((1, T, nIh), np.float32)
    qq[:, Q], qi[:, Q], wi[:, Q] = r(1, len(Q), nh, c), r(1, len(Q), nIh, cI), r(1, len(Q), nIh)
    sink = r(nh)
    comp = {}

    def csa_compress():
        comp["C"] = compress_kv_overlapped(Ca, Cb, Za, Zb, Ba, Bb, m)
        comp["K"] = compress_kv(Ki, Zi, Bi, m)

    def csa_queries():
        csa_core_at(Ca, Cb, Za, Zb, Ki, Zi, qq, qi, wi, Ba, Bb, Bi, m=m, topk=topk, queries=Q,
                    sliding_window=win, sink_logits=sink, C_comp=comp["C"], K_IComp=comp["K"])
    res["C2_csa_core"] = {}
    for th in (N, 1):
        tc, tq = _cpu_timed(csa_compress, th), _cpu_timed(csa_queries, th)
        res["C2_csa_core"][th] = 1.0 / (tc / T + tq / len(Q))
    samples.append("C2: csa core of 1 of 4 sequences (T=8192), compression of the whole "
                   "sequence + attention at 256 evenly spaced queries (numpy)")
    sel = _selection_vs_oracle((Ca, Cb, Za, Zb, Ki, Zi, qq, qi, wi), (Ba, Bb, Bi), Q, m, topk,
                               win, sink)

    # the HCA core of one sequence (T=32768), attention at 512 queries
    T, m2 = 32768, 128
    C, Z = r(1, T, c), r(1, T, c)
    Bp = 0.02 * r(m2, c)
    Q = np.linspace(0, T - 1, 512).astype(np.int64)
    qq = np.zeros((1, T, nh, c), np.float32)
    qq[:, Q] = r(1, len(Q), nh, c)

    def hca_compress():
        comp["H"] = compress_kv(C, Z, Bp, m2)

    def hca_queries():
        hca_core_at(C, Z, qq, Bp, m2=m2, queries=Q, sliding_window=win, sink_logits=sink,
                    C_comp=comp["H"])
    res["C3_hca_core"] = {}
    for th in (N, 1):
        tc, tq = _cpu_timed(hca_compress, th), _cpu_timed(hca_queries, th)
        res["C3_hca_core"][th] = 1.0 / (tc / T + tq / len(Q))
    samples.append("C3: hca core of 1 of 4 sequences (T=32768), compression of the whole "
                   "sequence + attention at 512 evenly spaced queries (numpy)")
    cfgs = {name: {"tokens_per_s": v[N], "tokens_per_s_1thread": v[1]} for name, v in res.items()}
    return {"value": res["C1_kda_chunk"][N], "unit": "tokens/s", "cores": N, "kind": "port",
            "sample": "; ".join(samples) + f"; 1 warm-up then the median of 3 runs; "
                      f"{N} threads ({n_aff} cores in the process's affinity) and 1 thread; "
                      f"host {_cpu_model()}",
            "value_1thread": res["C1_kda_chunk"][1], "cpu_model": _cpu_model(),
            "affinity_cores": n_aff, "configs": cfgs, "C2_selection_vs_oracle": sel}


# ----------------------------------------------------------------------------- extras

def _w(gen, o, i, dev):
    return (torch.randn(o, i, generator=gen) * i ** -0.5).to(dev, torch.bfloat16)


def csa_weights(d, c, nh, dc, nIh, cI, m, dev, seed=2):
    g = torch.Generator().manual_seed(seed)
    W = {n: _w(g, c, d, dev) for n in ('W_aKV', 'W_bKV', 'W_aZ', 'W_bZ')}
    W['Ba'] = (0.02 * torch.randn(m, c, generator=g)).to(dev, torch.bfloat16)
    W['Bb'] = (0.02 * torch.randn(m, c, generator=g)).to(dev, torch.bfloat16)
    W['W_DQ'] = _w(g, dc, d, dev)
    W['W_UQ'] = _w(g, c * nh, dc, dev)
    W['W_IUQ'] = _w(g, cI * nIh, dc, dev)
    W['W_w'] = _w(g, nIh, d, dev)
    W['W_KV_idx'] = _w(g, cI, d, dev)
    W['W_Z_idx'] = _w(g, cI, d, dev)
    W['B_idx'] = (0.02 * torch.randn(m, cI, generator=g)).to(dev, torch.bfloat16)
    W['sink'] = torch.randn(nh, generator=g).to(dev)
    return W


def csa_core_algorithmic(B, T, m, topk, win, nh, c, nIh, cI):
    t = np.arange(T, dtype=np.int64)
    vis = (t + 1) // m
    idx_entries = int(vis.sum())
    sel = int(np.minimum(vis, topk).sum())
    wslots = int(np.minimum(win, t + 1).sum())
    flops = B * (idx_entries * 2 * nIh * cI + (sel + wslots) * 4 * nh * c)
    nb = T // m
    # bf16 inputs of the core, bf16 out, int32 indices, fp32 indexer keys
    bytes_ = B * T * 2 * (4 * c + 2 * cI + nh * c + nIh * cI + nIh + nh * c) \
        + B * T * topk * 4 + B * nb * (c * 2 + cI * 4)
    return flops, bytes_


def hca_core_algorithmic(B, T, m2, win, nh, c):
    t = np.arange(T, dtype=np.int64)
    comp = int(((t + 1) // m2).sum())
    wslots = int(np.minimum(win, t + 1).sum())
    flops = B * (comp + wslots) * 4 * nh * c
    bytes_ = B * T * 2 * (2 * c + 2 * nh * c)
    return flops, bytes_


def _roof(flops, bytes_, ms):
    t = ms * 1e-3
    return {"tflops": flops / t / 1e12, "mfma_frac": flops / t / 1e12 / BF16_PEAK_TFLOPS,
            "gbs": bytes_ / t / 1e9, "hbm_frac": bytes_ / t / 1e9 / HBM_PEAK_GBS,
            "algorithmic_flops": flops, "algorithmic_bytes": bytes_}


def bench_kda(B, T, steps, warmup, dev):
    import kch
    H, K, V = 16, 128, 128
    xs, s0, _, _ = kda_inputs(B, T, H, K, V, dev=dev)
    ms, med, _ = time_steps(
        lambda: kch.naive_chunk_kda(*xs, initial_state=s0, output_final_state=True), steps, warmup)
    flops, bytes_ = kda_algorithmic(B, T, H, K, V)
    out = {"B": B, "T": T, "tokens_per_s": B * T / (ms * 1e-3), "ms": ms, "ms_median": med}
    out.update(_roof(flops, bytes_, ms))
    return out


def bench_csa(B, T, steps, warmup, dev):
    import kch
    d, c, nh, dc, nIh, cI, m, topk, win = 2048, 128, 16, 128, 4, 64, 4, 512, 128
    W = csa_weights(d, c, nh, dc, nIh, cI, m, dev)
    Hs = torch.randn(B, T, d, generator=torch.Generator().manual_seed(2)).to(dev, torch.bfloat16)
    args = [W[n] for n in ('W_aKV', 'W_bKV', 'W_aZ', 'W_bZ', 'Ba', 'Bb', 'W_DQ', 'W_UQ',
                           'W_IUQ', 'W_w', 'W_KV_idx', 'W_Z_idx', 'B_idx')]
    kw = dict(m=m, topk=topk, nh=nh, nIh=nIh, c=c, c_I=cI, dc=dc, sliding_window=win,
              sink_logits=W['sink'], normalize_qk=True)
    ms_full, _, _ = time_steps(lambda: kch.naive_csa(Hs, *args, **kw), steps, warmup)
    with torch.no_grad():
        comb = torch.nn.functional.linear(Hs, torch.cat(
            [W['W_aKV'], W['W_bKV'], W['W_aZ'], W['W_bZ'], W['W_KV_idx'], W['W_Z_idx']], 0))
        Ca, Cb, Za, Zb, Ki, Zi = comb.split([c, c, c, c, cI, cI], -1)
        cQ = torch.nn.functional.linear(Hs, W['W_DQ'])
        q_idx = torch.nn.functional.linear(cQ, W['W_IUQ']).view(B, T, nIh, cI)
        w_idx = torch.nn.functional.linear(Hs, W['W_w'])
        q = torch.nn.functional.linear(cQ, W['W_UQ']).view(B, T, nh, c)
    ms_core, _, _ = time_steps(
        lambda: kch.csa_core(Ca, Cb, Za, Zb, Ki, Zi, q, q_idx, w_idx, W['Ba'], W['Bb'],
                             W['B_idx'], m=m, topk=topk, sliding_window=win,
                             sink_logits=W['sink'], normalize_qk=True), steps, warmup)
    flops, bytes_ = csa_core_algorithmic(B, T, m, topk, win, nh, c, nIh, cI)
    core = {"ms": ms_core, "tokens_per_s": B * T / (ms_core * 1e-3)}
    core.update(_roof(flops, bytes_, ms_core))
    return {"B": B, "T": T, "tokens_per_s": B * T / (ms_full * 1e-3), "ms": ms_full,
            "includes": "projections (hipBLASLt; q up-projection kch_linear_up) + core", "core": core}


def bench_hca(B, T, steps, warmup, dev):
    import kch
    d, c, nh, dc, m2, win = 2048, 128, 16, 128, 128, 128
    g = torch.Generator().manual_seed(3)
    W_KV, W_Z, W_DQ = _w(g, c, d, dev), _w(g, c, d, dev), _w(g, dc, d, dev)
    W_UQ = _w(g, c * nh, dc, dev)
    B_pos = (0.02 * torch.randn(m2, c, generator=g)).to(dev, torch.bfloat16)
    sink = torch.randn(nh, generator=g).to(dev)
    Hs = torch.randn(B, T, d, generator=g).to(dev, torch.bfloat16)
    kw = dict(m2=m2, nh=nh, c=c, dc=dc, sliding_window=win, sink_logits=sink)
    ms_full, _, _ = time_steps(lambda: kch.naive_hca(Hs, W_KV, W_Z, B_pos, W_DQ, W_UQ, **kw),
                               steps, warmup)
    with torch.no_grad():
        CZ = torch.nn.functional.linear(Hs, torch.cat([W_KV, W_Z], 0))
        C, Z = CZ.split([c, c], -1)
        q = torch.nn.functional.linear(torch.nn.functional.linear(Hs, W_DQ), W_UQ).view(B, T, nh, c)
    ms_core, _, _ = time_steps(
        lambda: kch.hca_core(C, Z, q, B_pos, m2=m2, sliding_window=win, sink_logits=sink),
        steps, warmup)
    flops, bytes_ = hca_core_algorithmic(B, T, m2, win, nh, c)
    core = {"ms": ms_core, "tokens_per_s": B * T / (ms_core * 1e-3)}
    core.update(_roof(flops, bytes_, ms_core))
    return {"B": B, "T": T, "tokens_per_s": B * T / (ms_full * 1e-3), "ms": ms_full,
            "includes": "projections (hipBLASLt; q up-projection kch_linear_up) + core", "core": core}


def bench_training(dev, reps=3):
    """The training path's backward passes at the configs' shapes (one call
    each after a warm-up, mean of ``reps``): the KDA gradients at configs[1],
    the HCA core's at configs[3], the CSA attention's at configs[2] (on the
    kernel's own top-512 selection), and one forward + backward step of the
    configs[4] stack geometry at B=2, T=2048 (bf16)."""
    import kch
    from kch.ops_csa import csa_attn_grad
    from kch.ops_hca import hca_core_grad

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    g = torch.Generator().manual_seed(5)
    out = {}
    B, T, H, K, V = 8, 4096, 16, 128, 128
    xs, s0, _, _ = kda_inputs(B, T, H, K, V, dev=dev)
    do = torch.randn(B, T, H, V, generator=g).to(dev, torch.bfloat16)
    out["kda_C1_backward_ms"] = timed(
        lambda: kch.kda_recurrent_grad(*xs, do, initial_state=s0, chunked=True))
    out["kda_C1_recurrent_backward_ms"] = timed(
        lambda: kch.kda_recurrent_grad(*xs, do, initial_state=s0))
    del xs, s0, do
    B, T, nh, c, m2, win = 4, 32768, 16, 128, 128, 128
    C, Z = (torch.randn(B, T, c, generator=g).to(dev, torch.bfloat16) for _ in range(2))
    q = torch.randn(B, T, nh, c, generator=g).to(dev, torch.bfloat16)
    dq = torch.randn(B, T, nh, c, generator=g).to(dev, torch.bfloat16)
    Bp = (0.02 * torch.randn(m2, c, generator=g)).to(dev)
    sink = torch.randn(nh, generator=g).to(dev)
    out["hca_C3_core_backward_ms"] = timed(
        lambda: hca_core_grad(C, Z, q, Bp, dq, m2=m2, sliding_window=win, sink_logits=sink))
    del C, Z, q, dq
    B, T, nh, c, m, topk, win, cI, nIh = 4, 8192, 16, 128, 4, 512, 128, 64, 4
    X = [torch.randn(B, T, c, generator=g).to(dev, torch.bfloat16) for _ in range(4)]
    Ki, Zi = (torch.randn(B, T, cI, generator=g).to(dev, torch.bfloat16) for _ in range(2))
    q = torch.randn(B, T, nh, c, generator=g).to(dev, torch.bfloat16)
    qi = torch.randn(B, T, nIh, cI, generator=g).to(dev, torch.bfloat16)
    wi = torch.randn(B, T, nIh, generator=g).to(dev, torch.bfloat16)
    Ba, Bb = ((0.02 * torch.randn(m, c, generator=g)).to(dev) for _ in range(2))
    Bi = (0.02 * torch.randn(m, cI, generator=g)).to(dev)
    with torch.no_grad():
        _, idx = kch.csa_core(*X, Ki, Zi, q, qi, wi, Ba, Bb, Bi, m=m, topk=topk,
                              sliding_window=win, sink_logits=sink, normalize_qk=True,
                              return_indices=True)
    dq = torch.randn(B, T, nh, c, generator=g).to(dev, torch.bfloat16)
    out["csa_C2_attention_backward_ms"] = timed(
        lambda: csa_attn_grad(*X, q, Ba, Bb, idx, dq, m=m, sliding_window=win, sink_logits=sink,
                              normalize_qk=True))
    del X, q, dq, idx
    cfg = kch.HybridConfig(d_model=2048, n_heads_qk=16, n_heads_v=16, head_dim_k=128,
                           head_dim_v=128, kda_chunk_size=64, csa_m=4, csa_topk=512, csa_nh=16,
                           csa_c=128, csa_dc=128, csa_nIh=4, csa_cI=64, csa_sliding_window=128,
                           hca_m2=128, hca_nh=16, hca_c=128, hca_dc=128, hca_sliding_window=128)
    model = kch.HybridKCHAttention(cfg, total_layers=5).to(dev, torch.bfloat16).train()
    x = torch.randn(2, 2048, 2048, generator=g).to(dev, torch.bfloat16)

    def train_step():
        model.zero_grad(set_to_none=True)
        y, _, _ = model.forward_functional(x, None, [None] * model.n_kda_layers)
        y.float().square().mean().backward()

    out["hybrid_C4_B2_T2048_train_step_ms"] = timed(train_step)
    # algorithmic FLOPs of the backwards: the attention ones recompute the
    # scores and dp (2 x 2c per pair and head) and form dq and dk (2c + 4c):
    # 2.5x the forward's 4c; the KDA one runs the recurrence forward twice and
    # backward once, taken as 2x the chunk form's forward FLOPs. Against the
    # fp32 peak: these kernels compute to fp32 accuracy (split-bf16 MFMA
    # products, or fp32 on the vector units).
    fl = {"kda_C1_backward_ms": 2.0 * kda_algorithmic(8, 4096, 16, 128, 128)[0],
          "hca_C3_core_backward_ms": 2.5 * hca_core_algorithmic(4, 32768, 128, 128, 16, 128)[0],
          "csa_C2_attention_backward_ms": 2.5 * csa_core_algorithmic(
              4, 8192, 4, 512, 128, 16, 128, 4, 64)[0]}
    out["fp32_peak_tflops"] = FP32_PEAK_TFLOPS
    for k, f in fl.items():
        tf = f / (out[k] * 1e-3) / 1e12
        out[k.replace("_ms", "_tflops")] = tf
        out[k.replace("_ms", "_fp32_frac")] = tf / FP32_PEAK_TFLOPS
    # CPU beside it: the oracle's hand-written KDA backward (numpy, fp64) on a
    # slice of configs[1], scaled to tokens/s of the whole workload
    from oracle.kda import recurrent_kda_grad
    rng = np.random.default_rng(0)
    Tc, Hc = 2048, 4
    qa = rng.standard_normal((1, Tc, Hc, 128))
    qa /= np.linalg.norm(qa, axis=-1, keepdims=True)
    ka = rng.standard_normal((1, Tc, Hc, 128))
    ka /= np.linalg.norm(ka, axis=-1, keepdims=True)
    va, doa = rng.standard_normal((1, Tc, Hc, 128)), rng.standard_normal((1, Tc, Hc, 128))
    ga = -np.log1p(np.exp(-rng.standard_normal((1, Tc, Hc, 128))))
    ba = 1.0 / (1.0 + np.exp(-rng.standard_normal((1, Tc, Hc))))
    t0 = time.perf_counter()
    recurrent_kda_grad(qa, ka, va, ga, ba, doa)
    dt = time.perf_counter() - t0
    out["cpu_kda_backward"] = {
        "tokens_per_s": Tc * Hc / dt / 16, "sample": f"oracle.kda.recurrent_kda_grad, B=1 T={Tc} "
        f"H={Hc} K=V=128 fp64 (numpy), scaled to configs[1]'s 16 heads", "seconds": dt,
        "gpu_tokens_per_s": 8 * 4096 / (out["kda_C1_backward_ms"] * 1e-3)}
    return out


def bench_hybrid(dev, T=16384, B=2, n_decode=256):
    import kch
    cfg = kch.HybridConfig(d_model=2048, n_heads_qk=16, n_heads_v=16, head_dim_k=128,
                           head_dim_v=128, kda_chunk_size=64, csa_m=4, csa_topk=512, csa_nh=16,
                           csa_c=128, csa_dc=128, csa_nIh=4, csa_cI=64, csa_sliding_window=128,
                           hca_m2=128, hca_nh=16, hca_c=128, hca_dc=128, hca_sliding_window=128)
    torch.manual_seed(4)
    dec = kch.HybridDecoding(cfg=cfg, total_layers=5)
    with torch.no_grad():
        for layer in dec.model.layers:
            if hasattr(layer, 'sink'):
                layer.sink.normal_()
    dec = dec.to(dev, torch.bfloat16).eval()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, T, cfg.d_model, generator=g).to(dev, torch.bfloat16)
    xs = torch.randn(n_decode + 2, B, 1, cfg.d_model, generator=g).to(dev, torch.bfloat16)
    # warm-up pass (kernel loading, GEMM heuristics), then the measured run
    dec.reset()
    dec(x[:, :1024])
    dec(xs[0])
    torch.cuda.synchronize()
    dec.reset()
    stream = torch.cuda.current_stream()
    e0, e1, e2, e3 = (torch.cuda.Event(enable_timing=True) for _ in range(4))
    e0.record(stream)
    y = dec(x)
    e1.record(stream)
    # two untimed decode steps: the first captures the step's graphs
    n_untimed = 2
    for i in range(n_untimed):
        y = dec(xs[i])
    e2.record(stream)
    captures = dec._graph_captures
    h0 = time.perf_counter()
    for i in range(n_untimed, n_untimed + n_decode):
        y = dec(xs[i])
    e3.record(stream)
    h1 = time.perf_counter()
    torch.cuda.synchronize()
    captures = dec._graph_captures - captures
    assert bool(torch.isfinite(y).all())
    pre_ms, dec_ms = e0.elapsed_time(e1), e2.elapsed_time(e3)
    return {"B": B, "T": T, "layout": dec.model.layout_str(), "prefill_ms": pre_ms,
            "prefill_tokens_per_s": B * T / (pre_ms * 1e-3), "decode_steps": n_decode,
            "decode_untimed_steps": n_untimed, "decode_device_steps": dec._device_steps,
            "decode_graph_captures_timed": captures,
            "decode_host_ms_per_step": 1e3 * (h1 - h0) / n_decode,
            "decode_ms_per_step": dec_ms / n_decode,
            "decode_tokens_per_s": B * n_decode / (dec_ms * 1e-3)}


def bench_decode_bw(dev, reps=5):
    """Decode steps on long caches, timed one by one with the 256 MB MALL flushed
    before each by READING 512 MB (a write would leave dirty lines whose
    write-back then competes with the timed reads), so the reads come from HBM:
      CSA: B=64, 1M-token context (262144 blocks of m=4), indexer 4 x 64 top-512
           over bf16 key rows, 16 heads of 128, window 128 + sink;
      HCA: B=128, 1M-token context (8192 blocks of m'=128), 16 heads of 128,
           window 128 + sink; and the same at a 4M-token context (32768 blocks,
           1.08 GB per step).
    Algorithmic bytes: every key row, its inverse norm, the selected rows and the
    window for CSA; every compressed row and the window for HCA."""
    from kch import _lib
    lib = _lib.load()
    g = torch.Generator(device=dev).manual_seed(5)
    flush = torch.ones(128 << 20, device=dev, dtype=torch.float32)  # 512 MB
    torch.cuda.synchronize()

    def timed(fn):
        ts = []
        for i in range(reps + 1):
            flush.amax()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            if i:
                ts.append(a.elapsed_time(b))
        return float(np.median(ts))

    res = {}
    B, nb, c, cI, nh, nIh, topk, win = 64, 262144, 128, 64, 16, 4, 512, 128
    kr = torch.randn(B, nb, cI, device=dev, generator=g).to(torch.bfloat16)
    kinv = kr.float().norm(dim=-1).clamp_min(1e-12).reciprocal()
    kv = torch.nn.functional.normalize(torch.randn(B, nb, c, device=dev, generator=g), dim=-1).to(torch.bfloat16)
    ring = torch.nn.functional.normalize(torch.randn(B, win, c, device=dev, generator=g), dim=-1).to(torch.bfloat16)
    q = torch.randn(B, nh, c, device=dev, generator=g)
    qi = torch.randn(B, nIh, cI, device=dev, generator=g)
    wi = torch.randn(B, nIh, device=dev, generator=g)
    sink = torch.randn(nh, device=dev, generator=g)
    out = torch.empty(B, nh, c, device=dev)
    nbytes = lib.kch_decode_ws_bytes(B, nb, nh, c, topk, win, 1)
    ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    st = _lib.stream_of(q)

    def csa():
        _lib.call("kch_csa_decode", _lib.ptr(q), _lib.ptr(qi), _lib.ptr(wi), _lib.ptr(kv), nb * c,
                  _lib.ptr(kr), nb * cI, _lib.ptr(kinv), nb, _lib.ptr(ring), win * c, win,
                  _lib.ptr(sink), _lib.ptr(out), None, B, nb, nh, c, nIh, cI, topk, 1.0, 1.0, 1, 1,
                  0, 1, 0, _lib.ptr(ws), nbytes, st)
    ms = timed(csa)
    byts = B * (nb * (cI * 2 + 4) + (topk + win) * c * 2 + (nh * c + nIh * cI + nIh) * 4 + nh * c * 4)
    res["csa"] = {"B": B, "context": nb * 4, "blocks": nb, "topk": topk, "ms": ms,
                  "algorithmic_bytes": byts, "gbs": byts / (ms * 1e-3) / 1e9,
                  "hbm_frac": byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    del kr, kinv, kv, ring, ws
    torch.cuda.empty_cache()
    # HCA at two cache sizes: the step's fixed costs (launch, the first rows'
    # latency, the partials' merge launch: about 9 us) weigh on 275 MB and
    # much less on 1.08 GB
    for name, B, nb in (("hca", 128, 8192), ("hca_4M", 128, 32768)):
        kv = torch.nn.functional.normalize(torch.randn(B, nb, c, device=dev, generator=g), dim=-1).to(torch.bfloat16)
        ring = torch.nn.functional.normalize(torch.randn(B, win, c, device=dev, generator=g), dim=-1).to(torch.bfloat16)
        q = torch.randn(B, nh, c, device=dev, generator=g)
        out = torch.empty(B, nh, c, device=dev)
        nbytes = lib.kch_decode_ws_bytes(B, nb, nh, c, 0, win, 0)
        ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)

        def hca():
            _lib.call("kch_hca_decode", _lib.ptr(q), _lib.ptr(kv), nb * c, _lib.ptr(ring), win * c, win,
                      _lib.ptr(sink), _lib.ptr(out), B, nb, nh, c, 1.0, 1, 0, 0, _lib.ptr(ws), nbytes, st)
        ms = timed(hca)
        byts = B * ((nb + win) * c * 2 + nh * c * 4 * 2)
        res[name] = {"B": B, "context": nb * 128, "blocks": nb, "ms": ms, "algorithmic_bytes": byts,
                     "gbs": byts / (ms * 1e-3) / 1e9, "hbm_frac": byts / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
        del kv, ring, ws
        torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # the first tens of steps after idle run at lower clocks (~10% slower at C1)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--headline-only", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run three 1 GiB device-to-device copies (HBM counter scale)")
    ap.add_argument("--only-extra", choices=["decode_bw", "hybrid_C4", "kda_T8K", "csa_C2", "hca_C3",
                                             "training"],
                    help="run just this extra workload and print its JSON (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (every box has one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import kch

    dev = torch.device("cuda:0")
    if args.only_extra:
        fn = {"decode_bw": bench_decode_bw, "hybrid_C4": bench_hybrid, "training": bench_training,
              "kda_T8K": lambda d: bench_kda(4, 8192, args.steps, args.warmup, d),
              "csa_C2": lambda d: bench_csa(4, 8192, max(3, args.steps // 4), 1, d),
              "hca_C3": lambda d: bench_hca(4, 32768, max(3, args.steps // 4), 1, d)}[args.only_extra]
        print(json.dumps({args.only_extra: fn(dev)}))
        return
    B, T, H, K, V = 8, 4096, 16, 128, 128
    xs, s0, host, s0h = kda_inputs(B, T, H, K, V, dev=dev)

    def step():
        return kch.naive_chunk_kda(*xs, initial_state=s0, output_final_state=True)

    ms_mean, ms_med, _ = time_steps(step, args.steps, args.warmup, per_step=True)
    _log(f"kda C1: {ms_mean:.3f} ms/step")
    flops, bytes_ = kda_algorithmic(B, T, H, K, V)
    t = ms_mean * 1e-3
    achieved = bytes_ / t / 1e9
    rec = {
        "metric": METRIC,
        "value": B * T / t,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_settle_steps": SETTLE_STEPS.get("step", 0),
        "ms_per_step": ms_mean,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "kda_chunk_prefill", "B": B, "T": T, "H": H, "K": K, "V": V,
                   "chunk": 64, "state": "fp32", "baseline_config": "configs[1]"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": HEADLINE_TRAFFIC_BYTES,
                     "algorithmic_bytes": bytes_,
                     "kernel": "kda_prep_kernel<128,128,bf16> + kda_state_kernel<128,64,bf16>",
                     "mfma_tflops": flops / t / 1e12,
                     "mfma_frac": flops / t / 1e12 / BF16_PEAK_TFLOPS},
        "ms_per_step_median": ms_med,
    }
    del xs, s0
    if args.copy_calibration:
        src = torch.empty(1 << 29, device=dev, dtype=torch.bfloat16).normal_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        rec["copy_calibration_bytes"] = {"read": src.numel() * 2, "write": dst.numel() * 2}
        del src, dst
    if not args.headline_only:
        extra = {}
        extra["kda_T8K"] = bench_kda(4, 8192, args.steps, args.warmup, dev)
        _log(f"kda T8K: {extra['kda_T8K']['ms']:.3f} ms")
        # the metric is quoted at T=8K: its KDA figure beside the headline
        rec["value_T8K"] = extra["kda_T8K"]["tokens_per_s"]
        rec["ms_per_step_T8K"] = extra["kda_T8K"]["ms"]
        extra["csa_C2"] = bench_csa(4, 8192, max(3, args.steps // 4), 1, dev)
        _log(f"csa C2: {extra['csa_C2']['ms']:.3f} ms")
        extra["hca_C3"] = bench_hca(4, 32768, max(3, args.steps // 4), 1, dev)
        _log(f"hca C3: {extra['hca_C3']['ms']:.3f} ms")
        extra["hca_T8K"] = bench_hca(4, 8192, max(3, args.steps // 4), 1, dev)
        _log(f"hca T8K: {extra['hca_T8K']['ms']:.3f} ms")
        torch.cuda.empty_cache()
        extra["decode_bw"] = bench_decode_bw(dev)
        _log(f"decode bw: csa {extra['decode_bw']['csa']['ms']:.3f} ms "
             f"({extra['decode_bw']['csa']['hbm_frac']:.1%} of HBM), hca "
             f"{extra['decode_bw']['hca']['ms']:.3f} ms ({extra['decode_bw']['hca']['hbm_frac']:.1%})")
        torch.cuda.empty_cache()
        extra["hybrid_C4"] = bench_hybrid(dev)
        _log(f"hybrid C4: prefill {extra['hybrid_C4']['prefill_ms']:.2f} ms, decode "
             f"{extra['hybrid_C4']['decode_ms_per_step']:.3f} ms/step")
        torch.cuda.empty_cache()
        # the training path (gradients): not part of the headline metric
        extra["training"] = bench_training(dev)
        _log(f"training: KDA C1 backward {extra['training']['kda_C1_backward_ms']:.2f} ms, "
             f"stack step {extra['training']['hybrid_C4_B2_T2048_train_step_ms']:.2f} ms")
        rec["extra"] = extra
    if not args.no_cpu:
        rec["cpu_baseline"] = cpu_baselines(host, s0h)
        _log("cpu baseline done")
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
