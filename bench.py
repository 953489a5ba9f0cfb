"""Benchmark of the MI355X hybrid-attention forward path (one JSON line on stdout).

Headline workload: KDA chunked prefill, bf16 inputs
with fp32 state, B=8 T=4096 H=16 K=V=128, q/k L2-normalised N(0,1), v N(0,1),
g = logsigmoid(N(0,1)) per channel, beta = sigmoid(N(0,1)), S0 ~ 0.02 N(0,1).
A step is one ``kch.naive_chunk_kda`` call over that batch (inputs resident in
HBM). ``value`` is B*T tokens per second of step time, measured with HIP events
on the stream the kernel runs on.

``roofline``: algorithmic HBM bytes of the step (q,k,v,g,o bf16 + beta bf16 +
S0 read and S write fp32) over the measured kernel time, against 8 TB/s.
``cpu_baseline``: the numpy oracle (a from-scratch CPU restatement of the
reference algorithm) on a bounded sample of the same workload, one thread.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
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


def time_steps(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    t0 = time.perf_counter()
    for a, b in ev:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [a.elapsed_time(b) for a, b in ev]
    return float(np.mean(per)), float(np.median(per)), wall


def cpu_baseline_kda(host, s0, B, T, H):
    """Oracle on a bounded sample: the first ``nb`` batches, all heads, one thread."""
    from threadpoolctl import threadpool_limits

    from oracle.kda import chunk_kda
    nb = 2
    q, k, v, g, beta = (x[:nb] for x in host)
    with threadpool_limits(1):
        t0 = time.perf_counter()
        chunk_kda(q, k, v, g, beta, initial_state=s0[:nb], chunk_size=64)
        dt = time.perf_counter() - t0
    frac = nb / B
    tok_s = (B * T) / (dt / frac)
    return {"value": tok_s, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"numpy oracle chunk_kda, {nb} of {B} sequences (all {H} heads, "
                      f"T={T}) in {dt:.1f} s, scaled to the full batch; 1 thread; "
                      f"host {platform.processor() or platform.machine()}"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (every box has one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import kch

    B, T, H, K, V = 8, 4096, 16, 128, 128
    dev = torch.device("cuda:0")
    xs, s0, host, s0h = kda_inputs(B, T, H, K, V, dev=dev)

    def step():
        return kch.naive_chunk_kda(*xs, initial_state=s0, output_final_state=True)

    ms_mean, ms_med, _ = time_steps(step, args.steps, args.warmup)
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
        "ms_per_step": ms_mean,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "kda_chunk_prefill", "B": B, "T": T, "H": H, "K": K, "V": V,
                   "chunk": 64, "state": "fp32", "baseline_config": "configs[1]"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes": bytes_, "kernel": "kda_chunk_lp_kernel<128,bf16>",
                     "mfma_tflops": flops / t / 1e12,
                     "mfma_frac": flops / t / 1e12 / BF16_PEAK_TFLOPS},
        "ms_per_step_median": ms_med,
    }
    if not args.no_cpu:
        rec["cpu_baseline"] = cpu_baseline_kda(host, s0h, B, T, H)
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
