"""Benchmark of the MI355X decode path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload gemv]

Prints one JSON line. The roofline object is the batch-1 MXFP4 GEMV of the GEMV configuration
(W 8192 x 2048 MXFP4, x fp16, y fp16): 8,933,376 algorithmic bytes per launch (codes 8,388,608 +
scales 524,288 + x 4,096 + y 16,384), timed per launch with HIP events on the launching stream,
over 64 distinct weight copies (572 MB, past the 256 MB MALL) so that every launch reads HBM.
The CPU baseline is the oracle's restatement of the reference's CPU MXFP4 GEMV (mxfp4.Run with
the int8-quantized activation, internal/mxfp4/matvec.go:33-160), on the host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
GEMV_N, GEMV_K = 8192, 2048
GEMV_BYTES = GEMV_N * GEMV_K // 2 + GEMV_N * GEMV_K // 32 + GEMV_K * 2 + GEMV_N * 2  # 8,933,376
COPIES = 64


def gemv_roofline(steps: int, warmup: int):
    import torch

    from hwnpu_amd import ops, synth

    ws = [synth.mxfp4_uniform(GEMV_N, GEMV_K, f"bench.c1.{i}") for i in range(COPIES)]
    x = synth.normal(GEMV_K, "bench.c1.x", dtype=torch.float16)
    y = torch.empty(GEMV_N, dtype=torch.float16, device="cuda")
    for i in range(warmup):
        w, e = ws[i % COPIES]
        ops.mxfp4_gemv(w, e, x, "f16", y=y)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        w, e = ws[i % COPIES]
        starts[i].record()
        ops.mxfp4_gemv(w, e, x, "f16", y=y)
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = sorted(s.elapsed_time(e) * 1e3 for s, e in zip(starts, ends))  # us
    avg_us = sum(per) / len(per)
    return {
        "avg_us": avg_us,
        "median_us": per[len(per) // 2],
        "wall_s": wall,
        "gbs": GEMV_BYTES / (avg_us * 1e-6) / 1e9,
    }


def cpu_gemv_baseline(budget_s: float = 12.0):
    """The reference's CPU MXFP4 GEMV restated (oracle, test infrastructure): the int8-quantized
    activation and mxfp4.Run's 32-row spans over every host core, on one 8192 x 2048 GEMV."""
    import numpy as np

    from oracle import oracle

    rng = np.random.default_rng(0)
    w = rng.integers(0, 256, (GEMV_N, GEMV_K // 2), dtype=np.uint8)
    e = rng.integers(123, 130, (GEMV_N, GEMV_K // 32), dtype=np.uint8)
    x = rng.standard_normal(GEMV_K).astype(np.float16).astype(np.float32)
    threads = oracle.max_threads()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t = time.perf_counter()
        q, s = oracle.vec_quantize(x)
        oracle.mxfp4_run(w, e, q[None, :], s[None, :], threads=threads)
        times.append(time.perf_counter() - t)
        if len(times) >= 200:
            break
    times.sort()
    med = times[len(times) // 2]
    return {"value": round(GEMV_BYTES / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{len(times)} MXFP4 GEMVs 8192x2048 (int8 activation, mxfp4.Run), median"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="gemv", choices=["gemv"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(sharding is a design note, not a measured path)", file=sys.stderr)
        sys.exit(2)
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    r = gemv_roofline(args.steps, args.warmup)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    out = {
        "metric": "MXFP4 GEMV achieved HBM GB/s (batch-1 decode GEMV, 8192x2048)",
        "value": round(r["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall_s"] / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4*fp16->f32",
        "data": "synthetic (seeded splitmix64 draws on the GPU)",
        "config": {"workload": "mxfp4_gemv N=8192 K=2048, 64 rotating weight copies", "n": GEMV_N, "k": GEMV_K},
        "roofline": {"bound": "hbm", "achieved": round(r["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel_avg_us": round(r["avg_us"], 3), "bytes_per_launch": GEMV_BYTES},
        "cpu_baseline": None if args.no_cpu else cpu_gemv_baseline(),
        "wall_s": round(wall, 3),
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
