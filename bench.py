#!/usr/bin/env python3
"""Benchmark of the GRPO RL-step hot path on one MI355X.

Prints ONE JSON line (the driver's contract). Workloads:
  ce_stress  config[3]: fused log-softmax/CE/token-logprob over bf16
             [65536 x 131072] logits (HBM-bound).
Timing: W warmup steps, then K timed steps bracketed by synchronisation; kernel
durations come from HIP events recorded on the stream the kernels run on.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline_ce(rows: int, vocab: int, seconds: float = 10.0) -> dict:
    """Oracle (f64 two-pass C port, all host threads) on a bounded sample of config[3] rows."""
    import numpy as np

    import oracle

    rng = np.random.default_rng(0)
    sample_rows = 256
    x = oracle.bf16_bits(rng.normal(0, 3, (sample_rows, vocab)).astype(np.float32))
    t = rng.integers(0, vocab, sample_rows).astype(np.int32)
    oracle.ce_rows(x[:8], t[:8])
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.ce_rows(x, t)
        n += 1
    dt = (time.perf_counter() - t0) / n
    gbs = sample_rows * vocab * 2 / dt / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": os.cpu_count(), "kind": "port",
            "sample": f"{sample_rows} rows x {vocab} bf16, lp only, {n} reps"}


def bench_ce_stress(args) -> dict:
    import torch

    from summa_amd import ops

    rows, vocab = args.rows, 131072
    dev = torch.device("cuda:0")
    x = torch.empty(rows, vocab, dtype=torch.bfloat16, device=dev)
    t = torch.empty(rows, dtype=torch.int32, device=dev)
    ops.fill_ce_stress(x, t, 3.0, 8.0, seed=0)
    torch.cuda.synchronize()
    for _ in range(args.warmup):
        ops.ce_rows(x, t)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    t0 = time.perf_counter()
    for a, b in evs:
        a.record(st)
        ops.ce_rows(x, t)
        b.record(st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    kms = sum(a.elapsed_time(b) for a, b in evs) / len(evs)
    algo_bytes = rows * vocab * 2 + rows * 8
    achieved = algo_bytes / (kms * 1e-3) / 1e9
    res = {
        "metric": "fused CE/log-prob rows/s (config[3] bf16 65536x131072)",
        "value": rows / (wall / args.steps), "unit": "rows/s",
        "ms_per_step": wall / args.steps * 1e3, "dtype": "bf16",
        "config": {"workload": "ce_stress", "rows": rows, "vocab": vocab, "outputs": "lp+loss"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
    }
    # grad-in-place variant (1 read + 1 write)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    ops.ce_rows(x, t, grad_in_place=True, grad_scale=1.0 / rows)
    b.record(st)
    torch.cuda.synchronize()
    gms = a.elapsed_time(b)
    res["grad_in_place"] = {"ms": round(gms, 4),
                            "GB/s": round(2 * rows * vocab * 2 / (gms * 1e-3) / 1e9, 1)}
    return res


WORKLOADS = {"ce_stress": bench_ce_stress}


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="ce_stress", choices=sorted(WORKLOADS))
    p.add_argument("--rows", type=int, default=65536)
    p.add_argument("--no-cpu-baseline", action="store_true")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the RL step is "
              "sharded by whole GRPO groups across GPUs, which this build does not run.",
              file=sys.stderr)
        return 2
    log(f"bench: workload={args.workload} steps={args.steps} warmup={args.warmup}")
    res = WORKLOADS[args.workload](args)
    out = {"metric": res.pop("metric"), "value": round(res.pop("value"), 3), "unit": res.pop("unit"),
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(res.pop("ms_per_step"), 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": res.pop("dtype"), "data": "synthetic",
           "config": res.pop("config")}
    out.update(res)
    if not args.no_cpu_baseline:
        log("bench: cpu baseline")
        out["cpu_baseline"] = cpu_baseline_ce(256, 131072)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
