#!/usr/bin/env python3
"""Benchmark of the GRPO RL-step hot path on one MI355X.

Prints ONE JSON line (the driver's contract). Workloads:
  rl_step    config[1] (default): 12-layer d768 Q4G128 decoder, 16 prompts x 8
             rollouts, 128-token prompts, 256 sampled tokens at T=1.0, then the
             log-prob recompute of policy + frozen reference and the GRPO loss.
             value = rollout tok/s; ms_per_step = whole RL step.
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


def measured_gemv_traffic():
    """HBM bytes per launch of the LM-head GEMV from the committed rocprofv3
    --pmc summary (FETCH_SIZE / WRITE_SIZE, copy-calibrated), or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "q4_gemv_lm_head_traffic.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        return None
    return None


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


CFG1 = dict(layers=12, d_model=768, heads=12, kv_heads=12, head_dim=64, ffn=3072, vocab=32768)


CFG2 = dict(layers=24, d_model=2048, heads=16, kv_heads=4, head_dim=128, ffn=5632, vocab=65536)


# config[4]: attention geometry is not specified by the config; H16 = KVH16,
# head_dim 128 (d_model / heads). The dense FFN width is unused (all layers MoE).
CFG4 = dict(layers=16, d_model=2048, heads=16, kv_heads=16, head_dim=128, ffn=1408, vocab=65536,
            experts=32, expert_ffn=1408)

# (model, prompts, group, prompt_len, new_tokens, reward sampler)
RL_CONFIGS = {
    1: (CFG1, 16, 8, 128, 256, "bernoulli0.3"),
    2: (CFG2, 32, 8, 512, 512, "uniform"),
    4: (CFG4, 16, 8, 256, 256, "bernoulli0.3"),
}


def q4_gemv_sweep(model_cfg: dict, dev, reps: int = 10) -> dict:
    """M=1 Q4G128 GEMV over every linear of a model (whole-model weight sweep).

    All launches are captured once in a HIP graph and replayed, so the timing is
    GPU time, not Python launch overhead; HIP events on the capture/replay
    stream. The config[2] sweep (~627 MB of packed weights) exceeds the 256 MB
    MALL, so every matrix streams from HBM. Algorithmic bytes per launch =
    N*K*(0.5 + 2/128) + K*2 (x) + N*4 (y)."""
    import torch

    from summa_amd import ops

    d, F, V = model_cfg["d_model"], model_cfg["ffn"], model_cfg["vocab"]
    qn = (model_cfg["heads"] + 2 * model_cfg["kv_heads"]) * model_cfg["head_dim"]
    shapes = [(qn, d), (d, model_cfg["heads"] * model_cfg["head_dim"]), (2 * F, d), (d, F)]
    mats = []
    for layer in range(model_cfg["layers"]):
        for n, k in shapes:
            w = torch.empty(n, k, device=dev)
            ops.fill_normal(w, 0.0, 0.02, seed=layer * 10 + n)
            mats.append(ops.Q4Weight.quantize(w))
            mats[-1].drop_rowmajor()
            del w
    w = torch.empty(V, d, device=dev)
    ops.fill_normal(w, 0.0, 0.02, seed=99)
    mats.append(ops.Q4Weight.quantize(w))
    del w
    kmax = max(m.k for m in mats)
    x = torch.randn(1, kmax, device=dev).to(torch.float16)  # model activations are f16
    xs = [x[:, :m.k].contiguous() for m in mats]
    ys = [torch.empty(1, m.n, device=dev) for m in mats]
    torch.cuda.synchronize()
    for m, xi, y in zip(mats, xs, ys):  # warm (module load, first launch)
        ops.q4_matmul(m, xi, out=y)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for m, xi, y in zip(mats, xs, ys):
            ops.q4_matmul(m, xi, out=y)
    graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for _ in range(reps):
        graph.replay()
    b.record(st)
    torch.cuda.synchronize()
    sweep_ms = a.elapsed_time(b) / reps
    nbytes = sum(m.nbytes + m.k * 2 + m.n * 4 for m in mats)
    # The largest GEMV (LM head) sustained: 4 distinct copies (> 256 MB MALL)
    # replayed back to back, so each launch streams its matrix from HBM.
    heads = [mats[-1]]
    for i in range(3):
        w = torch.empty(V, d, device=dev)
        ops.fill_normal(w, 0.0, 0.02, seed=1000 + i)
        heads.append(ops.Q4Weight.quantize(w))
        heads[-1].drop_rowmajor()
        del w
    y_head = torch.empty(1, V, device=dev)
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        for _ in range(2):
            for m in heads:
                ops.q4_matmul(m, xs[-1], out=y_head)
    g2.replay()
    torch.cuda.synchronize()
    a.record(st)
    for _ in range(reps):
        g2.replay()
    b.record(st)
    torch.cuda.synchronize()
    head_us = a.elapsed_time(b) * 1e3 / (reps * 8)
    head_bytes = heads[0].nbytes + d * 2 + V * 4
    return {"sweep_ms": sweep_ms, "sweep_bytes": nbytes, "sweep_GBs": nbytes / sweep_ms / 1e6,
            "launches": len(mats), "avg_launch_us": sweep_ms * 1e3 / len(mats),
            "model": f"{model_cfg['layers']}L d{d} F{F} V{V}",
            "lm_head_shape": [V, d], "lm_head_us": head_us, "lm_head_bytes": head_bytes,
            "lm_head_GBs": head_bytes / head_us / 1e3}


def cpu_baseline_rl(config: int) -> dict:
    """Oracle (C restatement, OpenMP over the host cores) rollout on a bounded
    sample of the workload: 2 rollouts x (full-length prompt + 8 sampled tokens)
    for config[1], 1 x (prompt + 2) for the larger configs."""
    import numpy as np

    import oracle

    mcfg, _, _, P, _, _ = RL_CONFIGS[config]
    cfg = {"layers": mcfg["layers"], "d": mcfg["d_model"], "H": mcfg["heads"],
           "KVH": mcfg["kv_heads"], "hd": mcfg["head_dim"], "F": mcfg["ffn"], "V": mcfg["vocab"]}
    if mcfg.get("experts"):
        cfg.update(E=mcfg["experts"], Fe=mcfg["expert_ffn"])
    w = oracle.random_weights(cfg, seed=0, std=0.02)
    host = oracle.HostModel(cfg, w, quantized=True)
    del w
    S, N = (2, 8) if config == 1 else (1, 2)
    prompts = np.random.default_rng(0).integers(0, cfg["V"], (S, P)).astype(np.int32)
    t0 = time.perf_counter()
    host.generate(prompts, N, 1.0, 0)
    dt = time.perf_counter() - t0
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count()))
    return {"value": round(S * N / dt, 4), "unit": "rollout tok/s", "cores": threads,
            "kind": "port",
            "sample": f"config[{config}] Q4 model, {S} rollouts x ({P}-token prompt + {N} "
                      f"sampled), {dt:.1f} s (prefill included, as in the rollout)"}


def bench_rl_step(args) -> dict:
    import torch

    from summa_amd.model import Model, ModelConfig, batch_result, rl_prepare

    mcfg, groups, G, P, N, reward_kind = RL_CONFIGS[args.config]
    S = groups * G
    dev = torch.device("cuda:0")
    mc = ModelConfig(**mcfg, max_seq=P + N, quantized=True)
    policy = Model(mc)
    policy.init_random(seed=0, std=0.02)
    reference = Model(mc)
    reference.init_random(seed=0, std=0.02)  # frozen copy of the initial policy
    gen = torch.Generator().manual_seed(0)
    prompts = torch.randint(0, mc.vocab, (S, P), generator=gen, dtype=torch.int32).to(dev)
    if reward_kind == "uniform":
        rewards = torch.rand((groups, G), generator=gen).to(dev)
    else:
        rewards = torch.bernoulli(torch.full((groups, G), 0.3), generator=gen).to(dev)
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()

    def step(seed):
        tok, lp_beh = policy.generate(prompts, N, temperature=1.0, seed=seed)
        e_mid.record(st)
        out = rl_prepare(policy, reference, prompts, tok, lp_beh, rewards, clip_epsilon=0.2,
                         advantage_epsilon=1e-6, kl_coefficient=0.04)
        return out

    e0, e_mid, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    log("bench: warmup")
    for i in range(args.warmup):
        step(1000 + i)
    torch.cuda.synchronize()
    roll_ms, step_ms = [], []
    t0 = time.perf_counter()
    for i in range(args.steps):
        e0.record(st)
        out = step(i)
        e1.record(st)
        torch.cuda.synchronize()
        roll_ms.append(e0.elapsed_time(e_mid))
        step_ms.append(e0.elapsed_time(e1))
        log(f"bench: step {i} rollout {roll_ms[-1]:.1f} ms, RL step {step_ms[-1]:.1f} ms")
    wall = time.perf_counter() - t0
    res = batch_result(out)
    roll = sum(roll_ms) / len(roll_ms)
    full = sum(step_ms) / len(step_ms)
    del policy, reference
    torch.cuda.empty_cache()
    log("bench: q4 gemv sweep (config[2] weights, graph replay)")
    sweep = q4_gemv_sweep(CFG2, dev)
    achieved = sweep["lm_head_GBs"]
    return {
        "metric": "rollout tok/s + RL step ms on 1 MI355X; % HBM roofline of 4-bit GEMV",
        "value": S * N / (roll * 1e-3), "unit": "rollout tok/s",
        "ms_per_step": full, "dtype": "q4g128 weights, f16-pair (fp32-grade) matmul inputs, f16 KV, f32 accumulate",
        "config": {"workload": f"rl_step config[{args.config}]", **mcfg, "prompts": groups,
                   "group": G, "prompt_len": P, "new_tokens": N, "temperature": 1.0,
                   "weights": "Q4G128 (bf16 scales)",
                   "rewards": "U[0,1]" if reward_kind == "uniform" else "Bernoulli(0.3)"},
        "rl_step_ms": round(full, 3), "rollout_ms": round(roll, 3),
        "prepare_ms": round(full - roll, 3), "wall_s": round(wall, 3),
        "grpo": {k: (round(v, 6) if isinstance(v, float) else v) for k, v in res.items()},
        "roofline": {"bound": "hbm",
                     "kernel": "q4g128 GEMV M=1, config[2] LM head 65536x2048 (4 copies > MALL, "
                               "graph replay); whole-model sweep in q4_gemv",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_gemv_traffic()},
        "q4_gemv": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in sweep.items()},
    }


def bench_q4_gemv(args) -> dict:
    """The 4-bit GEMV alone (the metric's roofline part): config[2] weights,
    M=1, graph replay; see q4_gemv_sweep."""
    import torch

    dev = torch.device("cuda:0")
    sweep = q4_gemv_sweep(CFG2, dev, reps=max(args.steps, 1) * 10)
    achieved = sweep["lm_head_GBs"]
    # a plain device copy of known size (256 MiB read + 256 MiB written): the
    # calibration dispatch for the HBM byte counters of a rocprofv3 --pmc run
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev)
    torch.empty_like(src).copy_(src)
    torch.cuda.synchronize()
    return {
        "metric": "4-bit GEMV GB/s (config[2] LM head, M=1)", "value": achieved, "unit": "GB/s",
        "ms_per_step": sweep["sweep_ms"], "dtype": "q4g128 weights, f16 x, f32 accumulate",
        "config": {"workload": "q4_gemv config[2]", "lm_head": [CFG2["vocab"], CFG2["d_model"]]},
        "roofline": {"bound": "hbm", "kernel": "q4g128 GEMV M=1 (LM head 65536x2048)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_gemv_traffic()},
        "q4_gemv": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in sweep.items()},
    }


WORKLOADS = {"rl_step": bench_rl_step, "ce_stress": bench_ce_stress, "q4_gemv": bench_q4_gemv}


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--workload", default="rl_step", choices=sorted(WORKLOADS))
    p.add_argument("--rows", type=int, default=65536)
    p.add_argument("--config", type=int, default=1, choices=sorted(RL_CONFIGS),
                   help="rl_step: BASELINE config index (1 = the headline line)")
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
        if args.workload == "rl_step":
            out["cpu_baseline"] = cpu_baseline_rl(args.config)
        elif args.workload == "ce_stress":
            out["cpu_baseline"] = cpu_baseline_ce(256, 131072)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
