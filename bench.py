#!/usr/bin/env python3
"""Benchmark of the GRPO RL-step hot path on one MI355X.

Prints ONE JSON line (the driver's contract). Workloads:
  rl_step         (default) one GRPO step of a BASELINE config (--config, default
                  2: the 24-layer d2048 GQA Q4G128 decoder, 32 prompts x 8
                  rollouts, 512-token prompts, 512 sampled tokens at T = 1, then
                  the log-prob recompute of the policy and its frozen copy over
                  all 1023 positions and the GRPO loss). value = rollout tok/s
                  (S * N / rollout time); ms_per_step = the whole RL step.
                  Sub-results: decode HBM fraction, recompute MFMA fraction,
                  the dominant kernel's roofline, the config[3] fused CE, the
                  whole-model Q4 GEMV sweep at M = 1, 2, 4, 8, 16, config[0].
  ce_stress       config[3]: fused log-softmax/CE/token-logprob over bf16
                  [65536 x 131072] logits (lp + loss, and grad in place).
  q4_gemv         the whole-model M = 1 Q4 GEMV sweep (config[2] weights).
  recompute_gemm  the dominant kernel alone: the config[2] recompute FFN-in
                  GEMM (wide-tile kernel), for counter runs.
  decode_attention  config[2]'s decode attention, per-rollout vs shared
                  prompt, at t = 1, 256, 511 (value = speedup at t = 511).
Timing: W warmup steps, then K timed steps bracketed by synchronisation; GPU
durations come from HIP events recorded on the stream the work runs on.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_F16_PEAK_TFS = 2500.0   # MI355X dense f16 / bf16 MFMA


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def profile_figure(name: str, key: str):
    """An integer figure (``key: value`` line) from a committed profiles/ summary."""
    try:
        for line in open(ROOT / "profiles" / name):
            if line.startswith(key + ":"):
                return int(line.split(":")[1])
    except OSError:
        return None
    return None


def _events(n):
    import torch
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def _time_launches(fn, reps: int) -> float:
    """Average GPU ms per call of ``fn`` (events on the current stream)."""
    import torch
    st = torch.cuda.current_stream()
    fn()
    torch.cuda.synchronize()
    a, b = _events(2)
    a.record(st)
    for _ in range(reps):
        fn()
    b.record(st)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


# --------------------------------------------------------------- analysis ---

def linear_shapes(m: dict) -> list:
    """(N, K) of every per-layer linear of a dense model (out x in)."""
    d, qn = m["d_model"], (m["heads"] + 2 * m["kv_heads"]) * m["head_dim"]
    return [(qn, d), (d, m["heads"] * m["head_dim"]), (2 * m["ffn"], d), (d, m["ffn"])]


def q4_bytes(n: int, k: int) -> int:
    return n * k // 2 + n * k // 128 * 2  # 4-bit codes + one bf16 scale per 128


def recompute_flops(wl, prompt_pass: bool = True) -> float:
    """Algorithmic flops of one model's log-prob recompute of S = prompts x
    group rollouts of P + N - 1 positions, where a group's rollouts share one
    prompt (GRPO), so its P prompt positions are computed once per group:
    2 * tokens * per-layer linear params over prompts * P + S * (N - 1) token
    rows, the LM head over the S * N scored rows, causal attention (Q.K^T and
    P.V over the lower triangle: the prompt's triangle once per group, the
    completion rows' keys per rollout). prompt_pass=False leaves out the prompt
    rows and their triangle: the policy's recompute reuses the prompt pass of
    the generation that produced the tokens."""
    m = wl.model
    P, N, S = wl.prompt_len, wl.new_tokens, wl.rollouts
    L = P + N - 1
    pp = 1 if prompt_pass else 0
    tokens = pp * wl.prompts * P + S * (N - 1)
    lin = sum(n * k for n, k in linear_shapes(m)) * m["layers"]
    head = m["vocab"] * m["d_model"]
    keys = pp * wl.prompts * P * (P + 1) / 2 + S * (L * (L + 1) / 2 - P * (P + 1) / 2)
    attn = 4 * m["head_dim"] * keys * m["heads"] * m["layers"]
    return 2.0 * tokens * lin + 2.0 * S * N * head + attn


def decode_bytes(wl, shared_prompt: bool = True) -> float:
    """Algorithmic HBM bytes of the N - 1 cached decode steps: every packed
    weight once per step plus the K/V cache (f16) each step's attention needs,
    once per KV head per layer: a group's shared prompt keys once per group
    (shared_prompt) or once per rollout, and each rollout's t generated keys."""
    m = wl.model
    S, P, N = wl.rollouts, wl.prompt_len, wl.new_tokens
    w = sum(q4_bytes(n, k) for n, k in linear_shapes(m)) * m["layers"]
    w += q4_bytes(m["vocab"], m["d_model"])
    kv_tok = m["layers"] * m["kv_heads"] * m["head_dim"] * 2 * 2
    seqs_p = wl.prompts if shared_prompt else S
    ctx = sum(seqs_p * P + S * t for t in range(1, N))
    return (N - 1) * w + kv_tok * ctx


# --------------------------------------------------------------- kernels ---

def recompute_gemm(wl, dev, reps: int = 10) -> dict:
    """The dominant kernel of the config[2] step: the FFN-in projection of the
    log-prob recompute (SwiGLU f16-pair epilogue) at the shape of its
    continuation chunks (prompt groups: a chunk is 65536 // (N - 1) = 128
    rollouts of N - 1 = 511 continuation rows over the group's prompt K / V),
    M = 65408, N = 2F = 11264, K = 2048, on the wide-tile kernel.
    flops = 2 M N K per launch."""
    import torch

    from summa_amd import _lib, ops

    m = wl.model
    M = max(1, 65536 // (wl.new_tokens - 1)) * (wl.new_tokens - 1)
    N, K = 2 * m["ffn"], m["d_model"]
    w = torch.empty(N, K, device=dev)
    ops.fill_normal(w, 0.0, 0.02, seed=5)
    qw = ops.Q4Weight.quantize(w)
    qw.drop_rowmajor()
    del w
    x = torch.empty(M, K, device=dev)
    ops.fill_normal(x, 0.0, 1.0, seed=6)
    xp = ops.f16_pair(x)
    del x
    out = torch.empty(M, 2 * (N // 2), dtype=torch.float16, device=dev)

    def run():
        ops.q4_matmul(qw, xp, out=out, epilogue=_lib.SM_EPI_SWIGLU_F16X2, pair=True)

    ms = _time_launches(run, reps)
    flops = 2.0 * M * N * K
    achieved = flops / (ms * 1e-3) / 1e12
    return {"kernel": "q4_gemm_wide_kernel<2,5> (recompute FFN-in, SwiGLU f16-pair epilogue)",
            "shape": [M, N, K], "us": round(ms * 1e3, 2), "flops": flops,
            "TFLOPs": round(achieved, 1), "frac": round(achieved / MFMA_F16_PEAK_TFS, 4)}


def q4_gemv_sweep(model_cfg: dict, dev, ms=(1, 2, 4, 8, 16), reps: int = 10) -> dict:
    """Q4G128 GEMV over every linear of a model (whole-model weight sweep), at
    M = 1, 2, 4, 8, 16 activation rows (f16).

    All launches of one M are captured in a HIP graph and replayed, so the
    time is GPU time, not Python launch overhead (HIP events on the replay
    stream). The config[2] sweep (~627 MB of packed weights) exceeds the
    256 MB MALL, so every matrix streams from HBM. Algorithmic bytes per
    launch = N*K*(0.5 + 2/128) + M*K*2 (x) + M*N*4 (y, f32)."""
    import torch

    from summa_amd import _lib, ops

    d, V = model_cfg["d_model"], model_cfg["vocab"]
    mats = []
    for layer in range(model_cfg["layers"]):
        for n, k in linear_shapes(model_cfg):
            w = torch.empty(n, k, device=dev)
            ops.fill_normal(w, 0.0, 0.02, seed=layer * 10 + n)
            mats.append(ops.Q4Weight.quantize(w))
            mats[-1].drop_rowmajor()
            del w
    w = torch.empty(V, d, device=dev)
    ops.fill_normal(w, 0.0, 0.02, seed=99)
    mats.append(ops.Q4Weight.quantize(w))
    mats[-1].drop_rowmajor()
    del w
    kmax = max(m.k for m in mats)
    st = torch.cuda.current_stream()
    res = {"model": f"{model_cfg['layers']}L d{d} F{model_cfg['ffn']} V{V}",
           "launches": len(mats), "weight_bytes": sum(m.nbytes for m in mats), "by_M": {}}
    for M in ms:
        x = torch.randn(M, kmax, device=dev).to(torch.float16)
        xs = [x[:, :m.k].contiguous() for m in mats]
        ys = [torch.empty(M, m.n, device=dev) for m in mats]
        for m, xi, y in zip(mats, xs, ys):  # warm (module load, first launch)
            ops.q4_matmul(m, xi, out=y)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for m, xi, y in zip(mats, xs, ys):
                ops.q4_matmul(m, xi, out=y)
        graph.replay()
        torch.cuda.synchronize()
        a, b = _events(2)
        a.record(st)
        for _ in range(reps):
            graph.replay()
        b.record(st)
        torch.cuda.synchronize()
        sweep_ms = a.elapsed_time(b) / reps
        nbytes = sum(m.nbytes + M * m.k * 2 + M * m.n * 4 for m in mats)
        gbs = nbytes / sweep_ms / 1e6
        res["by_M"][str(M)] = {"sweep_ms": round(sweep_ms, 4), "bytes": nbytes,
                               "GBs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        if M == 1:
            # the same GEMVs as one sm_q4_gemv_multi launch (every matrix is
            # independent here), replayed the same way
            batch = ops.GemvBatch([(m, xi, y, _lib.SM_EPI_STORE_F32)
                                   for m, xi, y in zip(mats, xs, ys)])
            batch.launch()
            torch.cuda.synchronize()
            a, b = _events(2)
            a.record(st)
            for _ in range(reps):
                batch.launch()
            b.record(st)
            torch.cuda.synchronize()
            one_ms = a.elapsed_time(b) / reps
            res["by_M"]["1"].update(
                launches_ms=res["by_M"]["1"]["sweep_ms"], single_launch_ms=round(one_ms, 4),
                single_launch_GBs=round(nbytes / one_ms / 1e6, 1),
                single_launch_frac=round(nbytes / one_ms / 1e6 / HBM_PEAK_GBS, 4))
            del batch
        del graph, xs, ys, x
    # The largest GEMV (LM head) sustained: 8 distinct copies (556 MB, over
    # twice the 256 MB MALL) replayed back to back, so each launch streams its
    # matrix from HBM.
    heads = [mats[-1]]
    for i in range(7):
        w = torch.empty(V, d, device=dev)
        ops.fill_normal(w, 0.0, 0.02, seed=1000 + i)
        heads.append(ops.Q4Weight.quantize(w))
        heads[-1].drop_rowmajor()
        del w
    xh = torch.randn(1, d, device=dev).to(torch.float16)
    y_head = torch.empty(1, V, device=dev)
    torch.cuda.synchronize()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        for _ in range(2):
            for m in heads:
                ops.q4_matmul(m, xh, out=y_head)
    g2.replay()
    torch.cuda.synchronize()
    a, b = _events(2)
    a.record(st)
    for _ in range(reps):
        g2.replay()
    b.record(st)
    torch.cuda.synchronize()
    head_us = a.elapsed_time(b) * 1e3 / (reps * 2 * len(heads))
    head_bytes = heads[0].nbytes + d * 2 + V * 4
    res.update(lm_head_shape=[V, d], lm_head_us=round(head_us, 3), lm_head_bytes=head_bytes,
               lm_head_GBs=round(head_bytes / head_us / 1e3, 1))
    return res


def ce_stress(dev, rows: int, reps: int = 5, host_sample: int = 0) -> dict:
    """config[3]: fused log-softmax / CE / token log-prob over bf16
    [rows, 131072] logits ~ N(0, 3) with a +8 spike at the target. lp + loss
    read the logits once (algorithmic bytes rows * V * 2); grad in place reads
    and writes them once (2 * rows * V * 2). host_sample > 0: also returns
    (``_sample``) that many rows spread over the batch (bf16 bits, targets)
    copied to the host before any timing, for the CPU baseline."""
    import torch

    from summa_amd import ops
    from summa_amd.configs import CE_STRESS

    vocab = CE_STRESS["vocab"]
    x = torch.empty(rows, vocab, dtype=torch.bfloat16, device=dev)
    t = torch.empty(rows, dtype=torch.int32, device=dev)
    ops.fill_ce_stress(x, t, CE_STRESS["std"], CE_STRESS["spike"], seed=0)
    torch.cuda.synchronize()
    sample = None
    if host_sample:
        idx = torch.linspace(0, rows - 1, host_sample, device=dev).long()
        lp_gpu = ops.ce_rows(x, t)[0][idx]
        sample = (x[idx].view(torch.int16).cpu().numpy().view("uint16"),
                  t[idx].cpu().numpy(), lp_gpu.cpu().numpy().astype("float64"))
    lp_ms = _time_launches(lambda: ops.ce_rows(x, t), reps)
    g_ms = _time_launches(lambda: ops.ce_rows(x, t, grad_in_place=True, grad_scale=1.0 / rows),
                          reps)
    rb = rows * vocab * 2
    del x, t
    torch.cuda.empty_cache()
    out = {"_sample": sample} if host_sample else {}
    return {**out, "shape": [rows, vocab], "dtype": "bf16",
            "lp_loss": {"ms": round(lp_ms, 4), "bytes": rb,
                        "GBs": round(rb / lp_ms / 1e6, 1),
                        "frac": round(rb / lp_ms / 1e6 / HBM_PEAK_GBS, 4)},
            "grad_in_place": {"ms": round(g_ms, 4), "bytes": 2 * rb,
                              "GBs": round(2 * rb / g_ms / 1e6, 1),
                              "frac": round(2 * rb / g_ms / 1e6 / HBM_PEAK_GBS, 4)}}


# ---------------------------------------------------------------- RL step ---

def rl_inputs(wl, mc, dev, count: int = 1, seed: int = 0):
    """``count`` distinct GRPO batches (prompts, rewards), drawn before any
    timing: `prompts` prompts each rolled out `group` times (rows g*group ..
    g*group + group - 1 carry prompt g). Every step of a run takes its own
    batch, as every update of the reference's post-training loop generates on
    new examples (posttrain.rs:4339-4440), so no step can reuse the prompt
    pass of a step before it."""
    import torch
    gen = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(count):
        prompts = torch.randint(0, mc.vocab, (wl.prompts, wl.prompt_len), generator=gen,
                                dtype=torch.int32).repeat_interleave(wl.group, 0).to(dev)
        rewards = wl.sample_rewards(gen).to(dev)
        out.append((prompts, rewards))
    return out


def run_rl_step(wl, policy, reference, batches, steps, warmup, tag=""):
    """W + K GRPO steps, step i on batches[i] (W + K distinct batches);
    returns per-step rollout / prepare / step ms (events) and the last step's
    outputs and batch."""
    import torch

    from summa_amd.configs import ADVANTAGE_EPSILON, CLIP_EPSILON, KL_COEFFICIENT
    from summa_amd.model import rl_prepare

    assert len(batches) >= warmup + steps
    st = torch.cuda.current_stream()
    e0, e_mid, e1 = _events(3)

    def step(seed, batch):
        prompts, rewards = batch
        tok, lp_beh = policy.generate(prompts, wl.new_tokens, temperature=wl.temperature,
                                      seed=seed)
        e_mid.record(st)
        out = rl_prepare(policy, reference, prompts, tok, lp_beh, rewards,
                         clip_epsilon=CLIP_EPSILON, advantage_epsilon=ADVANTAGE_EPSILON,
                         kl_coefficient=KL_COEFFICIENT)
        out["tokens"], out["lp_beh"] = tok, lp_beh
        return out

    for i in range(warmup):
        step(1000 + i, batches[i])
    torch.cuda.synchronize()
    roll, full = [], []
    t0 = time.perf_counter()
    for i in range(steps):
        e0.record(st)
        out = step(i, batches[warmup + i])
        e1.record(st)
        torch.cuda.synchronize()
        roll.append(e0.elapsed_time(e_mid))
        full.append(e0.elapsed_time(e1))
        if tag:
            log(f"bench: {tag} step {i} rollout {roll[-1]:.1f} ms, RL step {full[-1]:.1f} ms")
    wall = time.perf_counter() - t0
    return roll, full, wall, out, batches[warmup + steps - 1]


def prefill_ms(wl, policy, prompts, reps: int = 3) -> float:
    """The rollout's prefill (plus its first sample): generate with N = 1."""
    return _time_launches(lambda: policy.generate(prompts, 1, temperature=wl.temperature,
                                                  seed=3), reps)


def config0_leg(dev, steps: int = 5) -> dict:
    """config[0] (2-layer fp32 decoder, 32 rollouts, greedy): the latency leg
    (median of ``steps`` RL steps after 2 warm-up steps)."""
    from summa_amd.configs import RL_WORKLOADS
    from summa_amd.model import Model
    wl = RL_WORKLOADS[0]
    mc = wl.model_config()
    policy, reference = Model(mc), Model(mc)
    for m in (policy, reference):  # each group's prompt computed once
        m.set_prompt_groups(wl.group)
    w = draw_weights(wl, [policy, reference], dev, seed=1)
    batches = rl_inputs(wl, mc, dev, count=steps + 2)
    roll, full, _, out, (prompts, _) = run_rl_step(wl, policy, reference, batches, steps, 2)
    r, f = statistics.median(roll), statistics.median(full)
    return {"rl_step_ms": round(f, 3), "rollout_ms": round(r, 3),
            "rollout_tok_s": round(wl.rollouts * wl.new_tokens / (r * 1e-3), 1),
            "prepare_ms": round(f - r, 3), "steps": steps,
            "_out": out, "_prompts": prompts, "_weights": w}


# -------------------------------------------------------------- baseline ---

def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


CPU_CE_ROWS = 512        # config[3] rows the CPU CE leg runs (spread over the batch)
CPU_RECOMPUTE_ROWS = 32  # continuation rows of the CPU recompute sample


def cpu_ce_leg(sample, gpu_ce) -> dict:
    """config[3] on the oracle (``or_ce_rows``: f64 two-pass log-softmax, the
    reference's CE restated) over CPU_CE_ROWS of the GPU's own logits rows
    (bf16, spread over the 65536-row batch): lp + loss at 1 thread and at
    every core, lp + loss + gradient at every core (the oracle writes an f32
    gradient array rather than bf16 in place), each the median of 3; ms and
    GB/s scaled to the full 65536 x 131072 batch by rows (the algorithmic
    bytes of the GPU leg); and the GPU's lp on those rows against the
    oracle's (1e-5)."""
    import numpy as np

    import oracle
    from summa_amd.configs import CE_STRESS

    logits, tgt, lp_gpu = sample
    R, V = logits.shape
    scale = CE_STRESS["rows"] / R
    out = {"sample_rows": R, "vocab": V}

    def med(fn):
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    for label, threads in (("1_thread", 1), ("all_threads", 0)):
        n = oracle.set_threads(threads)
        t = med(lambda: oracle.ce_rows(logits, tgt))
        full_ms = t * scale * 1e3
        out[f"lp_loss_{label}"] = {"threads": n, "sample_ms": round(t * 1e3, 2),
                                   "full_batch_ms": round(full_ms, 1),
                                   "GBs": round(gpu_ce["lp_loss"]["bytes"] / full_ms / 1e6, 2)}
    t = med(lambda: oracle.ce_rows(logits, tgt, grad=True, grad_scale=1.0 / CE_STRESS["rows"]))
    full_ms = t * scale * 1e3
    out["grad_all_threads"] = {"threads": oracle.set_threads(0), "sample_ms": round(t * 1e3, 2),
                               "full_batch_ms": round(full_ms, 1),
                               "GBs": round(gpu_ce["grad_in_place"]["bytes"] / full_ms / 1e6, 2)}
    lp_or, _, _ = oracle.ce_rows(logits, tgt)
    err = float(np.abs(lp_or - lp_gpu).max())
    out["parity"] = {"max_abs_lp_gpu_minus_oracle": err, "tolerance": 1e-5,
                     "verdict": "pass" if err <= 1e-5 else "fail"}
    out["gpu_speedup_lp_loss"] = round(out["lp_loss_all_threads"]["full_batch_ms"]
                                       / gpu_ce["lp_loss"]["ms"], 1)
    return out


def cpu_recompute_leg(wl, host) -> dict:
    """The log-prob recompute on the oracle at the config's real context: one
    rollout's last CPU_RECOMPUTE_ROWS continuation positions (pos P + N - 1 -
    rows .. P + N - 2, attending over a full cache of P + N - 1 positions
    filled with synthetic K / V, the same work as the recompute's last rows),
    then the LM head and the log-softmax over those rows; at every core,
    median of 3. Scaled to one RL step's recompute of the policy (continuation
    rows) and of the frozen copy (prompt rows once per group + continuation
    rows) by token rows, the attention at the end-of-context cost (an upper
    bound for the earlier rows)."""
    import numpy as np

    import oracle

    c = host.cfg
    P, N, S = wl.prompt_len, wl.new_tokens, wl.rollouts
    cap = P + N - 1
    R = CPU_RECOMPUTE_ROWS
    pos0 = cap - R
    rng = np.random.default_rng(3)
    kc = (rng.standard_normal(c["layers"] * c["KVH"] * cap * c["hd"], dtype=np.float32)
          * np.float32(0.5))
    vc = (rng.standard_normal(kc.size, dtype=np.float32) * np.float32(0.5))
    ids = rng.integers(0, c["V"], R).astype(np.int32)
    n = oracle.set_threads(0)
    t_fwd, t_head = [], []
    for _ in range(3):
        t0 = time.perf_counter()
        x = host.forward_at(ids, pos0, kc, vc, cap)
        t1 = time.perf_counter()
        oracle.ce_rows(host.logits(x), ids)
        t2 = time.perf_counter()
        t_fwd.append(t1 - t0)
        t_head.append(t2 - t1)
    f_row, h_row = statistics.median(t_fwd) / R, statistics.median(t_head) / R
    layer_rows = wl.prompts * P + 2 * S * (N - 1)  # frozen copy's prompt pass + 2 continuations
    head_rows = 2 * S * N
    return {"threads": n, "sample": (f"1 rollout, positions {pos0}..{cap - 1} of {cap} "
                                     f"(full synthetic cache), {R} rows"),
            "forward_ms_per_row": round(f_row * 1e3, 2), "head_ce_ms_per_row": round(h_row * 1e3, 2),
            "rl_step_recompute_s_extrapolated": round(f_row * layer_rows + h_row * head_rows, 1),
            "rows_extrapolated": {"layer_rows": layer_rows, "head_rows": head_rows}}


def cpu_rl_leg(wl, host_weights) -> dict:
    """One config's RL step on the C oracle (the reference CPU path restated:
    fp32, batch 1 per rollout, generate.rs:68-124) on the GPU box's host
    cores, on a bounded sample: one rollout, a 64-token prompt prefilled
    untimed, then cached decode steps (rollout tok/s = 1 / time per step, the
    rate of the reference's per-rollout loop); warm-up, then the median of 5
    reps, at 1 thread and at every core. Plus the log-prob recompute at the
    config's real context (cpu_recompute_leg), the GRPO loss over the full
    [S, N] arrays, and the RL step extrapolated from those (S * N tokens at
    the all-core rollout rate, the recompute, the loss)."""
    import numpy as np

    import oracle
    from summa_amd.configs import ADVANTAGE_EPSILON, CLIP_EPSILON, KL_COEFFICIENT

    cfg = wl.model_config().oracle_cfg()
    host = oracle.HostModel(cfg, host_weights, quantized=wl.quantized)
    prompt = np.random.default_rng(0).integers(0, cfg["V"], 64).astype(np.int32)
    out = {}
    for label, threads in (("1_thread", 1), ("all_threads", 0)):
        n = oracle.set_threads(threads)
        per_rep = 1 if threads == 1 else 2
        stamps = []
        host.decode_steps(prompt, 1 + 5 * per_rep, wl.temperature, 0,
                          on_step=lambda i: stamps.append(time.perf_counter()))
        stamps.append(time.perf_counter())
        # stamps[i] .. stamps[i + 1] is decode step i; step 0 is the warm-up
        reps = [(stamps[1 + r * per_rep + per_rep] - stamps[1 + r * per_rep]) / per_rep
                for r in range(5)]
        med = statistics.median(reps)
        out[label] = {"threads": n, "s_per_token": round(med, 4),
                      "rollout_tok_s": round(1.0 / med, 4)}
    oracle.set_threads(0)
    log(f"bench: cpu recompute sample (config[{wl.index}])")
    out["recompute"] = cpu_recompute_leg(wl, host)
    del host
    # GRPO loss over the whole batch's [S, N] arrays (f64 oracle)
    rng = np.random.default_rng(1)
    sh = (wl.prompts, wl.group, wl.new_tokens)
    cur = rng.normal(-5, 1, sh)
    beh = cur + rng.normal(0, 1e-3, sh)
    t0 = time.perf_counter()
    for _ in range(5):
        oracle.grpo_loss(rng.random(sh[:2]), cur, beh, cur, None, CLIP_EPSILON,
                         ADVANTAGE_EPSILON, KL_COEFFICIENT)
    out["grpo_loss_ms"] = round((time.perf_counter() - t0) / 5 * 1e3, 3)
    rollout_s = wl.rollouts * wl.new_tokens / out["all_threads"]["rollout_tok_s"]
    out["rl_step_s_extrapolated"] = round(
        rollout_s + out["recompute"]["rl_step_recompute_s_extrapolated"]
        + out["grpo_loss_ms"] / 1e3, 1)
    out["sample"] = (f"config[{wl.index}] model, 1 rollout: 64-token prompt prefilled untimed, "
                     f"then median of 5 reps of cached decode steps (1 thread: 1 step per rep, "
                     f"all threads: 2); recompute: {CPU_RECOMPUTE_ROWS} rows at the end of a "
                     f"{wl.prompt_len + wl.new_tokens - 1}-position context; GRPO loss over the "
                     f"full {list(sh)} arrays; RL step = {wl.rollouts} x {wl.new_tokens} tokens "
                     f"at the all-core rate + recompute + loss")
    return out


def cpu_baseline_rl(wl, host_weights, c0=None, ce=None, others=None) -> dict:
    """The C oracle on the host cores (cpu_rl_leg) for the line's config, then
    config[3]'s CE on a row sample (cpu_ce_leg), config[0]'s full RL step with
    its oracle parity verdict, and cpu_rl_leg for the other configs whose
    weights the line kept (``others``: config index -> device weights)."""
    out = cpu_rl_leg(wl, host_weights)
    sample = out.pop("sample")
    res = {"value": out["all_threads"]["rollout_tok_s"], "unit": "rollout tok/s",
           "cores": out["all_threads"]["threads"], "kind": "port",
           "sample": sample + f"; config[3] CE over {CPU_CE_ROWS} of its rows",
           "cpu_model": _cpu_model(), "nproc": os.cpu_count(), **out}
    if ce is not None:
        log("bench: cpu CE sample (config[3])")
        res["ce_config3"] = cpu_ce_leg(*ce)
    if c0 is not None:
        res["config0"] = c0
    from summa_amd.configs import RL_WORKLOADS
    for idx, dw in (others or {}).items():
        log(f"bench: cpu baseline config[{idx}]")
        host_w = _model_host_weights(dw)
        res[f"config{idx}"] = cpu_rl_leg(RL_WORKLOADS[idx], host_w)
        del host_w
    return res


def cpu_config0(c0_gpu) -> dict:
    """config[0] on the oracle at every core: the full RL step's rollouts and
    recompute (median of 3), and the GPU's log-probs against it (1e-5)."""
    import numpy as np

    import oracle
    from summa_amd.configs import RL_WORKLOADS

    wl = RL_WORKLOADS[0]
    mc = wl.model_config()
    weights = _model_host_weights(c0_gpu["_weights"])
    host = oracle.HostModel(mc.oracle_cfg(), weights, quantized=False)
    prompts = c0_gpu["_prompts"].cpu().numpy()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        tok, _ = host.generate(prompts, wl.new_tokens, 0.0, 0)
        lp = host.logprobs(prompts, tok)
        times.append(time.perf_counter() - t0)
    out = c0_gpu["_out"]
    gtok = out["tokens"].cpu().numpy()
    lp_or = host.logprobs(prompts, gtok)
    err_cur = float(np.abs(out["lp_cur"].cpu().numpy() - lp_or).max())
    err_beh = float(np.abs(out["lp_beh"].cpu().numpy() - lp_or).max())
    same = float((gtok == tok).mean())
    return {"cpu_rl_step_ms": round(statistics.median(times) * 1e3, 1),
            "parity": {"max_abs_lp_recompute": err_cur, "max_abs_lp_behaviour": err_beh,
                       "tolerance": 1e-5, "greedy_tokens_equal": same,
                       "verdict": "pass" if max(err_cur, err_beh) <= 1e-5 else "fail"}}


def _model_host_weights(dev_weights: dict) -> dict:
    return {k: v.cpu().numpy() for k, v in dev_weights.items()}


def draw_weights(wl, models, dev, seed: int = 0) -> dict:
    """Seeded N(0, 0.02) weights drawn on the device and installed into every
    model of ``models``; returns the device tensors (for the CPU baseline)."""
    import torch

    from summa_amd import ops

    mc = wl.model_config()
    Lr, d = mc.layers, mc.d_model
    out = {"attn_norm": torch.ones(Lr, d, device=dev), "ffn_norm": torch.ones(Lr, d, device=dev),
           "final_norm": torch.ones(d, device=dev)}
    n = [0]

    def draw(shape, sd=0.02):
        t = torch.empty(shape, device=dev)
        n[0] += 1
        ops.fill_normal(t, 0.0, sd, seed=seed * 1000003 + n[0])
        return t

    out["embed"], out["lm_head"] = draw((mc.vocab, d)), draw((mc.vocab, d))
    shapes = dict(zip(("qkv", "o", "in", "down"), linear_shapes(wl.model)))
    if mc.experts:
        del shapes["in"], shapes["down"]
        shapes.update(exp_in=(mc.experts, 2 * mc.expert_ffn, d),
                      exp_down=(mc.experts, d, mc.expert_ffn), router=(mc.experts, d))
    for k, shp in shapes.items():
        out[k] = draw((Lr, *shp), 1.0 / d ** 0.5 if k == "router" else 0.02)
    per_layer = ("attn_norm", "ffn_norm", "qkv", "o", "in", "down", "router", "exp_in",
                 "exp_down")
    for m in models:
        for k, t in out.items():
            if k in per_layer:
                for layer in range(Lr):
                    m.set_tensor(k, t[layer], layer)
            else:
                m.set_tensor(k, t)
    torch.cuda.synchronize()
    return out


# ------------------------------------------------------------- workloads ---

def rl_step_leg(wl, dev, steps: int, warmup: int, seed: int = 0) -> dict:
    """One BASELINE RL config on the GPU: the policy and its frozen copy (same
    weights) with prompt groups and bound workspaces, W warm-up and K timed
    GRPO steps, each on its own prompts (so the frozen copy always runs its
    prompt pass, and the policy reuses only the prompt pass of the generation
    of the same step). Returns the step's figures, the phase split and the
    decode-vs-recompute check, plus private keys for the CPU baseline."""
    import torch

    from summa_amd.model import Model, batch_result

    mc = wl.model_config()
    policy, reference = Model(mc), Model(mc)
    dweights = draw_weights(wl, [policy, reference], dev, seed=seed)
    for m in (policy, reference):  # hot calls carve their buffers from a bound workspace
        m.set_prompt_groups(wl.group)  # each group's prompt computed once
        m.bind_workspace(wl.rollouts, wl.prompt_len, wl.new_tokens)
    batches = rl_inputs(wl, mc, dev, count=warmup + steps, seed=seed)
    S, N = wl.rollouts, wl.new_tokens
    log(f"bench: config[{wl.index}] warmup")
    roll, full, wall, out, (prompts, _) = run_rl_step(wl, policy, reference, batches, steps,
                                                      warmup, tag=f"config[{wl.index}]")
    res = batch_result(out)
    gap = (out["lp_beh"] - out["lp_cur"]).abs()
    lp_gap = float(gap.max())
    within = float((gap <= 2e-3).float().mean())
    r_ms, f_ms = sum(roll) / len(roll), sum(full) / len(full)
    pre_ms = prefill_ms(wl, policy, prompts)
    dec_ms = r_ms - pre_ms
    dec_bytes = decode_bytes(wl)
    # the frozen reference's full recompute (its prompt pass included: every
    # step brings new prompts) + the policy's without its prompt pass (the
    # generation of the same step computed it, sm_model_set_prompt_groups)
    rec_flops = recompute_flops(wl) + recompute_flops(wl, prompt_pass=False)
    prep_ms = f_ms - r_ms
    leg = {
        "rollout_tok_s": round(S * N / (r_ms * 1e-3), 1),
        "rl_step_ms": round(f_ms, 3), "rollout_ms": round(r_ms, 3), "prepare_ms": round(prep_ms, 3),
        "steps": steps, "warmup": warmup, "wall_s": round(wall, 3),
        "prompts_per_step": "distinct (new prompts every warm-up and timed step)",
        "grpo": {k: (round(v, 6) if isinstance(v, float) else v) for k, v in res.items()},
        # cached decode vs the recompute over the whole batch (2e-3 bar); for
        # MoE models a router near-tie can pick another expert pair in one
        # path, after which that rollout's tokens differ (tests resolve those
        # through traced router decisions)
        "check": {"max_abs_lp_behaviour_minus_recompute": lp_gap,
                  "fraction_of_tokens_within_2e-3": within},
        "phases": {
            "prefill_ms": round(pre_ms, 3),
            "decode": {"ms": round(dec_ms, 3), "steps": N - 1,
                       "us_per_step": round(dec_ms * 1e3 / (N - 1), 1),
                       "algorithmic_bytes": dec_bytes,
                       "floor_ms": round(dec_bytes / HBM_PEAK_GBS / 1e6, 3),
                       "hbm_frac": round(dec_bytes / HBM_PEAK_GBS / 1e6 / dec_ms, 4)},
            "recompute_and_loss": {"ms": round(prep_ms, 3), "algorithmic_flops": rec_flops,
                                   "TFLOPs": round(rec_flops / (prep_ms * 1e-3) / 1e12, 1),
                                   "mfma_frac": round(rec_flops / (prep_ms * 1e-3) / 1e12
                                                      / MFMA_F16_PEAK_TFS, 4)}},
        "_value": S * N / (r_ms * 1e-3), "_f_ms": f_ms, "_weights": dweights,
    }
    if wl.model.get("experts"):
        leg["check"]["note"] = ("MoE: a router near-tie can flip a token's expert pair between "
                                "the decode and recompute paths; the GPU tests resolve each flip "
                                "through the traced router decisions")
    policy.close()
    reference.close()
    del policy, reference
    torch.cuda.empty_cache()
    return leg


def bench_rl_step(args) -> dict:
    import torch

    from summa_amd.configs import CE_STRESS, RL_WORKLOADS

    wl = RL_WORKLOADS[args.config]
    dev = torch.device("cuda:0")
    leg = rl_step_leg(wl, dev, args.steps, args.warmup)
    dweights = leg.pop("_weights")
    line = {
        "metric": "rollout tok/s + RL step ms on 1 MI355X; % HBM roofline of 4-bit GEMV",
        "value": leg.pop("_value"), "unit": "rollout tok/s", "ms_per_step": leg.pop("_f_ms"),
        "dtype": ("q4g128 weights, f16-pair (fp32-grade) matmul inputs, f16 KV, f32 accumulate"
                  if wl.quantized else "f32"),
        "config": {"workload": f"rl_step config[{wl.index}]", **wl.model, "prompts": wl.prompts,
                   "group": wl.group, "prompt_len": wl.prompt_len, "new_tokens": wl.new_tokens,
                   "temperature": wl.temperature,
                   "weights": "Q4G128 (bf16 scales)" if wl.quantized else "f32",
                   "rewards": wl.reward_label()},
    }
    for k in ("steps", "warmup", "rollout_tok_s"):
        leg.pop(k)
    line.update(leg)
    if args.leg_only:  # the chosen config's RL step alone (per-config kernel profiles)
        return line
    # the other quantized configs' RL steps (a few steps each: they run the
    # same kernels at other shapes)
    others = {}
    for idx in (1, 2, 4):
        if idx == args.config or args.config == 0:
            continue
        log(f"bench: config[{idx}]")
        sub = rl_step_leg(RL_WORKLOADS[idx], dev, steps=3, warmup=1, seed=idx)
        others[idx] = sub.pop("_weights")  # for its CPU baseline leg
        for k in ("_value", "_f_ms"):
            sub.pop(k)
        line[f"config{idx}"] = sub
    log("bench: dominant kernel (recompute FFN-in GEMM)")
    k = recompute_gemm(RL_WORKLOADS[2], dev)
    line["roofline"] = {"bound": "mfma", "kernel": k["kernel"], "shape": k["shape"],
                        "achieved": k["TFLOPs"], "peak": MFMA_F16_PEAK_TFS, "unit": "TFLOP/s",
                        "frac": k["frac"], "us": k["us"],
                        "traffic": profile_figure("recompute_gemm_ffn_in_traffic.md",
                                                  "traffic_bytes_per_launch")}
    log("bench: q4 gemv sweep (config[2] weights, M = 1..16, graph replay)")
    sweep = q4_gemv_sweep(RL_WORKLOADS[2].model, dev)
    sweep["lm_head_traffic"] = profile_figure("q4_gemv_lm_head_traffic.md",
                                              "traffic_bytes_per_launch")
    line["q4_gemv"] = sweep
    log("bench: fused CE (config[3])")
    ce = ce_stress(dev, CE_STRESS["rows"], host_sample=CPU_CE_ROWS)
    ce_sample = ce.pop("_sample")
    line["ce_config3"] = ce
    log("bench: config[0]")
    c0 = config0_leg(dev)
    line["config0"] = {k: v for k, v in c0.items() if not k.startswith("_")}
    line["_cpu"] = (dweights, c0, ce_sample, ce, others)
    return line


def bench_ce_stress(args) -> dict:
    import torch

    from summa_amd.configs import CE_STRESS
    dev = torch.device("cuda:0")
    r = ce_stress(dev, args.rows, reps=max(args.steps, 1))
    # calibration copy for the counter runs (256 MiB read + 256 MiB written)
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev)
    torch.empty_like(src).copy_(src)
    torch.cuda.synchronize()
    gbs = r["grad_in_place"]["GBs"]
    return {"metric": "fused CE grad-in-place GB/s (config[3] bf16 65536x131072)",
            "value": gbs, "unit": "GB/s", "ms_per_step": r["grad_in_place"]["ms"],
            "dtype": "bf16", "config": {"workload": "ce_stress", **CE_STRESS},
            "roofline": {"bound": "hbm", "kernel": "ce_grad (lp + loss + grad in place)",
                         "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": r["grad_in_place"]["frac"],
                         "traffic": profile_figure("ce_config3_traffic.md",
                                                   "traffic_bytes_per_launch")},
            "ce_config3": r}


def bench_q4_gemv(args) -> dict:
    import torch

    from summa_amd.configs import RL_WORKLOADS
    dev = torch.device("cuda:0")
    sweep = q4_gemv_sweep(RL_WORKLOADS[2].model, dev, reps=max(args.steps, 1) * 10)
    achieved = sweep["lm_head_GBs"]
    # a plain device copy of known size (256 MiB read + 256 MiB written): the
    # calibration dispatch for the HBM byte counters of a rocprofv3 --pmc run
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev)
    torch.empty_like(src).copy_(src)
    torch.cuda.synchronize()
    return {"metric": "4-bit GEMV GB/s (config[2] LM head, M=1)", "value": achieved,
            "unit": "GB/s", "ms_per_step": sweep["by_M"]["1"]["sweep_ms"],
            "dtype": "q4g128 weights, f16 x, f32 accumulate",
            "config": {"workload": "q4_gemv config[2]",
                       "lm_head": [RL_WORKLOADS[2].model["vocab"],
                                   RL_WORKLOADS[2].model["d_model"]]},
            "roofline": {"bound": "hbm", "kernel": "q4g128 GEMV M=1 (LM head 65536x2048)",
                         "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved / HBM_PEAK_GBS, 4),
                         "traffic": profile_figure("q4_gemv_lm_head_traffic.md",
                                                   "traffic_bytes_per_launch")},
            "q4_gemv": sweep}


def bench_recompute_gemm(args) -> dict:
    import torch

    from summa_amd.configs import RL_WORKLOADS
    dev = torch.device("cuda:0")
    k = recompute_gemm(RL_WORKLOADS[2], dev, reps=max(args.steps, 1))
    # calibration copy for the counter runs (256 MiB read + 256 MiB written)
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev)
    torch.empty_like(src).copy_(src)
    torch.cuda.synchronize()
    return {"metric": "recompute FFN-in GEMM TFLOP/s (config[2])", "value": k["TFLOPs"],
            "unit": "TFLOP/s", "ms_per_step": k["us"] / 1e3, "dtype": "q4g128 x f16 pairs",
            "config": {"workload": "recompute_gemm config[2]", "shape": k["shape"]},
            "roofline": {"bound": "mfma", "kernel": k["kernel"], "achieved": k["TFLOPs"],
                         "peak": MFMA_F16_PEAK_TFS, "unit": "TFLOP/s", "frac": k["frac"],
                         "traffic": profile_figure("recompute_gemm_ffn_in_traffic.md",
                                                   "traffic_bytes_per_launch")}}


def bench_decode_attention(args) -> dict:
    """Decode attention at the config[2] decode shape (256 rollouts in 32
    prompt groups of 8, 512-token prompt, 16 query / 4 KV heads, head dim
    128, f16 K/V cache of capacity 1023, f16-pair queries and output) at
    positions t = 1, 256, 511 after the prompt: the per-rollout kernel
    (sm_attn_decode, every rollout reads its own prompt K/V) against the
    shared-prompt path (sm_attn_decode_prefix: the prompt K/V once per
    group, then each rollout's t continuation keys). Algorithmic bytes:
    per-rollout 256 x 4 x (512 + t) x 128 x 2 B x 2 + queries + output;
    shared prompt 32 x 4 x 512 x 128 x 2 B x 2 + 256 x 4 x t x 128 x 2 B x 2
    + queries + output + the prompt partials written and read once."""
    import torch

    from summa_amd import _lib
    from summa_amd._lib import SM_F16, SM_F16X2, call
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream()
    S, G, P, H, KVH, hd, cap = 256, 8, 512, 16, 4, 128, 1023
    gen = torch.Generator(device=dev).manual_seed(0)
    rnd = lambda *sh: torch.randn(*sh, generator=gen, device=dev).half()  # noqa: E731
    q, kc, vc = rnd(S, H, hd), rnd(S, KVH, cap, hd), rnd(S, KVH, cap, hd)
    pk, pv = rnd(S // G, KVH, P, hd), rnd(S // G, KVH, P, hd)
    out = torch.empty(S, 2 * H * hd, dtype=torch.float16, device=dev)
    nws = int(_lib.lib().sm_attn_decode_prefix_workspace_bytes(S, G, P, H, KVH, hd))
    ws = torch.empty(nws // 4, device=dev)
    qo = S * H * hd * 4 + S * 2 * H * hd * 2           # f16-pair queries + output
    res = {}
    for t in (1, 256, 511):
        lens = torch.full((S,), P + t, dtype=torch.int32, device=dev)
        full = _time_launches(lambda: call(
            "sm_attn_decode", q.data_ptr(), kc.data_ptr(), vc.data_ptr(), lens.data_ptr(),
            out.data_ptr(), SM_F16, SM_F16X2, S, H, KVH, cap, hd, st.cuda_stream),
            max(args.steps, 1))
        pre = _time_launches(lambda: call(
            "sm_attn_decode_prefix", q.data_ptr(), pk.data_ptr(), pv.data_ptr(), kc.data_ptr(),
            vc.data_ptr(), lens.data_ptr(), out.data_ptr(), ws.data_ptr(), nws, SM_F16,
            SM_F16X2, S, G, P, H, KVH, cap, hd, st.cuda_stream), max(args.steps, 1))
        b_full = S * KVH * (P + t) * hd * 4 + qo
        b_pre = (S // G) * KVH * P * hd * 4 + S * KVH * t * hd * 4 + qo + 2 * nws
        res[str(t)] = {"per_rollout_us": round(full * 1e3, 2), "shared_prompt_us": round(pre * 1e3, 2),
                       "per_rollout_GBs": round(b_full / full / 1e6, 1),
                       "shared_prompt_GBs": round(b_pre / pre / 1e6, 1),
                       "speedup": round(full / pre, 3)}
    # calibration copy for the counter runs (256 MiB read + 256 MiB written)
    src = torch.empty(64 << 20, dtype=torch.float32, device=dev)
    torch.empty_like(src).copy_(src)
    torch.cuda.synchronize()
    top = res["511"]
    return {"metric": "decode attention speedup of the shared prompt (config[2] shape, t=511)",
            "value": top["speedup"], "unit": "x", "ms_per_step": top["shared_prompt_us"] / 1e3,
            "dtype": "f16 K/V, f16-pair q/out, f32 softmax",
            "config": {"workload": "decode_attention config[2]", "rollouts": S, "group": G,
                       "prompt_len": P, "heads": H, "kv_heads": KVH, "head_dim": hd},
            "roofline": {"bound": "hbm", "kernel": "sm_attn_decode_prefix at t=511",
                         "achieved": top["shared_prompt_GBs"], "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(top["shared_prompt_GBs"] / HBM_PEAK_GBS, 4),
                         "traffic": profile_figure("decode_attention_shared_prompt_traffic.md",
                                                   "traffic_bytes_per_launch")},
            "by_t": res}


def bench_policy_update(args) -> dict:
    """The GRPO policy update at config[2] scale (``--config 4``: the MoE
    config[4]) (sm_policy_prepare + sm_policy_optimizer_step): one group of 8
    rollouts x (prompt + new tokens) per call, recompute with activations kept,
    the frozen reference's log-probs, the loss and the whole backward into f32
    master gradients, then AdamW with the global-norm clip. The rollouts come
    from the installed Q4 model."""
    import torch

    from summa_amd import train
    from summa_amd.configs import RL_WORKLOADS
    from summa_amd.model import Model
    cfg_id = 4 if args.config == 4 else 2
    wl = RL_WORKLOADS[cfg_id]
    mc = wl.model_config()
    dev = torch.device("cuda:0")
    d, F, V, Ly = mc.d_model, mc.ffn, mc.vocab, mc.layers
    E, Fe = mc.experts, mc.expert_ffn
    qn = (mc.heads + 2 * mc.kv_heads) * mc.head_dim
    gen = torch.Generator(device=dev).manual_seed(0)
    nrm = lambda *sh: torch.randn(*sh, generator=gen, device=dev) * 0.02  # noqa: E731
    w = {"embed": nrm(V, d), "lm_head": nrm(V, d), "final_norm": torch.ones(d, device=dev),
         "attn_norm": torch.ones(Ly, d, device=dev), "ffn_norm": torch.ones(Ly, d, device=dev),
         "qkv": nrm(Ly, qn, d), "o": nrm(Ly, d, mc.heads * mc.head_dim)}
    if E:  # router logits ~ N(0, 1) (the configs' router init), stacked experts
        w.update(router=torch.randn(Ly, E, d, generator=gen, device=dev) / d ** 0.5,
                 exp_in=nrm(Ly, E, 2 * Fe, d), exp_down=nrm(Ly, E, d, Fe))
        ffn_params = E * (3 * Fe * d + d)
    else:
        w.update({"in": nrm(Ly, 2 * F, d), "down": nrm(Ly, d, F)})
        ffn_params = 3 * F * d
    pol = train.Policy(mc, w, dev)
    del w
    ref = Model(mc)
    pol.install(ref)
    G, P, N = wl.group, wl.prompt_len, wl.new_tokens
    # one GRPO group: G rollouts of one prompt
    prompts = torch.randint(0, V, (1, P), dtype=torch.int32, device=dev).repeat(G, 1)
    tok, beh = ref.generate(prompts, N, temperature=wl.temperature, seed=1)
    rewards = torch.rand(1, G, device=dev)
    st = torch.cuda.current_stream()
    e0, e1, e2 = _events(3)
    by_planes, lp_gap = {}, None
    # the f32-grade three-plane GEMMs (the headline), then 16-bit and bf16
    # operands (the reference's CUDA-path matmul precision)
    for planes in ((args.planes,) if args.planes else (3, 2, 1)):
        pol.set_matmul_planes(planes)
        prep, step = [], []
        for i in range(args.warmup + args.steps):
            e0.record(st)
            out = pol.prepare(ref, prompts, tok, beh, rewards)
            e1.record(st)
            pol.optimizer_step(1.0)
            e2.record(st)
            torch.cuda.synchronize()
            if lp_gap is None:  # the policy still equals the model that rolled out
                lp_gap = float((out["lp_cur"] - beh).abs().max())
            if i >= args.warmup:
                prep.append(e0.elapsed_time(e1))
                step.append(e1.elapsed_time(e2))
            log(f"bench: policy update planes={planes} {i}: prepare {e0.elapsed_time(e1):.1f} ms, "
                f"optimizer step {e1.elapsed_time(e2):.1f} ms")
        # the same prepare with the frozen model's log-probs given (as the RL
        # step's recompute returns them), so the update does not run it again
        ref_lp = out["lp_ref"].clone()
        prep_g = []
        for i in range(args.warmup + args.steps):
            e0.record(st)
            pol.prepare(None, prompts, tok, beh, rewards, reference_lp=ref_lp)
            e1.record(st)
            pol.optimizer_step(1.0)
            torch.cuda.synchronize()
            if i >= args.warmup:
                prep_g.append(e0.elapsed_time(e1))
        by_planes[str(planes)] = {"prepare_ms": round(sum(prep) / len(prep), 2),
                                  "optimizer_step_ms": round(sum(step) / len(step), 2),
                                  "prepare_given_reference_lp_ms":
                                      round(sum(prep_g) / len(prep_g), 2)}
    head = str(args.planes or 3)
    p_ms, s_ms = by_planes[head]["prepare_ms"], by_planes[head]["optimizer_step_ms"]
    positions = G * (P + N - 1)
    return {"metric": f"GRPO policy update positions/s (config[{cfg_id}], one group per call)",
            "value": positions / ((p_ms + s_ms) / 1e3), "unit": "positions/s",
            "ms_per_step": p_ms + s_ms,
            "dtype": (f"f32 masters, Q4G128 fake-quantized forward, {head}-plane bf16 GEMMs"),
            "config": {"workload": f"policy_update config[{cfg_id}]", "rollouts": G,
                       "prompt_len": P, "new_tokens": N},
            "prepare_ms": round(p_ms, 2), "optimizer_step_ms": round(s_ms, 2),
            "by_matmul_planes": by_planes,
            "parameters": int(Ly * (qn * d + d * mc.heads * mc.head_dim + ffn_params + 2 * d)
                              + 2 * V * d + d),
            "first_prepare_lp_vs_rollout_max_abs": lp_gap}


def bench_decode_gemms(args) -> dict:
    """config[2]'s decode projections at the decode shape (M 256 rollouts, f16-
    pair activations, synthetic Q4G128 weights), each launched 10 times (the
    launches the committed counter summaries of the decode GEMMs profile):
    FFN-in (2 x 5632 columns, SwiGLU f16-pair epilogue), a 3072-column store of
    the qkv shape, and o (2048 x 2048) and down (2048 x 5632) through the fused
    residual + RMSNorm path (sm_q4_matmul_add_rmsnorm). Value: the FFN-in's
    event-timed average per call."""
    import ctypes

    import torch

    from summa_amd import _lib, ops
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream()
    M = 256
    L = _lib.lib()

    def q4(n, k, seed):
        w = torch.empty(n, k, device=dev)
        ops.fill_normal(w, 0, 0.02, seed=seed)
        return ops.Q4Weight.quantize(w)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)
    x = torch.empty(M, 2048, device=dev)
    ops.fill_normal(x, 0, 1, seed=2)
    xp = ops.f16_pair(x)
    xf = torch.empty(M, 5632, device=dev)
    ops.fill_normal(xf, 0, 1, seed=3)
    xfp = ops.f16_pair(xf)
    w_in, w_qkv = q4(11264, 2048, 1), q4(3072, 2048, 4)
    w_o, w_dn = q4(2048, 2048, 5), q4(2048, 5632, 6)
    resid = torch.zeros(M, 2048, device=dev)
    gamma = torch.ones(2048, device=dev)
    h = torch.empty(M, 4096, dtype=torch.float16, device=dev)

    def addnorm(w, xx, K):
        _lib.check(L.sm_q4_matmul_add_rmsnorm(
            w.tcodes.data_ptr(), w.tscales.data_ptr(), 2048, K, xx.data_ptr(), _lib.SM_F16X2, M,
            2 * K, resid.data_ptr(), gamma.data_ptr(), ctypes.c_float(1e-5), h.data_ptr(),
            ws.data_ptr(), ws.numel(), ctypes.c_void_p(st.cuda_stream)))
    calls = {
        "ffn_in": lambda: ops.q4_matmul(w_in, xp, epilogue=_lib.SM_EPI_SWIGLU_F16X2, pair=True,
                                        workspace=ws),
        "qkv_shape": lambda: ops.q4_matmul(w_qkv, xp, pair=True, workspace=ws),
        "o_add_rmsnorm": lambda: addnorm(w_o, xp, 2048),
        "down_add_rmsnorm": lambda: addnorm(w_dn, xfp, 5632)}
    res = {}
    for name, fn in calls.items():
        res[name] = round(_time_launches(fn, 10) * 1e3, 2)
    return {"metric": "decode FFN-in us per call (config[2] decode shape, M 256)",
            "value": res["ffn_in"], "unit": "us", "higher_is_better": False,
            "ms_per_step": res["ffn_in"] / 1e3, "dtype": "q4g128 weights, f16-pair activations",
            "config": {"workload": "decode_gemms config[2]", "M": M},
            "us_per_call": res}


def bench_policy_gemms(args) -> dict:
    """The policy update's largest GEMM shapes at config[2] (one GRPO group:
    8 x 1023 positions, d 2048, F 5632, V 65536; the last group's 4096 scored
    rows for the LM head) through sm_gemm_planes_ws as the prepare runs them
    (operands whose k is not contiguous transposed into the scratch first,
    transposes inside the timing; the forward and data-gradient shapes with a
    fake-quantized B, exact in two bf16 planes, as in the quantized prepare),
    for 3, 2 and 1 bf16 planes. Per shape: the
    event-timed average of 5 calls, algorithmic f32 TF/s (2 M N K) and the
    fraction of the 2.5 PF/s bf16 MFMA peak in issued plane products (6, 3 or
    1 per f32 product; 5 at three planes with a two-plane B). Value: the
    smallest three-plane fraction among the
    backward (weight and data gradient) shapes."""
    import ctypes

    import torch

    from summa_amd import _lib
    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream()
    L = _lib.lib()
    M, d, F, V, R = 8 * 1023, 2048, 5632, 65536, 4096
    shapes = {  # name: (trans_a, trans_b, M, N, K)
        "fwd_ffn_in": (0, 1, M, 2 * F, d), "dW_ffn_in": (1, 0, 2 * F, d, M),
        "dX_ffn_in": (0, 0, M, d, 2 * F), "fwd_down": (0, 1, M, d, F),
        "dW_down": (1, 0, d, F, M), "dX_down": (0, 0, M, F, d),
        "dW_o": (1, 0, d, d, M), "dX_o": (0, 0, M, d, d),
        "fwd_lm_head": (0, 1, R, V, d), "dW_lm_head": (1, 0, V, d, R),
        "dX_lm_head": (0, 0, R, d, V)}
    need = max(int(L.sm_gemm_planes_scratch_bytes(ta, tb, m, n, k))
               for ta, tb, m, n, k in shapes.values())
    scratch = torch.empty(max(need, 16) // 4, device=dev)
    products = {3: 6, 2: 3, 1: 1}  # per f32 product (three planes with a two-plane B: 5)
    res = {}
    for planes in (3, 2, 1):
        res[str(planes)] = {}
        for name, (ta, tb, m, n, k) in shapes.items():
            a = torch.randn((k, m) if ta else (m, k), device=dev)
            b = torch.randn((n, k) if tb else (k, n), device=dev)
            c = torch.empty(m, n, device=dev)

            # forward and data gradients multiply by the fake-quantized weight
            # (B; exact in two bf16 planes), as the quantized policy's prepare does
            bp = 0 if name.startswith("dW") else 2
            if bp == 2:
                b = (torch.randint(-7, 8, b.shape, device=dev).float() * (1.0 / 128)).contiguous()

            def call():
                _lib.check(L.sm_gemm_planes_ws(
                    planes, bp, ta, tb, m, n, k, ctypes.c_float(1.0), a.data_ptr(), a.stride(0),
                    b.data_ptr(), b.stride(0), ctypes.c_float(0.0), c.data_ptr(), n,
                    scratch.data_ptr(), scratch.numel() * 4, ctypes.c_void_p(st.cuda_stream)))
            sec = _time_launches(call, 5) / 1e3
            tf = 2.0 * m * n * k / sec / 1e12
            npr = 5 if (planes == 3 and bp == 2) else products[planes]
            res[str(planes)][name] = {"us": round(sec * 1e6, 1), "f32_TFs": round(tf, 1),
                                      "mfma_frac": round(tf * npr / 2500.0, 3)}
            log(f"bench: policy GEMM planes={planes} {name}: {sec * 1e6:.1f} us, "
                f"{tf:.1f} TF/s, MFMA {tf * npr / 2500.0:.3f}")
            del a, b, c
    worst = min(v["mfma_frac"] for k_, v in res["3"].items() if not k_.startswith("fwd"))
    return {"metric": "policy-update backward GEMM MFMA fraction (config[2] shapes, 3 planes, min)",
            "value": worst, "unit": "fraction of 2.5 PF/s", "higher_is_better": True,
            "ms_per_step": sum(v["us"] for v in res["3"].values()) / 1e3,
            "dtype": "f32 via bf16 planes",
            "config": {"workload": "policy_gemms config[2]", "positions": M},
            "by_planes": res}


WORKLOADS = {"rl_step": bench_rl_step, "ce_stress": bench_ce_stress, "q4_gemv": bench_q4_gemv,
             "recompute_gemm": bench_recompute_gemm, "policy_update": bench_policy_update,
             "decode_attention": bench_decode_attention, "decode_gemms": bench_decode_gemms,
             "policy_gemms": bench_policy_gemms}


def main() -> int:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--workload", default="rl_step", choices=sorted(WORKLOADS))
    p.add_argument("--rows", type=int, default=65536)
    p.add_argument("--config", type=int, default=2, choices=[0, 1, 2, 4],
                   help="rl_step: BASELINE config index (2 = the headline line)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--planes", type=int, default=0, choices=[0, 1, 2, 3],
                   help="policy_update: only this matmul plane count (0: 3, 2 and 1)")
    p.add_argument("--leg-only", action="store_true",
                   help="rl_step: only the --config leg (no other configs, dominant-kernel, "
                        "GEMV, CE or CPU legs), for per-config kernel profiles")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the RL step is "
              "sharded by whole GRPO groups across GPUs, which this build does not run.",
              file=sys.stderr)
        return 2
    log(f"bench: workload={args.workload} steps={args.steps} warmup={args.warmup}")
    res = WORKLOADS[args.workload](args)
    cpu = res.pop("_cpu", None)
    out = {"metric": res.pop("metric"), "value": round(res.pop("value"), 3), "unit": res.pop("unit"),
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(res.pop("ms_per_step"), 4), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": res.pop("dtype"), "data": "synthetic",
           "config": res.pop("config")}
    out.update(res)
    if not args.no_cpu_baseline and cpu is not None:
        log("bench: cpu baseline (oracle on the host cores)")
        from summa_amd.configs import RL_WORKLOADS
        dweights, c0, ce_sample, ce, others = cpu
        host_w = _model_host_weights(dweights)
        del dweights
        out["cpu_baseline"] = cpu_baseline_rl(RL_WORKLOADS[args.config], host_w, cpu_config0(c0),
                                              (ce_sample, ce), others)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
