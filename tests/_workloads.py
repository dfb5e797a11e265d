"""Shared helpers for the GPU tests that run the BASELINE configs at size.

Weights are drawn on the device (``sm_fill_normal``, a pure function of seed
and index), installed into the device model(s) and copied to the host for the
CPU oracle: drawing 1.3 G normals with numpy would take minutes.
"""
from __future__ import annotations

import numpy as np
import torch

from summa_amd import ops
from summa_amd.model import Model


def _shapes(mc):
    d, H, KVH, hd, F, V = mc.d_model, mc.heads, mc.kv_heads, mc.head_dim, mc.ffn, mc.vocab
    qn = H * hd + 2 * KVH * hd
    lin = {"qkv": (qn, d), "o": (d, H * hd)}
    if mc.experts:
        lin.update(exp_in=(mc.experts, 2 * mc.expert_ffn, d),
                   exp_down=(mc.experts, d, mc.expert_ffn))
    else:
        lin.update({"in": (2 * F, d), "down": (d, F)})
    return lin


def device_weights(mc, models, seed: int, dev, std: float = 0.02) -> dict:
    """N(0, std) linears and embedding, unit norms, router ~ N(0, 1/sqrt(d))
    (the configs' synthetic init, as ``oracle.random_weights``), installed into
    every model of ``models``; returns the host copies in the oracle's dict
    layout ([layers, ...] per-layer tensors, linears [out, in])."""
    Lr, d = mc.layers, mc.d_model
    host = {"attn_norm": np.ones((Lr, d), np.float32), "ffn_norm": np.ones((Lr, d), np.float32),
            "final_norm": np.ones(d, np.float32)}
    counter = [0]

    def draw(shape, sd):
        t = torch.empty(shape, dtype=torch.float32, device=dev)
        counter[0] += 1
        ops.fill_normal(t, 0.0, sd, seed=seed * 1000003 + counter[0])
        return t

    for name, shape, sd in (("embed", (mc.vocab, d), std), ("lm_head", (mc.vocab, d), std)):
        t = draw(shape, sd)
        for m in models:
            m.set_tensor(name, t)
        host[name] = t.cpu().numpy()
    for name in ("attn_norm", "ffn_norm"):
        for layer in range(Lr):
            t = torch.from_numpy(host[name][layer]).to(dev)
            for m in models:
                m.set_tensor(name, t, layer)
    t = torch.from_numpy(host["final_norm"]).to(dev)
    for m in models:
        m.set_tensor("final_norm", t)
    shapes = _shapes(mc)
    if mc.experts:
        shapes["router"] = (mc.experts, d)
    for name, shape in shapes.items():
        arr = np.empty((Lr, *shape), np.float32)
        sd = 1.0 / np.sqrt(d) if name == "router" else std
        for layer in range(Lr):
            t = draw(shape, sd)
            for m in models:
                m.set_tensor(name, t, layer)
            arr[layer] = t.cpu().numpy()
        host[name] = arr
    torch.cuda.synchronize()
    return host


def build_models(wl, dev, seed: int = 0, count: int = 2):
    """``count`` device models of workload ``wl`` holding identical weights
    (policy and its frozen copy), plus the host weights."""
    mc = wl.model_config()
    models = [Model(mc) for _ in range(count)]
    host = device_weights(mc, models, seed, dev)
    return mc, models, host


def mix64(z):
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xbf58476d1ce4e5b9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94d049bb133111eb)
    return z ^ (z >> np.uint64(31))


def gumbel(seed, row, step, V):
    """Gumbel noise of the device's counter sampler for (seed, row, step)."""
    with np.errstate(over="ignore"):
        a = mix64(np.uint64(seed) + np.uint64(0x9e3779b97f4a7c15) * np.uint64(row + 1))
        cnt = np.uint64(step) * np.uint64(V) + np.arange(V, dtype=np.uint64)
        k = mix64(a ^ (cnt * np.uint64(0xd1b54a32d192ed03)))
    u = ((k >> np.uint64(40)).astype(np.float32) + np.float32(0.5)) * np.float32(1.0 / 16777216.0)
    with np.errstate(divide="ignore"):  # u rounds to 1 for the top counter value: key +inf
        return -np.log(-np.log(u.astype(np.float64)))


def check_sampled_tokens(tokens, logits, temperature, seed, rows, tol):
    """Every sampled token against the sampler's decision on the oracle's
    logits (teacher-forced on the device's own prefix): tokens[i, n] must be
    argmax(logits[i, n] / T + gumbel(seed, rows[i], n)) (greedy: argmax of the
    logits), or within ``tol`` of it (a near-tie). Returns the near-tie count."""
    ties = 0
    S, N, V = logits.shape
    for i in range(S):
        for n in range(N):
            lg = logits[i, n].astype(np.float64)
            key = lg / temperature + gumbel(seed, rows[i], n, V) if temperature > 0 else lg
            a, b = int(tokens[i, n]), int(np.argmax(key))
            if a != b:
                gap = key[b] - key[a]
                assert gap < tol, (f"rollout {rows[i]} step {n}: token {a} vs oracle {b}, "
                                   f"key gap {gap:.3e} is not a near-tie")
                ties += 1
    return ties
