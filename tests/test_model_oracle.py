"""Pins the oracle decoder (oracle/model.c) on the CPU.

Checks: an independent numpy forward (f64) of the same architecture,
cached-decode == stateless-forward (the reference invariant of
summa-llm/src/model/mod.rs:143-179, 1e-5), GQA head mapping against an
equivalent MHA model, the generation goldens of generate.rs:256-295 that apply
without a repetition penalty, and the seeded Gumbel sampler's distribution.
"""
import numpy as np
import pytest

import oracle

TINY = {"layers": 2, "d": 64, "H": 4, "KVH": 2, "hd": 16, "F": 96, "V": 50}


def _np_forward(cfg, w, ids):
    """Independent f64 numpy forward: logits [S, L, V]."""
    Lr, d, H, KVH, hd, F = (cfg[k] for k in ("layers", "d", "H", "KVH", "hd", "F"))
    S, L = ids.shape
    x = w["embed"][ids].astype(np.float64)
    pos = np.arange(L)
    freq = 1e4 ** (-2.0 * np.arange(hd // 2) / hd)
    ang = pos[:, None] * freq[None]
    cos, sin = np.cos(ang), np.sin(ang)

    def rope(t):  # [S, L, heads, hd], adjacent pairs
        a, b = t[..., 0::2], t[..., 1::2]
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        out = np.empty_like(t)
        out[..., 0::2] = a * c - b * s
        out[..., 1::2] = b * c + a * s
        return out

    def norm(v, g):
        return v / np.sqrt((v ** 2).mean(-1, keepdims=True) + 1e-5) * g

    mask = np.triu(np.ones((L, L), bool), 1)
    for l in range(Lr):
        h = norm(x, w["attn_norm"][l])
        qkv = h @ w["qkv"][l].T.astype(np.float64)
        q = rope(qkv[..., :H * hd].reshape(S, L, H, hd))
        k = rope(qkv[..., H * hd:(H + KVH) * hd].reshape(S, L, KVH, hd))
        v = qkv[..., (H + KVH) * hd:].reshape(S, L, KVH, hd)
        k = np.repeat(k, H // KVH, axis=2)
        v = np.repeat(v, H // KVH, axis=2)
        sc = np.einsum("slhd,sthd->shlt", q, k) / np.sqrt(hd)
        sc[:, :, mask] = -np.inf
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        att = np.einsum("shlt,sthd->slhd", p, v).reshape(S, L, H * hd)
        x = x + att @ w["o"][l].T
        h = norm(x, w["ffn_norm"][l])
        if cfg.get("E"):
            x = x + _np_moe(cfg, w, l, h)
            continue
        gv = h @ w["in"][l].T
        g, val = gv[..., :F], gv[..., F:]
        x = x + (g / (1 + np.exp(-g)) * val) @ w["down"][l].T
    return norm(x, w["final_norm"]) @ w["lm_head"].T


def _np_moe(cfg, w, l, h):
    """Top-2 MoE of SparseMoe::forward (ffn.rs:478-711) in f64: general CPU
    top-k (stable argsort: on equal logits the lower expert index ranks first,
    as the strict '>' scan of moe_topk.rs:74-104), softmax over the pair."""
    Fe = cfg["Fe"]
    lead = h.shape[:-1]
    h2 = h.reshape(-1, h.shape[-1])
    logits = h2 @ w["router"][l].T.astype(np.float64)
    top = np.argsort(-logits, axis=1, kind="stable")[:, :2]
    sel = np.take_along_axis(logits, top, 1)
    wts = np.exp(sel - sel[:, :1])
    wts /= wts.sum(1, keepdims=True)
    out = np.zeros_like(h2)
    for t in range(h2.shape[0]):
        for j in range(2):
            e = top[t, j]
            gv = w["exp_in"][l, e].astype(np.float64) @ h2[t]
            u = gv[:Fe] / (1 + np.exp(-gv[:Fe])) * gv[Fe:]
            out[t] += wts[t, j] * (w["exp_down"][l, e].astype(np.float64) @ u)
    return out.reshape(*lead, -1)


def test_forward_matches_independent_numpy():
    w = oracle.random_weights(TINY, seed=1, std=0.2)
    w["attn_norm"] = np.random.default_rng(2).uniform(0.5, 1.5, w["attn_norm"].shape).astype(np.float32)
    m = oracle.HostModel(TINY, w, quantized=False)
    ids = np.random.default_rng(3).integers(0, TINY["V"], (2, 11)).astype(np.int32)
    got = m.forward_logits(ids)
    ref = _np_forward(TINY, w, ids)
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-5)


TINY_MOE = dict(TINY, E=6, Fe=48)


def test_moe_forward_matches_independent_numpy():
    w = oracle.random_weights(TINY_MOE, seed=11, std=0.2)
    m = oracle.HostModel(TINY_MOE, w, quantized=False)
    ids = np.random.default_rng(12).integers(0, TINY["V"], (2, 9)).astype(np.int32)
    gaps = m.router_gaps(ids)
    assert gaps.min() > 1e-3  # no top-2 near-tie, so f32 vs f64 picks the same experts
    np.testing.assert_allclose(m.forward_logits(ids), _np_forward(TINY_MOE, w, ids),
                               rtol=1e-4, atol=1e-5)


def test_moe_router_ties_pick_lowest_index():
    # Router rows built so logits tie exactly: e0 = 3z, e1 = e4 = z, others -z
    # with z = h.r. For z > 0 experts 1 and 4 tie for second place and the
    # strict '>' scan keeps expert 1; for z < 0 experts 2, 3, 5 tie and 2, 3 win.
    # Expert 4 and 5 are therefore never used: their weights must not matter.
    cfg = dict(TINY_MOE, layers=1)
    w = oracle.random_weights(cfg, seed=13, std=0.2)
    r = np.random.default_rng(17).normal(0, 0.2, cfg["d"]).astype(np.float32)
    w["router"][0] = np.stack([3 * r, r, -r, -r, r, -r])
    ids = np.random.default_rng(14).integers(0, cfg["V"], (2, 7)).astype(np.int32)
    base = oracle.HostModel(cfg, w, quantized=False).forward_logits(ids)
    np.testing.assert_allclose(base, _np_forward(cfg, w, ids), rtol=1e-4, atol=1e-5)
    w2 = {k: v.copy() for k, v in w.items()}
    w2["exp_in"][0, 4] = w2["exp_in"][0, 0]
    w2["exp_down"][0, 5] *= -3.0
    np.testing.assert_array_equal(base, oracle.HostModel(cfg, w2, quantized=False).forward_logits(ids))
    w3 = {k: v.copy() for k, v in w.items()}
    w3["exp_down"][0, 1] *= -3.0  # expert 1 is used by the tokens with z > 0
    assert np.abs(oracle.HostModel(cfg, w3, quantized=False).forward_logits(ids) - base).max() > 1e-3


def test_moe_cached_decode_equals_stateless_forward():
    w = oracle.random_weights(TINY_MOE, seed=15, std=0.2)
    m = oracle.HostModel(TINY_MOE, w, quantized=False)
    prompts = np.random.default_rng(16).integers(0, TINY["V"], (2, 5)).astype(np.int32)
    tok, lp_gen = m.generate(prompts, 6, temperature=0.0)
    np.testing.assert_allclose(lp_gen, m.logprobs(prompts, tok), atol=1e-5)


def test_cached_decode_equals_stateless_forward():
    w = oracle.random_weights(TINY, seed=4, std=0.2)
    m = oracle.HostModel(TINY, w, quantized=False)
    prompts = np.random.default_rng(5).integers(0, TINY["V"], (3, 6)).astype(np.int32)
    tok, lp_gen = m.generate(prompts, 9, temperature=0.0)
    lp_re = m.logprobs(prompts, tok)
    np.testing.assert_allclose(lp_gen, lp_re, atol=1e-5)
    # greedy: each generated token is the argmax of the stateless logits
    full = m.forward_logits(np.concatenate([prompts, tok[:, :-1]], 1))
    P = prompts.shape[1]
    np.testing.assert_array_equal(full[:, P - 1:].argmax(-1), tok)


def test_gqa_mapping_equals_duplicated_mha():
    # KVH=2, H=4: query heads {0,1} read KV head 0, {2,3} read KV head 1 (h // (H/KVH)).
    g = dict(TINY)
    mha = dict(TINY, KVH=4)
    w = oracle.random_weights(g, seed=6, std=0.2)
    H, KVH, hd, d = 4, 2, 16, 64
    wq = w["qkv"][:, :H * hd]
    wk = w["qkv"][:, H * hd:(H + KVH) * hd].reshape(-1, KVH, hd, d)
    wv = w["qkv"][:, (H + KVH) * hd:].reshape(-1, KVH, hd, d)
    wm = dict(w)
    wm["qkv"] = np.concatenate([wq, np.repeat(wk, 2, 1).reshape(-1, H * hd, d),
                                np.repeat(wv, 2, 1).reshape(-1, H * hd, d)], 1)
    ids = np.random.default_rng(7).integers(0, g["V"], (2, 7)).astype(np.int32)
    a = oracle.HostModel(g, w, False).forward_logits(ids)
    b = oracle.HostModel(mha, wm, False).forward_logits(ids)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


def test_generation_goldens():
    # generate.rs:256-262: argmax of [0.1, 5, 0.2, -1] is 1; exact ties -> lowest index
    tok, lp = oracle.sample(np.array([[0.1, 5.0, 0.2, -1.0], [2.0, 7.0, 7.0, 1.0]], np.float32), 0.0, 0, 0)
    assert list(tok) == [1, 1]
    v = np.array([0.1, 5.0, 0.2, -1.0])
    assert abs(lp[0] - (5.0 - np.log(np.exp(v).sum()))) < 1e-6


def test_gumbel_sampler_distribution_and_determinism():
    base = np.array([0.0, 1.0, 2.0, 0.5], np.float32)
    rows = 40000
    t1, _ = oracle.sample(np.tile(base, (rows, 1)), 1.0, 9, 3)
    t2, _ = oracle.sample(np.tile(base, (rows, 1)), 1.0, 9, 3)
    np.testing.assert_array_equal(t1, t2)
    counts = np.bincount(t1, minlength=4) / rows
    p = np.exp(base) / np.exp(base).sum()
    assert np.all(np.abs(counts - p) < 0.01)


def test_quantized_oracle_close_to_dequantized_f32():
    # The Q4 path computes with dequantised weights (scale * code exact in f32)
    # and f16-rounded q/k/v: logits stay close to the f32 model whose weights
    # are the decoded Q4 values.
    cfg = dict(TINY, d=128, F=128, hd=32, H=4, KVH=4)
    w = oracle.random_weights(cfg, seed=8, std=0.05)
    q = oracle.HostModel(cfg, w, quantized=True)
    wd = dict(w)
    for k in ("qkv", "o", "in", "down"):
        codes, scales = q.packed[k]
        wd[k] = oracle.q4_decode(codes, scales, w[k].size).reshape(w[k].shape)
    codes, scales = q.packed["lm_head"]
    wd["lm_head"] = oracle.q4_decode(codes, scales, w["lm_head"].size).reshape(w["lm_head"].shape)
    wd["embed"] = oracle.round_bf16(w["embed"])
    f = oracle.HostModel(cfg, wd, quantized=False)
    ids = np.random.default_rng(9).integers(0, cfg["V"], (2, 9)).astype(np.int32)
    a, b = q.forward_logits(ids), f.forward_logits(ids)
    assert np.abs(a - b).max() < 2e-2 * max(1.0, np.abs(b).max())
    assert np.abs(a - b).max() > 0  # the f16 q/k/v rounding is really applied


def test_moe_quantized_oracle_close_to_dequantized_f32():
    # per-expert Q4G128 packing: decoding each expert's codes gives the f32
    # model the quantized MoE path approximates (f16 q/k/v rounding only)
    cfg = dict(TINY_MOE, d=128, Fe=128, hd=32, H=4, KVH=4)
    w = oracle.random_weights(cfg, seed=18, std=0.05)
    q = oracle.HostModel(cfg, w, quantized=True)
    wd = dict(w)
    for k in ("qkv", "o", "lm_head", "exp_in", "exp_down"):
        codes, scales = q.packed[k]
        wd[k] = oracle.q4_decode(codes, scales, w[k].size).reshape(w[k].shape)
    wd["embed"] = oracle.round_bf16(w["embed"])
    f = oracle.HostModel(cfg, wd, quantized=False)
    ids = np.random.default_rng(19).integers(0, cfg["V"], (2, 9)).astype(np.int32)
    assert min(q.router_gaps(ids).min(), f.router_gaps(ids).min()) > 1e-2
    a, b = q.forward_logits(ids), f.forward_logits(ids)
    assert 0 < np.abs(a - b).max() < 2e-2 * max(1.0, np.abs(b).max())
