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


def test_quantized_oracle_with_f32_kv_equals_dequantized_f32():
    """kv_f32 removes the only rounding the quantized path adds: with q, k and
    v kept in f32 it equals the f32 model on the decoded Q4 weights (both
    accumulating in f64), while the default rounds them to f16."""
    cfg = dict(TINY, d=128, F=128, hd=32, H=4, KVH=2)
    w = oracle.random_weights(cfg, seed=10, std=0.05)
    q = oracle.HostModel(cfg, w, quantized=True)
    qf = oracle.HostModel(cfg, w, quantized=True, kv_f32=True)
    wd = dict(w)
    for k in ("qkv", "o", "in", "down", "lm_head"):
        codes, scales = q.packed[k]
        wd[k] = oracle.q4_decode(codes, scales, w[k].size).reshape(w[k].shape)
    wd["embed"] = oracle.round_bf16(w["embed"])
    f = oracle.HostModel(cfg, wd, quantized=False, acc64=True)
    ids = np.random.default_rng(11).integers(0, cfg["V"], (2, 9)).astype(np.int32)
    a, b, c = qf.forward_logits(ids), f.forward_logits(ids), q.forward_logits(ids)
    assert np.abs(a - b).max() <= 1e-6 * max(1.0, np.abs(b).max())
    assert np.abs(c - b).max() > 10 * np.abs(a - b).max()


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


# ---- sampling options (generate.rs:127-250) --------------------------------

def test_repetition_penalty_golden_sign_aware_once_per_token():
    # generate.rs:279-284
    np.testing.assert_array_equal(oracle.apply_penalty([4.0, -2.0, 3.0, 1.0], [0, 1, 0], 2.0),
                                  [2.0, -4.0, 3.0, 1.0])
    with pytest.raises(ValueError):
        oracle.apply_penalty([1.0, 2.0], [2], 2.0)


def test_repetition_penalty_changes_greedy_golden():
    # generate.rs:286-295: [5, 4, 1], prior [0], p = 2 -> 1
    tok, _ = oracle.sample_ex(np.array([[5.0, 4.0, 1.0]], np.float32), temperature=0.0, seed=42,
                              step=0, repetition_penalty=2.0, prior=[[0]])
    assert tok[0] == 1
    tok, _ = oracle.sample_ex(np.array([[0.1, 5.0, 0.2, -1.0]], np.float32), temperature=0.0,
                              seed=0, step=0)
    assert tok[0] == 1  # generate.rs:260-265


def test_sample_ex_options_off_equals_plain_sampler():
    rng = np.random.default_rng(5)
    logits = rng.normal(0, 2, (8, 300)).astype(np.float32)
    for T in (0.0, 0.7, 1.3):
        a, la = oracle.sample(logits, T, 77, 4)
        b, lb = oracle.sample_ex(logits, temperature=T, seed=77, step=4)
        np.testing.assert_array_equal(a, b)
        np.testing.assert_allclose(la, lb, rtol=0, atol=1e-12)
        # top_k >= V is no restriction; top_k = 1 is the argmax
        c, _ = oracle.sample_ex(logits, temperature=T, seed=77, step=4, top_k=300)
        np.testing.assert_array_equal(a, c)
    g, _ = oracle.sample_ex(logits, temperature=1.0, seed=3, step=0, top_k=1)
    np.testing.assert_array_equal(g, logits.argmax(1))


def _topk_set(vals, k):
    # k largest by value, then lowest index (select_nth_unstable_by, generate.rs:218-225)
    order = np.lexsort((np.arange(vals.size), -vals.astype(np.float64)))
    return set(order[:k].tolist())


def test_top_k_draws_stay_in_the_k_largest_with_index_tie_break():
    vals = np.array([1.0, 3.0, 3.0, 0.5, 3.0, 2.0, -1.0, 3.0], np.float32)
    allowed = _topk_set(vals, 3)
    assert allowed == {1, 2, 4}
    seen = set()
    for seed in range(400):
        t, _ = oracle.sample_ex(vals[None], temperature=2.0, seed=seed, step=0, top_k=3)
        seen.add(int(t[0]))
    assert seen == allowed


def test_top_k_distribution_is_softmax_over_the_candidates():
    base = np.array([0.0, 1.0, 2.0, 0.5, 1.5, -0.5], np.float32)
    T, k, rows = 0.8, 3, 30000
    tok, _ = oracle.sample_ex(np.tile(base, (rows, 1)), temperature=T, seed=11, step=2, top_k=k)
    cand = sorted(_topk_set(base, k))
    w = np.zeros(base.size)
    w[cand] = np.exp((base[cand].astype(np.float64) - base.max()) / T)
    p = w / w.sum()
    counts = np.bincount(tok, minlength=base.size) / rows
    assert np.all(np.abs(counts - p) < 0.012), (counts, p)


def test_nucleus_keeps_the_smallest_prefix_reaching_top_p():
    # the opt-in nucleus filter, checked against its definition (f64 probs)
    rng = np.random.default_rng(21)
    for trial in range(40):
        V = int(rng.integers(5, 60))
        vals = rng.normal(0, 1.5, V).astype(np.float32)
        T, top_p = float(rng.uniform(0.5, 1.5)), float(rng.uniform(0.2, 0.95))
        order = np.lexsort((np.arange(V), -vals.astype(np.float64)))
        p = np.exp((vals[order].astype(np.float64) - vals.max()) / T)
        cum = np.cumsum(p / p.sum())
        keep = int(np.searchsorted(cum, top_p - 1e-12) + 1)
        if min(abs(cum - top_p)) < 1e-6:
            continue  # boundary within the fixed-point resolution
        allowed = set(order[:keep].tolist())
        got = set()
        for seed in range(60):
            t, _ = oracle.sample_ex(vals[None], temperature=T, seed=seed, step=trial,
                                    top_p=top_p, apply_top_p=True)
            got.add(int(t[0]))
        assert got <= allowed, (trial, got, allowed)
        # applied off: top_p is validated only (the reference has no nucleus sampler)
        t0, _ = oracle.sample_ex(vals[None], temperature=T, seed=5, step=trial, top_p=top_p)
        t1, _ = oracle.sample(vals[None], T, 5, trial)
        assert t0[0] == t1[0]


def test_generate_ex_stops_at_eos_and_penalises_the_context():
    cfg = dict(TINY)
    w = oracle.random_weights(cfg, seed=4, std=0.3)
    m = oracle.HostModel(cfg, w, quantized=False)
    prompts = np.array([[1, 2, 3], [4, 5, 6]], np.int32)
    tok, lp = m.generate(prompts, 12, temperature=0.0)
    eos = int(tok[0, 4])
    t2, lp2, lens = m.generate_ex(prompts, 12, temperature=0.0, eos_token=eos)
    first = [int(np.argmax(r == eos)) if (r == eos).any() else None for r in tok]
    for s in range(2):
        n = 12 if first[s] is None else first[s] + 1
        assert lens[s] == n
        np.testing.assert_array_equal(t2[s, :n], tok[s, :n])
        assert np.all(t2[s, n:] == eos) and np.all(lp2[s, n:] == 0.0)
    # with a strong penalty greedy decoding avoids repeating context tokens while
    # fresh ones remain
    t3, _, _ = m.generate_ex(prompts, 6, temperature=0.0, repetition_penalty=1e6)
    for s in range(2):
        ctx = list(prompts[s])
        for t in t3[s]:
            assert t not in ctx
            ctx.append(int(t))
