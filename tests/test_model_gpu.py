"""End-to-end RL-step pieces on the GPU vs the CPU oracle decoder.

Bars: sampled tokens bit-exact up to the first logit
near-tie; per-token log-probs within 1e-5 (fp32 model) / 2e-3 (bf16, Q4);
loss and advantages within 1e-4 relative.
"""
import numpy as np
import pytest
import torch

import oracle
from summa_amd.model import Model, ModelConfig, batch_result, rl_prepare

pytestmark = pytest.mark.gpu

CFG0 = ModelConfig(layers=2, d_model=256, heads=4, kv_heads=4, head_dim=64, ffn=1024, vocab=4096,
                   max_seq=128, quantized=False)


def _mask64(z):
    return z & np.uint64(0xFFFFFFFFFFFFFFFF)


def _mix64(z):
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xbf58476d1ce4e5b9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94d049bb133111eb)
    return z ^ (z >> np.uint64(31))


def _gumbel(seed, row, step, V):
    """Gumbel noise of the counter sampler for (seed, row, step) over the vocab."""
    with np.errstate(over="ignore"):
        a = _mix64(np.uint64(seed) + np.uint64(0x9e3779b97f4a7c15) * np.uint64(row + 1))
        cnt = np.uint64(step) * np.uint64(V) + np.arange(V, dtype=np.uint64)
        k = _mix64(a ^ (cnt * np.uint64(0xd1b54a32d192ed03)))
    u = ((k >> np.uint64(40)).astype(np.float32) + np.float32(0.5)) * np.float32(1.0 / 16777216.0)
    return -np.log(-np.log(u.astype(np.float64)))


def _build(cfg: ModelConfig, weights, dev):
    m = Model(cfg)
    m.load_host_weights(weights, dev)
    return m


def _check_tokens(host, prompts, tok_gpu, tok_or, temperature, seed, tol):
    """Tokens must agree until the first near-tie of the (perturbed) logits."""
    P = prompts.shape[1]
    V = host.cfg["V"]
    mismatched = 0
    for s in range(prompts.shape[0]):
        diff = np.nonzero(tok_gpu[s] != tok_or[s])[0]
        if diff.size == 0:
            continue
        mismatched += 1
        n = int(diff[0])
        ids = np.concatenate([prompts[s], tok_gpu[s, :n]])[None]
        logits = host.forward_logits(ids)[0, P - 1 + n].astype(np.float64)
        a, b = int(tok_gpu[s, n]), int(tok_or[s, n])
        if temperature > 0:
            key = logits / temperature + _gumbel(seed, s, n, V)
        else:
            key = logits
        assert abs(key[a] - key[b]) < tol, f"seq {s} step {n}: not a near-tie ({key[a]} vs {key[b]})"
    return mismatched


def test_config0_greedy_rollout_and_logprobs(dev):
    print("case config0 greedy fp32", flush=True)
    cfg = CFG0.oracle_cfg()
    w = oracle.random_weights(cfg, seed=0, std=0.02)
    host = oracle.HostModel(cfg, w, quantized=False)
    m = _build(CFG0, w, dev)
    prompts = np.random.default_rng(0).integers(0, cfg["V"], (32, 32)).astype(np.int32)
    pd = torch.from_numpy(prompts).to(dev)
    tok, lp_beh = m.generate(pd, 64, temperature=0.0)
    lp_cur = m.logprobs(pd, tok)
    tok_np = tok.cpu().numpy()
    lp_or = host.logprobs(prompts, tok_np)
    np.testing.assert_allclose(lp_cur.cpu().numpy(), lp_or, atol=1e-5)
    np.testing.assert_allclose(lp_beh.cpu().numpy(), lp_or, atol=1e-5)
    tok_or, _ = host.generate(prompts, 64, 0.0)
    mism = _check_tokens(host, prompts, tok_np, tok_or, 0.0, 0, 1e-4)
    print(f"sequences diverging at a near-tie: {mism}/32", flush=True)


def test_logprob_chunking_is_exact(dev):
    cfg = CFG0.oracle_cfg()
    w = oracle.random_weights(cfg, seed=1, std=0.02)
    m = _build(CFG0, w, dev)
    prompts = torch.randint(0, cfg["V"], (6, 10), dtype=torch.int32, device=dev)
    tok = torch.randint(0, cfg["V"], (6, 7), dtype=torch.int32, device=dev)
    a = m.logprobs(prompts, tok)
    b = m.logprobs(prompts, tok, max_tokens_per_forward=2 * 16)  # 2 sequences per forward
    assert torch.equal(a, b)


@pytest.mark.parametrize("geom", ["cfg1", "cfg2", "batch", "batch_cfg1"])
def test_quantized_rollout_and_logprobs(dev, geom):
    """cfg1 / cfg2 geometry at small batch; "batch" decodes 128 sequences at
    once, so every decode matmul runs the batch kernel (with split-K);
    "batch_cfg1" decodes 128 sequences of config[1]'s layer shapes, whose qkv
    (with RoPE) and SwiGLU projections run the LDS-staged decode kernel."""
    print(f"case quantized {geom}", flush=True)
    if geom == "cfg1":
        mc = ModelConfig(layers=2, d_model=768, heads=12, kv_heads=12, head_dim=64, ffn=3072,
                         vocab=32768, max_seq=64, quantized=True)
        S, P, N = 8, 16, 8
    elif geom == "batch":
        mc = ModelConfig(layers=2, d_model=768, heads=12, kv_heads=4, head_dim=64, ffn=3072,
                         vocab=4096, max_seq=64, quantized=True)
        S, P, N = 128, 8, 4
    elif geom == "batch_cfg1":
        mc = ModelConfig(layers=2, d_model=768, heads=12, kv_heads=12, head_dim=64, ffn=3072,
                         vocab=4096, max_seq=64, quantized=True)
        S, P, N = 128, 8, 4
    else:
        mc = ModelConfig(layers=2, d_model=2048, heads=16, kv_heads=4, head_dim=128, ffn=5632,
                         vocab=4096, max_seq=64, quantized=True)
        S, P, N = 4, 24, 6
    cfg = mc.oracle_cfg()
    w = oracle.random_weights(cfg, seed=2, std=0.02)
    host = oracle.HostModel(cfg, w, quantized=True)
    m = _build(mc, w, dev)
    prompts = np.random.default_rng(3).integers(0, cfg["V"], (S, P)).astype(np.int32)
    pd = torch.from_numpy(prompts).to(dev)
    tok, lp_beh = m.generate(pd, N, temperature=1.0, seed=11)
    lp_cur = m.logprobs(pd, tok)
    tok_np = tok.cpu().numpy()
    lp_or = host.logprobs(prompts, tok_np)
    err = np.abs(lp_cur.cpu().numpy() - lp_or).max()
    err_beh = np.abs(lp_beh.cpu().numpy() - lp_or).max()
    print(f"max |lp - oracle|: recompute {err:.2e}, behavior {err_beh:.2e}", flush=True)
    # 16-bit KV cache: 2e-3 abs on per-token log-probs
    np.testing.assert_allclose(lp_cur.cpu().numpy(), lp_or, atol=2e-3)
    np.testing.assert_allclose(lp_beh.cpu().numpy(), lp_or, atol=2e-3)
    tok_or, _ = host.generate(prompts, N, 1.0, 11)
    mism = _check_tokens(host, prompts, tok_np, tok_or, 1.0, 11, 4e-3)
    print(f"sequences diverging at a near-tie: {mism}/{S}", flush=True)


def test_rl_prepare_matches_oracle(dev):
    print("case rl_prepare config0", flush=True)
    cfg = CFG0.oracle_cfg()
    w = oracle.random_weights(cfg, seed=4, std=0.02)
    w_ref = oracle.random_weights(cfg, seed=5, std=0.02)  # frozen copy that differs
    host, host_ref = oracle.HostModel(cfg, w, False), oracle.HostModel(cfg, w_ref, False)
    policy, reference = _build(CFG0, w, dev), _build(CFG0, w_ref, dev)
    groups, G, P, N = 4, 8, 32, 16
    rng = np.random.default_rng(6)
    prompts = rng.integers(0, cfg["V"], (groups * G, P)).astype(np.int32)
    pd = torch.from_numpy(prompts).to(dev)
    tok, lp_beh = policy.generate(pd, N, temperature=1.0, seed=3)
    rewards = rng.binomial(1, 0.5, (groups, G)).astype(np.float32)
    out = rl_prepare(policy, reference, pd, tok, lp_beh, torch.from_numpy(rewards).to(dev),
                     clip_epsilon=0.2, advantage_epsilon=1e-6, kl_coefficient=0.04)
    res = batch_result(out)
    tok_np = tok.cpu().numpy()
    lp_cur = host.logprobs(prompts, tok_np)
    lp_ref = host_ref.logprobs(prompts, tok_np)
    np.testing.assert_allclose(out["lp_cur"].cpu().numpy(), lp_cur, atol=1e-5)
    np.testing.assert_allclose(out["lp_ref"].cpu().numpy(), lp_ref, atol=1e-5)
    beh = lp_beh.cpu().numpy().astype(np.float64)
    stats, adv, dlp, err = oracle.grpo_loss(rewards, lp_cur.reshape(groups, G, N),
                                            beh.reshape(groups, G, N),
                                            lp_ref.reshape(groups, G, N), None, 0.2, 1e-6, 0.04)
    assert err == 0
    got = out["stats"].cpu().numpy()
    np.testing.assert_allclose(got[:, 1:3], stats[:, 1:3], rtol=1e-6)
    # loss / KL: the inputs carry the fp32 log-prob differences (<= 1e-5)
    np.testing.assert_allclose(got[:, 0], stats[:, 0], rtol=1e-4, atol=2e-6)
    np.testing.assert_allclose(got[:, 3], stats[:, 3], rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(out["dlp"].cpu().numpy(), dlp.reshape(groups * G, N), rtol=1e-4,
                               atol=1e-7)
    assert abs(res["mean_reward_sum"] - stats[:, 1].sum()) < 1e-5
    assert res["rollouts"] == groups * G


@pytest.mark.parametrize("quantized,experts", [(True, 0), (False, 0), (True, 8)])
def test_prompt_groups_equal_per_rollout(dev, quantized, experts):
    """Prompt groups (sm_model_set_prompt_groups): generation (plain and with
    EOS / top-k / repetition penalty), the recompute (one and several chunks)
    and the GRPO prepare with each group's prompt computed once give the
    tokens of computing every rollout's prompt and its log-probs up to the
    order of f32 additions (the prompt GEMMs run at groups x P rows instead of
    S x P, which can pick another tiling or K split; through the 16-bit K / V
    cache that stays within 2e-4, 1e-5 for f32 models), P 40 not being a
    multiple of the attention tiles. A prompt that differs inside a group, or
    rollouts that are not whole groups, are rejected."""
    from summa_amd.sampling import SamplingConfig
    print(f"case prompt groups quantized={quantized} experts={experts}", flush=True)
    kw = dict(experts=experts, expert_ffn=256) if experts else {}
    cfg = ModelConfig(layers=2, d_model=256, heads=4, kv_heads=2, head_dim=64, ffn=512,
                      vocab=1024, max_seq=64, quantized=quantized, **kw)
    plain, grouped = Model(cfg), Model(cfg)
    for m in (plain, grouped):
        m.init_random(17, std=0.05)
    G, groups, P, N = 4, 3, 40, 12
    grouped.set_prompt_groups(G)
    gen = torch.Generator().manual_seed(3)
    base = torch.randint(0, cfg.vocab, (groups, P), generator=gen, dtype=torch.int32)
    prompts = base.repeat_interleave(G, 0).to(dev)
    tol = 2e-4 if quantized else 1e-5

    def close(a, b, what):
        err = float((a - b).abs().max())
        print(f"  {what}: max |grouped - per rollout| {err:.2e}", flush=True)
        assert err <= tol, what

    t1, l1 = plain.generate(prompts, N, temperature=1.0, seed=5)
    t2, l2 = grouped.generate(prompts, N, temperature=1.0, seed=5)
    assert torch.equal(t1, t2)
    close(l1, l2, "generate")
    sc = SamplingConfig(max_new_tokens=N, temperature=0.8, top_k=20, repetition_penalty=1.3,
                        eos_token=int(t1[0, 3]), seed=9)
    e1, e2 = plain.generate_ex(prompts, sc), grouped.generate_ex(prompts, sc)
    assert torch.equal(e1[0], e2[0]) and torch.equal(e1[2], e2[2])
    close(e1[1], e2[1], "generate_ex")
    for budget in (0, 100):  # one chunk; one rollout and two prompts per forward
        r1 = plain.logprobs(prompts, t1, max_tokens_per_forward=budget)
        r2 = grouped.logprobs(prompts, t1, max_tokens_per_forward=budget)
        close(r1, r2, f"logprobs (budget {budget})")
    rewards = torch.rand(groups, G, generator=gen).to(dev)
    o1 = rl_prepare(plain, plain, prompts, t1, l1, rewards)
    o2 = rl_prepare(grouped, grouped, prompts, t1, l1, rewards)
    close(o1["lp_cur"], o2["lp_cur"], "prepare lp_cur")
    assert torch.equal(o2["lp_cur"], o2["lp_ref"])
    bad = prompts.clone()
    bad[5, 7] = (bad[5, 7] + 1) % cfg.vocab
    with pytest.raises(Exception, match="differs from its group"):
        grouped.generate(bad, N, temperature=1.0, seed=5)
    with pytest.raises(Exception, match="whole groups"):
        grouped.logprobs(prompts[:10], t1[:10])


@pytest.mark.parametrize("quantized,experts", [(True, 0), (False, 0), (True, 8)])
def test_prompt_state_reuse(dev, quantized, experts):
    """A grouped recompute reuses the prompt pass of the generation (or
    recompute) before it when the prompts, the weights and the buffers are
    the same, and recomputes it otherwise: every result equals the recompute
    of a model created for that one call, bit for bit: after generating, for
    other prompts, for the first prompts again, after a weight change, with a
    budget that splits the prompt pass, after a split pass of other prompts,
    and (MoE) after a router-traced generation of other prompts."""
    print(f"case prompt state reuse quantized={quantized} experts={experts}", flush=True)
    kw = dict(experts=experts, expert_ffn=256) if experts else {}
    cfg = ModelConfig(layers=2, d_model=256, heads=4, kv_heads=2, head_dim=64, ffn=512,
                      vocab=1024, max_seq=64, quantized=quantized, **kw)
    a = Model(cfg)
    seed = [29]
    a.init_random(seed[0], std=0.05)
    a.set_prompt_groups(4)
    gen = torch.Generator().manual_seed(8)
    P, N = 24, 10

    def prompts():
        base = torch.randint(0, cfg.vocab, (3, P), generator=gen, dtype=torch.int32)
        return base.repeat_interleave(4, 0).to(dev)

    p1, p2 = prompts(), prompts()
    tok, _ = a.generate(p1, N, temperature=1.0, seed=2)

    def fresh(prm, budget):
        b = Model(cfg)
        b.init_random(seed[0], std=0.05)
        b.set_prompt_groups(4)
        out = b.logprobs(prm, tok, max_tokens_per_forward=budget)
        torch.cuda.synchronize()
        b.close()
        return out

    def same(prm, what, budget=0):
        la = a.logprobs(prm, tok, max_tokens_per_forward=budget)
        assert torch.equal(la, fresh(prm, budget)), what

    same(p1, "after the generation")
    same(p1, "again")
    same(p2, "other prompts")
    same(p1, "the first prompts again")
    # a prompt pass split by the budget overwrites the kept prompt K / V
    # without recording them: the next default-budget recompute of the old
    # prompts must not reuse them
    same(p1, "recorded p1")
    same(p2, "p2 in chunks", budget=30)
    same(p1, "p1 after a split pass of p2")
    if experts:
        # a traced generation runs a prompt pass it does not record
        a.generate(p1, N, temperature=1.0, seed=2)
        a.trace_routes(4096, logits=False)
        a.generate(p2, N, temperature=1.0, seed=2)
        a.stop_trace()
        same(p1, "p1 after a traced generation of p2")
    a.generate(p1, N, temperature=1.0, seed=3)
    seed[0] = 31
    a.init_random(seed[0], std=0.05)  # new weights: the generation's prompt pass is stale
    same(p1, "after a weight change")
    same(p1, "prompt pass in chunks", budget=30)
