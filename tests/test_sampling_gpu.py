"""Device sampler with the TextGenerator options (sm_sample_ex, sm_rl_generate_ex)
against the CPU oracle (generate.rs:127-250).

Bars: tokens bit-exact (a mismatch only at a near-tie of the Gumbel / greedy
keys, |d| < 1e-4 after the 1/T scale); log-probs of the raw logits within 1e-5;
EOS bookkeeping (done flags, lengths, padding) exact.
"""
import numpy as np
import pytest
import torch

import oracle
from summa_amd import sampling
from summa_amd.model import Model, ModelConfig
from summa_amd.sampling import SamplingConfig

pytestmark = pytest.mark.gpu


def _mix64(z):
    z = np.asarray(z, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xbf58476d1ce4e5b9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94d049bb133111eb)
    return z ^ (z >> np.uint64(31))


def _gumbel(seed, row, step, V):
    with np.errstate(over="ignore"):
        a = _mix64(np.uint64(seed) + np.uint64(0x9e3779b97f4a7c15) * np.uint64(row + 1))
        cnt = np.uint64(step) * np.uint64(V) + np.arange(V, dtype=np.uint64)
        k = _mix64(a ^ (cnt * np.uint64(0xd1b54a32d192ed03)))
    u = ((k >> np.uint64(40)).astype(np.float32) + np.float32(0.5)) * np.float32(1.0 / 16777216.0)
    return -np.log(-np.log(u.astype(np.float64)))


def _priors(rng, rows, V, n):
    return [rng.integers(0, V, n).astype(np.int32) for _ in range(rows)]


def _seen(dev, priors, V):
    n = max(len(p) for p in priors)
    ids = np.full((len(priors), n), -1, np.int32)
    for r, p in enumerate(priors):
        ids[r, :len(p)] = p
    return sampling.seen_tokens(torch.from_numpy(ids).to(dev), V)


CASES = [
    dict(temperature=0.0, repetition_penalty=1.5),
    dict(temperature=0.8, top_k=50),
    dict(temperature=1.0, top_k=7, repetition_penalty=1.3),
    dict(temperature=0.7, top_p=0.9, apply_top_p=True),
    dict(temperature=0.9, top_k=40, top_p=0.8, apply_top_p=True, repetition_penalty=1.1),
    dict(temperature=1.2, top_k=2000),
    dict(temperature=0.6, top_p=0.95),  # validated only: equals the plain sampler
]


@pytest.mark.parametrize("V", [4096, 32768])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_sample_ex_matches_oracle(dev, V, case):
    kw = CASES[case]
    print(f"case sample_ex V={V} {kw}", flush=True)
    rows = 12
    rng = np.random.default_rng(case * 7 + V)
    logits = rng.normal(0, 2, (rows, V)).astype(np.float32)
    priors = _priors(rng, rows, V, 60)
    cfg = SamplingConfig(**kw)
    ld = torch.from_numpy(logits).to(dev)
    seen = _seen(dev, priors, V) if cfg.repetition_penalty != 1.0 else None
    tok, lp = sampling.sample(ld, cfg, seed=99, step=3, seen=seen)
    rt, rlp = oracle.sample_ex(logits, temperature=cfg.temperature, seed=99, step=3,
                               top_k=-1 if cfg.top_k is None else cfg.top_k,
                               repetition_penalty=cfg.repetition_penalty, top_p=cfg.top_p,
                               apply_top_p=cfg.apply_top_p, prior=priors)
    np.testing.assert_array_equal(tok.cpu().numpy(), rt)
    np.testing.assert_allclose(lp.cpu().numpy(), rlp, atol=1e-5)
    if seen is not None:  # the chosen token is recorded in the bitmap
        bits = seen.cpu().numpy().view(np.uint32)
        for r, t in enumerate(rt):
            assert (bits[r, t >> 5] >> (t & 31)) & 1


@pytest.mark.parametrize("T", [0.0, 0.7])
def test_sample_ex_with_options_off_equals_sample(dev, T):
    from summa_amd._lib import call
    rows, V = 16, 32768
    g = torch.Generator(device=dev).manual_seed(11)
    logits = torch.randn(rows, V, device=dev, generator=g) * 3
    a = torch.empty(rows, dtype=torch.int32, device=dev)
    la = torch.empty(rows, device=dev)
    call("sm_sample", logits.data_ptr(), rows, V, V, T, 5, 9, a.data_ptr(), 1, la.data_ptr(), 1,
         None, torch.cuda.current_stream().cuda_stream)
    b, lb = sampling.sample(logits, SamplingConfig(temperature=T), seed=5, step=9)
    assert torch.equal(a, b)
    # The two kernels visit a row's elements in different per-thread orders
    # (sm_sample reads 16-byte groups), so the log-sum-exp behind the log-prob
    # is rounded differently: a few ulp of |lp| ~ 15 (ulp 9.5e-7).
    torch.testing.assert_close(la, lb, rtol=0, atol=1e-5)


def test_top_k_ties_keep_the_lowest_indices(dev):
    # many equal values across the k-th position: ties resolve by index
    rows, V, k = 8, 1000, 100
    rng = np.random.default_rng(3)
    logits = rng.integers(0, 6, (rows, V)).astype(np.float32)
    ld = torch.from_numpy(logits).to(dev)
    for seed in range(6):
        cfg = SamplingConfig(temperature=50.0, top_k=k)
        tok, _ = sampling.sample(ld, cfg, seed=seed, step=0)
        rt, _ = oracle.sample_ex(logits, temperature=50.0, seed=seed, step=0, top_k=k)
        np.testing.assert_array_equal(tok.cpu().numpy(), rt)
        for r in range(rows):
            order = np.lexsort((np.arange(V), -logits[r]))
            assert int(rt[r]) in set(order[:k].tolist())


def test_done_rows_emit_eos_and_lengths(dev):
    rows, V, eos = 4, 64, 7
    logits = torch.full((rows, V), -5.0, device=dev)
    logits[0, eos] = 5.0   # emits EOS now
    logits[1, 3] = 5.0     # another token
    logits[2, eos] = 5.0   # already done: padded, untouched length
    logits[3, eos] = 5.0
    done = torch.tensor([0, 0, 1, 0], dtype=torch.int32, device=dev)
    lengths = torch.full((rows,), 99, dtype=torch.int32, device=dev)
    cfg = SamplingConfig(temperature=0.0, eos_token=eos)
    tok, lp = sampling.sample(logits, cfg, seed=0, step=4, done=done, lengths=lengths)
    assert tok.tolist() == [eos, 3, eos, eos]
    assert done.tolist() == [1, 0, 1, 1]
    assert lengths.tolist() == [5, 99, 99, 5]
    assert lp[2].item() == 0.0 and lp[0].item() < 0.0


CFG0 = ModelConfig(layers=2, d_model=256, heads=4, kv_heads=4, head_dim=64, ffn=1024, vocab=4096,
                   max_seq=128, quantized=False)

GEN_CASES = [
    dict(temperature=0.0, repetition_penalty=1.3),
    dict(temperature=0.9, top_k=20, eos_token="auto"),
    dict(temperature=0.8, top_k=50, top_p=0.9, apply_top_p=True, repetition_penalty=1.2,
         eos_token="auto"),
]


@pytest.mark.parametrize("case", range(len(GEN_CASES)))
def test_generate_ex_teacher_forced_against_oracle(dev, case):
    """Every generated position is re-sampled by the oracle from the oracle's own
    logits for the device prefix (prompt and device tokens so far as the
    penalty context): same token unless the keys are a near-tie; EOS padding
    and lengths as TextGenerator::generate stops."""
    kw = dict(GEN_CASES[case])
    print(f"case generate_ex {kw}", flush=True)
    cfg = CFG0.oracle_cfg()
    w = oracle.random_weights(cfg, seed=case, std=0.05)
    host = oracle.HostModel(cfg, w, quantized=False)
    m = Model(CFG0)
    m.load_host_weights(w, dev)
    S, P, N, seed = 16, 8, 24, 1234 + case
    V = cfg["V"]
    prompts = np.random.default_rng(case).integers(0, V, (S, P)).astype(np.int32)
    pd = torch.from_numpy(prompts).to(dev)
    if kw.get("eos_token") == "auto":
        # an EOS that some rollouts do emit: a token of the plain rollout
        t0, _ = m.generate(pd, N, temperature=kw["temperature"], seed=seed)
        kw["eos_token"] = int(np.bincount(t0.cpu().numpy().ravel()).argmax())
    sc = SamplingConfig(max_new_tokens=N, **kw)
    tok, lp, lens = m.generate_ex(pd, sc, seed=seed)
    tok, lp, lens = tok.cpu().numpy(), lp.cpu().numpy(), lens.cpu().numpy()
    eos = -1 if sc.eos_token is None else sc.eos_token
    ids = np.concatenate([prompts, tok], axis=1)
    logits = host.forward_logits(ids)
    near = 0
    for s in range(S):
        n_s = int(lens[s])
        if eos >= 0 and n_s < N:
            assert tok[s, n_s - 1] == eos and not (tok[s, :n_s - 1] == eos).any()
            assert (tok[s, n_s:] == eos).all() and (lp[s, n_s:] == 0).all()
        else:
            assert n_s == N and not (tok[s] == eos).any()
        for n in range(n_s):
            row = logits[s, P - 1 + n][None].astype(np.float32)
            prior = [ids[s, :P + n]]
            rt, rlp = oracle.sample_ex(row, temperature=sc.temperature, seed=seed, step=n,
                                       top_k=-1 if sc.top_k is None else sc.top_k,
                                       repetition_penalty=sc.repetition_penalty, top_p=sc.top_p,
                                       apply_top_p=sc.apply_top_p, prior=prior, row0=s)
            assert abs(lp[s, n] - rlp[0]) < 1e-5, (s, n, lp[s, n], rlp[0])
            if rt[0] != tok[s, n]:
                val = oracle.apply_penalty(row[0], prior[0], sc.repetition_penalty).astype(np.float64)
                key = val / sc.temperature + _gumbel(seed, s, n, V) if sc.temperature > 0 else val
                a, b = int(tok[s, n]), int(rt[0])
                assert abs(key[a] - key[b]) < 1e-4, f"seq {s} step {n}: {key[a]} vs {key[b]}"
                near += 1
    print(f"near-tie positions: {near}", flush=True)


def test_eos_stopped_rollouts_through_rl_prepare(dev):
    """Rollouts that stop at EOS enter the GRPO loss through their completion
    mask (n < lengths[s]): rl_prepare(lengths=...) equals the oracle's loss on
    the masked rows, and the padded tail gets no gradient."""
    from summa_amd.model import completion_mask, rl_prepare
    cfg = CFG0.oracle_cfg()
    w = oracle.random_weights(cfg, seed=7, std=0.05)
    m, ref = Model(CFG0), Model(CFG0)
    m.load_host_weights(w, dev)
    ref.load_host_weights(oracle.random_weights(cfg, seed=8, std=0.05), dev)
    groups, G, P, N, seed = 2, 8, 8, 24, 99
    S = groups * G
    prompts = torch.from_numpy(np.random.default_rng(3).integers(0, cfg["V"], (S, P))
                               .astype(np.int32)).to(dev)
    kw = dict(max_new_tokens=N, temperature=0.9, top_k=20)
    # an EOS that rollout 0 emits at its third step at the latest: the token it
    # samples there without one (the draws do not depend on the EOS option)
    t0, _, _ = m.generate_ex(prompts, SamplingConfig(**kw), seed=seed)
    eos = int(t0[0, 2])
    tok, beh, lens = m.generate_ex(prompts, SamplingConfig(eos_token=eos, **kw), seed=seed)
    L = lens.cpu().numpy()
    assert (L < N).any(), "no rollout stopped at EOS"
    mask_h = (np.arange(N)[None, :] < L[:, None]).astype(np.float64)
    np.testing.assert_array_equal(completion_mask(lens, N).cpu().numpy(), mask_h)
    rewards = torch.from_numpy(np.random.default_rng(4).random((groups, G)).astype(np.float32)).to(dev)
    out = rl_prepare(m, ref, prompts, tok, beh, rewards, lengths=lens)
    with pytest.raises(ValueError, match="either mask or lengths"):
        rl_prepare(m, ref, prompts, tok, beh, rewards, mask=completion_mask(lens, N), lengths=lens)
    sh = (groups, G, N)
    st_or, _, dlp_or, err = oracle.grpo_loss(
        rewards.cpu().numpy(), out["lp_cur"].cpu().numpy().reshape(sh),
        beh.cpu().numpy().reshape(sh), out["lp_ref"].cpu().numpy().reshape(sh),
        mask_h.reshape(sh), 0.2, 1e-6, 0.04)
    assert err == 0
    np.testing.assert_allclose(out["stats"].cpu().numpy(), st_or, rtol=1e-4, atol=1e-6)
    dlp = out["dlp"].cpu().numpy()
    np.testing.assert_allclose(dlp, dlp_or.reshape(S, N), rtol=1e-4, atol=1e-9)
    assert (dlp[mask_h == 0] == 0).all()
