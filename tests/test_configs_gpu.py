"""The RL step of configs [0], [1], [2] and [4] at their full workloads on the GPU.

Each case runs one whole GRPO step at the config's depth, width, vocabulary,
batch and lengths (rollout generation, log-prob recompute of the policy and
its frozen copy, the GRPO loss) and checks:

* size-independent properties over the whole batch: token ids in range,
  every log-prob finite and <= 0, the decode-time (behaviour) log-probs equal
  to the recompute within 2e-3 (two kernel paths: the cached decode and the
  prefill-style recompute; the cached == stateless invariant of
  summa-llm/src/model/mod.rs:143-179), the frozen copy's log-probs bitwise
  equal to the policy's (so KL = 0 and rho = exp(lp_cur - lp_beh) ~ 1), no
  clipped tokens, advantages summing to 0 in every group;
* the GRPO loss on the full [S, N] arrays against the oracle's f64
  ``grpo_loss`` (posttrain.rs:720-868) at 1e-4 relative;
* two rollouts (the first and the last) against the CPU oracle at full depth
  and full length: per-token log-probs of both paths within 2e-3 (1e-5 for
  the fp32 config[0]), and every sampled token equal to the sampler's choice
  on the oracle's logits up to a near-tie.

The MoE config adds router near-ties: a token whose top-2 expert set is
decided by less than the two paths' rounding differences can pick different
experts in the decode and recompute paths (and the oracle). Its checks allow
that for a few rollouts and name each one.
"""
import numpy as np
import pytest
import torch

import oracle
from summa_amd.configs import ADVANTAGE_EPSILON, CLIP_EPSILON, KL_COEFFICIENT, RL_WORKLOADS
from summa_amd.model import batch_result, rl_prepare

from _workloads import build_models, check_sampled_tokens

pytestmark = pytest.mark.gpu

SEED = 7
# A router near-tie: second- and third-largest router logits closer than
# ROUTER_TIE in some layer at the first disagreeing token or the one before
# it. The two device paths (and the oracle) agree on the residual stream to a
# few 1e-5 relative, but their f16 K/V roundings differ by an ulp here and
# there, which moves router logits (~N(0, 1)) by up to ~1e-4: a top-2 set can
# flip only at a margin of that order. A margin under 1e-3 at two given
# tokens in one of 16 layers has a probability of about 10 %, so a
# disagreement without one points at a bug.
ROUTER_TIE = 1e-3
ROUTER_WINDOW = 1


def _run_step(wl, dev):
    mc, (policy, reference), host_w = build_models(wl, dev, seed=wl.index)
    gen = torch.Generator().manual_seed(wl.index)
    S, P, N = wl.rollouts, wl.prompt_len, wl.new_tokens
    prompts = torch.randint(0, mc.vocab, (S, P), generator=gen, dtype=torch.int32).to(dev)
    rewards = wl.sample_rewards(gen).to(dev)
    tok, lp_beh = policy.generate(prompts, N, temperature=wl.temperature, seed=SEED)
    out = rl_prepare(policy, reference, prompts, tok, lp_beh, rewards, clip_epsilon=CLIP_EPSILON,
                     advantage_epsilon=ADVANTAGE_EPSILON, kl_coefficient=KL_COEFFICIENT)
    res = batch_result(out)
    torch.cuda.synchronize()
    arrays = {k: v.cpu().numpy() for k, v in out.items() if v is not None}
    arrays.update(prompts=prompts.cpu().numpy(), tokens=tok.cpu().numpy(),
                  lp_beh=lp_beh.cpu().numpy(), rewards=rewards.cpu().numpy())
    del policy, reference
    torch.cuda.empty_cache()
    return mc, host_w, arrays, res


@pytest.mark.timeout(600)
@pytest.mark.parametrize("index", [0, 1, 2])
def test_full_workload_rl_step(dev, index):
    wl = RL_WORKLOADS[index]
    S, P, N, G = wl.rollouts, wl.prompt_len, wl.new_tokens, wl.group
    print(f"case config[{index}] full workload: S={S} P={P} N={N} layers={wl.model['layers']}",
          flush=True)
    mc, host_w, a, res = _run_step(wl, dev)
    V = mc.vocab
    tok, lp_beh, lp_cur, lp_ref = a["tokens"], a["lp_beh"], a["lp_cur"], a["lp_ref"]
    moe = bool(mc.experts)
    lp_tol = 2e-3 if wl.quantized else 1e-5

    # ---- whole-batch properties
    assert tok.shape == (S, N) and tok.min() >= 0 and tok.max() < V
    for name, lp in (("behaviour", lp_beh), ("recompute", lp_cur)):
        assert np.isfinite(lp).all(), f"{name} log-probs not finite"
        assert (lp <= 0).all(), f"{name} log-probs > 0: {lp.max()}"
    assert np.array_equal(lp_ref, lp_cur), "frozen copy with equal weights must match bitwise"
    dev_path = np.abs(lp_beh.astype(np.float64) - lp_cur).max(1)
    off = np.nonzero(dev_path > lp_tol)[0]
    print(f"max |behaviour - recompute| {dev_path.max():.2e} (median rollout "
          f"{np.median(dev_path):.2e}); rollouts over {lp_tol}: {off.tolist()}", flush=True)
    if not moe:
        assert off.size == 0
    host = oracle.HostModel(mc.oracle_cfg(), host_w, quantized=wl.quantized)
    del host_w
    if moe and off.size:
        # Each such rollout must have a router near-tie at (or just before)
        # its first token where the two paths disagree: the top-2 expert set
        # there is decided by less than the paths' rounding differences.
        assert off.size <= S // 4, f"too many rollouts off: {off.tolist()}"
        gaps = host.router_gaps(np.concatenate([a["prompts"][off], tok[off, :N - 1]], 1))
        for i, s in enumerate(off):
            n0 = int(np.argmax(np.abs(lp_beh[s].astype(np.float64) - lp_cur[s]) > lp_tol))
            window = gaps[:, i, max(0, P - 1 + n0 - ROUTER_WINDOW):P + n0]
            print(f"rollout {s}: paths disagree from token {n0}; smallest router gap at and "
                  f"before it {window.min():.2e}", flush=True)
            assert window.min() < ROUTER_TIE, f"rollout {s} token {n0}: no router near-tie"
    assert (a["flags"] == 0).all()
    stats = a["stats"]
    assert np.isfinite(stats).all()
    assert res["mean_kl_sum"] == 0.0
    assert res["clipped_fraction_sum"] == 0.0 or moe

    # ---- GRPO loss on the full arrays against the f64 oracle
    groups = wl.prompts
    sh = (groups, G, N)
    st_or, adv_or, dlp_or, err = oracle.grpo_loss(
        a["rewards"].astype(np.float64), lp_cur.reshape(sh).astype(np.float64),
        lp_beh.reshape(sh).astype(np.float64), lp_ref.reshape(sh).astype(np.float64), None,
        CLIP_EPSILON, ADVANTAGE_EPSILON, KL_COEFFICIENT)
    assert err == 0
    np.testing.assert_allclose(stats[:, 1:3], st_or[:, 1:3], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(stats[:, 0], st_or[:, 0], rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(stats[:, 3:], st_or[:, 3:], rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(a["dlp"], dlp_or.reshape(S, N), rtol=1e-4, atol=1e-9)
    adv = np.asarray(adv_or).reshape(groups, G)
    assert np.abs(adv.sum(1)).max() < 1e-4 * G
    r = a["rewards"].astype(np.float64)
    sd = r.std(1)
    expect = (r - r.mean(1, keepdims=True)) / np.maximum(sd, ADVANTAGE_EPSILON)[:, None]
    np.testing.assert_allclose(adv, expect, rtol=1e-6, atol=1e-9)

    # ---- two rollouts at full depth and length against the oracle
    rows = [0, S - 1]
    lp_or, logits_or = host.continuation(a["prompts"][rows], tok[rows])
    err_cur = np.abs(lp_cur[rows] - lp_or).max(1)
    err_beh = np.abs(lp_beh[rows] - lp_or).max(1)
    print(f"oracle rollouts {rows}: max |recompute - oracle| {err_cur.tolist()}, "
          f"|behaviour - oracle| {err_beh.tolist()}", flush=True)
    # MoE: a rollout may leave the comparison at its first token off the
    # oracle only at a router near-tie there (as above)
    upto = [N, N]
    if moe:
        gaps = host.router_gaps(np.concatenate([a["prompts"][rows], tok[rows, :N - 1]], 1))
        for i, s in enumerate(rows):
            bad = np.nonzero((np.abs(lp_cur[s] - lp_or[i]) > lp_tol) |
                             (np.abs(lp_beh[s] - lp_or[i]) > lp_tol))[0]
            if bad.size:
                n0 = int(bad[0])
                window = gaps[:, i, max(0, P - 1 + n0 - ROUTER_WINDOW):P + n0]
                print(f"rollout {s}: off the oracle from token {n0}; smallest router gap at "
                      f"and before it {window.min():.2e}", flush=True)
                assert window.min() < ROUTER_TIE, f"rollout {s} token {n0}: no router near-tie"
                upto[i] = n0
    else:
        assert err_cur.max() <= lp_tol and err_beh.max() <= lp_tol
    ties = 0
    for i in range(2):
        if upto[i]:
            ties += check_sampled_tokens(tok[rows[i]:rows[i] + 1, :upto[i]],
                                         logits_or[i:i + 1, :upto[i]], wl.temperature, SEED,
                                         [rows[i]], tol=4e-3 if wl.quantized else 1e-4)
    print(f"sampled tokens: {sum(upto)} checked, {ties} at near-ties", flush=True)
