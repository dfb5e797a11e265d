"""GRPO loss kernel (sm_grpo_loss) vs the f64 CPU oracle and the reference goldens."""
import math

import numpy as np
import pytest
import torch

import oracle
from summa_amd import ops

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.tensor(np.asarray(a, dtype=np.float32), device=dev)


def test_golden_clipping(dev):
    # posttrain.rs:5173-5204 / :5240-5256 (tensor core == scalar golden, 1e-6)
    loss = ops.grpo_loss_tensor(_t([1.0, 0.0], dev), _t([[math.log(1.5)], [math.log(0.5)]], dev),
                                _t([[0.0], [0.0]], dev), None, _t([[1.0], [1.0]], dev),
                                0.2, 1e-6, 0.0)
    assert abs(float(loss.cpu()[0]) + 0.2) < 1e-6


def test_golden_kl(dev):
    # posttrain.rs:5207-5237
    out = ops.grpo_loss_batched(_t([[1.0, 0.0]], dev), _t([[[0.0], [0.0]]], dev),
                                _t([[[0.0], [0.0]]], dev), _t([[[math.log(2)], [math.log(2)]]], dev),
                                None, 0.2, 1e-6, 0.5)
    kl = 2.0 - math.log(2.0) - 1.0
    s = out["stats"].cpu().numpy()[0]
    d = out["dlp"].cpu().numpy()[0, :, 0]
    assert abs(s[3] - kl) < 1e-6 and abs(s[0] - 0.5 * kl) < 1e-6
    assert abs(d[0] + 0.75) < 1e-6 and abs(d[1] - 0.25) < 1e-6


@pytest.mark.parametrize("B,G,T,ragged", [(4, 8, 64, False), (32, 8, 512, True), (3, 2, 1, False),
                                          (2, 16, 300, True)])
def test_matches_oracle(dev, B, G, T, ragged):
    print(f"case B={B} G={G} T={T} ragged={ragged}", flush=True)
    rng = np.random.default_rng(B * 100 + T)
    cur = rng.normal(-3, 1, (B, G, T)).astype(np.float32)
    beh = (cur + rng.normal(0, 0.3, (B, G, T))).astype(np.float32)
    ref = (cur + rng.normal(0, 0.2, (B, G, T))).astype(np.float32)
    r = rng.binomial(1, 0.3, (B, G)).astype(np.float32)
    r[0] = rng.uniform(0, 1, G)
    mask = np.ones((B, G, T), np.float32)
    if ragged:
        for b in range(B):
            for g in range(G):
                mask[b, g, rng.integers(1, T + 1):] = 0
    out = ops.grpo_loss_batched(_t(r, dev), _t(cur, dev), _t(beh, dev), _t(ref, dev),
                                _t(mask, dev), 0.2, 1e-6, 0.04)
    stats, adv, dlp, err = oracle.grpo_loss(r, cur, beh, ref, mask, 0.2, 1e-6, 0.04)
    assert err == 0
    # loss and advantages within 1e-4 relative (BASELINE bound); stats from f64 math
    np.testing.assert_allclose(out["advantages"].cpu().numpy(), adv, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(out["stats"].cpu().numpy(), stats, rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(out["dlp"].cpu().numpy(), dlp, rtol=1e-4, atol=1e-9)


@pytest.mark.parametrize("case,msg", [
    ("fractional_mask", "GRPO active_mask must contain only binary zero/one values"),
    ("empty_mask", "GRPO active_mask must contain at least one active token in every rollout"),
    ("unsafe_ratio", "GRPO importance log-ratio exceeds the safe exponential domain"),
    ("nan_reward", "GRPO rewards contain a non-finite value"),
])
def test_rejections(dev, case, msg):
    G, T = 2, 3
    r = np.array([1.0, 0.0])
    cur = np.zeros((G, T))
    beh = np.zeros((G, T))
    mask = np.ones((G, T))
    if case == "fractional_mask":
        mask[0, 1] = 0.5
    elif case == "empty_mask":
        mask[1] = 0
    elif case == "unsafe_ratio":
        cur[0, 0] = 81
    elif case == "nan_reward":
        r[0] = np.nan
    with pytest.raises(ops.GrpoValidationError, match=msg):
        ops.grpo_loss_tensor(_t(r, dev), _t(cur, dev), _t(beh, dev), None, _t(mask, dev),
                             0.2, 1e-6, 0.0)
