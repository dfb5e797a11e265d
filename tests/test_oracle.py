"""Pins the CPU oracle against the reference's golden vectors and closed forms.

Every oracle function used as a checker has at least one check here that a
plausible mistake (dropped term, wrong sign, transposed operand) would fail.
"""
import math

import numpy as np
import pytest
from scipy.special import log_softmax

import oracle


# ------------------------------------------------------------------ GRPO ---
# Golden literals from summa-train/src/posttrain.rs:5173-5256.

def test_grpo_golden_group_normalization_and_clipping():
    # posttrain.rs:5173-5204: lp = [ln 1.5], [ln 0.5], behavior 0, rewards [1, 0], beta 0.
    stats, adv, dlp, err = oracle.grpo_loss(
        rewards=[[1.0, 0.0]], lp_cur=[[[math.log(1.5)], [math.log(0.5)]]],
        lp_beh=[[[0.0], [0.0]]], lp_ref=None, clip=0.2, adv_eps=1e-6, beta=0.0)
    assert err == 0
    loss, mean_r, std_r, kl, clipped = stats[0]
    assert abs(mean_r - 0.5) < 1e-12 and abs(std_r - 0.5) < 1e-12
    assert list(adv[0]) == [1.0, -1.0]
    assert abs(loss - (-0.2)) < 1e-12
    assert abs(clipped - 1.0) < 1e-12
    assert abs(dlp[0, 0, 0]) < 1e-12 and abs(dlp[0, 1, 0]) < 1e-12


def test_grpo_unclipped_gradient_and_kl_estimator_are_exact():
    # posttrain.rs:5207-5237: lp = lp_beh = 0, lp_ref = ln 2, beta 0.5.
    stats, adv, dlp, err = oracle.grpo_loss(
        rewards=[[1.0, 0.0]], lp_cur=[[[0.0], [0.0]]], lp_beh=[[[0.0], [0.0]]],
        lp_ref=[[[math.log(2.0)], [math.log(2.0)]]], clip=0.2, adv_eps=1e-6, beta=0.5)
    assert err == 0
    kl = 2.0 - math.log(2.0) - 1.0
    assert abs(stats[0, 3] - kl) < 1e-12
    assert abs(stats[0, 0] - 0.5 * kl) < 1e-12
    assert abs(dlp[0, 0, 0] - (-0.75)) < 1e-12
    assert abs(dlp[0, 1, 0] - 0.25) < 1e-12


def test_grpo_tensor_core_masked_equals_unpadded():
    # grpo_loss_tensor masks padding (posttrain.rs:957-961): a padded batch must
    # equal the scalar oracle on the unpadded rollouts, with zero padded grads.
    rng = np.random.default_rng(3)
    G, lens = 4, [5, 2, 7, 3]
    T = max(lens)
    cur = rng.normal(-2, 0.3, (1, G, T))
    beh = cur + rng.normal(0, 0.1, (1, G, T))
    ref = cur + rng.normal(0, 0.1, (1, G, T))
    mask = np.zeros((1, G, T))
    for i, n in enumerate(lens):
        mask[0, i, :n] = 1
    r = rng.uniform(0, 1, (1, G))
    stats, adv, dlp, err = oracle.grpo_loss(r, cur, beh, ref, mask)
    assert err == 0
    # brute force on unpadded rollouts, straight from the formulas
    mean = r.mean()
    sd = math.sqrt(((r - mean) ** 2).mean())
    A = (r[0] - mean) / max(sd, 1e-6)
    obj = 0.0
    for i, n in enumerate(lens):
        c, b, f = cur[0, i, :n], beh[0, i, :n], ref[0, i, :n]
        rho = np.exp(c - b)
        surr = np.minimum(rho * A[i], np.clip(rho, 0.8, 1.2) * A[i])
        kl = np.exp(f - c) - (f - c) - 1
        obj += (surr - 0.04 * kl).mean() / G
        act = ((A[i] >= 0) & (rho <= 1.2)) | ((A[i] < 0) & (rho >= 0.8))
        g = (-(act * rho * A[i]) + 0.04 * (1 - np.exp(f - c))) / (G * n)
        np.testing.assert_allclose(dlp[0, i, :n], g, rtol=1e-12, atol=1e-15)
        assert np.all(dlp[0, i, n:] == 0)
    assert abs(stats[0, 0] - (-obj)) < 1e-12


@pytest.mark.parametrize("case,expect", [
    ("fractional_mask", 1 << 3), ("empty_mask", 1 << 4), ("unsafe_ratio", 1 << 6),
    ("nan_reward", 1 << 0), ("nan_current", 1 << 1), ("unsafe_ref", 1 << 11),
])
def test_grpo_rejections(case, expect):
    # posttrain.rs:5258-5435 rejection cases.
    G, T = 2, 3
    r = np.array([[1.0, 0.0]])
    cur = np.zeros((1, G, T))
    beh = np.zeros((1, G, T))
    ref = np.zeros((1, G, T))
    mask = np.ones((1, G, T))
    if case == "fractional_mask":
        mask[0, 0, 1] = 0.5
    elif case == "empty_mask":
        mask[0, 1, :] = 0
    elif case == "unsafe_ratio":
        cur[0, 0, 0] = 81.0
    elif case == "nan_reward":
        r[0, 0] = np.nan
    elif case == "nan_current":
        cur[0, 1, 2] = np.nan
    elif case == "unsafe_ref":
        ref[0, 0, 0] = 100.0
    _, _, _, err = oracle.grpo_loss(r, cur, beh, ref, mask)
    assert err & expect


def test_grpo_equal_rewards_give_zero_advantage():
    stats, adv, dlp, err = oracle.grpo_loss([[0.3] * 8], np.zeros((1, 8, 4)), np.zeros((1, 8, 4)),
                                            np.zeros((1, 8, 4)))
    assert err == 0 and np.all(adv == 0) and stats[0, 0] == 0 and np.all(dlp == 0)


# -------------------------------------------------------------------- CE ---

def _ce_inputs(rows, vocab, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 3, (rows, vocab)).astype(np.float32)
    t = rng.integers(0, vocab, rows).astype(np.int32)
    return x, t


def test_ce_matches_library_log_softmax():
    x, t = _ce_inputs(9, 1000)
    lp, lse, _ = oracle.ce_rows(x, t)
    ref = log_softmax(x.astype(np.float64), axis=1)[np.arange(9), t]
    np.testing.assert_allclose(lp, ref, rtol=0, atol=1e-12)


def test_ce_padded_columns_ignored_and_zero_grad():
    # linear_cross_entropy/tests.rs:19-126: stored {11, 16} with logical 11 must
    # agree with the unpadded computation; padded gradients are exactly zero.
    rows, lv = 7, 11
    targets = np.array([0, 3, 7, 2, 10, 4, 1], np.int32)
    hidden = (np.sin(np.arange(rows * 5) * 0.071) * 0.2).reshape(rows, 5).astype(np.float32)
    for stored in (11, 16):
        w = (np.cos(np.arange(stored * 5) * 0.113) * 0.3).reshape(stored, 5).astype(np.float32)
        logits = np.ascontiguousarray(hidden @ w.T)
        if stored > lv:
            logits[:, lv:] = 1e4  # garbage in padding must not matter
        lp, _, g = oracle.ce_rows(logits, targets, lv, grad=True, grad_scale=1.0 / rows)
        ref = log_softmax(logits[:, :lv].astype(np.float64), axis=1)[np.arange(rows), targets]
        np.testing.assert_allclose(lp, ref, atol=1e-12)
        assert np.all(g[:, lv:] == 0)
        # gradient closed form: (softmax - onehot)/rows; rows of the grad sum to 0
        p = np.exp(log_softmax(logits[:, :lv].astype(np.float64), axis=1))
        p[np.arange(rows), targets] -= 1
        np.testing.assert_allclose(g[:, :lv], p / rows, atol=1e-7)


def test_ce_closed_forms():
    # uniform row -> lp = -ln V ; spiked row -> lp = 8 - ln(V - 1 + e^8)
    V = 4096
    x = np.zeros((2, V), np.float32)
    x[1, 5] = 8.0
    lp, lse, _ = oracle.ce_rows(x, np.array([17, 5], np.int32))
    assert abs(lp[0] + math.log(V)) < 1e-12
    assert abs(lp[1] - (8 - math.log(V - 1 + math.exp(8)))) < 1e-12


def test_ce_bf16_input_matches_f32_of_rounded():
    x, t = _ce_inputs(4, 333, seed=1)
    b = oracle.bf16_bits(x)
    lp_b, _, _ = oracle.ce_rows(b, t)
    lp_f, _, _ = oracle.ce_rows(oracle.bf16_to_f32(b), t)
    np.testing.assert_array_equal(lp_b, lp_f)


def test_bf16_rounding_known_values():
    assert oracle.bf16_bits(np.array([1.0], np.float32))[0] == 0x3F80
    assert oracle.bf16_bits(np.array([1.005859375], np.float32))[0] == 0x3F81  # rounds up
    assert oracle.bf16_bits(np.array([1.00390625], np.float32))[0] == 0x3F80
    assert oracle.bf16_bits(np.array([1.01171875], np.float32))[0] == 0x3F82  # tie -> even
    assert oracle.bf16_bits(np.array([-2.5], np.float32))[0] == 0xC020


# ---------------------------------------------------------------- Q4G128 ---

def _codec_weights(n):
    # summa-train/src/quantization.rs:2287-2291 generator
    i = np.arange(n, dtype=np.float32)
    return (np.sin(i * np.float32(0.37)) * 2 + (np.arange(n) % 7) * np.float32(0.01)).astype(np.float32)


def test_q4_roundtrip_is_scale_times_code():
    w = _codec_weights(256 * 3)
    codes, scales = oracle.q4_quantize(w)
    assert codes.size == w.size // 2 and scales.size == w.size // 128
    dec = oracle.q4_decode(codes, scales, w.size)
    s = np.repeat(oracle.bf16_to_f32(scales), 128)
    q = dec / s
    assert np.all(q == np.round(q)) and q.min() >= -8 and q.max() <= 7
    # each group's absmax element maps to |code| 7 (scale = bf16(absmax/7))
    for g in range(w.size // 128):
        seg = w[g * 128:(g + 1) * 128]
        assert abs(q[g * 128 + np.argmax(np.abs(seg))]) == 7
    # quantisation error bounded by half a step (plus bf16 scale rounding)
    assert np.all(np.abs(dec - w) <= 0.5 * s * 1.0001 + np.abs(w) * 2 ** -8)


def test_q4_nibble_layout_and_twos_complement():
    # element 0 -> low nibble, element 1 -> high nibble; -1 stored as 0xF.
    w = np.zeros(128, np.float32)
    w[0], w[1], w[2], w[3] = 7.0, -7.0, -1.0, 3.0
    codes, scales = oracle.q4_quantize(w)
    assert oracle.bf16_to_f32(scales)[0] == 1.0
    assert codes[0] == 0x97  # low 7, high -7 = 0x9
    assert codes[1] == 0x3F  # low -1 = 0xF, high 3
    assert np.all(codes[2:] == 0)


def test_q4_partial_group_padded_in_storage_only():
    # quantization.rs:2571-2589: a 137-element tensor has 2 groups; decode
    # returns exactly 137 values.
    w = _codec_weights(137)
    codes, scales = oracle.q4_quantize(w)
    assert scales.size == 2 and codes.size == 128
    assert oracle.q4_decode(codes, scales, 137).size == 137


def test_q4_matvec_equals_decode_times_x():
    # quantization.rs:2591-2618: matrix_vector == decode . x within 1e-5.
    rows, cols = 6, 256
    w = _codec_weights(rows * cols)
    codes, scales = oracle.q4_quantize(w)
    x = np.cos(np.arange(cols) * 0.3).astype(np.float32)
    y = oracle.q4_matvec(codes, scales, rows, cols, x)
    dense = oracle.q4_decode(codes, scales, rows * cols).reshape(rows, cols).astype(np.float64)
    np.testing.assert_allclose(y, dense @ x, atol=1e-5)
    # transposed operand would differ
    assert not np.allclose(y, (dense.T[:rows, :rows] @ x[:rows]), atol=1e-3)


def test_f16_rounding_matches_numpy_float16():
    # IEEE binary16 round-to-nearest-even incl. subnormals and overflow
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.normal(0, 1, 2000), rng.normal(0, 1e-5, 500), rng.normal(0, 3e4, 500),
                        [65504.0, 65519.0, 65520.0, -70000.0, 0.0, -0.0, 2.0 ** -25, 3 * 2.0 ** -26]])
    v = v.astype(np.float32)
    got = np.array([oracle.lib().or_round_f16(float(x)) for x in v], np.float32)
    np.testing.assert_array_equal(got, v.astype(np.float16).astype(np.float32))
