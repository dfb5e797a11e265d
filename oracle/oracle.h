/*
 * CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's CPU path for the GRPO RL step.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker; the product path (summa_amd) never links
 * or calls it.
 *
 * Each function cites the reference file:line it restates. Parity pins (the
 * golden vectors and closed forms that check each function) are listed in
 * tests/test_oracle.py; functions without one say "parity unpinned".
 */
#ifndef SUMMA_ORACLE_H
#define SUMMA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* OpenMP thread count of the oracle's parallel loops (n <= 0: every core). */
void or_set_threads(int n);
int or_max_threads(void);

/* bf16 <-> f32 (round to nearest even), the rounding the device path uses. */
float or_bf16_to_f32(uint16_t b);
uint16_t or_f32_to_bf16(float f);
void or_bf16_bits(const float* x, int64_t n, uint16_t* out); /* elementwise or_f32_to_bf16 */
/* f32 -> nearest IEEE binary16 value (ties to even, subnormals, overflow to
 * inf), returned as f32. */
float or_round_f16(float f);

/* Row-wise log-softmax / CE in f64, two passes.
 * linear_cross_entropy/reference.rs:21-92 (mask_padded_logits + chunked_loss)
 * and gpu.rs:29-158 (row statistics / gradient). logits are f32 (dtype 0) or
 * bf16 bits (dtype 1); grad (nullable) is f32 [rows, stored]. */
void or_ce_rows(const void* logits, int dtype, const int32_t* targets, int64_t rows,
                int64_t stored, int64_t logical, double* lp, double* lse, float* grad,
                double grad_scale, const double* row_scale);

/* GRPO loss per group: posttrain.rs:720-868 (scalar grpo_loss) extended with
 * the active mask of grpo_loss_tensor (posttrain.rs:874-1028).
 * stats [groups*5]: loss, mean_reward, reward_stddev, mean_kl, clipped_fraction.
 * Returns 0, or the first validation failure code (SM_GRPO_* bit). */
int or_grpo_loss(const double* rewards, const double* lp_cur, const double* lp_beh,
                 const double* lp_ref, const double* mask, int64_t groups, int64_t G,
                 int64_t T, double clip, double adv_eps, double beta, double* stats,
                 double* adv, double* dlp);

/* Q4G128 codec (format tag 4 in the HQUANT family, defined by this build):
 * weight [rows, cols] row-major, groups of 128 over the flattened tensor
 * (quantization.rs:691-773 grouping), signed int4 two's-complement codes, low
 * nibble = even element, one bf16 scale per group = bf16(absmax / 7),
 * code = clamp(round_half_away(w / scale), -8, 7). */
void or_q4_quantize(const float* w, int64_t n, uint8_t* codes, uint16_t* scales);
void or_q4_decode(const uint8_t* codes, const uint16_t* scales, int64_t n, float* out);
/* y[r] = sum_c value(r*cols+c) * x[c], sequential f32 accumulation
 * (PackedTensor::matrix_vector, quantization.rs:630-654). */
void or_q4_matvec(const uint8_t* codes, const uint16_t* scales, int64_t rows, int64_t cols,
                  const float* x, float* y);

/* Sampling with the TextGenerator options (model.c; generate.rs:127-250).
 * or_apply_penalty: apply_repetition_penalty (:155-182); -1 for a token outside
 * [0, V). or_sample_ex_row: one row of select_next_token with top-k, penalty,
 * greedy and the opt-in nucleus filter (parity unpinned for the nucleus part:
 * the reference has no nucleus sampler). */
int or_apply_penalty(float* values, int64_t V, const int32_t* prior, int64_t n, float penalty);
int or_sample_ex_row(const float* logits, int64_t V, float temperature, int top_k, float penalty,
                     float top_p, int apply_top_p, uint64_t seed, int64_t row, int64_t step,
                     const int32_t* prior, int64_t n, int32_t* tok, double* lp);

/* HQUANT codec (hquant.c; quantization.rs:445-773, :934-978, :2274-2281). */
uint16_t or_f32_to_f16_bits(float f);
float or_f16_bits_to_f32(uint16_t b);
uint64_t or_fnv1a64(const uint8_t* p, int64_t n);
int64_t or_hq_bytes_per_group(int format);
int or_hq_quantize(const float* v, int64_t n, int format, uint16_t* scales, uint8_t* codes);
void or_hq_decode(int format, int64_t n, const uint16_t* scales, const uint8_t* codes,
                  float* out);

#ifdef __cplusplus
}
#endif
#endif
