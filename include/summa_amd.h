/*
 * summa_amd — C ABI of the MI355X (gfx950) RL-step engine.
 *
 * Every entry point takes caller-owned, contiguous device buffers (plain
 * pointers and sizes) plus an opaque HIP stream (`void* stream`, a
 * hipStream_t; NULL = the null stream). Calls enqueue work and return without
 * synchronising unless stated. Return value: SM_OK (0) or a negative
 * sm_status; sm_last_error() gives the calling thread's last message. Nothing
 * aborts or throws across this boundary.
 *
 * Each declaration cites the reference interface (SpaceFrontiers/summa) it
 * replaces as `path:line`.
 */
#ifndef SUMMA_AMD_H
#define SUMMA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum sm_status {
  SM_OK = 0,
  SM_ERR_INVALID = -1,     /* bad shape / argument: reference would panic or bail */
  SM_ERR_HIP = -2,         /* HIP runtime error */
  SM_ERR_UNSUPPORTED = -3, /* shape outside what the kernels implement */
  SM_ERR_NUMERIC = -4      /* device-side validation failed (non-finite, ratio > 80, ...) */
} sm_status;

typedef enum sm_dtype { SM_F32 = 0, SM_BF16 = 1, SM_F16 = 2 } sm_dtype;

/* Library identity / diagnostics. */
int sm_version(void);
const char* sm_last_error(void);

/* ------------------------------------------------------------------------
 * Fused row-wise log-softmax / cross-entropy / token log-prob.
 * Replaces LinearCrossEntropyBackend::linear_cross_entropy_inner's row
 * kernels ce_row_statistics + ce_row_gradient
 * (summa-llm/src/model/linear_cross_entropy/gpu.rs:29-158, mod.rs:33-57) and
 * the log_softmax(...).gather(targets) of the GRPO log-prob recompute
 * (summa-train/src/tensor_sleep.rs:2609-2614).
 *
 * logits: [rows, stored_vocab] of `dtype` (SM_BF16 or SM_F32). Only columns
 *   < logical_vocab are read (padded columns have probability exactly 0).
 * targets: [rows] int32 in [0, logical_vocab).
 * token_logprob (nullable): [rows] f32, log_softmax(row)[target].
 * row_lse (nullable): [rows] f32, log-sum-exp of the row.
 * grad (nullable): if non-NULL it must equal `logits` (in-place); receives
 *   (softmax - onehot(target)) * grad_scale * (row_scale ? row_scale[r] : 1)
 *   in `dtype`; padded columns receive exact zeros.
 * loss (nullable): [1] f32 = mean over rows of -token_logprob (needs
 *   token_logprob non-NULL). Deterministic (fixed-order reduction).
 */
int sm_ce_rows(const void* logits, int dtype, const int32_t* targets, int64_t rows,
               int64_t stored_vocab, int64_t logical_vocab, float* token_logprob,
               float* row_lse, void* grad, float grad_scale, const float* row_scale,
               float* loss, void* stream);

/* ------------------------------------------------------------------------
 * GRPO clipped policy-gradient + k3-KL loss, batched over prompt groups.
 * Replaces grpo_loss_tensor (summa-train/src/posttrain.rs:874-1028) and
 * follows the scalar oracle grpo_loss (posttrain.rs:720-868) for the
 * per-token gradient d loss / d current_log_prob.
 *
 * rewards [groups*G] f32; lp_cur, lp_beh, lp_ref (nullable), mask (nullable =
 * all active): [groups*G*T] f32. Advantages are normalised within each group.
 * group_stats (nullable) [groups*5] f32: loss, mean_reward, reward_stddev,
 *   mean_kl, clipped_fraction (as in GrpoLoss, posttrain.rs:706-717).
 * advantages (nullable) [groups*G] f32; dlp (nullable) [groups*G*T] f32.
 * flags (nullable) [groups] int32: validation bitmask (SM_GRPO_* below),
 *   0 when every check of grpo_loss_tensor passes. Decode on the host with
 *   sm_grpo_flags_message().
 */
enum {
  SM_GRPO_BAD_REWARD = 1 << 0,
  SM_GRPO_BAD_CURRENT = 1 << 1,
  SM_GRPO_BAD_BEHAVIOR = 1 << 2,
  SM_GRPO_MASK_NOT_BINARY = 1 << 3,
  SM_GRPO_MASK_EMPTY_ROW = 1 << 4,
  SM_GRPO_RATIO_NONFINITE = 1 << 5,
  SM_GRPO_RATIO_UNSAFE = 1 << 6,
  SM_GRPO_REWARD_OVERFLOW = 1 << 7,
  SM_GRPO_LOSS_OVERFLOW = 1 << 8,
  SM_GRPO_BAD_REFERENCE = 1 << 9,
  SM_GRPO_REF_RATIO_NONFINITE = 1 << 10,
  SM_GRPO_REF_RATIO_UNSAFE = 1 << 11
};
int sm_grpo_loss(const float* rewards, const float* lp_cur, const float* lp_beh,
                 const float* lp_ref, const float* mask, int64_t groups, int64_t group_size,
                 int64_t tokens, double clip_epsilon, double advantage_epsilon,
                 double kl_coefficient, float* group_stats, float* advantages, float* dlp,
                 int32_t* flags, void* stream);
/* Host-only: message of the first set validation bit (reference wording,
 * posttrain.rs:976-1006), or NULL when flags == 0. */
const char* sm_grpo_flags_message(int32_t flags);

/* ------------------------------------------------------------------------
 * Q4G128 weights (this build's HQUANT format tag 4): W[N, K] row-major
 * (out x in), groups of 128 along the flattened tensor, one bf16 scale per
 * group = bf16(absmax/7), int4 two's-complement codes, low nibble = even
 * element. codes: ceil(n/128)*64 bytes; scales: ceil(n/128) bf16.
 *
 * sm_q4_quantize replaces quantize_tensor (summa-train/src/quantization.rs:
 * 691-773) for the new format: code = clamp(round_half_away(w/scale), -8, 7).
 * bad_scales (nullable, device int32, caller-zeroed) counts groups whose
 * non-zero scale is outside the f16 normal range that the matmul needs.
 */
int sm_q4_quantize(const void* w, int dtype, int64_t n, uint8_t* codes, uint16_t* scales,
                   int32_t* bad_scales, void* stream);

/* y = x . W^T over Q4G128 weights, bf16 x [M, ldx], f32 accumulate. Replaces
 * the quantized-matmul dispatch: PackedTensor::matrix_vector
 * (quantization.rs:630-654) batched over M rows, i.e. Linear::forward
 * (summa-llm/src/model/matmul.rs:57-66) on a QuantizedModelBackend weight
 * (quantization.rs:1183-1189). K % 128 == 0. Epilogues:
 *   SM_EPI_STORE_F32   y f32 [M, ldy] = acc
 *   SM_EPI_STORE_BF16  y bf16 = acc
 *   SM_EPI_ADD_F32     y f32 += acc  (residual add, block.rs:103-157)
 *   SM_EPI_SWIGLU_BF16 W rows are [gate | value] (N = 2F); y bf16 [M, F] =
 *                      silu(gate) * value (ffn.rs:854-877, fused_swiglu.rs:110-126)
 */
enum { SM_EPI_STORE_F32 = 0, SM_EPI_STORE_BF16 = 1, SM_EPI_ADD_F32 = 2, SM_EPI_SWIGLU_BF16 = 3 };
int sm_q4_matmul(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                 const uint16_t* x, int64_t M, int64_t ldx, void* y, int64_t ldy, int epilogue,
                 void* stream);

/* ------------------------------------------------------------------------
 * Seeded synthetic data (no reference counterpart; bench/test inputs).
 * Values are a pure function of (seed, index), identical for any launch shape.
 */
int sm_fill_normal(void* out, int dtype, int64_t n, float mean, float std, uint64_t seed,
                   void* stream);
/* Config[3]-style CE stress rows: logits[r, :] ~ N(0, std) and
 * logits[r, targets[r]] += spike, targets[r] uniform in [0, vocab). */
int sm_fill_ce_stress(void* logits, int dtype, int32_t* targets, int64_t rows, int64_t vocab,
                      float std, float spike, uint64_t seed, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SUMMA_AMD_H */
