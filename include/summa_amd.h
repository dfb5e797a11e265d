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

/* SM_F16X2: an f16 pair carrying an fp32-grade activation. A row of K values
 * holds K f16 "hi" values followed by K f16 "lo" values, x = hi + lo with
 * hi = f16(x), lo = f16(x - hi) (about 22 significant bits); the row stride
 * (ldx / ldy) counts f16 elements and is >= 2K. Matmul inputs of quantized
 * models use it so the f16 MFMA path keeps fp32-level activation precision. */
typedef enum sm_dtype { SM_F32 = 0, SM_BF16 = 1, SM_F16 = 2, SM_F16X2 = 3 } sm_dtype;

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
 * Fused linear head + cross-entropy: the LinearCrossEntropyBackend seam
 * (summa-llm/src/model/linear_cross_entropy/mod.rs:33-57) that
 * Dispatch::linear_cross_entropy_inner calls (mod.rs:73), with the chunked
 * semantics of chunked_loss / chunked_backward (reference.rs:42-159) and
 * fused_loss / fused_backward (gpu.rs:264-426). f32 operands, f32-grade
 * GEMMs (sm_gemm_ex), so [chunk, stored_vocab] f32 logits exist only in the
 * workspace.
 *
 * hidden [tokens, d] f32, weight [stored_vocab, d] f32 (Burn's [vocab,
 *   hidden] head weight), bias [stored_vocab] f32 (read only when use_bias),
 *   targets [tokens] int32 in [0, logical_vocab) (the reference's Int tensor,
 *   narrowed), chunk > 0 rows per logits slab.
 * sm_linear_cross_entropy: loss [1] = mean over tokens of
 *   -log_softmax(hidden . W^T + b)[target] over the logical vocabulary
 *   (padded columns masked, mask_padded_logits reference.rs:21-40);
 *   token_logprob (nullable) [tokens] receives each row's log-prob.
 * sm_linear_cross_entropy_backward: grad_output [1] f32 on the device (the
 *   loss's upstream gradient); grad_hidden [tokens, d] =, grad_weight
 *   [stored_vocab, d] =, grad_bias [stored_vocab] = (when use_bias) the
 *   three gradients of linear_cross_entropy_backward; rows >= logical_vocab
 *   of grad_weight / grad_bias are exactly 0.
 * workspace: sm_linear_cross_entropy_workspace_bytes(...) bytes, 256-byte
 *   aligned (-1 for a bad shape); no call allocates.
 * Errors (no panic across the ABI): chunk <= 0 ("linear cross-entropy chunk
 *   size must be positive"), tokens == 0 ("linear cross-entropy requires at
 *   least one token"), logical_vocab outside 1..=stored_vocab.
 */
int64_t sm_linear_cross_entropy_workspace_bytes(int64_t tokens, int64_t d, int64_t stored_vocab,
                                                int64_t chunk, int use_bias);
int sm_linear_cross_entropy(const float* hidden, const float* weight, const float* bias,
                            const int32_t* targets, int64_t tokens, int64_t d,
                            int64_t stored_vocab, int64_t logical_vocab, int64_t chunk,
                            int use_bias, float* loss, float* token_logprob, void* workspace,
                            int64_t workspace_bytes, void* stream);
int sm_linear_cross_entropy_backward(const float* hidden, const float* weight, const float* bias,
                                     const int32_t* targets, const float* grad_output,
                                     int64_t tokens, int64_t d, int64_t stored_vocab,
                                     int64_t logical_vocab, int64_t chunk, int use_bias,
                                     float* grad_hidden, float* grad_weight, float* grad_bias,
                                     void* workspace, int64_t workspace_bytes, void* stream);

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

/* Prepared (tiled) device copy of a Q4G128 weight, the counterpart of
 * prepare_linear_for_inference (summa-llm/src/model/matmul.rs:20-35): 16 rows
 * x one 128-element group form one contiguous 1 KB tile (row r at byte 64*r),
 * tiles ordered [row_block][group]; scales 16 per tile in the same order.
 * Sizes: tiled_codes ceil(N/16)*16 * K/2 bytes, tiled_scales ceil(N/16)*16 *
 * K/128 bf16; rows beyond N are zero. K % 128 == 0. */
int sm_q4_pack(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
               uint8_t* tiled_codes, uint16_t* tiled_scales, void* stream);

/* y = x . W^T over Q4G128 weights in the prepared layout (sm_q4_pack), x [M,
 * ldx] bf16, f16 or f16 pairs (x_dtype SM_F16X2: two f16 MFMAs per step, hi
 * and lo), f32 accumulate. Replaces
 * the quantized-matmul dispatch: PackedTensor::matrix_vector
 * (quantization.rs:630-654) batched over M rows, i.e. Linear::forward
 * (summa-llm/src/model/matmul.rs:57-66) on a QuantizedModelBackend weight
 * (quantization.rs:1183-1189). K % 128 == 0. Epilogues:
 *   SM_EPI_STORE_F32   y f32 [M, ldy] = acc
 *   SM_EPI_STORE_BF16  y bf16 = acc
 *   SM_EPI_ADD_F32     y f32 += acc  (residual add, block.rs:103-157)
 *   SM_EPI_SWIGLU_BF16 W rows are [gate | value] (N = 2F); y bf16 [M, F] =
 *                      silu(gate) * value (ffn.rs:854-877, fused_swiglu.rs:110-126)
 *   SM_EPI_SWIGLU_F16  same with f16 output
 *   SM_EPI_SWIGLU_F16X2 same as an SM_F16X2 row: hi at [m, j], lo at [m, F + j]
 *                      (ldy >= 2F)
 */
enum {
  SM_EPI_STORE_F32 = 0,
  SM_EPI_STORE_BF16 = 1,
  SM_EPI_ADD_F32 = 2,
  SM_EPI_SWIGLU_BF16 = 3,
  SM_EPI_SWIGLU_F16 = 4,
  SM_EPI_SWIGLU_F16X2 = 5
};
int sm_q4_matmul(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                 const void* x, int x_dtype, int64_t M, int64_t ldx, void* y, int64_t ldy,
                 int epilogue, void* stream);
/* Same contract with a caller-owned device workspace (16-byte aligned): when
 * workspace_bytes >= sm_q4_matmul_workspace_bytes(M, N, K, epilogue) a batch
 * call whose grid would underfill the GPU splits K over several workgroups
 * and a second kernel sums the fp32 partials in split order (deterministic)
 * and applies the epilogue. A smaller workspace only limits the split. The
 * workspace contents are scratch; calls sharing one workspace must not
 * overlap. */
int64_t sm_q4_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K, int epilogue);
int sm_q4_matmul_ws(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                    const void* x, int x_dtype, int64_t M, int64_t ldx, void* y, int64_t ldy,
                    int epilogue, void* workspace, int64_t workspace_bytes, void* stream);
/* A residual projection and the RMSNorm that follows it (the pre-norm
 * decoder's x = x + Linear(h); h = RMSNorm(x) * gamma, block.rs / norm.rs:36-50,
 * with the Linear over a quantized weight, matmul.rs:57-66): resid [M, N] f32
 * += x . W^T (as sm_q4_matmul_ws with SM_EPI_ADD_F32, ldy = N), then h_out
 * [M, 2N] f16 pairs (SM_F16X2 rows) = RMSNorm(resid) * gamma (as sm_rmsnorm).
 * At decode batch sizes (the LDS-staged decode kernel's shapes, N a multiple
 * of 256 up to 4096, a workspace of sm_q4_matmul_workspace_bytes(M, N, K,
 * SM_EPI_ADD_F32) bytes) K is split and one kernel sums the partials in split
 * order into resid and normalises the rows; elsewhere the two steps run. The
 * results are those of the two calls wherever the matmul would split K
 * itself, and within f32 summation order otherwise. */
int sm_q4_matmul_add_rmsnorm(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                             const void* x, int x_dtype, int64_t M, int64_t ldx, float* resid,
                             const float* gamma, float eps, void* h_out, void* workspace,
                             int64_t workspace_bytes, void* stream);
/* sm_q4_matmul_add_rmsnorm for an MoE layer's FFN norm, with the router of
 * the normed rows (SparseMoe::forward's fp32 router and top-2, ffn.rs:489-514,
 * moe_topk.rs:74-104, over h as its f16 pairs hold it): top_idx / top_w
 * [M, 2] as sm_moe_router_top2 gives them, router_logits [M, experts] f32
 * (nullable) = h . w_router^T, w_router [experts, N] f32, 2 <= experts <= 64.
 * Where the fused form applies, the router runs in the same launch as the
 * norm (the row sums in a different order than sm_moe_router_top2's, within
 * f32 rounding of it); otherwise the two steps plus sm_moe_router_top2. */
int sm_q4_matmul_add_rmsnorm_router(const uint8_t* codes, const uint16_t* scales, int64_t N,
                                    int64_t K, const void* x, int x_dtype, int64_t M, int64_t ldx,
                                    float* resid, const float* gamma, float eps, void* h_out,
                                    const float* w_router, int64_t experts, float* router_logits,
                                    int32_t* top_idx, float* top_w, void* workspace,
                                    int64_t workspace_bytes, void* stream);
/* sm_q4_matmul_ws without a caller workspace and without any allocation, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The split-K partials live in a static device array of
 * SM_Q4_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends); results
 * are bit-identical to sm_q4_matmul_ws given a workspace of
 * sm_q4_matmul_workspace_bytes(M, N, K, epilogue) bytes. A call whose query
 * exceeds the scratch is rejected (SM_ERR_INVALID) before any launch. All
 * calls on one GPU share its scratch: calls that overlap on one GPU race. */
#define SM_Q4_NOALLOC_SCRATCH_BYTES (96LL * 1024 * 1024)
int64_t sm_q4_noalloc_scratch_bytes(void);
int sm_q4_matmul_noalloc(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                         const void* x, int x_dtype, int64_t M, int64_t ldx, void* y, int64_t ldy,
                         int epilogue, void* stream);

/* Many independent one-row Q4 GEMVs in one launch: job i computes
 * y_i[N_i] (=, or +=) x_i[K_i] . W_i^T, i.e. one decode-step Linear::forward
 * (summa-llm/src/model/matmul.rs:57-66) per job, for inputs that are ready
 * together (independent projections, a whole-model weight sweep). No
 * single-call counterpart in the reference (it launches one matmul per
 * linear). Each job's y equals sm_q4_matmul at M = 1 bit for bit when K >=
 * 512. Use: fill a host array of jobs, call sm_q4_gemv_multi_plan (checks
 * every job, sets first_block, returns the total number of 16-row blocks and,
 * given a host int32 array of that size, fills the block -> job table), copy
 * both arrays to device memory, then launch sm_q4_gemv_multi with the device
 * copies (no allocation; the tables can be reused for every launch while
 * the buffers they name stay valid). max_k >= every job's K, with
 * (1 or 2) * max_k * 2 bytes <= 64 KB. */
typedef struct sm_q4_gemv_job {
  const uint8_t* codes;    /* prepared tiled codes (sm_q4_pack), 16-byte aligned */
  const uint16_t* scales;  /* prepared tiled scales */
  const void* x;           /* K f16 (x_dtype SM_F16) or 2K (SM_F16X2: hi then lo), 16-byte aligned */
  void* y;                 /* N outputs: f32, or bf16 for SM_EPI_STORE_BF16 */
  int64_t N, K;            /* K a positive multiple of 128 */
  int32_t epilogue;        /* SM_EPI_STORE_F32, SM_EPI_STORE_BF16 or SM_EPI_ADD_F32 */
  int32_t first_block;     /* set by sm_q4_gemv_multi_plan */
} sm_q4_gemv_job;
int64_t sm_q4_gemv_multi_plan(sm_q4_gemv_job* jobs, int64_t njobs, int32_t* block_job);
int sm_q4_gemv_multi(const sm_q4_gemv_job* jobs, int64_t njobs, const int32_t* block_job,
                     int64_t nblocks, int64_t max_k, int x_dtype, void* stream);

/* qkv projection fused with RoPE and the KV-cache append: y = x . W^T over
 * the Q4 qkv weight (rows [q heads | k heads | v heads], N = (H + 2 KVH) hd)
 * for S sequences x L rows (row s*L + i at position pos0[s] + i), then q and
 * k rotated (adjacent-pair RoPE from rope_table [max_pos, hd/2, 2]) and q
 * written to q_out [S*L, H, hd], k and v to the caches [S, KVH, cap, hd] at
 * their positions (positions outside [0, cap) are skipped). Replaces
 * project_qkv + the AttnCache slice_assign (attention.rs:142-177, 331-356) as
 * sm_q4_matmul + sm_rope_append would, without the fp32 qkv round trip.
 * cache_dtype SM_F16; head_dim a power of two >= 16. */
int sm_q4_qkv_rope(const uint8_t* codes, const uint16_t* scales, int64_t H, int64_t KVH,
                   int64_t head_dim, int64_t K, const void* x, int x_dtype, int64_t S, int64_t L,
                   int64_t ldx, const float* rope_table, const int32_t* pos0, int64_t cap,
                   void* q_out, void* kcache, void* vcache, int cache_dtype, void* stream);

/* Dense fp32 y = x . W^T (fp32 models; matmul::linear, summa-llm/src/model/
 * matmul.rs:57-66). epilogue: SM_EPI_STORE_F32 or SM_EPI_ADD_F32. */
int sm_gemm_f32(const float* w, int64_t N, int64_t K, const float* x, int64_t M, int64_t ldx,
                float* y, int64_t ldy, int epilogue, void* stream);
/* out[r, c] = silu(gv[r, c]) * gv[r, F + c] (ffn.rs:854-886 gated activation). */
int sm_swiglu_f32(const float* gate_value, int64_t rows, int64_t F, float* out, void* stream);

/* ------------------------------------------------------------------------
 * Decoder elementwise ops.
 * sm_embed: x[r] = table[ids[r]] * scale, f32 out (Transformer::embed,
 *   summa-llm/src/model/transformer.rs:511-518); out-of-range ids give NaN rows.
 * sm_rmsnorm: y = x / sqrt(mean(x^2) + eps) * gamma, fp32 statistics
 *   (Norm::forward, summa-llm/src/model/norm.rs:36-50), y in out_dtype
 *   (SM_F32, SM_BF16 or SM_F16).
 * sm_rope_append: qkv [S*L, (H+2KVH)*hd] f32 -> q_out [S*L, H, hd] with RoPE,
 *   K (RoPE) and V written to caches [S, KVH, cap, hd] at position pos0[s]+i;
 *   q_dtype / cache_dtype: (f32, f32), (f32 or bf16, bf16) or (f16, f16)
 *   (project_qkv + AttnCache slice_assign, attention.rs:142-177, 331-356).
 *   rope_table [max_pos, hd/2, 2] f32 (cos, sin), adjacent-pair convention.
 */
int sm_embed(const void* table, int dtype, const int32_t* ids, int64_t rows, int64_t d,
             int64_t vocab, float scale, float* x, void* stream);
int sm_rmsnorm(const float* x, const float* gamma, int64_t rows, int64_t d, float eps, void* y,
               int out_dtype, void* stream);
int sm_rope_append(const float* qkv, const float* rope_table, const int32_t* pos0, int64_t S,
                   int64_t L, int64_t H, int64_t KVH, int64_t head_dim, int64_t cap, void* q_out,
                   int q_dtype, void* kcache, void* vcache, int cache_dtype, void* stream);

/* ------------------------------------------------------------------------
 * Attention over the KV cache [S, KVH, cap, hd] (AttnCache, attention.rs:20-40).
 * sm_attn_decode: one query per sequence, q/out [S, H, hd], keys 0..lens[s]-1
 *   (forward_cached -> sdpa -> attention(q, repeat_kv(k), repeat_kv(v)),
 *   attention.rs:216-265, 318-371; repeat_kv fused_attention.rs:114-125).
 * sm_attn_prefill: causal, q/out [S, L, H, hd], row i at position pos0[s]+i
 *   attends keys 0..=pos0[s]+i (fused_attention / CubeK flash forward,
 *   attention.rs:250, cube_attention.rs:127-220).
 * dtype (q and cache) SM_BF16 or SM_F16 (MFMA kernels; out_dtype SM_BF16,
 * SM_F16 or SM_F16X2 rows of 2*H*hd f16) or SM_F32 (VALU, out_dtype SM_F32);
 * head_dim 64 or 128.
 */
int sm_attn_decode(const void* q, const void* kcache, const void* vcache, const int32_t* lens,
                   void* out, int dtype, int out_dtype, int64_t S, int64_t H, int64_t KVH,
                   int64_t cap, int64_t head_dim, void* stream);
int sm_attn_prefill(const void* q, const void* kcache, const void* vcache, const int32_t* pos0,
                    void* out, int dtype, int out_dtype, int64_t S, int64_t L, int64_t H,
                    int64_t KVH, int64_t cap, int64_t head_dim, void* stream);
/* Decode attention for rollouts in groups of G that share a prompt of P
 * tokens (GrpoGenerationBatchRequest: one example per group,
 * posttrain.rs:1206-1216; per rollout the semantics of sm_attn_decode, i.e.
 * forward_cached, attention.rs:216-265): rollout s attends keys 0..P-1 from
 * prefix_k / prefix_v [S/G, KVH, P, hd] (its group's prompt, stored once) and
 * keys P..lens[s]-1 from kcache / vcache [S, KVH, cap, hd] (its own
 * continuation); every lens[s] must be >= P. The prompt keys are read once per
 * (group, KV head) for all G * H/KVH query heads of the group. dtype SM_F16 or
 * SM_BF16, out_dtype SM_F16X2; G * H / KVH <= 32. workspace: at least
 * sm_attn_decode_prefix_workspace_bytes(S, G, P, H, KVH, head_dim) bytes,
 * 16-byte aligned (per-(query head, key split) partials; no allocation). */
int64_t sm_attn_decode_prefix_workspace_bytes(int64_t S, int64_t G, int64_t P, int64_t H,
                                              int64_t KVH, int64_t head_dim);
int sm_attn_decode_prefix(const void* q, const void* prefix_k, const void* prefix_v,
                          const void* kcache, const void* vcache, const int32_t* lens, void* out,
                          void* workspace, int64_t workspace_bytes, int dtype, int out_dtype,
                          int64_t S, int64_t G, int64_t P, int64_t H, int64_t KVH, int64_t cap,
                          int64_t head_dim, void* stream);
/* Same, also writing the per-row log-sum-exp of the scaled, masked scores
 * (natural log) to lse [S*H, L] f32 (nullable): the convention of the flash
 * forward and attention_log_sum_exp (fused_attention.rs:166-172), which the
 * attention backward consumes. */
int sm_attn_prefill_lse(const void* q, const void* kcache, const void* vcache,
                        const int32_t* pos0, void* out, float* lse, int dtype, int out_dtype,
                        int64_t S, int64_t L, int64_t H, int64_t KVH, int64_t cap,
                        int64_t head_dim, void* stream);

/* Full-sequence attention in the reference's tensor layout: the
 * AttentionBackend::attention_inner / attention_backward pair
 * (summa-llm/src/model/fused_attention.rs:37-74; portable definitions
 * reference_attention :177-217 and reference_attention_backward :219-261)
 * that Dispatch::attention_inner calls (:103-110).
 * q, out [B, H, S, hd]; k, v [B, KVH, S, hd] with KVH dividing H (KVH == H is
 * the repeat_kv'd form the reference hands over; a smaller KVH is read in
 * place, query head h using key/value head h / (H / KVH)); scale 1/sqrt(hd);
 * causal = 1 masks keys after the query's position. lse (nullable) [B*H, S]
 * f32: the per-row log-sum-exp of the scaled, masked scores (natural log).
 * sm_attention: dtype SM_F32 (VALU), SM_BF16 or SM_F16 (MFMA; out in the
 *   same dtype); head_dim 64 or 128.
 * sm_attention_backward: f32; from the forward's output and lse; dq [B, H,
 *   S, hd], dk / dv [B, KVH, S, hd] (summed over each head group, as
 *   reduce_kv_grad :127-138); delta_scratch [B*H*S] f32. */
int sm_attention(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H,
                 int64_t KVH, int64_t S, int64_t head_dim, int causal, void* out, float* lse,
                 void* stream);
int sm_attention_backward(const float* q, const float* k, const float* v, const float* out,
                          const float* grad_out, const float* lse, int64_t B, int64_t H,
                          int64_t KVH, int64_t S, int64_t head_dim, int causal, float* dq,
                          float* dk, float* dv, float* delta_scratch, void* stream);

/* Next-token selection for `rows` logits rows (select_next_token /
 * sample_from_logits, summa-llm/src/generate.rs:127-202). temperature <= 0:
 * greedy, first max wins ties; otherwise Gumbel-max sampling from
 * softmax(logits / T) with the counter RNG keyed (seed, row, step) — one
 * substream per rollout, as ModelExecutionRngRange (posttrain.rs:1043).
 * tokens[r*tok_stride] <- token; logprobs[r*lp_stride] (nullable) <-
 * log_softmax(logits)[token]; next_ids[r] (nullable) <- token. */
int sm_sample(const float* logits, int64_t rows, int64_t ld, int64_t vocab, float temperature,
              uint64_t seed, int64_t step, int32_t* tokens, int64_t tok_stride, float* logprobs,
              int64_t lp_stride, int32_t* next_ids, void* stream);

/* Sampling options of a rollout (SamplingConfig, summa-llm/src/generate.rs:12-23,
 * and RolloutSampling, summa-train/src/posttrain.rs:353-387). */
typedef struct sm_sampling {
  float temperature;        /* <= 0: greedy; NaN is rejected */
  int32_t top_k;            /* < 0: off (None); 0 is rejected; k >= 1 samples among the k
                               largest logits (value, then lowest index) */
  float repetition_penalty; /* 1: off; must be finite and >= 1 */
  int32_t eos_token;        /* -1: none */
  float top_p;              /* must be finite and in (0, 1] (RolloutSampling::validate) */
  int32_t apply_top_p;      /* 0: top_p is validated only, as in the reference, which has no
                               nucleus sampler; 1: keep the smallest value-ordered prefix of the
                               candidates whose softmax(logits / T) mass reaches top_p */
} sm_sampling;

/* Next-token selection with the full option set (select_next_token,
 * apply_repetition_penalty, sample_from_values; generate.rs:127-250).
 * Per row: the penalty divides (positive) or multiplies (negative) the logit of
 * every token set in seen[r] (a bitmap [rows, seen_ld] u32, bit v of word v/32;
 * required when the penalty is on), then greedy argmax (lowest index on ties) or
 * a Gumbel-max draw among the top-k / nucleus candidates with the counter RNG of
 * sm_sample (with the options off, the draw equals sm_sample's). The chosen
 * token is set in seen (when non-null). done [rows] (nullable, needs eos_token):
 * a row with done != 0 emits eos_token with log-prob 0; a row that emits
 * eos_token gets done = 1 and lengths[r] (nullable) = step + 1.
 * logprobs <- log_softmax(logits)[token] of the raw logits. Validation errors
 * carry the reference's messages ("top_k must be >= 1 (got 0)", "temperature
 * must not be NaN", "repetition_penalty must be finite and >= 1 (got x)",
 * "rollout top_p must be finite and in (0, 1]"). */
int sm_sample_ex(const float* logits, int64_t rows, int64_t ld, int64_t vocab,
                 const sm_sampling* sampling, uint64_t seed, int64_t step, uint32_t* seen,
                 int64_t seen_ld, int32_t* done, int32_t* lengths, int32_t* tokens,
                 int64_t tok_stride, float* logprobs, int64_t lp_stride, int32_t* next_ids,
                 void* stream);
/* seen[r] |= {ids[r, 0..n)} (ids [rows, ids_ld] int32; ids outside [0, vocab)
 * mark nothing); clear != 0 zeroes the rows first. The prior_tokens set of
 * apply_repetition_penalty (generate.rs:155-182). */
int sm_seen_tokens(const int32_t* ids, int64_t rows, int64_t n, int64_t ids_ld, int64_t vocab,
                   uint32_t* seen, int64_t seen_ld, int clear, void* stream);

/* ------------------------------------------------------------------------
 * Top-2 mixture of experts (SparseMoe::forward, summa-llm/src/model/ffn.rs:
 * 478-711), all on the device with no host round trip.
 * sm_moe_router_top2: logits = f32 h . W_r^T (W_r [E, d] f32), top-2 with a
 *   strict '>' scan (top2_indices_kernel, moe_topk.rs:74-104), weights =
 *   softmax over the pair. top_idx/top_w [tokens, 2]; logits_out nullable
 *   (or logits only: top_idx and top_w both NULL, logits_out required).
 *   h f32, f16 or f16 pairs [tokens, d], d <= 8192, 2 <= E <= 64.
 * sm_moe_route_plan_logits: top-2 routing from router logits [tokens, E]
 *   (as sm_moe_router_top2 takes it: top_idx / top_w [tokens, 2]) and the
 *   route plan of those routes (as sm_moe_route_plan with top_k = 2), in one
 *   launch for up to 512 tokens (moe_topk.rs:36-104 + moe_route.rs:22-142).
 * sm_moe_route_plan: stable sort of routes r = t*k + j by expert
 *   (host_route_plan ffn.rs:888-929 / route_plan moe_route.rs:22-142) into the
 *   int32 `plan` buffer of sm_moe_plan_words() words: counts[E],
 *   offsets[E+1], order[R], inverse[R], src_rows[R], then 16- and 128-row
 *   tile lists used by sm_q4_grouped_matmul. error (device int32, caller-zeroed)
 *   gets bit 0 set for an expert index outside [0, E); such a route is left
 *   out of the plan (inverse = -1) and contributes nothing in sm_moe_combine.
 *   One workgroup; E <= 64.
 * sm_q4_grouped_matmul: per expert e, rows offsets[e]..offsets[e+1]-1 of y =
 *   A . W_e^T with W_e the e-th of `experts` stacked prepared Q4 weights
 *   [N, K]; A row p = x[src_rows[p]] when gather != 0 (the token gather,
 *   route_gather moe_dispatch.rs:57, folded into the matmul) else x[p]
 *   (grouped_linear / grouped_swiglu_mlp, grouped_linear.rs:65-104).
 *   Epilogues: SM_EPI_STORE_F32/BF16 or SM_EPI_SWIGLU_BF16/F16/F16X2; x
 *   bf16, f16 or f16 pairs.
 * sm_moe_combine: x[t] += sum_j top_w[t,j] * routed[inverse[t*k+j]] (f32)
 *   (route_combine_forward, moe_dispatch.rs:290-312).
 */
int64_t sm_moe_plan_words(int64_t tokens, int64_t top_k, int64_t experts);
int sm_moe_router_top2(const void* h, int h_dtype, const float* w_router, int64_t tokens,
                       int64_t d, int64_t experts, float* logits_out, int32_t* top_idx,
                       float* top_w, void* stream);
int sm_moe_route_plan(const int32_t* top_idx, int64_t tokens, int64_t top_k, int64_t experts,
                      int32_t* plan, int32_t* error, void* stream);
int sm_moe_route_plan_logits(const float* logits, int64_t tokens, int64_t experts,
                             int32_t* top_idx, float* top_w, int32_t* plan, int32_t* error,
                             void* stream);
int sm_q4_grouped_matmul(const uint8_t* codes, const uint16_t* scales, int64_t experts, int64_t N,
                         int64_t K, const void* x, int x_dtype, int64_t ldx, int gather,
                         const int32_t* plan, int64_t tokens, int64_t top_k, void* y, int64_t ldy,
                         int epilogue, void* stream);
int sm_moe_combine(const float* routed, const float* top_w, const int32_t* plan, int64_t tokens,
                   int64_t top_k, int64_t experts, int64_t d, float* x, void* stream);
/* The combine and the next RMSNorm (block.rs: x = x + MoE(h); h = RMSNorm(x) *
 * gamma, norm.rs:36-50): x as sm_moe_combine, then h_out [tokens, 2d] f16
 * pairs (SM_F16X2 rows) = RMSNorm(x) * gamma as sm_rmsnorm, in one launch for
 * d a multiple of 256 up to 4096 (the two steps otherwise); the same results
 * as the two calls. */
int sm_moe_combine_rmsnorm(const float* routed, const float* top_w, const int32_t* plan,
                           int64_t tokens, int64_t top_k, int64_t experts, int64_t d, float* x,
                           const float* gamma, float eps, void* h_out, void* stream);

/* MoE training kernels (route_gather_* / route_combine_*,
 * summa-llm/src/model/moe_dispatch.rs:244-384; swiglu_forward / _backward,
 * fused_swiglu.rs:106-150). Tensors f32 or bf16 (dtype SM_F32 / SM_BF16), f32
 * arithmetic; routing weights top_w [tokens, k] f32; `plan` from
 * sm_moe_route_plan.
 * sm_moe_gather: routed[p] = x[order[p] / k] ([R, d], sorted route order).
 * sm_moe_gather_backward: grad_x[t] = sum_j grad_routed[inverse[t*k + j]].
 * sm_moe_combine_backward: grad_routed[inverse[r]] = grad_x[r / k] * top_w[r]
 *   and grad_w[r] = <grad_x[r / k], routed[inverse[r]]> (either output
 *   nullable; the weight gradient needs `routed`).
 * sm_swiglu / sm_swiglu_backward over [gate | value] rows [rows, 2F]:
 *   out = silu(g) * v; d gate = dy * v * s (1 + g (1 - s)) with s = sigmoid(g),
 *   d value = dy * silu(g). */
int sm_moe_gather(const void* x, int dtype, const int32_t* plan, int64_t tokens, int64_t top_k,
                  int64_t experts, int64_t d, void* routed, void* stream);
int sm_moe_gather_backward(const void* grad_routed, int dtype, const int32_t* plan,
                           int64_t tokens, int64_t top_k, int64_t experts, int64_t d,
                           void* grad_x, void* stream);
int sm_moe_combine_backward(const void* grad_x, const void* routed, int dtype, const float* top_w,
                            const int32_t* plan, int64_t tokens, int64_t top_k, int64_t experts,
                            int64_t d, void* grad_routed, float* grad_w, void* stream);
int sm_swiglu(const void* gate_value, int dtype, int64_t rows, int64_t F, void* out,
              void* stream);
int sm_swiglu_backward(const void* gate_value, const void* grad, int dtype, int64_t rows,
                       int64_t F, void* grad_gate_value, void* stream);

/* ------------------------------------------------------------------------
 * Float-weight grouped expert projections and the route permutation at the
 * reference's dispatch seam (GroupedLinearBackend, grouped_linear.rs:23-60;
 * RowPermutationBackend, row_permute.rs:33-41). All f32, f32-grade products
 * (sm_gemm_ex per expert with rows, in expert order; no allocation).
 * counts: HOST array [experts] of the rows per expert, as
 *   grouped_linear_inner takes them (Vec<usize>); they must sum to routes.
 * sm_row_permute: out[i] = input[order[i]] over rows of `cols` elements
 *   (row_permute_inner; its backward is the same call with the inverse
 *   permutation); order entries outside [0, rows) give zero rows; out must
 *   not alias input. dtype SM_F32, SM_BF16 or SM_F16 (bits copied).
 * sm_grouped_linear: out [routes, d_out] = input [routes, d_in] rows of expert
 *   e (counts[e] consecutive rows, experts in order) times weight[e]
 *   ([E, d_in, d_out] row-major) (grouped_linear_inner).
 * sm_grouped_linear_backward: grad_input = grad W_e^T and grad_weight[e] =
 *   input_e^T grad_e, zero for an expert without rows; either output
 *   nullable (grouped_linear_backward, grouped_linear.rs:30-37, 524-570).
 * sm_grouped_swiglu_mlp: projected [routes, 2I] = grouped_linear(input,
 *   in_weight [E, d, 2I]) as [gate | value], hidden [routes, I] =
 *   silu(gate) * value, out [routes, d_out] = grouped_linear(hidden,
 *   down_weight [E, I, d_out]) (grouped_swiglu_mlp_inner, :779-799).
 * sm_grouped_swiglu_mlp_backward: grad_input, grad_in_weight,
 *   grad_down_weight from the forward's projected and hidden
 *   (grouped_swiglu_mlp_backward, :801-826); scratch: routes * 3 * I floats. */
int sm_row_permute(const void* input, int dtype, int64_t rows, int64_t cols,
                   const int32_t* order, void* out, void* stream);
int sm_grouped_linear(const float* input, const float* weight, const int64_t* counts,
                      int64_t experts, int64_t routes, int64_t d_in, int64_t d_out, float* out,
                      void* stream);
int sm_grouped_linear_backward(const float* input, const float* weight, const float* grad,
                               const int64_t* counts, int64_t experts, int64_t routes,
                               int64_t d_in, int64_t d_out, float* grad_input,
                               float* grad_weight, void* stream);
int sm_grouped_swiglu_mlp(const float* input, const float* in_weight, const float* down_weight,
                          const int64_t* counts, int64_t experts, int64_t routes, int64_t d,
                          int64_t intermediate, int64_t d_out, float* out, float* projected,
                          float* hidden, void* stream);
int sm_grouped_swiglu_mlp_backward(const float* input, const float* in_weight,
                                   const float* down_weight, const int64_t* counts,
                                   int64_t experts, int64_t routes, int64_t d,
                                   int64_t intermediate, int64_t d_out, const float* projected,
                                   const float* hidden, const float* grad, float* grad_input,
                                   float* grad_in_weight, float* grad_down_weight,
                                   float* scratch, void* stream);

/* ------------------------------------------------------------------------
 * Policy-update kernels (backward of the recompute and the optimizer step:
 * prepare_device_batch autodiff + optimizer_step, posttrain.rs:1288-1305,
 * trainer.rs:1974-1975), f32 with f32 accumulation.
 * sm_gemm_ex: C = alpha op(A) op(B) + beta C, op(A) [M, K] (A stored [M, K],
 *   or [K, M] when trans_a), op(B) [K, N] (B stored [K, N], or [N, K] when
 *   trans_b): the data / weight gradients of Linear::forward (matmul.rs:57-66).
 *   Problems of at least 2^27 multiply-adds run on the matrix cores as
 *   sm_gemm_mfma does; smaller ones on an f32 FMA kernel.
 * sm_gemm_mfma: the same contract (K > 0) always on the matrix cores: each f32
 *   operand is split exactly into three bf16 planes and the six plane
 *   products of weight >= 2^-16 are accumulated in f32, an f32 GEMM up to the
 *   order of its additions (the bf16 operands of matmul_2 / linear on the
 *   reference's CUDA path, matmul.rs:73-82, 132-143, with f32 results).
 * sm_gemm_planes: sm_gemm_mfma with `planes` bf16 planes per operand: 3 as
 *   sm_gemm_mfma; 2: hi + lo planes, three products (16-bit operands, each
 *   product within about 2^-15 relative); 1: the bf16-rounded operands' product
 *   accumulated in f32, which is the reference's CUDA-path matmul
 *   (matmul.rs:73-82, 132-143: bf16 operands). Other values fail.
 * sm_rmsnorm_backward: dx (= or += with accumulate) and dgamma (nullable; =
 *   or += ; summed over rows in order) of y = x / sqrt(mean x^2 + eps) * gamma
 *   (norm.rs:36-50); rinv_scratch [rows].
 * sm_rope_qk: rotate the q and k heads of qkv rows [S*L, (H+2KVH)*hd] in place
 *   at positions pos0[s] + i (backward = 1: the transposed rotation, for
 *   gradients) (attention.rs:142-177).
 * sm_attn_backward_f32: causal GQA attention backward from the forward's
 *   log-sum-exp (sm_attn_prefill_lse): q/o/dout [S*L, H, hd], k/v/dk/dv
 *   [S, KVH, L, hd] (positions 0..L-1), lse [S*H, L]; delta_scratch [S*H*L]
 *   (fused_attention.rs:219-405).
 * sm_embed_backward: dtable[ids[r]] += dx[r] (atomic f32 adds).
 * sm_adamw_step: m, v moments, bias correction at `step` (from 1), decoupled
 *   weight decay: p = p (1 - lr wd) - lr mhat / (sqrt(vhat) + eps).
 * sm_muon_momentum: velocity = g + mu velocity (g on the first step), update =
 *   mu velocity + g (BatchedMuon, muon.rs:200-204); sm_axpby: y = a x + b y;
 *   sm_frobenius_normalize: x /= max(||x||_F, eps), the norm to norm_out[0]
 *   (zeropower_via_newton_schulz, muon.rs:257-285). */
int sm_gemm_ex(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
               const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
               int64_t ldc, void* stream);
int sm_gemm_mfma(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                 const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
                 int64_t ldc, void* stream);
int sm_gemm_planes(int planes, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                   float alpha, const float* A, int64_t lda, const float* B, int64_t ldb,
                   float beta, float* C, int64_t ldc, void* stream);
/* sm_gemm_planes with a scratch (16-byte aligned) of at least
 * sm_gemm_planes_scratch_bytes(trans_a, trans_b, M, N, K) bytes: an operand
 * whose k is not contiguous (op(A) of a transposed A, op(B) of an
 * untransposed B) is transposed into it first, so that both operands stream
 * along k (at one plane both operands are converted once into bf16 copies
 * there instead); the result is sm_gemm_planes' bit for bit. A smaller
 * scratch runs sm_gemm_planes as is. b_planes 2 (with planes 3) declares every B value
 * exact in two bf16 planes (value - bf16(value) is itself a bf16, as for a
 * bf16 scale times a 4-bit code): the zero third plane of B is then not
 * multiplied (five plane products instead of six, the same bits); 0 or 3:
 * no such claim. (The policy update's GEMMs run this way.) */
int64_t sm_gemm_planes_scratch_bytes(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K);
int sm_gemm_planes_ws(int planes, int b_planes, int trans_a, int trans_b, int64_t M, int64_t N,
                      int64_t K, float alpha, const float* A, int64_t lda, const float* B,
                      int64_t ldb, float beta, float* C, int64_t ldc, void* scratch,
                      int64_t scratch_bytes, void* stream);
int sm_rmsnorm_backward(const float* x, const float* gamma, const float* dy, int64_t rows,
                        int64_t d, float eps, int accumulate, float* dx, float* dgamma,
                        float* rinv_scratch, void* stream);
int sm_rope_qk(float* qkv, const float* rope_table, const int32_t* pos0, int64_t S, int64_t L,
               int64_t H, int64_t KVH, int64_t head_dim, int backward, void* stream);
int sm_attn_backward_f32(const float* q, const float* k, const float* v, const float* o,
                         const float* dout, const float* lse, int64_t S, int64_t L, int64_t H,
                         int64_t KVH, int64_t head_dim, float* dq, float* dk, float* dv,
                         float* delta_scratch, void* stream);
/* The f32 attention forward (sm_attn_prefill_lse with dtype SM_F32: causal,
 * positions pos0[s] + i, log-sum-exp out) and its backward
 * (sm_attn_backward_f32) with bf16 matrix-core operands: every product takes
 * its f32 operands rounded to bf16 (nearest even) and accumulates in f32. This
 * is the 16-bit precision of the reference's CUDA-path flash attention (F16
 * in, F32 accumulate, cube_attention.rs:127-220) and of its backward, which
 * forms P and dS in bf16 (cube_attention.rs:53-95); the policy update runs it
 * with one-plane (bf16) matmuls (sm_policy_set_matmul_planes 1). Rows shorter
 * than 32 positions keep the f32 kernels. Same arguments as the f32 calls. */
int sm_attn_prefill_lse_bf16ops(const float* q, const float* kcache, const float* vcache,
                                const int32_t* pos0, float* out, float* lse, int64_t S,
                                int64_t L, int64_t H, int64_t KVH, int64_t cap, int64_t head_dim,
                                void* stream);
int sm_attn_backward_bf16ops(const float* q, const float* k, const float* v, const float* o,
                             const float* dout, const float* lse, int64_t S, int64_t L,
                             int64_t H, int64_t KVH, int64_t head_dim, float* dq, float* dk,
                             float* dv, float* delta_scratch, void* stream);
int sm_embed_backward(const int32_t* ids, const float* dx, int64_t rows, int64_t d,
                      int64_t vocab, float* dtable, void* stream);
int sm_adamw_step(float* param, const float* grad, float* m, float* v, int64_t n, float lr,
                  float beta1, float beta2, float eps, float weight_decay, int64_t step,
                  void* stream);
int sm_muon_momentum(const float* grad, float* velocity, float* update, int64_t n,
                     float momentum, int first_step, void* stream);
int sm_axpby(const float* x, float* y, int64_t n, float a, float b, void* stream);
int sm_frobenius_normalize(float* x, int64_t n, float eps, float* norm_out, void* stream);

/* ------------------------------------------------------------------------
 * Decoder model (the MAL Transformer subset the configs use,
 * summa-llm/src/model/transformer.rs, block.rs, attention.rs, ffn.rs) and the
 * RL-step runtime behind GrpoDeviceBatchRuntime (posttrain.rs:1288-1305).
 */
typedef struct sm_model_config {
  int32_t layers, d_model, heads, kv_heads, head_dim, ffn, vocab;
  int32_t max_seq;   /* RoPE table rows = largest cache capacity */
  float norm_eps;    /* RMSNorm epsilon (MAL default 1e-5) */
  float rope_theta;  /* MAL default 1e4 */
  int32_t quantized; /* 1: Q4G128 linears, f16 matmul inputs, bf16 q/KV/embedding;
                        0: all fp32 */
  int32_t experts;    /* 0: dense SwiGLU FFN; > 0: top-2 MoE FFN in every layer */
  int32_t expert_ffn; /* expert intermediate width (MoE only) */
} sm_model_config;

typedef struct sm_model sm_model;

/* Tensor kinds for sm_model_set_tensor. Linear weights are [out, in]
 * (transpose of Burn's Linear [d_in, d_out]); QKV rows are [q | k | v]
 * (attention.rs:92), IN rows are [gate | value] (ffn.rs:64-88). */
enum {
  SM_W_EMBED = 0,      /* [vocab, d] */
  SM_W_ATTN_NORM = 1,  /* [d] per layer */
  SM_W_QKV = 2,        /* [H*hd + 2*KVH*hd, d] per layer */
  SM_W_O = 3,          /* [d, H*hd] per layer */
  SM_W_FFN_NORM = 4,   /* [d] per layer */
  SM_W_IN = 5,         /* [2F, d] per layer */
  SM_W_DOWN = 6,       /* [d, F] per layer */
  SM_W_FINAL_NORM = 7, /* [d] */
  SM_W_LM_HEAD = 8,    /* [vocab, d] */
  SM_W_ROUTER = 9,     /* [E, d] per layer, kept f32 (router math is fp32, ffn.rs:489) */
  SM_W_EXPERT_IN = 10, /* [E, 2Fe, d] per layer ([gate | value] rows per expert) */
  SM_W_EXPERT_DOWN = 11 /* [E, d, Fe] per layer */
};

int sm_model_create(const sm_model_config* cfg, sm_model** out);
int sm_model_destroy(sm_model* model);
int64_t sm_model_weight_bytes(const sm_model* model);
/* Load one tensor from a dense f32 device buffer; quantized models quantize
 * linears on the device (QuantizedModelBackend::load_quantized_matrix /
 * load_floating_tensor, quantization.rs:1183-1189). Synchronises `stream`
 * for quantized linears (range check of the scales). */
int sm_model_set_tensor(sm_model* model, int kind, int layer, const float* src, void* stream);
/* MoE router trace, a diagnostic with no reference counterpart (the
 * reference reports router statistics only as training-side auxiliary losses,
 * ffn.rs:478-711). While a trace is set, every MoE layer of every forward run
 * on this model appends, per token, its top-2 expert ids (idx [capacity, 2]
 * int32, device) and its router logits (logits [capacity, experts] f32,
 * device, nullable), in call order: forward by forward, layer by layer, tokens
 * in row order (a prefill or recompute chunk: sequence-major; a decode step:
 * one token per sequence). Entries past `capacity` tokens are dropped and
 * counted. idx = NULL ends tracing. Setting a trace resets both counts. */
int sm_model_trace_routes(sm_model* model, int32_t* idx, float* logits, int64_t capacity);
int sm_model_route_trace_count(const sm_model* model, int64_t* recorded, int64_t* dropped);
/* Synthetic weights: every linear and the embedding ~ N(0, std) from the
 * counter RNG, norms = 1, router ~ N(0, 1/sqrt(d)) so router logits are
 * ~N(0, 1) (the BASELINE configs' random init). */
int sm_model_init_random(sm_model* model, uint64_t seed, float std, void* stream);

/* ------------------------------------------------------------------------
 * HQUANT packed tensors (PackedTensor, summa-train/src/quantization.rs:414-689;
 * container to_bytes / from_bytes :502-597). Formats 1-3 are the reference's
 * (binary / ternary / ternary-entropy g128, FP16 group scales); 4 is this
 * build's Q4G128 (two's-complement nibbles, low nibble first, bf16 scales),
 * which has no counterpart in the reference codec. */
enum {
  SM_HQ_BINARY = 1,
  SM_HQ_TERNARY = 2,
  SM_HQ_TERNARY_ENTROPY = 3,
  SM_HQ_Q4G128 = 4
};
typedef struct sm_hquant {
  int32_t format;       /* SM_HQ_* */
  int32_t group_size;   /* 128 */
  int32_t rank;         /* 1..32 */
  int64_t shape[32];
  int64_t elements;
  const uint16_t* scales; /* one per group: FP16 bits (formats 1-3), bf16 bits (4) */
  int64_t nscales;
  const uint8_t* codes;
  int64_t ncodes;
} sm_hquant;
/* FNV-1a 64 of a byte range (the container checksum, quantization.rs:2274). */
uint64_t sm_fnv1a64(const uint8_t* bytes, int64_t n);
/* Parse and validate a container held in host memory (from_bytes +
 * validate_packed, :530-597, :980-1071): `out` points into `bytes` (which must
 * stay alive and be 2-byte aligned). Errors carry the reference's messages
 * ("quantized tensor checksum mismatch", "invalid quantized tensor magic",
 * "packed tensor contains reserved ternary code 3", ...). */
int sm_hquant_parse(const uint8_t* bytes, int64_t n, sm_hquant* out);
/* Serialized size of `t`, and the serialisation itself (to_bytes, :502-528):
 * validates `t` (host pointers) first. */
int64_t sm_hquant_bytes(const sm_hquant* t);
int sm_hquant_write(const sm_hquant* t, uint8_t* out, int64_t cap, int64_t* written);
/* Device decode (PackedTensor::decode, :445-497): t->scales / t->codes are
 * device pointers; out [elements] f32, or with transpose = 1 a rank-2 [r, c]
 * tensor written as [c, r]. */
int sm_hquant_decode(const sm_hquant* t, float* out, int transpose, void* stream);
/* QuantizedModelBackend::load_quantized_matrix (:1183-1189): install a packed
 * tensor (device scales / codes) as model tensor `kind` / `layer`.
 * layout 0: rows are [out, in] as sm_model_set_tensor; 1: [in, out] (Burn's
 * Linear weight layout, the layout of reference archives). A Q4G128 tensor in
 * layout 0 is installed bit for bit into a quantized model; everything else is
 * decoded and stored like sm_model_set_tensor (a quantized model re-quantizes
 * binary / ternary weights to Q4G128: not exact, FP16 scales are not bf16). */
int sm_model_load_packed(sm_model* model, int kind, int layer, const sm_hquant* tensor,
                         int layout, void* stream);

/* Device workspace of the RL calls (no hidden allocation in hot calls, the
 * workspace-query convention the Burn kernels lack). sm_rl_workspace_bytes:
 * bytes that sm_rl_generate / sm_rl_generate_ex of S rollouts with P prompt
 * and N new tokens, and sm_rl_logprobs / sm_rl_prepare of the same shapes
 * (max_tokens_per_forward as they are given it), need at most; -1 on bad
 * arguments. sm_model_bind_workspace hands the model a caller-owned device
 * buffer of at least that many bytes (256-byte aligned) sized for those
 * bounds: every later hot call on this model carves its buffers from it and
 * never allocates, and a call with larger shapes fails with SM_ERR_INVALID.
 * ws = NULL returns the model to its own grow-only buffers (the default,
 * which allocates on the first call at a new size). Binding synchronises the
 * device. Weight loading (sm_model_set_tensor, sm_model_load_packed,
 * sm_model_init_random) allocates temporaries either way. */
int64_t sm_rl_workspace_bytes(sm_model* model, int64_t S, int64_t P, int64_t N,
                              int64_t max_tokens_per_forward);
int sm_model_bind_workspace(sm_model* model, void* ws, int64_t bytes, int64_t S, int64_t P,
                            int64_t N, int64_t max_tokens_per_forward);

/* Prompt groups (GrpoGenerationBatchRequest: one example per group of
 * group_size rollouts, posttrain.rs:1206-1216; padded_group_log_probabilities
 * takes one prefix per group, summa-train/src/tensor_sleep.rs:2642-2689):
 * with group_size G > 1, later sm_rl_generate / sm_rl_generate_ex /
 * sm_rl_logprobs / sm_rl_prepare calls on this model take rollouts
 * g*G .. g*G+G-1 to share one prompt and compute the prompt positions once
 * per group (the prefill, and the recompute's prompt part), copying their
 * K / V to the group's rollouts: the same values as per rollout, since a
 * prompt position depends on the prompt alone. Each call checks on the device
 * that S is whole groups and every prompt row equals its group's first (one
 * host synchronisation; SM_ERR_INVALID otherwise). A grouped recompute whose
 * prompts, weights and buffers equal those of the model's last grouped prompt
 * pass (a generation's prefill, or a recompute) reuses that pass's K / V and
 * last rows instead of computing them again (the same values). 1 (the
 * default) computes every rollout's prompt. Set it before sm_rl_workspace_bytes
 * / sm_model_bind_workspace, whose sizes depend on it. */
int sm_model_set_prompt_groups(sm_model* model, int64_t group_size);

/* Batched rollouts (generate_device_batch, posttrain.rs:1191-1216; per rollout
 * the semantics of TextGenerator::generate, generate.rs:68-124, with no EOS):
 * prompts [S, P] int32 -> tokens [S, N] int32 and behavior_lp [S, N] f32
 * (nullable), one prefill then N-1 cached decode steps. */
int sm_rl_generate(sm_model* model, const int32_t* prompts, int64_t S, int64_t P, int64_t N,
                   float temperature, uint64_t seed, int32_t* tokens, float* behavior_lp,
                   void* stream);
/* Same with the full sampling options (TextGenerator::generate, generate.rs:68-124,
 * for S rollouts at once): the repetition penalty counts the prompt and every
 * generated token of the rollout; a rollout that emits eos_token stops (its later
 * tokens are eos_token with behavior log-prob 0, lengths[s] = tokens generated
 * including the EOS; N when none), and the loop ends once every rollout has
 * stopped (checked every 16 steps). lengths [S] int32 nullable. */
int sm_rl_generate_ex(sm_model* model, const int32_t* prompts, int64_t S, int64_t P, int64_t N,
                      const sm_sampling* sampling, uint64_t seed, int32_t* tokens,
                      float* behavior_lp, int32_t* lengths, void* stream);
/* The completion mask of rollouts that stop at EOS: mask[s, n] = 1 while
 * n < lengths[s] (the tokens generated, EOS included, as sm_rl_generate_ex
 * reports them), else 0, f32 [S, N] (the active mask grpo_loss_tensor takes,
 * posttrain.rs:874-1028; the padded tail must not enter the loss). */
int sm_completion_mask(const int32_t* lengths, int64_t S, int64_t N, float* mask, void* stream);
/* Log-prob recompute (padded_group_log_probabilities /
 * equal_length_continuation_log_probabilities, tensor_sleep.rs:2531-2689):
 * lp_out[s, n] = log_softmax(model(prompt ‖ tokens[:, :N-1]))[P-1+n][tokens[s, n]].
 * Sequences are processed in chunks of <= max_tokens_per_forward tokens
 * (0 = 65536, the reference's bound, tensor_sleep.rs:52). */
int sm_rl_logprobs(sm_model* model, const int32_t* prompts, const int32_t* tokens, int64_t S,
                   int64_t P, int64_t N, int64_t max_tokens_per_forward, float* lp_out,
                   void* stream);
/* prepare_device_batch numerics (posttrain.rs:4420, 1234-1244): recompute the
 * current (policy) and frozen (reference, nullable when kl_coefficient == 0)
 * log-probs, then sm_grpo_loss over groups x group_size rollouts. */
int sm_rl_prepare(sm_model* policy, sm_model* reference, const int32_t* prompts,
                  const int32_t* tokens, const float* behavior_lp, const float* rewards,
                  const float* mask, int64_t groups, int64_t group_size, int64_t P, int64_t N,
                  double clip_epsilon, double advantage_epsilon, double kl_coefficient,
                  int64_t max_tokens_per_forward, float* lp_cur, float* lp_ref,
                  float* group_stats, float* dlp, int32_t* flags, void* stream);

/* ------------------------------------------------------------------------
 * Trainable policy: the gradient and optimizer half of GrpoDeviceBatchRuntime
 * (posttrain.rs:1288-1305): prepare_device_batch stages gradients,
 * optimizer_step(learning_rate_scale) applies them. f32 master weights of a
 * dense decoder ([out, in] rows, tensor kinds SM_W_EMBED .. SM_W_LM_HEAD) or
 * of a top-2 MoE decoder (no SM_W_IN / SM_W_DOWN; SM_W_ROUTER, SM_W_EXPERT_IN,
 * SM_W_EXPERT_DOWN per layer: SparseMoe, ffn.rs:478-711, trained through its
 * combine, per-expert GEMM, gather and pair-softmax router gradients); a
 * quantized config runs its forward on fake-quantized weights (Q4G128
 * linears, bf16 embedding: what sm_policy_install puts into a quantized
 * model) with straight-through gradients (trainer.rs:312-318).
 * sm_optimizer_config: AdamW (lr, beta1, beta2, eps, weight_decay; the
 * trainer's 3e-4, 0.9, 0.95, 1e-8, 0.1: trainer.rs:1124-1129, main.rs:171-174)
 * for every tensor, or with muon_lr > 0 Muon for the per-layer projections
 * (BatchedMuon, muon.rs:196-285; trainer.rs:1974-1975); grad_clip > 0 clips the
 * global gradient norm (gradient_norm_and_clip, main.rs:667-694; default 1.0).
 * sm_policy_prepare: the recompute with activations kept (lp_cur), the
 *   frozen reference's log-probs (sm_rl_logprobs on `reference`), the GRPO
 *   loss (as sm_grpo_loss) and the backward of sum(dlp * lp_cur), added to the
 *   staged gradients. Arguments as sm_rl_prepare.
 * sm_policy_prepare_with_ref: the same with the frozen reference's log-probs
 *   given, reference_lp [S, N] f32 over the same tokens (as sm_rl_prepare or
 *   sm_rl_logprobs returned them for the step's recompute; nullable when
 *   kl_coefficient is 0), so the update does not run the frozen model again:
 *   grpo_loss_tensor's reference_token_log_probs input (posttrain.rs:874-1028).
 *   With the same log-probs the results equal sm_policy_prepare's bit for bit.
 * sm_policy_optimizer_step: clip, optimizer update at lr * scale, staged
 *   gradients cleared; grad_norm (nullable, host) gets the pre-clip norm; a
 *   non-finite norm fails with the reference's message (trainer.rs:1959-1964).
 *   Synchronises the stream once (the norm readback).
 * sm_policy_install: the master weights into an inference model
 *   (sm_model_set_tensor per tensor: quantized models re-quantize).
 * sm_policy_get_tensor: a master weight (gradient = 0) or its staged
 *   gradient (gradient = 1) into dst.
 * sm_policy_set_matmul_planes: the bf16 planes per operand of the prepare's
 *   GEMMs (sm_gemm_planes): 3 (the default, f32-grade), 2 (16-bit operands) or
 *   1 (bf16 operands with f32 accumulation: the precision of the reference's
 *   CUDA-path training matmul, matmul.rs:73-82, 132-143). */
typedef struct sm_policy sm_policy;
typedef struct sm_optimizer_config {
  float lr, beta1, beta2, eps, weight_decay;
  float muon_lr;   /* 0: AdamW for every tensor */
  float grad_clip; /* <= 0: no clipping */
} sm_optimizer_config;
int sm_policy_create(const sm_model_config* cfg, const sm_optimizer_config* opt,
                     sm_policy** out);
int sm_policy_destroy(sm_policy* policy);
int sm_policy_set_matmul_planes(sm_policy* policy, int planes);
int sm_policy_set_tensor(sm_policy* policy, int kind, int layer, const float* src, void* stream);
int sm_policy_get_tensor(const sm_policy* policy, int kind, int layer, float* dst, int gradient,
                         void* stream);
int sm_policy_install(const sm_policy* policy, sm_model* model, void* stream);
int sm_policy_prepare(sm_policy* policy, sm_model* reference, const int32_t* prompts,
                      const int32_t* tokens, const float* behavior_lp, const float* rewards,
                      const float* mask, int64_t groups, int64_t group_size, int64_t P, int64_t N,
                      double clip_epsilon, double advantage_epsilon, double kl_coefficient,
                      float* lp_cur, float* lp_ref, float* group_stats, float* dlp,
                      int32_t* flags, void* stream);
int sm_policy_prepare_with_ref(sm_policy* policy, const float* reference_lp,
                               const int32_t* prompts, const int32_t* tokens,
                               const float* behavior_lp, const float* rewards, const float* mask,
                               int64_t groups, int64_t group_size, int64_t P, int64_t N,
                               double clip_epsilon, double advantage_epsilon,
                               double kl_coefficient, float* lp_cur, float* group_stats,
                               float* dlp, int32_t* flags, void* stream);
int sm_policy_optimizer_step(sm_policy* policy, double learning_rate_scale, float* grad_norm,
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
