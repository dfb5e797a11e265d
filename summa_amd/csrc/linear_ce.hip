// Fused linear head + cross-entropy (the LinearCrossEntropyBackend seam).
//
// Forward: per chunk of `chunk` token rows, logits = hidden[rows] . W^T (+ b)
// into a workspace slab of [chunk, stored_vocab] f32 (the full [tokens, V]
// logits never exist), then the row kernel of sm_ce_rows (online max / sum,
// token log-prob, padded columns never read); the loss is -mean(lp) over
// every token, one fixed-order reduction. Backward: the same logits per
// chunk, the row kernel's gradient in place scaled by grad_output / tokens
// (read on the device), then dhidden[rows] = G . W, dW (+)= G^T . hidden[rows]
// and db (+)= column sums of G, so padded rows of dW and db stay exactly 0.
// The GEMMs are sm_gemm_ex (f32-grade; the three-plane bf16 matrix-core
// kernel at these sizes).
//
// Reference: LinearCrossEntropyBackend (summa-llm/src/model/linear_cross_entropy/mod.rs:33-57),
// chunked_loss / chunked_backward (reference.rs:42-159), fused_loss /
// fused_backward (gpu.rs:264-426).
#include "common.hpp"

namespace sm {
namespace {

constexpr size_t kLceAlign = 256;
size_t lce_align(size_t v) { return (v + kLceAlign - 1) / kLceAlign * kLceAlign; }

// Workspace layout: logits [chunk, Vs] f32 | lp [tokens] f32 | row scale
// [chunk] f32 | bias-gradient partials [kColParts, Vs] f32.
constexpr int kColParts = 64;

struct LceLayout {
  size_t logits, lp, rscale, parts, total;
};

LceLayout lce_layout(int64_t tokens, int64_t stored, int64_t chunk, bool use_bias) {
  LceLayout l{};
  const int64_t rows = std::min(chunk, tokens);
  l.logits = 0;
  l.lp = l.logits + lce_align((size_t)rows * stored * 4);
  l.rscale = l.lp + lce_align((size_t)tokens * 4);
  l.parts = l.rscale + lce_align((size_t)rows * 4);
  l.total = l.parts + (use_bias ? lce_align((size_t)kColParts * stored * 4) : 0);
  return l;
}

// logits[r, c] += bias[c] over the stored columns.
__global__ void add_bias_kernel(float* __restrict__ logits, const float* __restrict__ bias,
                                int64_t rows, int64_t stored) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * stored) return;
  logits[i] += bias[i % stored];
}

// scale[r] = grad_output[0] / tokens for the chunk's rows.
__global__ void fill_scale_kernel(float* __restrict__ scale, int64_t rows,
                                  const float* __restrict__ grad_output, float inv_tokens) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < rows) scale[i] = grad_output[0] * inv_tokens;
}

// Column sums of G [rows, Vs] in kColParts row slices (part p sums rows
// p, p + kColParts, ... in order), then db (+)= the parts summed in order:
// deterministic, no atomics.
__global__ void colsum_parts_kernel(const float* __restrict__ g, int64_t rows, int64_t stored,
                                    float* __restrict__ parts) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int p = blockIdx.y;
  if (c >= stored) return;
  float acc = 0.f;
  for (int64_t r = p; r < rows; r += kColParts) acc += g[r * stored + c];
  parts[(int64_t)p * stored + c] = acc;
}

__global__ void colsum_finish_kernel(const float* __restrict__ parts, int64_t stored,
                                     int accumulate, float* __restrict__ db) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= stored) return;
  float acc = 0.f;
  for (int p = 0; p < kColParts; ++p) acc += parts[(int64_t)p * stored + c];
  db[c] = accumulate ? db[c] + acc : acc;
}

// loss = -mean(lp) over every token (f64, fixed order).
__global__ __launch_bounds__(1024) void lce_mean_neg_kernel(const float* __restrict__ lp,
                                                            int64_t n, float* __restrict__ loss) {
  __shared__ double part[1024 / kWave];
  double acc = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 1024) acc += (double)lp[i];
  acc = wave_sum_f64(acc);
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < 1024 / kWave; ++w) t += part[w];
    loss[0] = (float)(-t / (double)n);
  }
}

int lce_check(const float* hidden, const float* weight, const float* bias,
              const int32_t* targets, int64_t tokens, int64_t d, int64_t stored,
              int64_t logical, int64_t chunk, int use_bias, void* ws, int64_t ws_bytes,
              const char* who) {
  SM_REQUIRE(hidden && weight && targets && ws, "%s: null argument", who);
  SM_REQUIRE(chunk > 0, "linear cross-entropy chunk size must be positive");
  SM_REQUIRE(tokens > 0, "linear cross-entropy requires at least one token");
  SM_REQUIRE(d > 0 && d < (1 << 30) && stored > 0 && stored < (1 << 30), "%s: bad shape", who);
  SM_REQUIRE(logical > 0 && logical <= stored, "logical vocabulary %lld must be in 1..=%lld",
             (long long)logical, (long long)stored);
  SM_REQUIRE(!use_bias || bias, "%s: use_bias needs a bias vector", who);
  SM_REQUIRE(reinterpret_cast<uintptr_t>(ws) % kLceAlign == 0, "%s: workspace must be 256-byte aligned",
             who);
  const LceLayout l = lce_layout(tokens, stored, chunk, use_bias != 0);
  SM_REQUIRE(ws_bytes >= 0 && (size_t)ws_bytes >= l.total,
             "%s: workspace holds %lld bytes, %zu needed (sm_linear_cross_entropy_workspace_bytes)",
             who, (long long)ws_bytes, l.total);
  return SM_OK;
}

// logits of rows [start, start + rows) into the workspace slab (+ bias).
int lce_logits(const float* hidden, const float* weight, const float* bias, int64_t start,
               int64_t rows, int64_t d, int64_t stored, int use_bias, float* logits,
               hipStream_t st) {
  SM_TRY(sm_gemm_ex(0, 1, rows, stored, d, 1.0f, hidden + start * d, d, weight, d, 0.0f, logits,
                    stored, st));
  if (use_bias) {
    const int64_t n = rows * stored;
    add_bias_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(logits, bias, rows, stored);
    SM_LAUNCH_CHECK();
  }
  return SM_OK;
}

}  // namespace
}  // namespace sm

using namespace sm;

extern "C" int64_t sm_linear_cross_entropy_workspace_bytes(int64_t tokens, int64_t d,
                                                           int64_t stored_vocab, int64_t chunk,
                                                           int use_bias) {
  if (tokens <= 0 || d <= 0 || stored_vocab <= 0 || chunk <= 0) return -1;
  return (int64_t)lce_layout(tokens, stored_vocab, chunk, use_bias != 0).total;
}

extern "C" int sm_linear_cross_entropy(const float* hidden, const float* weight,
                                       const float* bias, const int32_t* targets, int64_t tokens,
                                       int64_t d, int64_t stored_vocab, int64_t logical_vocab,
                                       int64_t chunk, int use_bias, float* loss,
                                       float* token_logprob, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
  SM_TRY(lce_check(hidden, weight, bias, targets, tokens, d, stored_vocab, logical_vocab, chunk,
                   use_bias, workspace, workspace_bytes, "sm_linear_cross_entropy"));
  SM_REQUIRE(loss, "sm_linear_cross_entropy: null loss");
  hipStream_t st = as_stream(stream);
  const LceLayout l = lce_layout(tokens, stored_vocab, chunk, use_bias != 0);
  char* ws = static_cast<char*>(workspace);
  float* logits = reinterpret_cast<float*>(ws + l.logits);
  float* lp = token_logprob ? token_logprob : reinterpret_cast<float*>(ws + l.lp);
  for (int64_t s0 = 0; s0 < tokens; s0 += chunk) {
    const int64_t rows = std::min(chunk, tokens - s0);
    SM_TRY(lce_logits(hidden, weight, bias, s0, rows, d, stored_vocab, use_bias, logits, st));
    SM_TRY(sm_ce_rows(logits, SM_F32, targets + s0, rows, stored_vocab, logical_vocab, lp + s0,
                      nullptr, nullptr, 1.0f, nullptr, nullptr, st));
  }
  lce_mean_neg_kernel<<<1, 1024, 0, st>>>(lp, tokens, loss);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_linear_cross_entropy_backward(
    const float* hidden, const float* weight, const float* bias, const int32_t* targets,
    const float* grad_output, int64_t tokens, int64_t d, int64_t stored_vocab,
    int64_t logical_vocab, int64_t chunk, int use_bias, float* grad_hidden, float* grad_weight,
    float* grad_bias, void* workspace, int64_t workspace_bytes, void* stream) {
  SM_TRY(lce_check(hidden, weight, bias, targets, tokens, d, stored_vocab, logical_vocab, chunk,
                   use_bias, workspace, workspace_bytes, "sm_linear_cross_entropy_backward"));
  SM_REQUIRE(grad_output && grad_hidden && grad_weight,
             "sm_linear_cross_entropy_backward: null gradient buffer");
  SM_REQUIRE(!use_bias || grad_bias, "sm_linear_cross_entropy_backward: use_bias needs grad_bias");
  hipStream_t st = as_stream(stream);
  const LceLayout l = lce_layout(tokens, stored_vocab, chunk, use_bias != 0);
  char* ws = static_cast<char*>(workspace);
  float* logits = reinterpret_cast<float*>(ws + l.logits);
  float* lp = reinterpret_cast<float*>(ws + l.lp);
  float* rscale = reinterpret_cast<float*>(ws + l.rscale);
  float* parts = reinterpret_cast<float*>(ws + l.parts);
  const float inv_tokens = (float)(1.0 / (double)tokens);
  for (int64_t s0 = 0; s0 < tokens; s0 += chunk) {
    const int64_t rows = std::min(chunk, tokens - s0);
    const bool first = s0 == 0;
    SM_TRY(lce_logits(hidden, weight, bias, s0, rows, d, stored_vocab, use_bias, logits, st));
    fill_scale_kernel<<<(unsigned)ceil_div(rows, 256), 256, 0, st>>>(rscale, rows, grad_output,
                                                                     inv_tokens);
    SM_LAUNCH_CHECK();
    // G = (softmax - onehot) * grad_output / tokens in place; padded columns 0
    SM_TRY(sm_ce_rows(logits, SM_F32, targets + s0, rows, stored_vocab, logical_vocab, lp + s0,
                      nullptr, logits, 1.0f, rscale, nullptr, st));
    // dhidden[rows] = G . W          ([rows, Vs] x [Vs, d])
    SM_TRY(sm_gemm_ex(0, 0, rows, d, stored_vocab, 1.0f, logits, stored_vocab, weight, d, 0.0f,
                      grad_hidden + s0 * d, d, st));
    // dW (+)= G^T . hidden[rows]     ([Vs, rows] x [rows, d])
    SM_TRY(sm_gemm_ex(1, 0, stored_vocab, d, rows, 1.0f, logits, stored_vocab, hidden + s0 * d, d,
                      first ? 0.0f : 1.0f, grad_weight, d, st));
    if (use_bias) {
      const dim3 grid((unsigned)ceil_div(stored_vocab, 256), kColParts);
      colsum_parts_kernel<<<grid, 256, 0, st>>>(logits, rows, stored_vocab, parts);
      colsum_finish_kernel<<<(unsigned)ceil_div(stored_vocab, 256), 256, 0, st>>>(
          parts, stored_vocab, first ? 0 : 1, grad_bias);
      SM_LAUNCH_CHECK();
    }
  }
  return SM_OK;
}
