// Trainable policy: the gradient and optimizer half of GrpoDeviceBatchRuntime
// (summa-train/src/posttrain.rs:1288-1305). prepare_device_batch recomputes
// the policy's token log-probs with its activations kept, evaluates the GRPO
// loss (grpo_loss_tensor, posttrain.rs:874-1028) and stages the gradient of
// every parameter; optimizer_step(learning_rate_scale) clips the global
// gradient norm and applies the trainer's optimizers (gradient_norm_and_clip,
// summa-train/src/main.rs:667-694; Muon for the per-layer projections and
// AdamW for the rest, trainer.rs:1124-1129, 1974-1975; muon.rs:196-285).
//
// Weights are f32 master copies of a dense or top-2 MoE decoder in the
// model's [out, in] rows (an MoE layer: f32 router [E, d], experts stacked
// [E * 2Fe, d] and [E * d, Fe]). For a quantized configuration the forward
// runs on fake-quantized weights (Q4G128 linears and experts, bf16 embedding,
// f32 router: the values the inference model holds after sm_policy_install)
// and the gradient passes straight through to the masters (the fake-quantized
// parameter leaves of trainer.rs:312-318), so the recomputed log-probs are
// those of the model that produced the rollouts.
//
// Host composition over the library's kernels (the same steps as the Python
// composition in summa_amd/train.py for dense layers): embedding, RMSNorm,
// GEMMs, RoPE, attention with its log-sum-exp, SwiGLU (dense, or per expert
// over the routes sorted by expert: router top-2, route plan, gather,
// combine), fused CE; backward through the CE gradient, GEMM data / weight
// gradients, RMSNorm, RoPE, attention, SwiGLU, the MoE combine / gather /
// router gradients and embedding backward kernels.
#include <cmath>
#include <vector>

#include "common.hpp"

extern "C" {
int sm_embed(const void*, int, const int32_t*, int64_t, int64_t, int64_t, float, float*, void*);
int sm_rmsnorm(const float*, const float*, int64_t, int64_t, float, void*, int, void*);
int sm_gemm_ex(int, int, int64_t, int64_t, int64_t, float, const float*, int64_t, const float*,
               int64_t, float, float*, int64_t, void*);
int sm_rope_qk(float*, const float*, const int32_t*, int64_t, int64_t, int64_t, int64_t, int64_t,
               int, void*);
int sm_attn_prefill_lse(const void*, const void*, const void*, const int32_t*, void*, float*, int,
                        int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void*);
int sm_swiglu(const void*, int, int64_t, int64_t, void*, void*);
int sm_swiglu_backward(const void*, const void*, int, int64_t, int64_t, void*, void*);
int sm_ce_rows(const void*, int, const int32_t*, int64_t, int64_t, int64_t, float*, float*, void*,
               float, const float*, float*, void*);
int sm_rmsnorm_backward(const float*, const float*, const float*, int64_t, int64_t, float, int,
                        float*, float*, float*, void*);
int sm_attn_backward_f32(const float*, const float*, const float*, const float*, const float*,
                         const float*, int64_t, int64_t, int64_t, int64_t, int64_t, float*, float*,
                         float*, float*, void*);
int sm_attn_prefill_lse_bf16ops(const float*, const float*, const float*, const int32_t*, float*,
                                float*, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t,
                                void*);
int sm_attn_backward_bf16ops(const float*, const float*, const float*, const float*, const float*,
                             const float*, int64_t, int64_t, int64_t, int64_t, int64_t, float*,
                             float*, float*, float*, void*);
int sm_embed_backward(const int32_t*, const float*, int64_t, int64_t, int64_t, float*, void*);
int sm_adamw_step(float*, const float*, float*, float*, int64_t, float, float, float, float, float,
                  int64_t, void*);
int sm_muon_momentum(const float*, float*, float*, int64_t, float, int, void*);
int sm_axpby(const float*, float*, int64_t, float, float, void*);
int sm_frobenius_normalize(float*, int64_t, float, float*, void*);
int sm_grpo_loss(const float*, const float*, const float*, const float*, const float*, int64_t,
                 int64_t, int64_t, double, double, double, float*, float*, float*, int32_t*, void*);
int sm_rl_logprobs(sm_model*, const int32_t*, const int32_t*, int64_t, int64_t, int64_t, int64_t,
                   float*, void*);
int sm_model_set_tensor(sm_model*, int, int, const float*, void*);
int sm_q4_quantize(const void*, int, int64_t, uint8_t*, uint16_t*, int32_t*, void*);
int64_t sm_moe_plan_words(int64_t, int64_t, int64_t);
int sm_moe_router_top2(const void*, int, const float*, int64_t, int64_t, int64_t, float*, int32_t*,
                       float*, void*);
int sm_moe_route_plan(const int32_t*, int64_t, int64_t, int64_t, int32_t*, int32_t*, void*);
int sm_moe_gather(const void*, int, const int32_t*, int64_t, int64_t, int64_t, int64_t, void*,
                  void*);
int sm_moe_gather_backward(const void*, int, const int32_t*, int64_t, int64_t, int64_t, int64_t,
                           void*, void*);
int sm_moe_combine(const float*, const float*, const int32_t*, int64_t, int64_t, int64_t, int64_t,
                   float*, void*);
int sm_moe_combine_backward(const void*, const void*, int, const float*, const int32_t*, int64_t,
                            int64_t, int64_t, int64_t, void*, float*, void*);
}

namespace sm {
int gemm_ex_planes(int planes, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                   float alpha, const float* A, int64_t lda, const float* B, int64_t ldb,
                   float beta, float* C, int64_t ldc, void* stream, float* scratch = nullptr,
                   int64_t scratch_floats = 0, int b_planes = 3);  // train.hip
int64_t gemm_planes_scratch_floats(bool ta, bool tb, int64_t M, int64_t N,
                                   int64_t K);  // gemm_mfma.hip
int64_t rmsnorm_dgamma_chunks(int64_t rows);                          // train.hip
int rmsnorm_backward_parts(const float* x, const float* gamma, const float* dy, int64_t rows,
                           int64_t d, float eps, int accumulate, float* dx, float* dgamma,
                           float* rinv_scratch, float* parts, hipStream_t st);
namespace {

constexpr int kKinds = 12;  // SM_W_EMBED .. SM_W_EXPERT_DOWN (a dense policy has no MoE kinds,
                            // an MoE policy no dense FFN: those kinds have no elements)
constexpr float kMuonMomentum = 0.95f;                          // muon.rs:10
constexpr float kNsA = 3.4445f, kNsB = -4.775f, kNsC = 2.0315f;  // muon.rs:11
constexpr int kNsSteps = 5;                                     // muon.rs:12
constexpr float kMuonEps = 1e-7f;                               // muon.rs:13

bool is_layer_kind(int k) {
  return k == SM_W_ATTN_NORM || k == SM_W_QKV || k == SM_W_O || k == SM_W_FFN_NORM ||
         k == SM_W_IN || k == SM_W_DOWN || k == SM_W_ROUTER || k == SM_W_EXPERT_IN ||
         k == SM_W_EXPERT_DOWN;
}
// the kinds a quantized model holds as Q4G128 (the router stays f32, ffn.rs:489)
bool is_linear_kind(int k) {
  return k == SM_W_QKV || k == SM_W_O || k == SM_W_IN || k == SM_W_DOWN || k == SM_W_LM_HEAD ||
         k == SM_W_EXPERT_IN || k == SM_W_EXPERT_DOWN;
}
bool is_muon_kind(int k) {  // the per-layer 2-D projections (trainer.rs:1974)
  return k == SM_W_QKV || k == SM_W_O || k == SM_W_IN || k == SM_W_DOWN;
}

__global__ void gather_rows_f32(const float* __restrict__ src, const int64_t* __restrict__ rows,
                                int64_t n, int d, float* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n * d) dst[i] = src[rows[i / d] * d + i % d];
}
__global__ void scatter_rows_f32(const float* __restrict__ src, const int64_t* __restrict__ rows,
                                 int64_t n, int d, float* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n * d) dst[rows[i / d] * d + i % d] = src[i];
}
// rows [S*L, (H + 2 KVH) hd] -> q [S*L, H*hd], k / v [S, KVH, L, hd]
__global__ void split_qkv_f32(const float* __restrict__ qkv, int S, int L, int H, int KVH, int hd,
                              float* __restrict__ q, float* __restrict__ k, float* __restrict__ v) {
  const int qn = (H + 2 * KVH) * hd;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)S * L * qn) return;
  const int64_t row = i / qn;
  const int c = i % qn;
  const float x = qkv[i];
  if (c < H * hd) { q[row * H * hd + c] = x; return; }
  const int s = row / L, r = row % L;
  const int c2 = c - H * hd;
  const int which = c2 / (KVH * hd), kh = (c2 % (KVH * hd)) / hd, e = c2 % hd;
  (which ? v : k)[(((size_t)s * KVH + kh) * L + r) * hd + e] = x;
}
// the inverse: dq, dk, dv -> dqkv rows
__global__ void merge_qkv_f32(const float* __restrict__ q, const float* __restrict__ k,
                              const float* __restrict__ v, int S, int L, int H, int KVH, int hd,
                              float* __restrict__ qkv) {
  const int qn = (H + 2 * KVH) * hd;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)S * L * qn) return;
  const int64_t row = i / qn;
  const int c = i % qn;
  if (c < H * hd) { qkv[i] = q[row * H * hd + c]; return; }
  const int s = row / L, r = row % L;
  const int c2 = c - H * hd;
  const int which = c2 / (KVH * hd), kh = (c2 % (KVH * hd)) / hd, e = c2 % hd;
  qkv[i] = (which ? v : k)[(((size_t)s * KVH + kh) * L + r) * hd + e];
}
// ids [S, L] = prompt ‖ tokens[:, :N-1]; scored rows s*L + P-1+n
__global__ void build_ids_rows(const int32_t* __restrict__ prompts,
                               const int32_t* __restrict__ tokens, int S, int P, int N,
                               int32_t* __restrict__ ids, int64_t* __restrict__ rows) {
  const int L = P + N - 1;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < (int64_t)S * L) {
    const int64_t s = i / L;
    const int t = i % L;
    ids[i] = (t < P) ? prompts[s * P + t] : tokens[s * N + (t - P)];
  }
  if (i < (int64_t)S * N) rows[i] = (i / N) * L + P - 1 + i % N;
}
__global__ void neg_f32(const float* __restrict__ a, int64_t n, float* __restrict__ b) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) b[i] = -a[i];
}
__global__ void transpose_f32(const float* __restrict__ a, int R, int C, float* __restrict__ b) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // a [R, C] -> b [C, R]
  if (i < (int64_t)R * C) b[(i % C) * R + i / C] = a[i];
}
__global__ void zero_f32(float* p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}
__global__ void round_bf16_f32(const float* __restrict__ a, int64_t n, float* __restrict__ b) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) b[i] = bf16_to_f32(f32_to_bf16(a[i]));
}
// Q4G128 codec decode (row-major codes, bf16 scales): value = scale * code
__global__ void q4_decode_f32(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ sc,
                              int64_t n, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int q = (codes[i / 2] >> ((i & 1) * 4)) & 0xf;
  if (q >= 8) q -= 16;
  out[i] = bf16_to_f32(sc[i / 128]) * (float)q;
}
// sum of squares (f64) of each 64 K-value chunk of `a` -> part[blockIdx.x]
constexpr int64_t kSumChunk = 65536;
// d logits of the top-2 router (weights = softmax over the two selected
// logits, ffn.rs:494-507): dl[t, e] = p_j (g_j - sum_i p_i g_i) for the expert
// e = idx[t, j] chosen in slot j, 0 for the unselected experts.
__global__ void router_grad_kernel(const float* __restrict__ top_w, const float* __restrict__ gw,
                                   const int32_t* __restrict__ idx, int64_t tokens, int E,
                                   float* __restrict__ dl) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tokens * E) return;
  const int64_t t = i / E;
  const int e = (int)(i % E);
  const float p0 = top_w[2 * t], p1 = top_w[2 * t + 1];
  const float g0 = gw[2 * t], g1 = gw[2 * t + 1];
  const float mean = p0 * g0 + p1 * g1;
  float v = 0.f;
  if (idx[2 * t] == e) v = p0 * (g0 - mean);
  else if (idx[2 * t + 1] == e) v = p1 * (g1 - mean);
  dl[i] = v;
}
__global__ __launch_bounds__(256) void sumsq_kernel(const float* __restrict__ a, int64_t n,
                                                    double* __restrict__ part) {
  __shared__ double wp[256 / kWave];
  double s = 0.0;
  const int64_t base = (int64_t)blockIdx.x * kSumChunk;
  const int64_t end = std::min<int64_t>(n, base + kSumChunk);
  for (int64_t i = base + threadIdx.x; i < end; i += 256) s += (double)a[i] * a[i];
  s = wave_sum_f64(s);
  if (threadIdx.x % kWave == 0) wp[threadIdx.x / kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < 256 / kWave; ++w) t += wp[w];
    part[blockIdx.x] = t;
  }
}
// acc[0] = sum of part[0..n): one workgroup, thread t adding parts t, t + 256,
// ... in order, then the 256 sums in a fixed tree (deterministic). A single
// thread adding the parts one after another took 1.4 ms at config[2]'s
// 21k parts.
__global__ __launch_bounds__(256) void sum_parts_kernel(const double* __restrict__ part,
                                                        int64_t n, double* __restrict__ acc) {
  __shared__ double sh[256];
  double t = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 256) t += part[i];
  sh[threadIdx.x] = t;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) sh[threadIdx.x] += sh[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) acc[0] = sh[0];
}
// g *= max_norm / norm when the norm (sqrt(acc[0])) exceeds max_norm > 0
__global__ void clip_scale_kernel(float* __restrict__ g, int64_t n, const double* __restrict__ acc,
                                  float max_norm) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const float norm = (float)sqrt(acc[0]);
  if (i < n && max_norm > 0.f && norm > max_norm) g[i] *= max_norm / norm;
}

// One pass of the AdamW step over a clipped gradient, which it then clears
// for the next accumulation: g' = g * (max_norm / norm) when the norm
// exceeds max_norm > 0 (clip_scale_kernel's arithmetic), then adamw_kernel's
// update with g', then g = 0; four elements per thread with 16-byte accesses
// (the scalar tail of n % 4 elements by the last threads). Replaces the clip,
// AdamW and clearing passes (40 -> 32 bytes per parameter).
__device__ inline void adamw_one(float& p, float& m, float& v, float g, float lr, float b1,
                                 float b2, float eps, float wd, float c1, float c2) {
  const float mi = b1 * m + (1.f - b1) * g;
  const float vi = b2 * v + (1.f - b2) * g * g;
  m = mi;
  v = vi;
  const float upd = (mi / c1) / (sqrtf(vi / c2) + eps);
  p = p * (1.f - lr * wd) - lr * upd;
}
typedef float f4 __attribute__((ext_vector_type(4)));
__global__ void adamw_clip_clear_kernel(float* __restrict__ p, float* __restrict__ g,
                                        float* __restrict__ m, float* __restrict__ v, int64_t n,
                                        float norm, float max_norm, float lr, float b1, float b2,
                                        float eps, float wd, float c1, float c2) {
  const int64_t i4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool clip = max_norm > 0.f && norm > max_norm;
  const float f = clip ? max_norm / norm : 1.f;
  if (4 * i4 + 3 < n) {
    f4 pp = reinterpret_cast<f4*>(p)[i4], gg = reinterpret_cast<f4*>(g)[i4];
    f4 mm = reinterpret_cast<f4*>(m)[i4], vv = reinterpret_cast<f4*>(v)[i4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float pe = pp[e], me = mm[e], ve = vv[e];
      const float ge = clip ? gg[e] * f : gg[e];
      adamw_one(pe, me, ve, ge, lr, b1, b2, eps, wd, c1, c2);
      pp[e] = pe;
      mm[e] = me;
      vv[e] = ve;
    }
    reinterpret_cast<f4*>(p)[i4] = pp;
    reinterpret_cast<f4*>(m)[i4] = mm;
    reinterpret_cast<f4*>(v)[i4] = vv;
    reinterpret_cast<f4*>(g)[i4] = f4{0.f, 0.f, 0.f, 0.f};
  } else {
    for (int64_t i = 4 * i4; i < n; ++i) {
      const float ge = clip ? g[i] * f : g[i];
      adamw_one(p[i], m[i], v[i], ge, lr, b1, b2, eps, wd, c1, c2);
      g[i] = 0.f;
    }
  }
}

unsigned blocks256(int64_t n) { return (unsigned)ceil_div(n > 0 ? n : 1, 256); }

struct Buf {
  void* p = nullptr;
  size_t n = 0;
};
int grow(Buf& b, size_t bytes) {
  if (b.n >= bytes) return SM_OK;
  if (b.p) SM_HIP(hipFree(b.p));
  b.p = nullptr;
  b.n = 0;
  SM_HIP(hipMalloc(&b.p, bytes ? bytes : 16));
  b.n = bytes;
  return SM_OK;
}

}  // namespace
}  // namespace sm

struct sm_policy {
  sm_model_config cfg;
  sm_optimizer_config opt;
  int64_t qdim = 0, kvdim = 0, qn = 0;
  int64_t rows_per_layer[sm::kKinds] = {};  // per-layer tensor shape [N, K]
  int64_t cols[sm::kKinds] = {};
  int64_t count[sm::kKinds] = {};           // elements over all layers
  float* w[sm::kKinds] = {};    // f32 masters
  float* g[sm::kKinds] = {};    // staged gradients
  float* wq[sm::kKinds] = {};   // fake-quantized copies (quantized configs)
  float* m1[sm::kKinds] = {};   // AdamW moments / Muon velocity in m1
  float* m2[sm::kKinds] = {};
  int64_t adam_step = 0, muon_step = 0;
  int planes = 3;  // bf16 planes per GEMM operand in sm_policy_prepare
  float* rope = nullptr;
  std::vector<void*> owned;
  // forward activations and scratch (grow-only)
  sm::Buf act, scratch;
  int64_t fS = 0, fP = 0, fN = 0;
  bool staged = false;
};

namespace sm {
namespace {

int palloc(sm_policy* p, float** out, int64_t n) {
  SM_HIP(hipMalloc((void**)out, (size_t)std::max<int64_t>(n, 1) * 4));
  p->owned.push_back(*out);
  zero_f32<<<blocks256(n), 256>>>(*out, n);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

// the weights the forward uses: masters, or their fake-quantized copies
const float* fw(const sm_policy* p, int kind) {
  return (p->cfg.quantized && p->wq[kind]) ? p->wq[kind] : p->w[kind];
}
const float* fwl(const sm_policy* p, int kind, int layer) {
  return fw(p, kind) + (size_t)layer * p->rows_per_layer[kind] * p->cols[kind];
}
float* gl(const sm_policy* p, int kind, int layer) {
  return p->g[kind] + (size_t)layer * p->rows_per_layer[kind] * p->cols[kind];
}

// Refresh the fake-quantized copies from the masters: Q4G128 per [N, K]
// linear (the inference model's quantizer, sm_q4_quantize) and bf16 for the
// embedding table.
int fake_quantize(sm_policy* p, hipStream_t st) {
  const auto& c = p->cfg;
  int64_t maxn = 0;
  for (int k = 0; k < kKinds; ++k)
    if (is_linear_kind(k)) maxn = std::max(maxn, p->rows_per_layer[k] * p->cols[k]);
  const int64_t groups = ceil_div(maxn, 128);
  SM_TRY(grow(p->scratch, (size_t)groups * 64 + (size_t)groups * 2 + 64));
  uint8_t* codes = (uint8_t*)p->scratch.p;
  uint16_t* scales = (uint16_t*)(codes + groups * 64);
  for (int k = 0; k < kKinds; ++k) {
    if (!is_linear_kind(k) || p->count[k] == 0) continue;
    const int64_t n = p->rows_per_layer[k] * p->cols[k];
    const int layers = (k == SM_W_LM_HEAD) ? 1 : c.layers;
    for (int l = 0; l < layers; ++l) {
      SM_TRY(sm_q4_quantize(p->w[k] + (size_t)l * n, SM_F32, n, codes, scales, nullptr, st));
      q4_decode_f32<<<blocks256(n), 256, 0, st>>>(codes, scales, n, p->wq[k] + (size_t)l * n);
    }
  }
  round_bf16_f32<<<blocks256(p->count[SM_W_EMBED]), 256, 0, st>>>(
      p->w[SM_W_EMBED], p->count[SM_W_EMBED], p->wq[SM_W_EMBED]);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

// zeropower_via_newton_schulz (muon.rs:257-285) of one [N, K] matrix in place
// of `upd`, in the orientation the reference sees it (Burn's [d_in, d_out] =
// this matrix transposed): the short side first, Frobenius-normalised, five
// quintic steps. tmp holds 2 N K + 2 min(N, K)^2 + 1 floats.
int newton_schulz(float* upd, int64_t N, int64_t K, float* tmp, hipStream_t st) {
  // Burn orientation X0 = upd^T [K, N]; with K > N iterate on X0^T = upd.
  const bool as_is = K > N;
  const int64_t r = as_is ? N : K, cdim = as_is ? K : N;
  float* x = tmp;
  float* x2 = x + N * K;
  float* gram = x2 + N * K;
  float* poly = gram + r * r;
  float* norm = poly + r * r;
  if (as_is) SM_HIP(hipMemcpyAsync(x, upd, (size_t)N * K * 4, hipMemcpyDeviceToDevice, st));
  else transpose_f32<<<blocks256(N * K), 256, 0, st>>>(upd, (int)N, (int)K, x);
  SM_TRY(sm_frobenius_normalize(x, r * cdim, kMuonEps, norm, st));
  for (int i = 0; i < kNsSteps; ++i) {
    SM_TRY(sm_gemm_ex(0, 1, r, r, cdim, 1.f, x, cdim, x, cdim, 0.f, gram, r, st));  // X X^T
    SM_TRY(sm_gemm_ex(0, 0, r, r, r, kNsC, gram, r, gram, r, 0.f, poly, r, st));    // c A A
    SM_TRY(sm_axpby(gram, poly, r * r, kNsB, 1.f, st));                              // + b A
    SM_HIP(hipMemcpyAsync(x2, x, (size_t)r * cdim * 4, hipMemcpyDeviceToDevice, st));
    SM_TRY(sm_gemm_ex(0, 0, r, cdim, r, 1.f, poly, r, x2, cdim, kNsA, x, cdim, st));  // a X + B X
  }
  if (as_is) SM_HIP(hipMemcpyAsync(upd, x, (size_t)N * K * 4, hipMemcpyDeviceToDevice, st));
  else transpose_f32<<<blocks256(N * K), 256, 0, st>>>(x, (int)K, (int)N, upd);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace
}  // namespace sm

using namespace sm;

extern "C" int sm_policy_create(const sm_model_config* cfg, const sm_optimizer_config* opt,
                                sm_policy** out) {
  SM_REQUIRE(cfg && opt && out, "sm_policy_create: null argument");
  const sm_model_config& c = *cfg;
  SM_REQUIRE(c.layers > 0 && c.d_model > 0 && c.heads > 0 && c.kv_heads > 0 &&
                 c.heads % c.kv_heads == 0 && c.ffn > 0 && c.vocab > 0 && c.max_seq > 0,
             "sm_policy_create: invalid model config");
  SM_REQUIRE(c.head_dim == 64 || c.head_dim == 128, "sm_policy_create: head_dim must be 64 or 128");
  SM_REQUIRE(c.experts == 0 || (c.experts >= 2 && c.experts <= 64 && c.expert_ffn > 0),
             "sm_policy_create: MoE configs need 2..=64 experts and expert_ffn > 0");
  if (c.quantized)
    SM_REQUIRE(c.d_model % 128 == 0 && c.ffn % 128 == 0 && (c.heads * c.head_dim) % 128 == 0 &&
                   (c.experts == 0 || c.expert_ffn % 128 == 0),
               "sm_policy_create: quantized models need d_model, ffn, heads*head_dim (and "
               "expert_ffn) %% 128 == 0");
  SM_REQUIRE(std::isfinite(opt->lr) && opt->lr >= 0.f && opt->beta1 >= 0.f && opt->beta1 < 1.f &&
                 opt->beta2 >= 0.f && opt->beta2 < 1.f && opt->eps > 0.f &&
                 opt->weight_decay >= 0.f && opt->muon_lr >= 0.f && std::isfinite(opt->grad_clip),
             "sm_policy_create: invalid optimizer settings");
  sm_policy* p = new sm_policy();
  p->cfg = c;
  p->opt = *opt;
  p->qdim = (int64_t)c.heads * c.head_dim;
  p->kvdim = (int64_t)c.kv_heads * c.head_dim;
  p->qn = p->qdim + 2 * p->kvdim;
  const int64_t d = c.d_model, F = c.ffn, E = c.experts, Fe = c.expert_ffn;
  const bool moe = E > 0;
  // per-layer [rows, cols]: an MoE layer's experts stack along the rows
  // ([E * 2Fe, d] and [E * d, Fe]) and replace the dense FFN
  const int64_t shape[kKinds][2] = {{c.vocab, d}, {1, d}, {p->qn, d}, {d, p->qdim}, {1, d},
                                    {moe ? 0 : 2 * F, d}, {moe ? 0 : d, F}, {1, d},
                                    {c.vocab, d}, {E, d}, {E * 2 * Fe, d}, {E * d, Fe}};
  auto fail = [&](int s) { sm_policy_destroy(p); return s; };
  for (int k = 0; k < kKinds; ++k) {
    p->rows_per_layer[k] = shape[k][0];
    p->cols[k] = shape[k][1];
    p->count[k] = shape[k][0] * shape[k][1] * (is_layer_kind(k) ? c.layers : 1);
    if (p->count[k] == 0) continue;
    int s;
    if ((s = palloc(p, &p->w[k], p->count[k])) || (s = palloc(p, &p->g[k], p->count[k])) ||
        (s = palloc(p, &p->m1[k], p->count[k])) || (s = palloc(p, &p->m2[k], p->count[k])))
      return fail(s);
    if (c.quantized && (is_linear_kind(k) || k == SM_W_EMBED))
      if ((s = palloc(p, &p->wq[k], p->count[k]))) return fail(s);
  }
  const int half = c.head_dim / 2;
  std::vector<float> tab((size_t)c.max_seq * half * 2);
  for (int pos = 0; pos < c.max_seq; ++pos)
    for (int q = 0; q < half; ++q) {
      const double ang = (double)pos * std::pow((double)c.rope_theta, -2.0 * q / c.head_dim);
      tab[((size_t)pos * half + q) * 2] = (float)std::cos(ang);
      tab[((size_t)pos * half + q) * 2 + 1] = (float)std::sin(ang);
    }
  int s;
  if ((s = palloc(p, &p->rope, (int64_t)tab.size()))) return fail(s);
  if (hipMemcpy(p->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
    set_error("sm_policy_create: rope upload failed");
    return fail(SM_ERR_HIP);
  }
  if (hipDeviceSynchronize() != hipSuccess) {
    set_error("sm_policy_create: initialisation failed");
    return fail(SM_ERR_HIP);
  }
  *out = p;
  return SM_OK;
}

extern "C" int sm_policy_destroy(sm_policy* p) {
  if (!p) return SM_OK;
  hipDeviceSynchronize();
  for (void* q : p->owned) hipFree(q);
  if (p->act.p) hipFree(p->act.p);
  if (p->scratch.p) hipFree(p->scratch.p);
  delete p;
  return SM_OK;
}

extern "C" int sm_policy_set_matmul_planes(sm_policy* p, int planes) {
  SM_REQUIRE(p, "sm_policy_set_matmul_planes: null policy");
  SM_REQUIRE(planes >= 1 && planes <= 3, "matmul planes must be 1, 2 or 3 (got %d)", planes);
  p->planes = planes;
  return SM_OK;
}

extern "C" int sm_policy_set_tensor(sm_policy* p, int kind, int layer, const float* src,
                                    void* stream) {
  SM_REQUIRE(p && src, "sm_policy_set_tensor: null argument");
  SM_REQUIRE(kind >= 0 && kind < kKinds, "sm_policy_set_tensor: tensor kind %d", kind);
  SM_REQUIRE(p->count[kind] > 0, "sm_policy_set_tensor: tensor kind %d is not part of this policy", kind);
  const int64_t n = p->rows_per_layer[kind] * p->cols[kind];
  float* dst = p->w[kind];
  if (is_layer_kind(kind)) {
    SM_REQUIRE(layer >= 0 && layer < p->cfg.layers, "layer %d out of range", layer);
    dst += (size_t)layer * n;
  }
  SM_HIP(hipMemcpyAsync(dst, src, (size_t)n * 4, hipMemcpyDeviceToDevice, as_stream(stream)));
  return SM_OK;
}

extern "C" int sm_policy_get_tensor(const sm_policy* p, int kind, int layer, float* dst,
                                    int gradient, void* stream) {
  SM_REQUIRE(p && dst, "sm_policy_get_tensor: null argument");
  SM_REQUIRE(kind >= 0 && kind < kKinds, "sm_policy_get_tensor: tensor kind %d", kind);
  SM_REQUIRE(p->count[kind] > 0, "sm_policy_get_tensor: tensor kind %d is not part of this policy", kind);
  const int64_t n = p->rows_per_layer[kind] * p->cols[kind];
  const float* src = gradient ? p->g[kind] : p->w[kind];
  if (is_layer_kind(kind)) {
    SM_REQUIRE(layer >= 0 && layer < p->cfg.layers, "layer %d out of range", layer);
    src += (size_t)layer * n;
  }
  SM_HIP(hipMemcpyAsync(dst, src, (size_t)n * 4, hipMemcpyDeviceToDevice, as_stream(stream)));
  return SM_OK;
}

extern "C" int sm_policy_install(const sm_policy* p, sm_model* model, void* stream) {
  SM_REQUIRE(p && model, "sm_policy_install: null argument");
  for (int k = 0; k < kKinds; ++k) {
    if (p->count[k] == 0) continue;
    const int64_t n = p->rows_per_layer[k] * p->cols[k];
    const int layers = is_layer_kind(k) ? p->cfg.layers : 1;
    for (int l = 0; l < layers; ++l)
      SM_TRY(sm_model_set_tensor(model, k, is_layer_kind(k) ? l : -1, p->w[k] + (size_t)l * n,
                                 stream));
  }
  return SM_OK;
}

namespace {
// sm_policy_prepare's body. The frozen reference's log-probs come from
// `reference` (computed here into lp_ref) or, with no reference model, from
// ref_lp_in (computed by the caller over the same tokens).
int policy_prepare(sm_policy* p, sm_model* reference, const float* ref_lp_in,
                   const int32_t* prompts, const int32_t* tokens, const float* behavior_lp,
                   const float* rewards, const float* mask, int64_t groups, int64_t group_size,
                   int64_t P, int64_t N, double clip_epsilon, double advantage_epsilon,
                   double kl_coefficient, float* lp_cur, float* lp_ref, float* group_stats,
                   float* dlp, int32_t* flags, void* stream) {
  SM_REQUIRE(p && prompts && tokens && behavior_lp && rewards && lp_cur && dlp,
             "sm_policy_prepare: null argument");
  SM_REQUIRE(kl_coefficient == 0.0 || (reference && lp_ref) || ref_lp_in,
             "GRPO rollout needs reference log-probs for positive KL coefficient");
  SM_REQUIRE(groups > 0 && group_size > 0 && P > 0 && N > 0, "sm_policy_prepare: bad shape");
  const auto& c = p->cfg;
  const int64_t S = groups * group_size, L = P + N - 1, M = S * L, R = S * N;
  SM_REQUIRE(L <= c.max_seq, "sequence length %lld exceeds max_seq_len %d", (long long)L,
             c.max_seq);
  hipStream_t st = as_stream(stream);
  const int64_t d = c.d_model, H = c.heads, KVH = c.kv_heads, hd = c.head_dim, F = c.ffn;
  const int64_t V = c.vocab, qn = p->qn, qdim = p->qdim;
  // the prepare's GEMMs on the policy's plane count, with room for their
  // transposed operands (tps: the largest need of the backward's (1, 0) and
  // (0, 0) products below)
  float* tps = nullptr;
  int64_t tps_floats = 0;
  auto pgemm = [&](int ta, int tb, int64_t m, int64_t n, int64_t k, float alpha, const float* A,
                   int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc,
                   void* sp) {
    return gemm_ex_planes(p->planes, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, sp,
                          tps, tps_floats, 3);
  };
  // the same with B a weight the forward uses: a quantized policy's are its
  // fake-quantized copies (a bf16 scale times a 4-bit code), exact in two bf16
  // planes, so three-plane products skip B's zero third plane (same bits)
  const int wb_planes = c.quantized ? 2 : 3;
  auto wgemm = [&](int ta, int tb, int64_t m, int64_t n, int64_t k, float alpha, const float* A,
                   int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc,
                   void* sp) {
    return gemm_ex_planes(p->planes, ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, sp,
                          tps, tps_floats, wb_planes);
  };
  if (c.quantized) SM_TRY(fake_quantize(p, st));
  // ---- activation arena: per layer x0, h, qkv, q, k, v, o, lse, x1, h2 and the
  // FFN's u, a (dense) or its routing and routed rows (MoE: top-2 indices and
  // weights, route plan, gathered input, [gate | value], SwiGLU, expert output)
  const int64_t E = c.experts, Fe = c.expert_ffn, RT = 2 * M;  // MoE routes (top-2)
  const bool moe = E > 0;
  const int64_t plan_words = moe ? sm_moe_plan_words(M, 2, E) : 0;
  const int64_t ffn_layer = moe ? 2 * M + 2 * M + plan_words + RT * (d + 2 * Fe + Fe + d)
                                : M * (2 * F + F);
  const int64_t ffn_fixed = moe ? RT * d /*dyr*/ + 2 * M /*gw*/ + RT * Fe /*dar*/ +
                                      RT * 2 * Fe /*dur*/ + RT * d /*drt*/ + M * E /*dlog*/ + 1
                                : M * 2 * F /*du*/ + M * F /*da*/;
  // transposed operands of the backward's weight (1, 0) and data (0, 0) GEMMs
  auto tneed = [](bool ta, bool tb, int64_t m, int64_t n, int64_t k) {
    return gemm_planes_scratch_floats(ta, tb, m, n, k);
  };
  int64_t tp_need = std::max(tneed(true, false, V, d, R), tneed(false, false, R, d, V));
  const int64_t lin[4][2] = {{qn, d}, {d, qdim}, {2 * F, d}, {d, F}};  // {out, in}
  for (int i = 0; i < (moe ? 2 : 4); ++i)
    tp_need = std::max({tp_need, tneed(true, false, lin[i][0], lin[i][1], M),
                        tneed(false, false, M, lin[i][1], lin[i][0])});
  if (moe)
    tp_need = std::max({tp_need, tneed(true, false, d, Fe, RT), tneed(false, false, RT, Fe, d),
                        tneed(true, false, 2 * Fe, d, RT), tneed(false, false, RT, d, 2 * Fe)});
  const int64_t per_layer =
      M * (d + d + qn + qdim + 2 * p->kvdim + qdim + H + d + d) + ffn_layer;
  const int64_t fixed = M * d /*x*/ + M * d /*hf*/ + R * d /*hr*/ + R * V /*logits*/ +
                        M * d /*dx*/ + M * d /*dhf*/ + R * d /*dhr*/ + ffn_fixed +
                        M * d /*dh*/ + M * qdim /*do*/ + M * qdim /*dq*/ +
                        2 * S * KVH * L * hd /*dk dv*/ + M * qn /*dqkv*/ + M /*rinv*/ +
                        S * H * L /*delta*/ + R /*row scale*/ + d /*dgamma final*/ + S /*pos0*/ +
                        rmsnorm_dgamma_chunks(M) * d /*dgamma parts*/ + tp_need;
  const size_t bytes = (size_t)(per_layer * c.layers + fixed) * 4 + (size_t)M * 4 /*ids*/ +
                       (size_t)R * 8 /*rows*/ + (size_t)(20 * c.layers + 48) * 256;
  SM_TRY(grow(p->act, bytes));
  char* cur = (char*)p->act.p;
  auto take = [&](int64_t n, size_t elem = 4) {
    char* r = cur;
    cur += ((size_t)n * elem + 255) / 256 * 256;
    return (void*)r;
  };
  struct Saved {
    float *x0, *h, *qkv, *q, *k, *v, *o, *lse, *x1, *h2, *u, *a;
    int32_t *tidx, *plan;
    float *tw, *rt, *ur, *ar, *yr;
    std::vector<int32_t> off;  // MoE: first sorted route of each expert (host)
  };
  std::vector<Saved> sv(c.layers);
  for (auto& s : sv) {
    s.x0 = (float*)take(M * d); s.h = (float*)take(M * d); s.qkv = (float*)take(M * qn);
    s.q = (float*)take(M * qdim); s.k = (float*)take(S * KVH * L * hd);
    s.v = (float*)take(S * KVH * L * hd); s.o = (float*)take(M * qdim);
    s.lse = (float*)take(S * H * L); s.x1 = (float*)take(M * d); s.h2 = (float*)take(M * d);
    if (moe) {
      s.tidx = (int32_t*)take(2 * M); s.tw = (float*)take(2 * M);
      s.plan = (int32_t*)take(plan_words); s.rt = (float*)take(RT * d);
      s.ur = (float*)take(RT * 2 * Fe); s.ar = (float*)take(RT * Fe); s.yr = (float*)take(RT * d);
      s.off.assign(E + 1, 0);
    } else {
      s.u = (float*)take(M * 2 * F); s.a = (float*)take(M * F);
    }
  }
  float* x = (float*)take(M * d);
  float* hf = (float*)take(M * d);
  float* hr = (float*)take(R * d);
  float* logits = (float*)take(R * V);
  float* dx = (float*)take(M * d);
  float* dhf = (float*)take(M * d);
  float* dhr = (float*)take(R * d);
  float *du = nullptr, *da = nullptr, *dyr = nullptr, *gw = nullptr, *dar = nullptr;
  float *dur = nullptr, *drt = nullptr, *dlog = nullptr;
  int32_t* perr = nullptr;
  if (moe) {
    dyr = (float*)take(RT * d); gw = (float*)take(2 * M); dar = (float*)take(RT * Fe);
    dur = (float*)take(RT * 2 * Fe); drt = (float*)take(RT * d); dlog = (float*)take(M * E);
    perr = (int32_t*)take(1);
  } else {
    du = (float*)take(M * 2 * F); da = (float*)take(M * F);
  }
  float* dh = (float*)take(M * d);
  float* dO = (float*)take(M * qdim);
  float* dq = (float*)take(M * qdim);
  float* dk = (float*)take(S * KVH * L * hd);
  float* dv = (float*)take(S * KVH * L * hd);
  float* dqkv = (float*)take(M * qn);
  float* rinv = (float*)take(M);
  float* delta = (float*)take(S * H * L);
  float* rscale = (float*)take(R);
  float* dgf = (float*)take(d);
  float* dgparts = (float*)take(rmsnorm_dgamma_chunks(M) * d);
  tps = (float*)take(tp_need);
  tps_floats = tp_need;
  int32_t* pos0 = (int32_t*)take(S);
  int32_t* ids = (int32_t*)take(M);
  int64_t* rows = (int64_t*)take(R, 8);
  SM_HIP(hipMemsetAsync(pos0, 0, (size_t)S * 4, st));
  build_ids_rows<<<blocks256(std::max(M, R)), 256, 0, st>>>(prompts, tokens, (int)S, (int)P,
                                                            (int)N, ids, rows);
  // ---- forward (recompute with activations kept)
  SM_TRY(sm_embed(fw(p, SM_W_EMBED), SM_F32, ids, M, d, V, 1.0f, x, stream));
  for (int l = 0; l < c.layers; ++l) {
    Saved& s = sv[l];
    SM_HIP(hipMemcpyAsync(s.x0, x, (size_t)M * d * 4, hipMemcpyDeviceToDevice, st));
    SM_TRY(sm_rmsnorm(s.x0, fwl(p, SM_W_ATTN_NORM, l), M, d, c.norm_eps, s.h, SM_F32, stream));
    SM_TRY(wgemm(0, 1, M, qn, d, 1.f, s.h, d, fwl(p, SM_W_QKV, l), d, 0.f, s.qkv, qn, stream));
    SM_TRY(sm_rope_qk(s.qkv, p->rope, pos0, S, L, H, KVH, hd, 0, stream));
    split_qkv_f32<<<blocks256(M * qn), 256, 0, st>>>(s.qkv, (int)S, (int)L, (int)H, (int)KVH,
                                                     (int)hd, s.q, s.k, s.v);
    // one plane (bf16 matmul operands): attention on bf16 operands as well
    if (p->planes == 1)
      SM_TRY(sm_attn_prefill_lse_bf16ops(s.q, s.k, s.v, pos0, s.o, s.lse, S, L, H, KVH, L, hd,
                                         stream));
    else
      SM_TRY(sm_attn_prefill_lse(s.q, s.k, s.v, pos0, s.o, s.lse, SM_F32, SM_F32, S, L, H, KVH,
                                 L, hd, stream));
    SM_HIP(hipMemcpyAsync(s.x1, s.x0, (size_t)M * d * 4, hipMemcpyDeviceToDevice, st));
    SM_TRY(wgemm(0, 1, M, d, qdim, 1.f, s.o, qdim, fwl(p, SM_W_O, l), qdim, 1.f, s.x1, d,
                      stream));
    SM_TRY(sm_rmsnorm(s.x1, fwl(p, SM_W_FFN_NORM, l), M, d, c.norm_eps, s.h2, SM_F32, stream));
    SM_HIP(hipMemcpyAsync(x, s.x1, (size_t)M * d * 4, hipMemcpyDeviceToDevice, st));
    if (moe) {
      // SparseMoe::forward (ffn.rs:478-711): f32 router, top-2 with the weights
      // a softmax over the pair, dropless expert SwiGLU FFNs over the routes
      // sorted by expert, weighted combine into the residual
      SM_TRY(sm_moe_router_top2(s.h2, SM_F32, fwl(p, SM_W_ROUTER, l), M, d, E, nullptr, s.tidx,
                                s.tw, stream));
      SM_HIP(hipMemsetAsync(perr, 0, 4, st));
      SM_TRY(sm_moe_route_plan(s.tidx, M, 2, E, s.plan, perr, stream));
      SM_TRY(sm_moe_gather(s.h2, SM_F32, s.plan, M, 2, E, d, s.rt, stream));
      // the expert row ranges on the host, for one GEMM per expert (as the
      // reference reads its counts, ffn.rs:586-598)
      SM_HIP(hipMemcpyAsync(s.off.data(), s.plan + E, (size_t)(E + 1) * 4,
                            hipMemcpyDeviceToHost, st));
      SM_HIP(hipStreamSynchronize(st));
      const float* win = fwl(p, SM_W_EXPERT_IN, l);
      const float* wdn = fwl(p, SM_W_EXPERT_DOWN, l);
      for (int64_t e = 0; e < E; ++e) {
        const int64_t o0 = s.off[e], n = s.off[e + 1] - o0;
        if (n <= 0) continue;
        SM_TRY(wgemm(0, 1, n, 2 * Fe, d, 1.f, s.rt + o0 * d, d, win + e * 2 * Fe * d, d, 0.f,
                     s.ur + o0 * 2 * Fe, 2 * Fe, stream));
      }
      SM_TRY(sm_swiglu(s.ur, SM_F32, RT, Fe, s.ar, stream));
      for (int64_t e = 0; e < E; ++e) {
        const int64_t o0 = s.off[e], n = s.off[e + 1] - o0;
        if (n <= 0) continue;
        SM_TRY(wgemm(0, 1, n, d, Fe, 1.f, s.ar + o0 * Fe, Fe, wdn + e * d * Fe, Fe, 0.f,
                     s.yr + o0 * d, d, stream));
      }
      SM_TRY(sm_moe_combine(s.yr, s.tw, s.plan, M, 2, E, d, x, stream));
    } else {
      SM_TRY(wgemm(0, 1, M, 2 * F, d, 1.f, s.h2, d, fwl(p, SM_W_IN, l), d, 0.f, s.u, 2 * F,
                   stream));
      SM_TRY(sm_swiglu(s.u, SM_F32, M, F, s.a, stream));
      SM_TRY(wgemm(0, 1, M, d, F, 1.f, s.a, F, fwl(p, SM_W_DOWN, l), F, 1.f, x, d, stream));
    }
  }
  SM_TRY(sm_rmsnorm(x, fw(p, SM_W_FINAL_NORM), M, d, c.norm_eps, hf, SM_F32, stream));
  gather_rows_f32<<<blocks256(R * d), 256, 0, st>>>(hf, rows, R, (int)d, hr);
  SM_TRY(wgemm(0, 1, R, V, d, 1.f, hr, d, fw(p, SM_W_LM_HEAD), d, 0.f, logits, V, stream));
  SM_TRY(sm_ce_rows(logits, SM_F32, tokens, R, V, V, lp_cur, nullptr, nullptr, 1.f, nullptr,
                    nullptr, stream));
  // ---- the frozen reference and the loss
  const float* ref_lp = ref_lp_in;
  if (reference && lp_ref) {
    SM_TRY(sm_rl_logprobs(reference, prompts, tokens, S, P, N, 0, lp_ref, stream));
    ref_lp = lp_ref;
  }
  SM_TRY(sm_grpo_loss(rewards, lp_cur, behavior_lp, ref_lp, mask, groups, group_size, N,
                      clip_epsilon, advantage_epsilon, kl_coefficient, group_stats, nullptr, dlp,
                      flags, stream));
  // ---- backward of sum(dlp * lp), gradients added to the staged ones.
  // d lp / d logits = onehot - softmax: the CE gradient with scale -dlp per row
  neg_f32<<<blocks256(R), 256, 0, st>>>(dlp, R, rscale);
  SM_TRY(sm_ce_rows(logits, SM_F32, tokens, R, V, V, nullptr, nullptr, logits, 1.f, rscale,
                    nullptr, stream));
  SM_TRY(pgemm(1, 0, V, d, R, 1.f, logits, V, hr, d, 1.f, p->g[SM_W_LM_HEAD], d, stream));
  SM_TRY(wgemm(0, 0, R, d, V, 1.f, logits, V, fw(p, SM_W_LM_HEAD), d, 0.f, dhr, d, stream));
  SM_HIP(hipMemsetAsync(dhf, 0, (size_t)M * d * 4, st));
  scatter_rows_f32<<<blocks256(R * d), 256, 0, st>>>(dhr, rows, R, (int)d, dhf);
  SM_TRY(rmsnorm_backward_parts(x, fw(p, SM_W_FINAL_NORM), dhf, M, d, c.norm_eps, 0, dx, dgf,
                                rinv, dgparts, st));
  SM_TRY(sm_axpby(dgf, p->g[SM_W_FINAL_NORM], d, 1.f, 1.f, stream));
  for (int l = c.layers - 1; l >= 0; --l) {
    Saved& s = sv[l];
    if (moe) {
      // x = x1 + sum_j w_j expert_{i_j}(h2): the combine's gradient to the
      // routed outputs and to the weights, the experts' data and weight
      // gradients per expert, the gather's sum back to the tokens, then the
      // router (d logits of the pair through the pair softmax; f32-grade GEMMs
      // as the reference keeps router math in f32)
      SM_TRY(sm_moe_combine_backward(dx, s.yr, SM_F32, s.tw, s.plan, M, 2, E, d, dyr, gw,
                                     stream));
      const float* win = fwl(p, SM_W_EXPERT_IN, l);
      const float* wdn = fwl(p, SM_W_EXPERT_DOWN, l);
      float* gin = gl(p, SM_W_EXPERT_IN, l);
      float* gdn = gl(p, SM_W_EXPERT_DOWN, l);
      for (int64_t e = 0; e < E; ++e) {
        const int64_t o0 = s.off[e], n = s.off[e + 1] - o0;
        if (n <= 0) continue;
        SM_TRY(wgemm(0, 0, n, Fe, d, 1.f, dyr + o0 * d, d, wdn + e * d * Fe, Fe, 0.f,
                     dar + o0 * Fe, Fe, stream));
        SM_TRY(pgemm(1, 0, d, Fe, n, 1.f, dyr + o0 * d, d, s.ar + o0 * Fe, Fe, 1.f,
                     gdn + e * d * Fe, Fe, stream));
      }
      SM_TRY(sm_swiglu_backward(s.ur, dar, SM_F32, RT, Fe, dur, stream));
      for (int64_t e = 0; e < E; ++e) {
        const int64_t o0 = s.off[e], n = s.off[e + 1] - o0;
        if (n <= 0) continue;
        SM_TRY(pgemm(1, 0, 2 * Fe, d, n, 1.f, dur + o0 * 2 * Fe, 2 * Fe, s.rt + o0 * d, d, 1.f,
                     gin + e * 2 * Fe * d, d, stream));
        SM_TRY(wgemm(0, 0, n, d, 2 * Fe, 1.f, dur + o0 * 2 * Fe, 2 * Fe, win + e * 2 * Fe * d,
                     d, 0.f, drt + o0 * d, d, stream));
      }
      SM_TRY(sm_moe_gather_backward(drt, SM_F32, s.plan, M, 2, E, d, dh, stream));
      router_grad_kernel<<<blocks256(M * E), 256, 0, st>>>(s.tw, gw, s.tidx, M, (int)E, dlog);
      SM_TRY(gemm_ex_planes(3, 0, 0, M, d, E, 1.f, dlog, E, fwl(p, SM_W_ROUTER, l), d, 1.f, dh,
                            d, stream));
      SM_TRY(gemm_ex_planes(3, 1, 0, E, d, M, 1.f, dlog, E, s.h2, d, 1.f,
                            gl(p, SM_W_ROUTER, l), d, stream));
    } else {
      // FFN: x = x1 + swiglu(h2 W_in^T) W_down^T
      SM_TRY(wgemm(0, 0, M, F, d, 1.f, dx, d, fwl(p, SM_W_DOWN, l), F, 0.f, da, F, stream));
      SM_TRY(pgemm(1, 0, d, F, M, 1.f, dx, d, s.a, F, 1.f, gl(p, SM_W_DOWN, l), F, stream));
      SM_TRY(sm_swiglu_backward(s.u, da, SM_F32, M, F, du, stream));
      SM_TRY(pgemm(1, 0, 2 * F, d, M, 1.f, du, 2 * F, s.h2, d, 1.f, gl(p, SM_W_IN, l), d,
                   stream));
      SM_TRY(wgemm(0, 0, M, d, 2 * F, 1.f, du, 2 * F, fwl(p, SM_W_IN, l), d, 0.f, dh, d,
                   stream));
    }
    SM_TRY(rmsnorm_backward_parts(s.x1, fwl(p, SM_W_FFN_NORM, l), dh, M, d, c.norm_eps, 1, dx,
                                  gl(p, SM_W_FFN_NORM, l), rinv, dgparts, st));
    // attention: x1 = x0 + attn(rope(h W_qkv^T)) W_o^T
    SM_TRY(wgemm(0, 0, M, qdim, d, 1.f, dx, d, fwl(p, SM_W_O, l), qdim, 0.f, dO, qdim,
                      stream));
    SM_TRY(pgemm(1, 0, d, qdim, M, 1.f, dx, d, s.o, qdim, 1.f, gl(p, SM_W_O, l), qdim,
                      stream));
    SM_TRY((p->planes == 1 ? sm_attn_backward_bf16ops : sm_attn_backward_f32)(
        s.q, s.k, s.v, s.o, dO, s.lse, S, L, H, KVH, hd, dq, dk, dv, delta, stream));
    merge_qkv_f32<<<blocks256(M * qn), 256, 0, st>>>(dq, dk, dv, (int)S, (int)L, (int)H,
                                                     (int)KVH, (int)hd, dqkv);
    SM_TRY(sm_rope_qk(dqkv, p->rope, pos0, S, L, H, KVH, hd, 1, stream));
    SM_TRY(pgemm(1, 0, qn, d, M, 1.f, dqkv, qn, s.h, d, 1.f, gl(p, SM_W_QKV, l), d, stream));
    SM_TRY(wgemm(0, 0, M, d, qn, 1.f, dqkv, qn, fwl(p, SM_W_QKV, l), d, 0.f, dh, d, stream));
    SM_TRY(rmsnorm_backward_parts(s.x0, fwl(p, SM_W_ATTN_NORM, l), dh, M, d, c.norm_eps, 1, dx,
                                  gl(p, SM_W_ATTN_NORM, l), rinv, dgparts, st));
  }
  SM_TRY(sm_embed_backward(ids, dx, M, d, V, p->g[SM_W_EMBED], stream));
  SM_LAUNCH_CHECK();
  p->staged = true;
  return SM_OK;
}
}  // namespace

extern "C" int sm_policy_prepare(sm_policy* p, sm_model* reference, const int32_t* prompts,
                                 const int32_t* tokens, const float* behavior_lp,
                                 const float* rewards, const float* mask, int64_t groups,
                                 int64_t group_size, int64_t P, int64_t N, double clip_epsilon,
                                 double advantage_epsilon, double kl_coefficient, float* lp_cur,
                                 float* lp_ref, float* group_stats, float* dlp, int32_t* flags,
                                 void* stream) {
  return policy_prepare(p, reference, nullptr, prompts, tokens, behavior_lp, rewards, mask,
                        groups, group_size, P, N, clip_epsilon, advantage_epsilon,
                        kl_coefficient, lp_cur, lp_ref, group_stats, dlp, flags, stream);
}

extern "C" int sm_policy_prepare_with_ref(sm_policy* p, const float* reference_lp,
                                          const int32_t* prompts, const int32_t* tokens,
                                          const float* behavior_lp, const float* rewards,
                                          const float* mask, int64_t groups, int64_t group_size,
                                          int64_t P, int64_t N, double clip_epsilon,
                                          double advantage_epsilon, double kl_coefficient,
                                          float* lp_cur, float* group_stats, float* dlp,
                                          int32_t* flags, void* stream) {
  return policy_prepare(p, nullptr, reference_lp, prompts, tokens, behavior_lp, rewards, mask,
                        groups, group_size, P, N, clip_epsilon, advantage_epsilon,
                        kl_coefficient, lp_cur, nullptr, group_stats, dlp, flags, stream);
}

extern "C" int sm_policy_optimizer_step(sm_policy* p, double learning_rate_scale,
                                        float* grad_norm, void* stream) {
  SM_REQUIRE(p, "sm_policy_optimizer_step: null policy");
  SM_REQUIRE(std::isfinite(learning_rate_scale) && learning_rate_scale >= 0.0,
             "learning rate scale must be finite and non-negative");
  hipStream_t st = as_stream(stream);
  // global gradient norm over every staged gradient, then the clip
  int64_t maxn = 0;
  for (int k = 0; k < kKinds; ++k) maxn = std::max(maxn, p->rows_per_layer[k] * p->cols[k]);
  int64_t ns_floats = 0;  // Newton-Schulz scratch: 2 N K + 2 min(N, K)^2 + 1 per projection
  for (int k = 0; k < kKinds; ++k)
    if (is_muon_kind(k) && p->count[k] > 0) {
      const int64_t n = p->rows_per_layer[k], kk = p->cols[k], r = std::min(n, kk);
      ns_floats = std::max(ns_floats, 2 * n * kk + 2 * r * r + 1);
    }
  int64_t nparts = 0;
  for (int k = 0; k < kKinds; ++k) nparts += ceil_div(p->count[k], kSumChunk);
  const size_t head = ((size_t)(nparts + 1) * 8 + 255) / 256 * 256;
  SM_TRY(grow(p->scratch, head + (size_t)(ns_floats + maxn) * 4));
  double* acc = (double*)p->scratch.p;
  double* parts = acc + 1;
  float* upd = (float*)((char*)p->scratch.p + head);
  float* ns_tmp = upd + maxn;
  for (int k = 0, off = 0; k < kKinds; ++k) {
    const int64_t nb = ceil_div(p->count[k], kSumChunk);
    if (nb == 0) continue;
    sumsq_kernel<<<(unsigned)nb, 256, 0, st>>>(p->g[k], p->count[k], parts + off);
    off += (int)nb;
  }
  sum_parts_kernel<<<1, 256, 0, st>>>(parts, nparts, acc);
  SM_LAUNCH_CHECK();
  double sumsq = 0.0;
  SM_HIP(hipMemcpyAsync(&sumsq, acc, 8, hipMemcpyDeviceToHost, st));
  SM_HIP(hipStreamSynchronize(st));
  const float norm = (float)std::sqrt(sumsq);
  if (grad_norm) *grad_norm = norm;
  SM_REQUIRE(std::isfinite(norm), "non-finite gradient norm at optimizer step %lld: %g",
             (long long)(p->adam_step + 1), (double)norm);
  const auto& o = p->opt;
  const float lr = (float)(o.lr * learning_rate_scale);
  const float muon_lr = (float)(o.muon_lr * learning_rate_scale);
  const bool muon = o.muon_lr > 0.f;
  // the clip runs on its own only ahead of Muon's momentum; AdamW applies it
  // inside its pass
  for (int k = 0; k < kKinds; ++k)
    if (p->count[k] > 0 && muon && is_muon_kind(k))
      clip_scale_kernel<<<blocks256(p->count[k]), 256, 0, st>>>(p->g[k], p->count[k], acc,
                                                                p->opt.grad_clip);
  SM_LAUNCH_CHECK();
  ++p->adam_step;
  if (muon) ++p->muon_step;
  for (int k = 0; k < kKinds; ++k) {
    if (p->count[k] == 0) continue;
    if (muon && is_muon_kind(k)) {
      // BatchedMuon::step (muon.rs:196-215): momentum, Newton-Schulz, and the
      // learning rate scaled by sqrt(max(1, d_in / d_out)) of Burn's [d_in, d_out]
      const int64_t N = p->rows_per_layer[k], K = p->cols[k], n = N * K;
      const float adj = muon_lr * std::sqrt(std::max(1.0f, (float)K / (float)N));
      for (int l = 0; l < p->cfg.layers; ++l) {
        float* w = p->w[k] + (size_t)l * n;
        float* gr = p->g[k] + (size_t)l * n;
        float* vel = p->m1[k] + (size_t)l * n;
        SM_TRY(sm_muon_momentum(gr, vel, upd, n, kMuonMomentum, p->muon_step == 1 ? 1 : 0, stream));
        SM_TRY(newton_schulz(upd, N, K, ns_tmp, st));
        SM_TRY(sm_axpby(upd, w, n, -adj, 1.f, stream));
      }
      zero_f32<<<blocks256(p->count[k]), 256, 0, st>>>(p->g[k], p->count[k]);
    } else {
      SM_REQUIRE(std::isfinite(lr) && o.beta1 >= 0.f && o.beta1 < 1.f && o.beta2 >= 0.f &&
                     o.beta2 < 1.f && o.eps > 0.f && o.weight_decay >= 0.f,
                 "sm_adamw_step: invalid hyperparameters");
      const float c1 = 1.f - powf(o.beta1, (float)p->adam_step);
      const float c2 = 1.f - powf(o.beta2, (float)p->adam_step);
      adamw_clip_clear_kernel<<<blocks256(ceil_div(p->count[k], 4)), 256, 0, st>>>(
          p->w[k], p->g[k], p->m1[k], p->m2[k], p->count[k], norm, o.grad_clip, lr, o.beta1,
          o.beta2, o.eps, o.weight_decay, c1, c2);
    }
  }
  SM_LAUNCH_CHECK();
  p->staged = false;
  return SM_OK;
}
