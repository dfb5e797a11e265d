// Decoder model + RL-step runtime (host C++ over the HIP kernels).
//
// This is the device side of GrpoDeviceBatchRuntime
// (summa-train/src/posttrain.rs:1288-1305): batched rollout generation
// (generate_device_batch; the reference runs TextGenerator::generate batch 1
// per rollout, summa-llm/src/generate.rs:53-124), log-prob recompute for the
// current and frozen policies (padded_group_log_probabilities,
// summa-train/src/tensor_sleep.rs:2531-2689) and the GRPO loss
// (prepare_device_batch). The model is the MAL Transformer restricted to what
// the configs use: pre-norm blocks x += Attn(RMSNorm(x)); x += FFN(RMSNorm(x))
// (block.rs:80-157), RoPE GQA attention (attention.rs:66-371), SwiGLU FFN
// (ffn.rs:854-886), final RMSNorm + LM head (transformer.rs:802-909).
//
// Precision policy. fp32 models: everything fp32 (the reference CPU path).
// Quantized models: Q4G128 linears (incl. LM head), bf16 embedding table,
// fp32 residual stream (the reference's decode stream, transformer.rs:588-592),
// matmul inputs as f16 hi/lo pairs (SM_F16X2: x = hi + lo, about 22
// significant bits, so activation roundings add no log-prob noise; a single
// f16 or bf16 rounding per matmul input drifts past the 2e-3 parity bar at
// 24 layers), f16 q and KV cache (3 more significand bits than bf16 in the
// same bytes), fp32 logits.
#include <cmath>
#include <cstring>
#include <vector>

#include "common.hpp"
#include "sampling.hpp"

extern "C" {
int sm_q4_matmul(const uint8_t*, const uint16_t*, int64_t, int64_t, const void*, int, int64_t,
                 int64_t, void*, int64_t, int, void*);
int sm_q4_qkv_rope(const uint8_t*, const uint16_t*, int64_t, int64_t, int64_t, int64_t,
                   const void*, int, int64_t, int64_t, int64_t, const float*, const int32_t*,
                   int64_t, void*, void*, void*, int, void*);
int64_t sm_q4_matmul_workspace_bytes(int64_t, int64_t, int64_t, int);
int sm_q4_matmul_ws(const uint8_t*, const uint16_t*, int64_t, int64_t, const void*, int, int64_t,
                    int64_t, void*, int64_t, int, void*, int64_t, void*);
int sm_q4_quantize(const void*, int, int64_t, uint8_t*, uint16_t*, int32_t*, void*);
int sm_q4_pack(const uint8_t*, const uint16_t*, int64_t, int64_t, uint8_t*, uint16_t*, void*);
int sm_gemm_f32(const float*, int64_t, int64_t, const float*, int64_t, int64_t, float*, int64_t,
                int, void*);
int sm_swiglu_f32(const float*, int64_t, int64_t, float*, void*);
int sm_embed(const void*, int, const int32_t*, int64_t, int64_t, int64_t, float, float*, void*);
int sm_rmsnorm(const float*, const float*, int64_t, int64_t, float, void*, int, void*);
int sm_rope_append(const float*, const float*, const int32_t*, int64_t, int64_t, int64_t, int64_t,
                   int64_t, int64_t, void*, int, void*, void*, int, void*);
int sm_attn_decode(const void*, const void*, const void*, const int32_t*, void*, int, int,
                   int64_t, int64_t, int64_t, int64_t, int64_t, void*);
int sm_attn_prefill(const void*, const void*, const void*, const int32_t*, void*, int, int,
                    int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, void*);
int sm_moe_combine_rmsnorm(const float*, const float*, const int32_t*, int64_t, int64_t, int64_t,
                           int64_t, float*, const float*, float, void*, void*);
int sm_q4_matmul_add_rmsnorm(const uint8_t*, const uint16_t*, int64_t, int64_t, const void*, int,
                             int64_t, int64_t, float*, const float*, float, void*, void*, int64_t,
                             void*);
int64_t sm_attn_decode_prefix_workspace_bytes(int64_t, int64_t, int64_t, int64_t, int64_t,
                                              int64_t);
int sm_attn_decode_prefix(const void*, const void*, const void*, const void*, const void*,
                          const int32_t*, void*, void*, int64_t, int, int, int64_t, int64_t,
                          int64_t, int64_t, int64_t, int64_t, int64_t, void*);
int sm_sample(const float*, int64_t, int64_t, int64_t, float, uint64_t, int64_t, int32_t*, int64_t,
              float*, int64_t, int32_t*, void*);
int sm_ce_rows(const void*, int, const int32_t*, int64_t, int64_t, int64_t, float*, float*, void*,
               float, const float*, float*, void*);
int sm_grpo_loss(const float*, const float*, const float*, const float*, const float*, int64_t,
                 int64_t, int64_t, double, double, double, float*, float*, float*, int32_t*, void*);
int sm_fill_normal(void*, int, int64_t, float, float, uint64_t, void*);
int64_t sm_moe_plan_words(int64_t, int64_t, int64_t);
int sm_moe_router_top2(const void*, int, const float*, int64_t, int64_t, int64_t, float*, int32_t*,
                       float*, void*);
int sm_moe_route_plan(const int32_t*, int64_t, int64_t, int64_t, int32_t*, int32_t*, void*);
int sm_q4_matmul_add_rmsnorm_router(const uint8_t*, const uint16_t*, int64_t, int64_t, const void*,
                                    int, int64_t, int64_t, float*, const float*, float, void*,
                                    const float*, int64_t, float*, int32_t*, float*, void*,
                                    int64_t, void*);
int sm_q4_grouped_matmul(const uint8_t*, const uint16_t*, int64_t, int64_t, int64_t, const void*,
                         int, int64_t, int, const int32_t*, int64_t, int64_t, void*, int64_t, int,
                         void*);
int sm_moe_combine(const float*, const float*, const int32_t*, int64_t, int64_t, int64_t, int64_t,
                   float*, void*);
}

namespace sm {
namespace {

// A workspace buffer of the model: grow-only device memory the model
// allocates itself, or (fixed) a slice of a caller-bound workspace, which is
// never reallocated: a call that needs more fails instead.
struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
  bool fixed = false;
  // bumped whenever p changes (growth, release, binding): a prompt state
  // recorded in this buffer is stale once its generation moved
  uint64_t gen = 0;
};

int ensure(DevBuf& b, size_t bytes) {
  if (b.n >= bytes) return SM_OK;
  ++b.gen;
  SM_REQUIRE(!b.fixed,
             "the bound workspace holds %zu bytes for a buffer this call needs %zu of: query "
             "sm_rl_workspace_bytes for the larger shape and bind again",
             b.n, bytes);
  if (b.p) SM_HIP(hipFree(b.p));
  b.p = nullptr;
  b.n = 0;
  SM_HIP(hipMalloc(&b.p, bytes ? bytes : 16));
  b.n = bytes;
  return SM_OK;
}

struct Linear {
  int64_t N = 0, K = 0;
  uint8_t* codes = nullptr;
  uint16_t* scales = nullptr;
  float* w = nullptr;
};

struct Layer {
  float* attn_norm = nullptr;
  float* ffn_norm = nullptr;
  Linear qkv, o, in, down;
  // MoE layers: router [E, d] f32 and E stacked experts (prepared Q4), each
  // expert's weights at codes + e * (rows(N) * K/2), scales + e * (rows(N) * K/128)
  float* router = nullptr;
  Linear exp_in, exp_down;  // N/K are one expert's shape
};

__global__ void fill_f32_kernel(float* p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void set_positions_kernel(int32_t* pos, int32_t* lens, int S, int value) {
  const int s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s < S) {
    pos[s] = value;
    lens[s] = value + 1;
  }
}

// rows [S, d] <- x[s*L + off, :]
__global__ void gather_rows_kernel(const float* __restrict__ x, int S, int L, int off, int d,
                                   float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)S * d) return;
  const int64_t s = i / d;
  const int c = i % d;
  out[i] = x[(s * L + off) * d + c];
}

// out [S, N, d] <- x[s*L + P-1 + n, :] for n < N
__global__ void gather_span_kernel(const float* __restrict__ x, int S, int L, int first, int N,
                                   int d, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)S * N * d) return;
  const int c = i % d;
  const int64_t sn = i / d;
  const int64_t s = sn / N;
  const int n = sn % N;
  out[i] = x[(s * L + first + n) * d + c];
}

// ids [S, P+N-1] <- prompt ‖ tokens[:, :N-1]
__global__ void build_ids_kernel(const int32_t* __restrict__ prompts,
                                 const int32_t* __restrict__ tokens, int S, int P, int N,
                                 int32_t* __restrict__ ids) {
  const int L = P + N - 1;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)S * L) return;
  const int64_t s = i / L;
  const int t = i % L;
  ids[i] = (t < P) ? prompts[s * P + t] : tokens[s * N + (t - P)];
}

__global__ void zero_i32_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// ---- prompt groups: G consecutive rollouts share one prompt
// flag[0] = 1 where a prompt row differs from its group's first row (every
// writer stores the same value)
// flag[0] = 1 if a prompt row differs from its group's first; with cached
// ([groups, P] ids of the prompt state), flag[1] = 1 if a group's prompt
// differs from the cached one.
__global__ void check_groups_kernel(const int32_t* __restrict__ prompts, int64_t S, int G, int P,
                                    const int32_t* __restrict__ cached,
                                    int32_t* __restrict__ flag) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= S * P) return;
  const int64_t s = i / P, t = i % P;
  if (prompts[i] != prompts[(s / G) * G * P + t]) flag[0] = 1;
  if (cached && prompts[i] != cached[(s / G) * P + t]) flag[1] = 1;
}

// out [groups, P] <- prompt row g * G
__global__ void group_prompts_kernel(const int32_t* __restrict__ prompts, int64_t groups, int G,
                                     int P, int32_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= groups * P) return;
  const int64_t g = i / P, t = i % P;
  out[i] = prompts[g * G * P + t];
}

// K or V cache rows of positions 0..P-1 for `nl` layers: sequence s of dst
// ([S][KVH][cap][hd] per layer, layer stride dls bytes) <- group
// (s0 + s) / G - g0 of src ([groups][KVH][P][hd], layer stride sls bytes);
// rows of rb bytes, copied in 16-byte chunks
__global__ void broadcast_prefix_kernel(const char* __restrict__ src, char* __restrict__ dst,
                                        int nl, int64_t S, int64_t s0, int64_t g0, int G, int KVH,
                                        int P, int cap, int rb, int64_t sls, int64_t dls) {
  const int q16 = rb / 16;
  const int64_t n = (int64_t)nl * S * KVH * P * q16;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int q = i % q16;
  int64_t r = i / q16;
  const int pos = r % P;
  r /= P;
  const int kh = r % KVH;
  r /= KVH;
  const int64_t s = r % S;
  const int l = (int)(r / S);
  const int64_t g = (s0 + s) / G - g0;
  const char* from = src + l * sls + ((g * KVH + kh) * P + pos) * (int64_t)rb + q * 16;
  char* to = dst + l * dls + ((s * KVH + kh) * (int64_t)cap + pos) * rb + q * 16;
  *reinterpret_cast<u32x4*>(to) = *reinterpret_cast<const u32x4*>(from);
}

// rows [S, d] <- x[((s / G) * L + off), :] (the group's hidden row)
__global__ void gather_group_rows_kernel(const float* __restrict__ x, int64_t S, int G, int L,
                                         int off, int d, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= S * d) return;
  const int64_t s = i / d;
  const int c = i % d;
  out[i] = x[((s / G) * L + off) * d + c];
}

// continuation ids [S, N-1] <- tokens[:, :N-1]
__global__ void cont_ids_kernel(const int32_t* __restrict__ tokens, int64_t S, int N,
                                int32_t* __restrict__ ids) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= S * (N - 1)) return;
  ids[i] = tokens[(i / (N - 1)) * N + i % (N - 1)];
}

// scored rows [S, N, d] of rollouts s0..s0+S-1: n = 0 from the group's last
// prompt row prow[(s0 + s) / G], n >= 1 from the continuation pass xc[s, n-1]
__global__ void gather_cont_rows_kernel(const float* __restrict__ prow,
                                        const float* __restrict__ xc, int64_t S, int64_t s0,
                                        int G, int N, int d, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= S * N * d) return;
  const int c = i % d;
  const int64_t sn = i / d, s = sn / N;
  const int n = sn % N;
  out[i] = n == 0 ? prow[((s0 + s) / G) * d + c] : xc[(s * (N - 1) + n - 1) * d + c];
}

unsigned blocks_for(int64_t n) { return (unsigned)ceil_div(n > 0 ? n : 1, 256); }

}  // namespace
}  // namespace sm

struct sm_model {
  sm_model_config cfg;
  int act = SM_F32;       // matmul-input activation dtype (f16 pairs when quantized)
  int kvt = SM_F32;       // q / KV cache dtype (f16 when quantized)
  int embt = SM_F32;      // embedding table dtype (bf16 when quantized)
  size_t act_size = 4;    // bytes per activation value (f32, or an f16 pair)
  size_t kv_size = 4;     // bytes per q / cache value
  size_t emb_size = 4;
  // f16 elements (or f32 values) per activation row of `width` values
  int64_t act_ld(int64_t width) const { return act == SM_F16X2 ? 2 * width : width; }
  int64_t qdim = 0, kvdim = 0, qkv_n = 0;
  void* embed = nullptr;
  float* final_norm = nullptr;
  sm::Linear lm_head;
  std::vector<sm::Layer> layers;
  float* rope = nullptr;
  std::vector<void*> owned;
  size_t weight_bytes = 0;
  // workspace
  sm::DevBuf x, h, qkv, qb, attn, u, gv, logits, rows, ids, pos, lens, next_ids, kc, vc, rkc, rvc,
      lp_tmp, flags, moe_idx, moe_w, moe_plan, moe_u, moe_y, moe_err, moe_lg, mmws, seen, done;
  // prompt groups (sm_model_set_prompt_groups): rollouts g*G .. g*G+G-1 share
  // one prompt, whose positions are computed once per group: their K / V for
  // every layer [layers][groups][KVH][P][hd] and last hidden rows [groups, d]
  int64_t prompt_group = 1;
  sm::DevBuf pkc, pvc, prow;
  // the grouped prompt pass last computed (by a generation's prefill or a
  // recompute): its group prompt ids [groups, P] (pids), K / V (pkc, pvc) and
  // last hidden rows (prow) serve a later grouped recompute of the same
  // prompts with the same weights and buffers, which then skips its prompt pass
  sm::DevBuf pids;
  bool pstate_valid = false;
  uint64_t pstate_weights = 0;
  uint64_t pstate_gens[4] = {0, 0, 0, 0};  // pkc, pvc, prow, pids generations
  int64_t pstate_groups = 0, pstate_G = 0, pstate_P = 0;
  uint64_t weights_version = 1;  // bumped by every weight write
  // partials of the shared-prompt decode attention (sm_attn_decode_prefix)
  sm::DevBuf apart;
  int64_t gen_cap = 0, gen_S = 0;
  // caller-bound workspace (sm_model_bind_workspace): the buffers above are
  // fixed slices of it
  void* ws_base = nullptr;
  int64_t ws_bytes = 0;
  // MoE router trace (sm_model_trace_routes): top-2 ids [cap, 2], logits [cap, E]
  int32_t* trace_idx = nullptr;
  float* trace_logits = nullptr;
  int64_t trace_cap = 0, trace_used = 0, trace_dropped = 0;
};

namespace sm {
namespace {

int dalloc(sm_model* m, void** p, size_t bytes, bool weight) {
  SM_HIP(hipMalloc(p, bytes ? bytes : 16));
  m->owned.push_back(*p);
  if (weight) m->weight_bytes += bytes;
  return SM_OK;
}

int alloc_linear(sm_model* m, Linear& L, int64_t N, int64_t K, int64_t count = 1) {
  L.N = N;
  L.K = K;
  if (m->cfg.quantized) {
    // prepared tiled layout (sm_q4_pack): rows padded to a multiple of 16
    const int64_t rows = q4t_rows(N);
    SM_TRY(dalloc(m, (void**)&L.codes, (size_t)count * rows * K / 2, true));
    SM_TRY(dalloc(m, (void**)&L.scales, (size_t)count * rows * (K / 128) * 2, true));
  } else {
    SM_TRY(dalloc(m, (void**)&L.w, (size_t)(N * K) * 4, true));
  }
  return SM_OK;
}

// Split-K workspace for batch-size Q4 matmuls (capped: the split is only used
// when a grid underfills the GPU, i.e. at decode batch sizes).
constexpr int64_t kMatmulWs = 64ll << 20;

int q4_linear(sm_model* m, const Linear& L, const void* x, int64_t M, void* y, int64_t ldy,
              int epi, hipStream_t st) {
  const int64_t want = std::min(kMatmulWs, sm_q4_matmul_workspace_bytes(M, L.N, L.K, epi));
  if (want > 0) SM_TRY(ensure(m->mmws, (size_t)want));
  return sm_q4_matmul_ws(L.codes, L.scales, L.N, L.K, x, m->act, M, m->act_ld(L.K), y, ldy, epi,
                         want > 0 ? m->mmws.p : nullptr, want, st);
}

// y (+)= x . W^T. x: activation dtype [M, K]; y f32 [M, N] (ADD or STORE).
int linear_f32out(sm_model* m, const Linear& L, const void* x, int64_t M, float* y, bool add,
                  hipStream_t st) {
  const int epi = add ? SM_EPI_ADD_F32 : SM_EPI_STORE_F32;
  if (m->cfg.quantized) return q4_linear(m, L, x, M, y, L.N, epi, st);
  return sm_gemm_f32(L.w, L.N, L.K, (const float*)x, M, L.K, y, L.N, epi, st);
}

// x += xin . W^T, then m->h = RMSNorm(x) * gamma in the activation dtype (a
// residual projection and the norm that follows it). Quantized models make it
// one call, which at decode batch sizes sums the projection's split-K partials
// into x and normalises the rows in one launch; elsewhere the two steps.
// router (MoE layers, quantized models): also the router's top-2 of the normed
// rows into m->moe_idx / m->moe_w (and, under a router trace, the logits into
// m->moe_lg; sm_q4_matmul_add_rmsnorm_router).
int linear_add_norm(sm_model* m, const Linear& L, const void* xin, int64_t M, float* x,
                    const float* gamma, hipStream_t st, const float* router = nullptr) {
  const auto& c = m->cfg;
  if (c.quantized && m->act == SM_F16X2) {
    const int64_t want =
        std::min(kMatmulWs, sm_q4_matmul_workspace_bytes(M, L.N, L.K, SM_EPI_ADD_F32));
    if (want > 0) SM_TRY(ensure(m->mmws, (size_t)want));
    if (router) {  // top-2 into moe_idx / moe_w; the logits only for a router trace
      SM_TRY(ensure(m->moe_idx, (size_t)M * 2 * 4));
      SM_TRY(ensure(m->moe_w, (size_t)M * 2 * 4));
      if (m->trace_logits) SM_TRY(ensure(m->moe_lg, (size_t)M * c.experts * 4));
      return sm_q4_matmul_add_rmsnorm_router(
          L.codes, L.scales, L.N, L.K, xin, m->act, M, m->act_ld(L.K), x, gamma, c.norm_eps,
          m->h.p, router, c.experts, m->trace_logits ? (float*)m->moe_lg.p : nullptr,
          (int32_t*)m->moe_idx.p, (float*)m->moe_w.p, want > 0 ? m->mmws.p : nullptr, want, st);
    }
    return sm_q4_matmul_add_rmsnorm(L.codes, L.scales, L.N, L.K, xin, m->act, M, m->act_ld(L.K),
                                    x, gamma, c.norm_eps, m->h.p, want > 0 ? m->mmws.p : nullptr,
                                    want, st);
  }
  SM_TRY(linear_f32out(m, L, xin, M, x, true, st));
  return sm_rmsnorm(x, gamma, M, c.d_model, c.norm_eps, m->h.p, m->act, st);
}

// u = silu(x W_gate^T) * (x W_value^T) in the activation dtype.
int linear_swiglu(sm_model* m, const Linear& L, const void* x, int64_t M, void* u,
                  hipStream_t st) {
  if (m->cfg.quantized)
    return q4_linear(m, L, x, M, u, m->act_ld(L.N / 2), SM_EPI_SWIGLU_F16X2, st);
  SM_TRY(ensure(m->gv, (size_t)M * L.N * 4));
  SM_TRY(sm_gemm_f32(L.w, L.N, L.K, (const float*)x, M, L.K, (float*)m->gv.p, L.N,
                     SM_EPI_STORE_F32, st));
  return sm_swiglu_f32((const float*)m->gv.p, M, L.N / 2, (float*)u, st);
}

// x += MoE(h) for `rows` tokens: router + top-2, route plan, two grouped Q4
// matmuls (gathered SwiGLU in, down), combine. All device side. With
// next_norm, the combine also leaves RMSNorm(x) * next_norm in m->h (the next
// layer's attention norm, one launch). routed: the FFN norm already ran the
// router (linear_add_norm with the router: top-2 in m->moe_idx / m->moe_w,
// logits in m->moe_lg under a trace).
int moe_ffn(sm_model* m, const Layer& Ly, int64_t rows, hipStream_t st,
            const float* next_norm = nullptr, bool routed = false) {
  const auto& c = m->cfg;
  const int64_t E = c.experts, Fe = c.expert_ffn, d = c.d_model, k = 2;
  const int64_t routes = rows * k;
  SM_TRY(ensure(m->moe_idx, (size_t)routes * 4));
  SM_TRY(ensure(m->moe_w, (size_t)routes * 4));
  SM_TRY(ensure(m->moe_plan, (size_t)sm_moe_plan_words(rows, k, E) * 4));
  SM_TRY(ensure(m->moe_u, (size_t)routes * Fe * m->act_size));
  SM_TRY(ensure(m->moe_y, (size_t)routes * d * 4));
  SM_TRY(ensure(m->moe_err, 4));
  int32_t* plan = (int32_t*)m->moe_plan.p;
  int32_t* trace_idx = nullptr;
  float* trace_lg = nullptr;
  if (m->trace_idx) {
    if (m->trace_used + rows <= m->trace_cap) {
      trace_idx = m->trace_idx + m->trace_used * 2;
      if (m->trace_logits) trace_lg = m->trace_logits + m->trace_used * E;
      m->trace_used += rows;
    } else {
      m->trace_dropped += rows;
    }
  }
  if (!routed)
    SM_TRY(sm_moe_router_top2(m->h.p, m->act, Ly.router, rows, d, E, trace_lg,
                              (int32_t*)m->moe_idx.p, (float*)m->moe_w.p, st));
  else if (trace_lg)
    SM_HIP(hipMemcpyAsync(trace_lg, m->moe_lg.p, (size_t)rows * E * 4, hipMemcpyDeviceToDevice,
                          st));
  SM_TRY(sm_moe_route_plan((const int32_t*)m->moe_idx.p, rows, k, E, plan,
                           (int32_t*)m->moe_err.p, st));
  if (trace_idx)
    SM_HIP(hipMemcpyAsync(trace_idx, m->moe_idx.p, (size_t)routes * 4, hipMemcpyDeviceToDevice,
                          st));
  SM_TRY(sm_q4_grouped_matmul(Ly.exp_in.codes, Ly.exp_in.scales, E, 2 * Fe, d, m->h.p, m->act,
                              m->act_ld(d), 1, plan, rows, k, m->moe_u.p, m->act_ld(Fe),
                              SM_EPI_SWIGLU_F16X2, st));
  SM_TRY(sm_q4_grouped_matmul(Ly.exp_down.codes, Ly.exp_down.scales, E, d, Fe, m->moe_u.p,
                              m->act, m->act_ld(Fe), 0, plan, rows, k, m->moe_y.p, d,
                              SM_EPI_STORE_F32, st));
  if (next_norm && m->act == SM_F16X2)
    return sm_moe_combine_rmsnorm((const float*)m->moe_y.p, (const float*)m->moe_w.p, plan, rows,
                                  k, E, d, (float*)m->x.p, next_norm, c.norm_eps, m->h.p, st);
  SM_TRY(sm_moe_combine((const float*)m->moe_y.p, (const float*)m->moe_w.p, plan, rows, k, E, d,
                        (float*)m->x.p, st));
  return next_norm ? sm_rmsnorm((const float*)m->x.p, next_norm, rows, d, c.norm_eps, m->h.p,
                                m->act, st)
                   : SM_OK;
}

size_t cache_layer_elems(const sm_model* m, int64_t S, int64_t cap) {
  return (size_t)S * m->cfg.kv_heads * cap * m->cfg.head_dim;
}

// The K / V of prompt positions 0..P-1 computed once per group of G rollouts
// (src [layers][groups][KVH][P][hd], layer stride `layer_bytes`), for
// run_layers over rollouts s0, s0 + 1, ... of a continuation (copied into
// cache positions 0..P-1 before each layer), or, at decode, read in place by
// the shared-prompt attention (sm_attn_decode_prefix).
struct PrefixKV {
  const void* k;
  const void* v;
  int64_t layer_bytes;
  int G, P;
  int64_t s0;
};

// Rollouts per continuation chunk of the grouped recompute: as many whole
// rollouts as keep their N - 1 new rows within the token budget.
int64_t grouped_chunk(int64_t budget, int64_t N) {
  return std::max<int64_t>(1, budget / std::max<int64_t>(N - 1, 1));
}

// Whether decode attention reads a group's prompt K / V in place
// (sm_attn_decode_prefix) instead of per-rollout copies: 16-bit caches with
// f16-pair attention output (the quantized models), at most 32 query heads per
// (group, KV head).
bool prefix_attention(const sm_model* m, int64_t S) {
  const auto& c = m->cfg;
  const int64_t G = m->prompt_group;
  return G > 1 && S % G == 0 && c.quantized && G * (c.heads / c.kv_heads) <= 32;
}

// All decoder layers over S sequences x L tokens (ids [S*L]) at positions
// pos0[s] + i. K/V go to caches (per-layer stride `layer_elems`, 0 = one
// buffer reused by every layer). decode: L == 1 and attention uses `lens`.
// pre: before each layer, its prompt K / V go into cache positions 0..P-1 of
// every sequence (the continuation of a group's prompt, pos0 = P).
int run_layers(sm_model* m, const int32_t* ids, int64_t S, int64_t L, const int32_t* pos0,
               const int32_t* lens, void* kc, void* vc, size_t layer_elems, int64_t cap,
               bool decode, hipStream_t st, const PrefixKV* pre = nullptr) {
  const auto& c = m->cfg;
  const int64_t rows = S * L;
  const int64_t d = c.d_model;
  SM_TRY(ensure(m->x, (size_t)rows * d * 4));
  SM_TRY(ensure(m->h, (size_t)rows * std::max<int64_t>(d, m->qdim) * m->act_size));
  if (!c.quantized) SM_TRY(ensure(m->qkv, (size_t)rows * m->qkv_n * 4));
  SM_TRY(ensure(m->qb, (size_t)rows * m->qdim * m->kv_size));
  SM_TRY(ensure(m->attn, (size_t)rows * m->qdim * m->act_size));
  SM_TRY(ensure(m->u, (size_t)rows * c.ffn * m->act_size));
  float* x = (float*)m->x.p;
  SM_TRY(sm_embed(m->embed, m->embt, ids, rows, d, c.vocab, 1.0f, x, st));
  bool normed = false;  // m->h already holds this layer's attention-norm output
  for (int l = 0; l < c.layers; ++l) {
    const Layer& Ly = m->layers[l];
    char* kl = (char*)kc + (size_t)l * layer_elems * m->kv_size;
    char* vl = (char*)vc + (size_t)l * layer_elems * m->kv_size;
    if (pre && !decode) {
      const int rb = c.head_dim * (int)m->kv_size;
      const int64_t n = S * c.kv_heads * pre->P * (rb / 16);
      for (int kv = 0; kv < 2; ++kv)
        broadcast_prefix_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(
            (const char*)(kv ? pre->v : pre->k) + l * pre->layer_bytes, kv ? vl : kl, 1, S,
            pre->s0, 0, pre->G, c.kv_heads, pre->P, (int)cap, rb, 0, 0);
    }
    if (!normed) SM_TRY(sm_rmsnorm(x, Ly.attn_norm, rows, d, c.norm_eps, m->h.p, m->act, st));
    normed = false;
    if (c.quantized) {  // qkv projection with RoPE + cache append in its epilogue
      SM_TRY(sm_q4_qkv_rope(Ly.qkv.codes, Ly.qkv.scales, c.heads, c.kv_heads, c.head_dim, d,
                            m->h.p, m->act, S, L, m->act_ld(d), m->rope, pos0, cap, m->qb.p, kl,
                            vl, m->kvt, st));
    } else {
      SM_TRY(linear_f32out(m, Ly.qkv, m->h.p, rows, (float*)m->qkv.p, false, st));
      SM_TRY(sm_rope_append((const float*)m->qkv.p, m->rope, pos0, S, L, c.heads, c.kv_heads,
                            c.head_dim, cap, m->qb.p, m->kvt, kl, vl, m->kvt, st));
    }
    if (decode && pre)  // the group's prompt keys from the shared prefix, the rest per rollout
      SM_TRY(sm_attn_decode_prefix(
          m->qb.p, (const char*)pre->k + l * pre->layer_bytes,
          (const char*)pre->v + l * pre->layer_bytes, kl, vl, lens, m->attn.p, m->apart.p,
          (int64_t)m->apart.n, m->kvt, m->act, S, pre->G, pre->P, c.heads, c.kv_heads, cap,
          c.head_dim, st));
    else if (decode)
      SM_TRY(sm_attn_decode(m->qb.p, kl, vl, lens, m->attn.p, m->kvt, m->act, S, c.heads,
                            c.kv_heads, cap, c.head_dim, st));
    else
      SM_TRY(sm_attn_prefill(m->qb.p, kl, vl, pos0, m->attn.p, m->kvt, m->act, S, L, c.heads,
                             c.kv_heads, cap, c.head_dim, st));
    // MoE layers: the FFN norm also computes the router logits
    const bool fused_router = c.experts > 0 && c.quantized && m->act == SM_F16X2;
    SM_TRY(linear_add_norm(m, Ly.o, m->attn.p, rows, x, Ly.ffn_norm, st,
                           fused_router ? Ly.router : nullptr));
    if (c.experts > 0) {  // the combine with the next layer's attention norm
      if (l + 1 < c.layers) {
        SM_TRY(moe_ffn(m, Ly, rows, st, m->layers[l + 1].attn_norm, fused_router));
        normed = true;
      } else {
        SM_TRY(moe_ffn(m, Ly, rows, st, nullptr, fused_router));
      }
    } else {
      SM_TRY(linear_swiglu(m, Ly.in, m->h.p, rows, m->u.p, st));
      if (l + 1 < c.layers) {  // the down projection with the next layer's attention norm
        SM_TRY(linear_add_norm(m, Ly.down, m->u.p, rows, x, m->layers[l + 1].attn_norm, st));
        normed = true;
      } else {
        SM_TRY(linear_f32out(m, Ly.down, m->u.p, rows, x, true, st));
      }
    }
  }
  return SM_OK;
}

// logits [M, V] f32 = LM_head(RMSNorm_final(xrows))
int head(sm_model* m, const float* xrows, int64_t M, float* logits, hipStream_t st) {
  SM_TRY(ensure(m->h, (size_t)M * std::max<int64_t>(m->cfg.d_model, m->qdim) * m->act_size));
  SM_TRY(sm_rmsnorm(xrows, m->final_norm, M, m->cfg.d_model, m->cfg.norm_eps, m->h.p, m->act, st));
  return linear_f32out(m, m->lm_head, m->h.p, M, logits, false, st);
}

// Whether the buffers holding the prompt state are those it was recorded in.
bool pstate_bufs_same(const sm_model* m) {
  return m->pstate_gens[0] == m->pkc.gen && m->pstate_gens[1] == m->pvc.gen &&
         m->pstate_gens[2] == m->prow.gen && m->pstate_gens[3] == m->pids.gen;
}

// Whether the model's prompt state was computed for groups of G x P with the
// current weights and buffers (its prompts still to be compared).
bool pstate_matches(const sm_model* m, int64_t groups, int64_t P) {
  return m->pstate_valid && m->pstate_weights == m->weights_version && pstate_bufs_same(m) &&
         m->pstate_groups == groups && m->pstate_G == m->prompt_group && m->pstate_P == P;
}

// Prompt groups: S must be whole groups of G and every prompt row equal to
// its group's first (checked on the device; one host synchronisation). With
// cached_out, also whether the prompts are those of the model's prompt state.
int check_prompt_groups(sm_model* m, const int32_t* prompts, int64_t S, int64_t P,
                        hipStream_t st, bool* cached_out = nullptr) {
  const int64_t G = m->prompt_group;
  SM_REQUIRE(S % G == 0, "prompt groups of %lld: %lld rollouts are not whole groups",
             (long long)G, (long long)S);
  const bool cmp = cached_out && pstate_matches(m, S / G, P);
  SM_TRY(ensure(m->flags, 8));
  int32_t* f = (int32_t*)m->flags.p;
  zero_i32_kernel<<<1, 64, 0, st>>>(f, 2);
  check_groups_kernel<<<blocks_for(S * P), 256, 0, st>>>(
      prompts, S, (int)G, (int)P, cmp ? (const int32_t*)m->pids.p : nullptr, f);
  int32_t bad[2] = {0, 0};
  SM_HIP(hipMemcpyAsync(bad, f, 8, hipMemcpyDeviceToHost, st));
  SM_HIP(hipStreamSynchronize(st));
  SM_REQUIRE(bad[0] == 0, "prompt groups of %lld: a rollout's prompt differs from its group's first",
             (long long)G);
  if (cached_out) *cached_out = cmp && bad[1] == 0;
  return SM_OK;
}

// Record the grouped prompt pass just computed (group prompt ids in ids
// [groups, P], K / V in pkc / pvc, last rows in prow) as the prompt state.
int record_pstate(sm_model* m, const int32_t* ids, int64_t groups, int64_t P, hipStream_t st) {
  m->pstate_valid = false;
  SM_TRY(ensure(m->pids, (size_t)groups * P * 4));
  SM_HIP(hipMemcpyAsync(m->pids.p, ids, (size_t)groups * P * 4, hipMemcpyDeviceToDevice, st));
  m->pstate_valid = true;
  m->pstate_weights = m->weights_version;
  m->pstate_gens[0] = m->pkc.gen;
  m->pstate_gens[1] = m->pvc.gen;
  m->pstate_gens[2] = m->prow.gen;
  m->pstate_gens[3] = m->pids.gen;
  m->pstate_groups = groups;
  m->pstate_G = m->prompt_group;
  m->pstate_P = P;
  return SM_OK;
}

// The prompt prefill of a generation: cache positions 0..P-1 of every
// rollout and its last prompt hidden row in m->rows [S, d]. With prompt
// groups each group's prompt runs once and is copied to its rollouts (the
// same values: a prompt position depends on the prompt alone).
int prefill_prompts(sm_model* m, const int32_t* prompts, int64_t S, int64_t P, int64_t cap,
                    size_t layer_elems, hipStream_t st) {
  const auto& c = m->cfg;
  int32_t* pos = (int32_t*)m->pos.p;
  int32_t* lens = (int32_t*)m->lens.p;
  const int64_t G = m->prompt_group;
  if (G <= 1) {
    set_positions_kernel<<<blocks_for(S), 256, 0, st>>>(pos, lens, (int)S, 0);
    SM_TRY(run_layers(m, prompts, S, P, pos, nullptr, m->kc.p, m->vc.p, layer_elems, cap, false,
                      st));
    gather_rows_kernel<<<blocks_for(S * c.d_model), 256, 0, st>>>(
        (const float*)m->x.p, (int)S, (int)P, (int)P - 1, c.d_model, (float*)m->rows.p);
    return SM_OK;
  }
  SM_TRY(check_prompt_groups(m, prompts, S, P, st));
  const int64_t groups = S / G;
  const size_t pl = (size_t)groups * c.kv_heads * P * c.head_dim;  // elements per layer
  SM_TRY(ensure(m->pkc, pl * c.layers * m->kv_size));
  SM_TRY(ensure(m->pvc, pl * c.layers * m->kv_size));
  SM_TRY(ensure(m->prow, (size_t)groups * c.d_model * 4));
  SM_TRY(ensure(m->ids, (size_t)groups * P * 4));
  int32_t* ids = (int32_t*)m->ids.p;
  group_prompts_kernel<<<blocks_for(groups * P), 256, 0, st>>>(prompts, groups, (int)G, (int)P,
                                                                ids);
  set_positions_kernel<<<blocks_for(groups), 256, 0, st>>>(pos, lens, (int)groups, 0);
  // this pass overwrites the prompt state's K / V and rows: it holds again
  // only if the pass is recorded below
  m->pstate_valid = false;
  SM_TRY(run_layers(m, ids, groups, P, pos, nullptr, m->pkc.p, m->pvc.p, pl, P, false, st));
  const int rb = c.head_dim * (int)m->kv_size;
  const int64_t n = (int64_t)c.layers * S * c.kv_heads * P * (rb / 16);
  // the shared-prompt decode attention reads the group's prompt K / V in place
  for (int kv = 0; kv < (prefix_attention(m, S) ? 0 : 2); ++kv)
    broadcast_prefix_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(
        (const char*)(kv ? m->pvc.p : m->pkc.p), (char*)(kv ? m->vc.p : m->kc.p), c.layers, S, 0,
        0, (int)G, c.kv_heads, (int)P, (int)cap, rb, (int64_t)(pl * m->kv_size),
        (int64_t)(layer_elems * m->kv_size));
  gather_group_rows_kernel<<<blocks_for(S * c.d_model), 256, 0, st>>>(
      (const float*)m->x.p, S, (int)G, (int)P, (int)P - 1, c.d_model, (float*)m->rows.p);
  // the same prompt pass as a recompute's (one chunk of all groups): kept for it
  gather_rows_kernel<<<blocks_for(groups * c.d_model), 256, 0, st>>>(
      (const float*)m->x.p, (int)groups, (int)P, (int)P - 1, c.d_model, (float*)m->prow.p);
  if (!m->trace_idx) SM_TRY(record_pstate(m, ids, groups, P, st));
  return SM_OK;
}

// After prefill_prompts: the group prompts' K / V that the decode steps'
// attention reads in place (out.k == nullptr when it reads per-rollout caches).
int decode_prefix(sm_model* m, int64_t S, int64_t P, PrefixKV& out) {
  out = PrefixKV{};
  if (!prefix_attention(m, S)) return SM_OK;
  const auto& c = m->cfg;
  const int64_t G = m->prompt_group;
  SM_TRY(ensure(m->apart, (size_t)sm_attn_decode_prefix_workspace_bytes(
                              S, G, P, c.heads, c.kv_heads, c.head_dim)));
  const int64_t layer_bytes = (S / G) * c.kv_heads * P * c.head_dim * (int64_t)m->kv_size;
  out = PrefixKV{m->pkc.p, m->pvc.p, layer_bytes, (int)G, (int)P, 0};
  return SM_OK;
}

}  // namespace
}  // namespace sm

using namespace sm;

extern "C" int sm_model_create(const sm_model_config* cfg, sm_model** out) {
  SM_REQUIRE(cfg && out, "sm_model_create: null argument");
  const sm_model_config& c = *cfg;
  SM_REQUIRE(c.layers > 0 && c.d_model > 0 && c.heads > 0 && c.kv_heads > 0 &&
                 c.heads % c.kv_heads == 0 && c.head_dim > 0 && c.head_dim % 2 == 0 &&
                 c.ffn > 0 && c.vocab > 0 && c.max_seq > 0,
             "sm_model_create: invalid model config");
  SM_REQUIRE(c.head_dim == 64 || c.head_dim == 128, "sm_model_create: head_dim must be 64 or 128");
  if (c.quantized)
    SM_REQUIRE(c.d_model % 128 == 0 && c.ffn % 128 == 0 && (c.heads * c.head_dim) % 128 == 0,
               "sm_model_create: quantized models need d_model, ffn and heads*head_dim %% 128 == 0");
  SM_REQUIRE(c.experts >= 0 && c.experts <= 64, "sm_model_create: experts must be in 0..=64");
  if (c.experts > 0) {
    SM_REQUIRE(c.quantized, "sm_model_create: MoE layers are built for quantized models");
    SM_REQUIRE(c.experts >= 2 && c.expert_ffn > 0 && c.expert_ffn % 128 == 0,
               "sm_model_create: MoE needs >= 2 experts and expert_ffn %% 128 == 0");
  }
  sm_model* m = new sm_model();
  m->cfg = c;
  m->act = c.quantized ? SM_F16X2 : SM_F32;
  m->kvt = c.quantized ? SM_F16 : SM_F32;
  m->embt = c.quantized ? SM_BF16 : SM_F32;
  m->act_size = 4;
  m->kv_size = c.quantized ? 2 : 4;
  m->emb_size = c.quantized ? 2 : 4;
  m->qdim = (int64_t)c.heads * c.head_dim;
  m->kvdim = (int64_t)c.kv_heads * c.head_dim;
  m->qkv_n = m->qdim + 2 * m->kvdim;
  auto fail = [&](int s) { sm_model_destroy(m); return s; };
  int s;
  if ((s = dalloc(m, &m->embed, (size_t)c.vocab * c.d_model * m->emb_size, true))) return fail(s);
  if ((s = dalloc(m, (void**)&m->final_norm, (size_t)c.d_model * 4, true))) return fail(s);
  if ((s = alloc_linear(m, m->lm_head, c.vocab, c.d_model))) return fail(s);
  m->layers.resize(c.layers);
  for (auto& Ly : m->layers) {
    if ((s = dalloc(m, (void**)&Ly.attn_norm, (size_t)c.d_model * 4, true))) return fail(s);
    if ((s = dalloc(m, (void**)&Ly.ffn_norm, (size_t)c.d_model * 4, true))) return fail(s);
    if ((s = alloc_linear(m, Ly.qkv, m->qkv_n, c.d_model))) return fail(s);
    if ((s = alloc_linear(m, Ly.o, c.d_model, m->qdim))) return fail(s);
    if (c.experts > 0) {
      if ((s = dalloc(m, (void**)&Ly.router, (size_t)c.experts * c.d_model * 4, true))) return fail(s);
      if ((s = alloc_linear(m, Ly.exp_in, 2 * (int64_t)c.expert_ffn, c.d_model, c.experts)))
        return fail(s);
      if ((s = alloc_linear(m, Ly.exp_down, c.d_model, c.expert_ffn, c.experts))) return fail(s);
    } else {
      if ((s = alloc_linear(m, Ly.in, 2 * (int64_t)c.ffn, c.d_model))) return fail(s);
      if ((s = alloc_linear(m, Ly.down, c.d_model, c.ffn))) return fail(s);
    }
  }
  // RoPE table: adjacent pairs, theta^(-2p/hd), angle = pos * freq, computed in
  // double and rounded to f32 (cos, sin) per (pos, pair).
  const int half = c.head_dim / 2;
  std::vector<float> tab((size_t)c.max_seq * half * 2);
  for (int pos = 0; pos < c.max_seq; ++pos)
    for (int p = 0; p < half; ++p) {
      const double freq = std::pow((double)c.rope_theta, -2.0 * p / (double)c.head_dim);
      const double ang = (double)pos * freq;
      tab[((size_t)pos * half + p) * 2] = (float)std::cos(ang);
      tab[((size_t)pos * half + p) * 2 + 1] = (float)std::sin(ang);
    }
  if ((s = dalloc(m, (void**)&m->rope, tab.size() * 4, false))) return fail(s);
  if (hipMemcpy(m->rope, tab.data(), tab.size() * 4, hipMemcpyHostToDevice) != hipSuccess) {
    set_error("sm_model_create: rope upload failed");
    return fail(SM_ERR_HIP);
  }
  *out = m;
  return SM_OK;
}

namespace sm {
namespace {

// Every workspace buffer of a model, in the order a bound workspace lays
// them out.
std::vector<DevBuf*> model_bufs(sm_model* m) {
  return {&m->x, &m->h, &m->qkv, &m->qb, &m->attn, &m->u, &m->gv, &m->logits, &m->rows,
          &m->ids, &m->pos, &m->lens, &m->next_ids, &m->kc, &m->vc, &m->rkc, &m->rvc,
          &m->lp_tmp, &m->flags, &m->moe_idx, &m->moe_w, &m->moe_plan, &m->moe_u, &m->moe_y,
          &m->moe_err, &m->moe_lg, &m->mmws, &m->seen, &m->done, &m->pkc, &m->pvc, &m->prow,
          &m->apart,
          &m->pids};
}

void release_bufs(sm_model* m) {
  m->pstate_valid = false;
  for (DevBuf* b : model_bufs(m)) {
    if (b->p && !b->fixed) hipFree(b->p);
    const uint64_t gen = b->gen + 1;
    *b = DevBuf{};
    b->gen = gen;
  }
  m->ws_base = nullptr;
  m->ws_bytes = 0;
}

// Largest size each buffer reaches in sm_rl_generate(_ex) of S rollouts with
// P prompt and N new tokens, and in sm_rl_logprobs / sm_rl_prepare of the
// same shapes, for any smaller shape too (each entry is monotone in S, P, N
// and max_tokens_per_forward); the same expressions the calls pass to ensure().
struct WsPlan {
  std::vector<size_t> bytes;  // parallel to model_bufs()
};

void plan_max(size_t& slot, size_t v) { slot = std::max(slot, v); }

WsPlan plan_workspace(sm_model* m, int64_t S, int64_t P, int64_t N, int64_t mtpf) {
  const auto& c = m->cfg;
  auto bufs = model_bufs(m);
  WsPlan plan;
  plan.bytes.assign(bufs.size(), 0);
  auto at = [&](DevBuf& b) -> size_t& {
    for (size_t i = 0; i < bufs.size(); ++i)
      if (bufs[i] == &b) return plan.bytes[i];
    return plan.bytes[0];  // unreachable: every buffer is listed
  };
  const int64_t d = c.d_model;
  auto mm = [&](int64_t M, int64_t Nn, int64_t K, int epi) {
    if (!c.quantized) return;
    const int64_t want = std::min(kMatmulWs, sm_q4_matmul_workspace_bytes(M, Nn, K, epi));
    if (want > 0) plan_max(at(m->mmws), (size_t)want);
  };
  auto layers = [&](int64_t rows) {  // run_layers over `rows` tokens
    plan_max(at(m->x), (size_t)rows * d * 4);
    plan_max(at(m->h), (size_t)rows * std::max<int64_t>(d, m->qdim) * m->act_size);
    if (!c.quantized) plan_max(at(m->qkv), (size_t)rows * m->qkv_n * 4);
    plan_max(at(m->qb), (size_t)rows * m->qdim * m->kv_size);
    plan_max(at(m->attn), (size_t)rows * m->qdim * m->act_size);
    plan_max(at(m->u), (size_t)rows * c.ffn * m->act_size);
    if (!c.quantized) plan_max(at(m->gv), (size_t)rows * 2 * c.ffn * 4);
    mm(rows, d, m->qdim, SM_EPI_ADD_F32);
    if (c.experts > 0) {
      const int64_t routes = rows * 2;
      plan_max(at(m->moe_idx), (size_t)routes * 4);
      plan_max(at(m->moe_w), (size_t)routes * 4);
      plan_max(at(m->moe_plan), (size_t)sm_moe_plan_words(rows, 2, c.experts) * 4);
      plan_max(at(m->moe_u), (size_t)routes * c.expert_ffn * m->act_size);
      plan_max(at(m->moe_y), (size_t)routes * d * 4);
      plan_max(at(m->moe_err), 4);
      plan_max(at(m->moe_lg), (size_t)rows * c.experts * 4);
    } else {
      mm(rows, 2 * (int64_t)c.ffn, d, SM_EPI_SWIGLU_F16X2);
      mm(rows, d, c.ffn, SM_EPI_ADD_F32);
    }
  };
  auto head = [&](int64_t M) {
    plan_max(at(m->h), (size_t)M * std::max<int64_t>(d, m->qdim) * m->act_size);
    mm(M, c.vocab, d, SM_EPI_STORE_F32);
  };
  // generation: prefill S*P rows (groups*P with prompt groups), decode steps
  // S rows, head S rows
  const int64_t cap = P + N - 1;
  const int64_t G = m->prompt_group;
  const bool grouped = G > 1 && S % G == 0;
  const int64_t groups = grouped ? S / G : S;
  layers(groups * P);
  layers(S);
  head(S);
  const size_t cache = (size_t)S * c.kv_heads * cap * c.head_dim * c.layers * m->kv_size;
  plan_max(at(m->kc), cache);
  plan_max(at(m->vc), cache);
  plan_max(at(m->pos), (size_t)S * 4);
  plan_max(at(m->lens), (size_t)S * 4);
  plan_max(at(m->next_ids), (size_t)S * 4);
  plan_max(at(m->rows), (size_t)S * d * 4);
  plan_max(at(m->logits), (size_t)S * c.vocab * 4);
  plan_max(at(m->seen), (size_t)S * ceil_div(c.vocab, 32) * 4);
  plan_max(at(m->done), (size_t)(S + 1) * 4);
  // recompute: chunks of at most max(budget, L) token rows (one sequence when
  // a sequence is longer than the budget)
  const int64_t L = P + N - 1;
  const int64_t budget = mtpf > 0 ? mtpf : 65536;
  const int64_t rows = std::min<int64_t>(S * L, std::max<int64_t>(budget, L));
  layers(rows);
  plan_max(at(m->rkc), (size_t)rows * c.kv_heads * c.head_dim * m->kv_size);
  plan_max(at(m->rvc), (size_t)rows * c.kv_heads * c.head_dim * m->kv_size);
  plan_max(at(m->ids), (size_t)rows * 4);
  plan_max(at(m->pos), (size_t)S * 4);
  plan_max(at(m->lens), (size_t)S * 4);
  plan_max(at(m->rows), (size_t)rows * d * 4);
  const int64_t rchunk = std::max<int64_t>(1, ((int64_t)1 << 29) / c.vocab);
  head(std::min(rows, rchunk));
  plan_max(at(m->logits), (size_t)std::min(rows, rchunk) * c.vocab * 4);
  if (grouped) {
    // every group's prompt K / V for all layers, its last hidden rows; the
    // recompute's prompt chunks of whole prompts
    const size_t prefix = (size_t)groups * c.kv_heads * P * c.head_dim * c.layers * m->kv_size;
    plan_max(at(m->pkc), prefix);
    plan_max(at(m->pvc), prefix);
    plan_max(at(m->prow), (size_t)groups * d * 4);
    plan_max(at(m->pids), (size_t)groups * P * 4);
    // continuation chunks: cc rollouts x (N - 1) rows (within the budget, so
    // covered by layers(rows) above) over a K / V buffer of cc x L positions
    const int64_t cc = std::min(S, grouped_chunk(budget, N));
    plan_max(at(m->rkc), (size_t)cc * c.kv_heads * L * c.head_dim * m->kv_size);
    plan_max(at(m->rvc), (size_t)cc * c.kv_heads * L * c.head_dim * m->kv_size);
    plan_max(at(m->ids), (size_t)cc * (N - 1) * 4);
    plan_max(at(m->rows), (size_t)cc * N * d * 4);
    plan_max(at(m->pos), (size_t)cc * 4);
    plan_max(at(m->lens), (size_t)cc * 4);
    // a continuation chunk scores cc * N rows (its N - 1 new rows plus the
    // group's last prompt row per rollout), which can exceed the budget
    head(std::min(cc * N, rchunk));
    plan_max(at(m->logits), (size_t)std::min(cc * N, rchunk) * c.vocab * 4);
    if (prefix_attention(m, S))
      plan_max(at(m->apart), (size_t)sm_attn_decode_prefix_workspace_bytes(
                                 S, G, P, c.heads, c.kv_heads, c.head_dim));
    const int64_t gchunk = std::max<int64_t>(1, budget / P);
    const int64_t prow_rows = std::min(groups, gchunk) * P;
    layers(prow_rows);
    plan_max(at(m->ids), (size_t)std::max(groups * P, prow_rows) * 4);
    plan_max(at(m->pos), (size_t)groups * 4);
    plan_max(at(m->lens), (size_t)groups * 4);
    plan_max(at(m->flags), 8);
  }
  return plan;
}

constexpr size_t kWsAlign = 256;
size_t align_up(size_t v) { return (v + kWsAlign - 1) / kWsAlign * kWsAlign; }

size_t plan_total(const WsPlan& p) {
  size_t t = 0;
  for (size_t b : p.bytes) t += align_up(b);
  return t;
}

}  // namespace
}  // namespace sm

extern "C" int sm_model_destroy(sm_model* m) {
  if (!m) return SM_OK;
  hipDeviceSynchronize();
  for (void* p : m->owned) hipFree(p);
  release_bufs(m);
  delete m;
  return SM_OK;
}

extern "C" int64_t sm_rl_workspace_bytes(sm_model* m, int64_t S, int64_t P, int64_t N,
                                         int64_t max_tokens_per_forward) {
  if (!m || S <= 0 || P <= 0 || N <= 0 || max_tokens_per_forward < 0) return -1;
  return (int64_t)plan_total(plan_workspace(m, S, P, N, max_tokens_per_forward));
}

extern "C" int sm_model_bind_workspace(sm_model* m, void* ws, int64_t bytes, int64_t S,
                                       int64_t P, int64_t N, int64_t max_tokens_per_forward) {
  SM_REQUIRE(m, "sm_model_bind_workspace: null model");
  SM_HIP(hipDeviceSynchronize());  // no call may still use the old buffers
  release_bufs(m);
  if (!ws) return SM_OK;  // back to the model's own grow-only buffers
  SM_REQUIRE(S > 0 && P > 0 && N > 0 && max_tokens_per_forward >= 0,
             "sm_model_bind_workspace: bad shape");
  SM_REQUIRE(reinterpret_cast<uintptr_t>(ws) % kWsAlign == 0,
             "sm_model_bind_workspace: the workspace must be 256-byte aligned");
  const WsPlan plan = plan_workspace(m, S, P, N, max_tokens_per_forward);
  const size_t need = plan_total(plan);
  SM_REQUIRE(bytes >= 0 && (size_t)bytes >= need,
             "sm_model_bind_workspace: %lld bytes given, %zu needed (sm_rl_workspace_bytes)",
             (long long)bytes, need);
  auto bufs = model_bufs(m);
  size_t off = 0;
  for (size_t i = 0; i < bufs.size(); ++i) {
    bufs[i]->fixed = true;
    ++bufs[i]->gen;
    bufs[i]->n = plan.bytes[i];
    bufs[i]->p = plan.bytes[i] ? static_cast<char*>(ws) + off : nullptr;
    off += align_up(plan.bytes[i]);
  }
  m->ws_base = ws;
  m->ws_bytes = bytes;
  return SM_OK;
}

extern "C" int64_t sm_model_weight_bytes(const sm_model* m) { return m ? (int64_t)m->weight_bytes : 0; }

extern "C" int sm_model_set_prompt_groups(sm_model* m, int64_t group_size) {
  SM_REQUIRE(m, "sm_model_set_prompt_groups: null model");
  SM_REQUIRE(group_size >= 1 && group_size <= (1 << 20),
             "sm_model_set_prompt_groups: group size must be in 1..2^20");
  m->prompt_group = group_size;
  return SM_OK;
}

extern "C" int sm_model_trace_routes(sm_model* m, int32_t* idx, float* logits, int64_t capacity) {
  SM_REQUIRE(m, "sm_model_trace_routes: null model");
  SM_REQUIRE(m->cfg.experts > 0 || !idx, "sm_model_trace_routes: the model has no MoE layers");
  SM_REQUIRE(!idx || capacity >= 0, "sm_model_trace_routes: negative capacity");
  SM_REQUIRE(idx || !logits, "sm_model_trace_routes: logits need an index buffer");
  m->trace_idx = idx;
  m->trace_logits = idx ? logits : nullptr;
  m->trace_cap = idx ? capacity : 0;
  m->trace_used = 0;
  m->trace_dropped = 0;
  return SM_OK;
}

extern "C" int sm_model_route_trace_count(const sm_model* m, int64_t* recorded, int64_t* dropped) {
  SM_REQUIRE(m && recorded && dropped, "sm_model_route_trace_count: null argument");
  *recorded = m->trace_used;
  *dropped = m->trace_dropped;
  return SM_OK;
}

static int tensor_target(sm_model* m, int kind, int layer, Linear** lin, void** dense,
                         int64_t* n, int64_t* count) {
  const auto& c = m->cfg;
  *lin = nullptr;
  *dense = nullptr;
  *count = 1;
  const bool moe_kind = kind == SM_W_ROUTER || kind == SM_W_EXPERT_IN || kind == SM_W_EXPERT_DOWN;
  const bool per_layer = kind == SM_W_ATTN_NORM || kind == SM_W_FFN_NORM || kind == SM_W_QKV ||
                         kind == SM_W_O || kind == SM_W_IN || kind == SM_W_DOWN || moe_kind;
  if (moe_kind) SM_REQUIRE(c.experts > 0, "tensor kind %d needs an MoE model", kind);
  if (kind == SM_W_IN || kind == SM_W_DOWN)
    SM_REQUIRE(c.experts == 0, "MoE models have no dense FFN (tensor kind %d)", kind);
  if (per_layer) SM_REQUIRE(layer >= 0 && layer < c.layers, "layer %d out of range", layer);
  switch (kind) {
    case SM_W_EMBED: *dense = m->embed; *n = (int64_t)c.vocab * c.d_model; break;
    case SM_W_FINAL_NORM: *dense = m->final_norm; *n = c.d_model; break;
    case SM_W_LM_HEAD: *lin = &m->lm_head; break;
    case SM_W_ATTN_NORM: *dense = m->layers[layer].attn_norm; *n = c.d_model; break;
    case SM_W_FFN_NORM: *dense = m->layers[layer].ffn_norm; *n = c.d_model; break;
    case SM_W_QKV: *lin = &m->layers[layer].qkv; break;
    case SM_W_O: *lin = &m->layers[layer].o; break;
    case SM_W_IN: *lin = &m->layers[layer].in; break;
    case SM_W_DOWN: *lin = &m->layers[layer].down; break;
    case SM_W_ROUTER: *dense = m->layers[layer].router; *n = (int64_t)c.experts * c.d_model; break;
    case SM_W_EXPERT_IN: *lin = &m->layers[layer].exp_in; *count = c.experts; break;
    case SM_W_EXPERT_DOWN: *lin = &m->layers[layer].exp_down; *count = c.experts; break;
    default: set_error("unknown tensor kind %d", kind); return SM_ERR_INVALID;
  }
  if (*lin) *n = (*lin)->N * (*lin)->K;
  return SM_OK;
}

namespace sm {
namespace {
__global__ void f32_to_bf16_kernel(const float* __restrict__ a, int64_t n, uint16_t* __restrict__ b) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) b[i] = f32_to_bf16(a[i]);
}
}  // namespace
}  // namespace sm

extern "C" int sm_model_set_tensor(sm_model* m, int kind, int layer, const float* src,
                                   void* stream) {
  SM_REQUIRE(m && src, "sm_model_set_tensor: null argument");
  ++m->weights_version;  // a cached prompt pass is stale from here
  Linear* lin;
  void* dense;
  int64_t n, count;
  SM_TRY(tensor_target(m, kind, layer, &lin, &dense, &n, &count));
  hipStream_t st = as_stream(stream);
  if (lin) {
    if (m->cfg.quantized) {
      // quantize to the row-major codec in a temporary, then prepare (tile);
      // stacked experts: one [N, K] weight after the other
      const int64_t groups = ceil_div(n, 128);
      DevBuf tmp;
      SM_TRY(ensure(tmp, (size_t)groups * 64 + (size_t)groups * 2 + 16));
      uint8_t* codes = (uint8_t*)tmp.p;
      uint16_t* scales = (uint16_t*)(codes + groups * 64);
      int32_t* bad = (int32_t*)(codes + groups * 64 + groups * 2 + (groups * 2) % 4);
      SM_HIP(hipMemsetAsync(bad, 0, 4, st));
      const size_t cstride = (size_t)q4t_rows(lin->N) * (lin->K / 2);
      const size_t sstride = (size_t)q4t_rows(lin->N) * (lin->K / 128);
      int s = SM_OK;
      for (int64_t e = 0; e < count && s == SM_OK; ++e) {
        s = sm_q4_quantize(src + e * n, SM_F32, n, codes, scales, bad, stream);
        if (s == SM_OK)
          s = sm_q4_pack(codes, scales, lin->N, lin->K, lin->codes + e * cstride,
                         lin->scales + e * sstride, stream);
      }
      int32_t nbad = 0;
      if (s == SM_OK && hipMemcpyAsync(&nbad, bad, 4, hipMemcpyDeviceToHost, st) != hipSuccess)
        s = SM_ERR_HIP;
      hipStreamSynchronize(st);
      hipFree(tmp.p);
      if (s != SM_OK) return s;
      SM_REQUIRE(nbad == 0, "%d Q4 groups have a scale outside the f16 normal range", nbad);
      return SM_OK;
    }
    SM_REQUIRE(count == 1, "stacked expert weights need a quantized model");
    SM_HIP(hipMemcpyAsync(lin->w, src, (size_t)n * 4, hipMemcpyDeviceToDevice, st));
    return SM_OK;
  }
  if (kind == SM_W_EMBED && m->embt == SM_BF16) {
    f32_to_bf16_kernel<<<blocks_for(n), 256, 0, st>>>(src, n, (uint16_t*)dense);
    SM_LAUNCH_CHECK();
    return SM_OK;
  }
  SM_HIP(hipMemcpyAsync(dense, src, (size_t)n * 4, hipMemcpyDeviceToDevice, st));
  return SM_OK;
}

namespace sm {
int hquant_decode_device(const sm_hquant* t, float* out, int transpose, hipStream_t st);
}

extern "C" int sm_model_load_packed(sm_model* m, int kind, int layer, const sm_hquant* t,
                                    int layout, void* stream) {
  SM_REQUIRE(m && t && t->scales && t->codes, "sm_model_load_packed: null argument");
  ++m->weights_version;  // a cached prompt pass is stale from here
  SM_REQUIRE(layout == 0 || layout == 1,
             "sm_model_load_packed: layout must be 0 ([out, in]) or 1 ([in, out])");
  Linear* lin;
  void* dense;
  int64_t n, count;
  SM_TRY(tensor_target(m, kind, layer, &lin, &dense, &n, &count));
  SM_REQUIRE(t->group_size == 128, "packed tensor is not g128");
  SM_REQUIRE(t->elements == n * count,
             "packed tensor has %lld elements; model tensor kind %d needs %lld",
             (long long)t->elements, kind, (long long)(n * count));
  SM_REQUIRE(t->nscales == ceil_div(t->elements, 128), "packed tensor scale count mismatch");
  if (layout == 1)
    SM_REQUIRE(lin && count == 1 && t->rank == 2 && t->shape[0] == lin->K && t->shape[1] == lin->N,
               "an [in, out] packed tensor must be a rank-2 linear weight [%lld, %lld]",
               lin ? (long long)lin->K : 0ll, lin ? (long long)lin->N : 0ll);
  else if (lin)
    SM_REQUIRE(t->rank >= 2 && t->shape[t->rank - 1] == lin->K,
               "an [out, in] packed tensor must end in the input width %lld", (long long)lin->K);
  hipStream_t st = as_stream(stream);
  if (lin && m->cfg.quantized && t->format == SM_HQ_Q4G128 && layout == 0) {
    // the row-major Q4G128 codec is this model's interchange format: tile it
    // as is (K % 128 == 0, so no group straddles two rows)
    SM_REQUIRE(t->ncodes == t->nscales * 64, "packed tensor code size mismatch");
    const size_t cstride = (size_t)q4t_rows(lin->N) * (lin->K / 2);
    const size_t sstride = (size_t)q4t_rows(lin->N) * (lin->K / 128);
    for (int64_t e = 0; e < count; ++e)
      SM_TRY(sm_q4_pack(t->codes + e * (n / 2), t->scales + e * (n / 128), lin->N, lin->K,
                        lin->codes + e * cstride, lin->scales + e * sstride, stream));
    return SM_OK;
  }
  DevBuf tmp;
  SM_TRY(ensure(tmp, (size_t)(n * count) * 4));
  int s = hquant_decode_device(t, (float*)tmp.p, layout == 1, st);
  if (s == SM_OK) s = sm_model_set_tensor(m, kind, layer, (const float*)tmp.p, stream);
  hipStreamSynchronize(st);
  hipFree(tmp.p);
  return s;
}

extern "C" int sm_model_init_random(sm_model* m, uint64_t seed, float std, void* stream) {
  SM_REQUIRE(m, "sm_model_init_random: null model");
  ++m->weights_version;  // a cached prompt pass is stale from here
  hipStream_t st = as_stream(stream);
  const auto& c = m->cfg;
  int64_t maxn = (int64_t)c.vocab * c.d_model;
  for (const auto& Ly : m->layers) {
    for (const Linear* L : {&Ly.qkv, &Ly.o, &Ly.in, &Ly.down}) maxn = std::max(maxn, L->N * L->K);
    for (const Linear* L : {&Ly.exp_in, &Ly.exp_down})
      maxn = std::max(maxn, L->N * L->K * (int64_t)c.experts);
  }
  DevBuf tmp;
  SM_TRY(ensure(tmp, (size_t)maxn * 4));
  auto fill_ones = [&](float* p) {
    fill_f32_kernel<<<blocks_for(c.d_model), 256, 0, st>>>(p, c.d_model, 1.0f);
  };
  uint64_t tid = 0;
  auto randn = [&](int kind, int layer, float sd) -> int {
    Linear* lin;
    void* dense;
    int64_t n, count;
    SM_TRY(tensor_target(m, kind, layer, &lin, &dense, &n, &count));
    SM_TRY(sm_fill_normal(tmp.p, SM_F32, n * count, 0.f, sd, mix64(seed ^ (0x51ed27ull * ++tid)),
                          stream));
    return sm_model_set_tensor(m, kind, layer, (const float*)tmp.p, stream);
  };
  auto body = [&]() -> int {
    SM_TRY(randn(SM_W_EMBED, -1, std));
    fill_ones(m->final_norm);
    SM_TRY(randn(SM_W_LM_HEAD, -1, std));
    for (int l = 0; l < c.layers; ++l) {
      fill_ones(m->layers[l].attn_norm);
      fill_ones(m->layers[l].ffn_norm);
      for (int k : {SM_W_QKV, SM_W_O}) SM_TRY(randn(k, l, std));
      if (c.experts > 0) {
        SM_TRY(randn(SM_W_ROUTER, l, 1.0f / std::sqrt((float)c.d_model)));
        SM_TRY(randn(SM_W_EXPERT_IN, l, std));
        SM_TRY(randn(SM_W_EXPERT_DOWN, l, std));
      } else {
        SM_TRY(randn(SM_W_IN, l, std));
        SM_TRY(randn(SM_W_DOWN, l, std));
      }
    }
    return SM_OK;
  };
  const int s = body();
  hipStreamSynchronize(st);
  hipFree(tmp.p);
  return s;
}

// ---------------------------------------------------------------- generate ---

extern "C" int sm_rl_generate(sm_model* m, const int32_t* prompts, int64_t S, int64_t P,
                              int64_t N, float temperature, uint64_t seed, int32_t* tokens,
                              float* behavior_lp, void* stream) {
  SM_REQUIRE(m && prompts && tokens, "sm_rl_generate: null argument");
  SM_REQUIRE(S > 0 && P > 0, "cannot generate from an empty prompt");
  SM_REQUIRE(N > 0, "sm_rl_generate: max_new_tokens must be positive");
  SM_REQUIRE(!std::isnan(temperature), "temperature must not be NaN");
  const int64_t cap = P + N - 1;
  SM_REQUIRE(cap <= m->cfg.max_seq, "attention cache capacity %lld exceeds max_seq_len %d",
             (long long)cap, m->cfg.max_seq);
  hipStream_t st = as_stream(stream);
  const auto& c = m->cfg;
  const size_t layer_elems = cache_layer_elems(m, S, cap);
  SM_TRY(ensure(m->kc, layer_elems * c.layers * m->kv_size));
  SM_TRY(ensure(m->vc, layer_elems * c.layers * m->kv_size));
  SM_TRY(ensure(m->pos, (size_t)S * 4));
  SM_TRY(ensure(m->lens, (size_t)S * 4));
  SM_TRY(ensure(m->next_ids, (size_t)S * 4));
  SM_TRY(ensure(m->rows, (size_t)S * c.d_model * 4));
  SM_TRY(ensure(m->logits, (size_t)S * c.vocab * 4));
  int32_t* pos = (int32_t*)m->pos.p;
  int32_t* lens = (int32_t*)m->lens.p;
  // prefill over the prompts at positions 0..P-1
  SM_TRY(prefill_prompts(m, prompts, S, P, cap, layer_elems, st));
  PrefixKV dpre{};
  SM_TRY(decode_prefix(m, S, P, dpre));
  SM_TRY(head(m, (const float*)m->rows.p, S, (float*)m->logits.p, st));
  SM_TRY(sm_sample((const float*)m->logits.p, S, c.vocab, c.vocab, temperature, seed, 0, tokens, N,
                   behavior_lp, N, (int32_t*)m->next_ids.p, st));
  // cached single-token steps
  for (int64_t t = 1; t < N; ++t) {
    set_positions_kernel<<<blocks_for(S), 256, 0, st>>>(pos, lens, (int)S, (int)(P + t - 1));
    SM_TRY(run_layers(m, (const int32_t*)m->next_ids.p, S, 1, pos, lens, m->kc.p, m->vc.p,
                      layer_elems, cap, true, st, dpre.k ? &dpre : nullptr));
    SM_TRY(head(m, (const float*)m->x.p, S, (float*)m->logits.p, st));
    SM_TRY(sm_sample((const float*)m->logits.p, S, c.vocab, c.vocab, temperature, seed, t,
                     tokens + t, N, behavior_lp ? behavior_lp + t : nullptr, N,
                     (int32_t*)m->next_ids.p, st));
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

namespace sm {
namespace {

// Rollouts that stopped: tokens[s, t0..N) = eos, behavior log-prob 0.
__global__ void pad_tail_kernel(int32_t* tokens, float* lp, int S, int N, int t0, int eos) {
  const int w = N - t0;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)S * w) return;
  const int64_t at = (i / w) * N + t0 + i % w;
  tokens[at] = eos;
  if (lp) lp[at] = 0.f;
}

constexpr int64_t kEosPoll = 16;  // decode steps between all-stopped checks

}  // namespace
}  // namespace sm

extern "C" int sm_rl_generate_ex(sm_model* m, const int32_t* prompts, int64_t S, int64_t P,
                                 int64_t N, const sm_sampling* sp, uint64_t seed, int32_t* tokens,
                                 float* behavior_lp, int32_t* lengths, void* stream) {
  SM_REQUIRE(m && prompts && tokens, "sm_rl_generate_ex: null argument");
  SM_REQUIRE(S > 0 && P > 0, "cannot generate from an empty prompt");
  SM_REQUIRE(N > 0, "sm_rl_generate_ex: max_new_tokens must be positive");
  const auto& c = m->cfg;
  SM_TRY(validate_sampling(sp, c.vocab));
  const int64_t cap = P + N - 1;
  SM_REQUIRE(cap <= c.max_seq, "attention cache capacity %lld exceeds max_seq_len %d",
             (long long)cap, c.max_seq);
  hipStream_t st = as_stream(stream);
  const size_t layer_elems = cache_layer_elems(m, S, cap);
  SM_TRY(ensure(m->kc, layer_elems * c.layers * m->kv_size));
  SM_TRY(ensure(m->vc, layer_elems * c.layers * m->kv_size));
  SM_TRY(ensure(m->pos, (size_t)S * 4));
  SM_TRY(ensure(m->lens, (size_t)S * 4));
  SM_TRY(ensure(m->next_ids, (size_t)S * 4));
  SM_TRY(ensure(m->rows, (size_t)S * c.d_model * 4));
  SM_TRY(ensure(m->logits, (size_t)S * c.vocab * 4));
  const bool pen = sp->repetition_penalty != 1.f;
  const bool eos = sp->eos_token >= 0;
  const int64_t seen_ld = ceil_div(c.vocab, 32);
  uint32_t* seen = nullptr;
  int32_t* done = nullptr;
  if (pen) {
    SM_TRY(ensure(m->seen, (size_t)S * seen_ld * 4));
    seen = (uint32_t*)m->seen.p;
    SM_TRY(seen_tokens(prompts, S, P, P, c.vocab, seen, seen_ld, true, st));
  }
  if (eos) {
    SM_TRY(ensure(m->done, (size_t)(S + 1) * 4));  // S flags, then the stopped count
    done = (int32_t*)m->done.p;
    SM_TRY(fill_i32(done, S + 1, 0, st));
  }
  if (lengths) SM_TRY(fill_i32(lengths, S, (int32_t)N, st));
  int32_t* next = (int32_t*)m->next_ids.p;
  int32_t* pos = (int32_t*)m->pos.p;
  int32_t* lens = (int32_t*)m->lens.p;
  SM_TRY(prefill_prompts(m, prompts, S, P, cap, layer_elems, st));
  PrefixKV dpre{};
  SM_TRY(decode_prefix(m, S, P, dpre));
  SM_TRY(head(m, (const float*)m->rows.p, S, (float*)m->logits.p, st));
  SM_TRY(sample_ex_launch((const float*)m->logits.p, S, c.vocab, c.vocab, sp, seed, 0, seen,
                          seen_ld, done, eos ? lengths : nullptr, eos ? done + S : nullptr, tokens,
                          N, behavior_lp, N, next, st));
  for (int64_t t = 1; t < N; ++t) {
    if (eos && t % kEosPoll == 0) {
      int32_t stopped = 0;
      SM_HIP(hipMemcpyAsync(&stopped, done + S, 4, hipMemcpyDeviceToHost, st));
      SM_HIP(hipStreamSynchronize(st));
      if (stopped >= S) {
        const int64_t n = S * (N - t);
        pad_tail_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(tokens, behavior_lp, (int)S,
                                                                    (int)N, (int)t, sp->eos_token);
        break;
      }
    }
    set_positions_kernel<<<blocks_for(S), 256, 0, st>>>(pos, lens, (int)S, (int)(P + t - 1));
    SM_TRY(run_layers(m, next, S, 1, pos, lens, m->kc.p, m->vc.p, layer_elems, cap, true, st,
                      dpre.k ? &dpre : nullptr));
    SM_TRY(head(m, (const float*)m->x.p, S, (float*)m->logits.p, st));
    SM_TRY(sample_ex_launch((const float*)m->logits.p, S, c.vocab, c.vocab, sp, seed, t, seen,
                            seen_ld, done, eos ? lengths : nullptr, eos ? done + S : nullptr,
                            tokens + t, N, behavior_lp ? behavior_lp + t : nullptr, N, next, st));
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

// ---------------------------------------------------------------- logprobs ---

namespace sm {
namespace {

// LM head + CE over scored rows [rows, d] (m->rows) in chunks bounding the
// [rows, V] logits to ~2 GiB: lp of tokens (row-major as the rows).
int score_rows(sm_model* m, int64_t rows, const int32_t* tokens, float* lp, hipStream_t st) {
  const auto& c = m->cfg;
  const int64_t rchunk = std::max<int64_t>(1, ((int64_t)1 << 29) / c.vocab);
  SM_TRY(ensure(m->logits, (size_t)std::min(rows, rchunk) * c.vocab * 4));
  for (int64_t r0 = 0; r0 < rows; r0 += rchunk) {
    const int64_t rn = std::min(rchunk, rows - r0);
    SM_TRY(head(m, (const float*)m->rows.p + r0 * c.d_model, rn, (float*)m->logits.p, st));
    SM_TRY(sm_ce_rows(m->logits.p, SM_F32, tokens + r0, rn, c.vocab, c.vocab, lp + r0, nullptr,
                      nullptr, 1.0f, nullptr, nullptr, st));
  }
  return SM_OK;
}

// The recompute with prompt groups: each group's prompt runs once (its K / V
// for every layer and its last hidden row kept), then every rollout's
// continuation tokens[:, :N-1] runs from position P over a cache whose
// positions 0..P-1 receive the group's prompt K / V before each layer. The
// scored row of token 0 is the group's last prompt row; those of tokens
// 1..N-1 come from the continuation. A prompt position depends on the prompt
// alone, so the values are those of the per-rollout forward.
int logprobs_grouped(sm_model* m, const int32_t* prompts, const int32_t* tokens, int64_t S,
                     int64_t P, int64_t N, int64_t budget, int64_t chunk, float* lp_out,
                     hipStream_t st) {
  const auto& c = m->cfg;
  const int64_t G = m->prompt_group, L = P + N - 1;
  bool cached = false;
  SM_TRY(check_prompt_groups(m, prompts, S, P, st, &cached));
  const int64_t groups = S / G;
  // continuations in chunks of whole rollouts whose N - 1 new rows fit the
  // token budget (the prompt rows come from the group's prompt K / V)
  chunk = grouped_chunk(budget, N);
  const size_t pl = (size_t)groups * c.kv_heads * P * c.head_dim;  // elements per layer
  SM_TRY(ensure(m->pkc, pl * c.layers * m->kv_size));
  SM_TRY(ensure(m->pvc, pl * c.layers * m->kv_size));
  SM_TRY(ensure(m->prow, (size_t)groups * c.d_model * 4));
  SM_TRY(ensure(m->pos, (size_t)std::max(groups, std::min(chunk, S)) * 4));
  SM_TRY(ensure(m->lens, (size_t)std::max(groups, std::min(chunk, S)) * 4));
  cached = cached && pstate_bufs_same(m);  // no prompt-state buffer moved since the check
  int32_t* pos = (int32_t*)m->pos.p;
  int32_t* lens = (int32_t*)m->lens.p;
  // prompts, once per group, in chunks of whole prompts within the budget;
  // skipped when the model's prompt state holds these prompts' pass (the same
  // single-chunk pass, so the same values), e.g. from the generation that
  // produced the tokens
  const int64_t gchunk = std::max<int64_t>(1, budget / P);
  const bool one_chunk = gchunk >= groups && !m->trace_idx;
  for (int64_t g0 = 0; g0 < groups && !(cached && one_chunk); g0 += gchunk) {
    const int64_t gc = std::min(gchunk, groups - g0);
    // the pass overwrites the prompt state: valid again only once a whole
    // single-chunk untraced pass is recorded
    m->pstate_valid = false;
    SM_TRY(ensure(m->ids, (size_t)gc * P * 4));
    int32_t* ids = (int32_t*)m->ids.p;
    group_prompts_kernel<<<blocks_for(gc * P), 256, 0, st>>>(prompts + g0 * G * P, gc, (int)G,
                                                              (int)P, ids);
    set_positions_kernel<<<blocks_for(gc), 256, 0, st>>>(pos, lens, (int)gc, 0);
    const size_t off = (size_t)g0 * c.kv_heads * P * c.head_dim * m->kv_size;
    SM_TRY(run_layers(m, ids, gc, P, pos, nullptr, (char*)m->pkc.p + off, (char*)m->pvc.p + off,
                      pl, P, false, st));
    gather_rows_kernel<<<blocks_for(gc * c.d_model), 256, 0, st>>>(
        (const float*)m->x.p, (int)gc, (int)P, (int)P - 1, c.d_model,
        (float*)m->prow.p + g0 * c.d_model);
    if (one_chunk) SM_TRY(record_pstate(m, ids, groups, P, st));
  }
  // continuations, in chunks of rollouts
  const PrefixKV pre0{m->pkc.p, m->pvc.p, (int64_t)(pl * m->kv_size), (int)G, (int)P, 0};
  for (int64_t s0 = 0; s0 < S; s0 += chunk) {
    const int64_t cs = std::min(chunk, S - s0);
    const int64_t rows = cs * N;
    if (N > 1) {
      const size_t layer_elems = cache_layer_elems(m, cs, L);
      SM_TRY(ensure(m->rkc, layer_elems * m->kv_size));
      SM_TRY(ensure(m->rvc, layer_elems * m->kv_size));
      SM_TRY(ensure(m->ids, (size_t)cs * (N - 1) * 4));
      int32_t* ids = (int32_t*)m->ids.p;
      cont_ids_kernel<<<blocks_for(cs * (N - 1)), 256, 0, st>>>(tokens + s0 * N, cs, (int)N, ids);
      set_positions_kernel<<<blocks_for(cs), 256, 0, st>>>(pos, lens, (int)cs, (int)P);
      PrefixKV pre = pre0;
      pre.s0 = s0;
      SM_TRY(run_layers(m, ids, cs, N - 1, pos, nullptr, m->rkc.p, m->rvc.p, 0, L, false, st,
                        &pre));
    }
    SM_TRY(ensure(m->rows, (size_t)rows * c.d_model * 4));
    gather_cont_rows_kernel<<<blocks_for(rows * c.d_model), 256, 0, st>>>(
        (const float*)m->prow.p, (const float*)m->x.p, cs, s0, (int)G, (int)N, c.d_model,
        (float*)m->rows.p);
    SM_TRY(score_rows(m, rows, tokens + s0 * N, lp_out + s0 * N, st));
  }
  return SM_OK;
}

}  // namespace
}  // namespace sm


extern "C" int sm_rl_logprobs(sm_model* m, const int32_t* prompts, const int32_t* tokens,
                              int64_t S, int64_t P, int64_t N, int64_t max_tokens_per_forward,
                              float* lp_out, void* stream) {
  SM_REQUIRE(m && prompts && tokens && lp_out, "sm_rl_logprobs: null argument");
  SM_REQUIRE(S > 0 && P > 0 && N > 0, "sm_rl_logprobs: bad shape");
  const int64_t L = P + N - 1;
  SM_REQUIRE(L <= m->cfg.max_seq, "sequence length %lld exceeds max_seq_len %d", (long long)L,
             m->cfg.max_seq);
  hipStream_t st = as_stream(stream);
  const auto& c = m->cfg;
  const int64_t budget = max_tokens_per_forward > 0 ? max_tokens_per_forward : 65536;
  const int64_t chunk = std::max<int64_t>(1, budget / L);
  if (m->prompt_group > 1)
    return logprobs_grouped(m, prompts, tokens, S, P, N, budget, chunk, lp_out, st);
  for (int64_t s0 = 0; s0 < S; s0 += chunk) {
    const int64_t cs = std::min(chunk, S - s0);
    const size_t layer_elems = cache_layer_elems(m, cs, L);
    SM_TRY(ensure(m->rkc, layer_elems * m->kv_size));
    SM_TRY(ensure(m->rvc, layer_elems * m->kv_size));
    SM_TRY(ensure(m->ids, (size_t)cs * L * 4));
    SM_TRY(ensure(m->pos, (size_t)cs * 4));
    SM_TRY(ensure(m->lens, (size_t)cs * 4));
    int32_t* ids = (int32_t*)m->ids.p;
    build_ids_kernel<<<blocks_for(cs * L), 256, 0, st>>>(prompts + s0 * P, tokens + s0 * N, (int)cs,
                                                         (int)P, (int)N, ids);
    set_positions_kernel<<<blocks_for(cs), 256, 0, st>>>((int32_t*)m->pos.p, (int32_t*)m->lens.p,
                                                         (int)cs, 0);
    // one K/V buffer reused by every layer (layer stride 0)
    SM_TRY(run_layers(m, ids, cs, L, (const int32_t*)m->pos.p, nullptr, m->rkc.p, m->rvc.p, 0, L,
                      false, st));
    // hidden states that predict tokens[:, n] sit at positions P-1+n
    const int64_t rows = cs * N;
    SM_TRY(ensure(m->rows, (size_t)rows * c.d_model * 4));
    gather_span_kernel<<<blocks_for(rows * c.d_model), 256, 0, st>>>(
        (const float*)m->x.p, (int)cs, (int)L, (int)P - 1, (int)N, c.d_model, (float*)m->rows.p);
    // LM head + CE in row chunks bounding the [rows, V] logits to ~2 GiB
    const int64_t rchunk = std::max<int64_t>(1, ((int64_t)1 << 29) / c.vocab);
    SM_TRY(ensure(m->logits, (size_t)std::min(rows, rchunk) * c.vocab * 4));
    for (int64_t r0 = 0; r0 < rows; r0 += rchunk) {
      const int64_t rn = std::min(rchunk, rows - r0);
      SM_TRY(head(m, (const float*)m->rows.p + r0 * c.d_model, rn, (float*)m->logits.p, st));
      SM_TRY(sm_ce_rows(m->logits.p, SM_F32, tokens + s0 * N + r0, rn, c.vocab, c.vocab,
                        lp_out + s0 * N + r0, nullptr, nullptr, 1.0f, nullptr, nullptr, st));
    }
  }
  return SM_OK;
}

// ----------------------------------------------------------------- prepare ---

extern "C" int sm_rl_prepare(sm_model* policy, sm_model* reference, const int32_t* prompts,
                             const int32_t* tokens, const float* behavior_lp,
                             const float* rewards, const float* mask, int64_t groups,
                             int64_t group_size, int64_t P, int64_t N, double clip_epsilon,
                             double advantage_epsilon, double kl_coefficient,
                             int64_t max_tokens_per_forward, float* lp_cur, float* lp_ref,
                             float* group_stats, float* dlp, int32_t* flags, void* stream) {
  SM_REQUIRE(policy && prompts && tokens && behavior_lp && rewards && lp_cur,
             "sm_rl_prepare: null argument");
  SM_REQUIRE(kl_coefficient == 0.0 || (reference && lp_ref),
             "GRPO rollout needs reference log-probs for positive KL coefficient");
  const int64_t S = groups * group_size;
  SM_TRY(sm_rl_logprobs(policy, prompts, tokens, S, P, N, max_tokens_per_forward, lp_cur, stream));
  const bool use_ref = reference && lp_ref;
  if (use_ref)
    SM_TRY(sm_rl_logprobs(reference, prompts, tokens, S, P, N, max_tokens_per_forward, lp_ref,
                          stream));
  return sm_grpo_loss(rewards, lp_cur, behavior_lp, use_ref ? lp_ref : nullptr, mask, groups,
                      group_size, N, clip_epsilon, advantage_epsilon, kl_coefficient, group_stats,
                      nullptr, dlp, flags, stream);
}
