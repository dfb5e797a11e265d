// Decoder elementwise ops and token selection.
//
//   embed        Transformer::embed (summa-llm/src/model/transformer.rs:511-518)
//   rmsnorm      Norm::forward -> Burn RmsNorm, fp32 statistics
//                (summa-llm/src/model/norm.rs:36-50): y = x / sqrt(mean(x^2) + eps) * gamma
//   rope_append  project_qkv's [q | k | v] split + RoPE (adjacent-pair convention,
//                attention.rs:142-177; docs/uni-stack-inference.md:24) + the
//                AttnCache slice_assign (attention.rs:331-356)
//   sample       select_next_token (summa-llm/src/generate.rs:127-202): greedy
//                first-max argmax, or a temperature sample, plus the token's
//                log-prob under log_softmax(logits) (the quantity the GRPO
//                recompute produces, summa-train/src/tensor_sleep.rs:2609-2614)
//
// The residual stream is fp32; activations that feed a matmul are emitted in
// the model's activation dtype (f16 pairs for quantized models, fp32 otherwise).
#include <cmath>

#include "common.hpp"

namespace sm {
namespace {

template <typename T> __device__ inline float to_f(T v);
template <> __device__ inline float to_f<float>(float v) { return v; }
template <> __device__ inline float to_f<uint16_t>(uint16_t v) { return bf16_to_f32(v); }
template <> __device__ inline float to_f<_Float16>(_Float16 v) { return (float)v; }
template <typename T> __device__ inline T from_f(float v);
template <> __device__ inline float from_f<float>(float v) { return v; }
template <> __device__ inline uint16_t from_f<uint16_t>(float v) { return f32_to_bf16(v); }
template <> __device__ inline _Float16 from_f<_Float16>(float v) { return (_Float16)v; }

// x[r, :] = table[ids[r], :] * scale  (f32 out)
template <typename T>
__global__ void embed_kernel(const T* __restrict__ table, const int32_t* __restrict__ ids,
                             int64_t rows, int d, int vocab, float scale, float* __restrict__ x) {
  const int64_t r = blockIdx.x;
  const int32_t id = ids[r];
  const bool ok = id >= 0 && id < vocab;
  for (int c = threadIdx.x; c < d; c += blockDim.x)
    x[r * d + c] = ok ? to_f(table[(size_t)id * d + c]) * scale : NAN;
}

// One 256-thread workgroup per row. PAIR: y rows are SM_F16X2 (hi | lo).
template <typename TO, bool PAIR = false>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ gamma, int d,
                                                      float eps, TO* __restrict__ y) {
  __shared__ float part[4];
  const int64_t r = blockIdx.x;
  const float* xr = x + r * d;
  float ss = 0.f;
  for (int c = threadIdx.x; c < d; c += 256) ss = fmaf(xr[c], xr[c], ss);
  ss = wave_sum(ss);
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float rms = sqrtf(tot / (float)d + eps);
  if constexpr (PAIR) {
    _Float16* yr = reinterpret_cast<_Float16*>(y) + r * 2 * d;
    for (int c = threadIdx.x; c < d; c += 256) split_f16(xr[c] / rms * gamma[c], yr[c], yr[d + c]);
  } else {
    for (int c = threadIdx.x; c < d; c += 256) y[r * d + c] = from_f<TO>(xr[c] / rms * gamma[c]);
  }
}

// One wave per row for d = 256 * V (the models' widths): the row stays in
// registers (V float4 per lane, lane l holding columns 4*(64*i + l) + 0..3, so
// every load and store instruction covers a contiguous 1 KB of the row), one
// read of x, a shuffle reduction, no barrier. Four rows per workgroup.
template <typename TO, bool PAIR, int V>
__global__ __launch_bounds__(256) void rmsnorm_wave_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ gamma,
                                                           int64_t rows, float eps,
                                                           TO* __restrict__ y) {
  constexpr int D = 256 * V;
  const int64_t r = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  if (r >= rows) return;  // uniform per wave
  const int lane = threadIdx.x % kWave;
  const float4* xr = reinterpret_cast<const float4*>(x + r * D);
  const float4* gr = reinterpret_cast<const float4*>(gamma);
  float4 v[V], gm[V];  // gamma is loaded with x: one memory round trip
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) v[i] = xr[i * kWave + lane];
#pragma unroll
  for (int i = 0; i < V; ++i) gm[i] = gr[i * kWave + lane];
#pragma unroll
  for (int i = 0; i < V; ++i)
    ss = fmaf(v[i].w, v[i].w, fmaf(v[i].z, v[i].z, fmaf(v[i].y, v[i].y, fmaf(v[i].x, v[i].x, ss))));
  ss = wave_sum(ss);
  const float rms = sqrtf(ss / (float)D + eps);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const float o[4] = {v[i].x / rms * gm[i].x, v[i].y / rms * gm[i].y, v[i].z / rms * gm[i].z,
                        v[i].w / rms * gm[i].w};
    const int c = 4 * (i * kWave + lane);
    if constexpr (PAIR) {
      _Float16 hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) split_f16(o[e], hi[e], lo[e]);
      _Float16* yr = reinterpret_cast<_Float16*>(y) + r * 2 * D;
      *reinterpret_cast<h4*>(yr + c) = h4{hi[0], hi[1], hi[2], hi[3]};
      *reinterpret_cast<h4*>(yr + D + c) = h4{lo[0], lo[1], lo[2], lo[3]};
    } else if constexpr (sizeof(TO) == 4) {
      *reinterpret_cast<float4*>(y + r * D + c) = float4{o[0], o[1], o[2], o[3]};
    } else {
      TO t[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] = from_f<TO>(o[e]);
      uint2 u;
      __builtin_memcpy(&u, t, 8);
      *reinterpret_cast<uint2*>(y + r * D + c) = u;
    }
  }
}

// qkv: [rows, (H + 2*KVH) * hd] f32, row = s*L + i at position pos0[s] + i.
// One thread per (row, head slot, pair).
template <typename TA, typename TC>
__global__ void rope_append_kernel(const float* __restrict__ qkv, const float2* __restrict__ rope,
                                   const int32_t* __restrict__ pos0, int L, int H, int KVH,
                                   int hd, int cap, int64_t rows, TA* __restrict__ q_out,
                                   TC* __restrict__ kc, TC* __restrict__ vc) {
  const int half = hd / 2;
  const int slots = H + 2 * KVH;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * slots * half) return;
  const int p = idx % half;
  const int slot = (idx / half) % slots;
  const int64_t row = idx / ((int64_t)half * slots);
  const int s = (int)(row / L), i = (int)(row % L);
  const int pos = pos0[s] + i;
  if (pos < 0 || pos >= cap) return;
  const float* src = qkv + row * (int64_t)slots * hd + (int64_t)slot * hd + 2 * p;
  const float a = src[0], b = src[1];
  if (slot >= H + KVH) {  // value: no rotation
    const int kvh = slot - H - KVH;
    TC* dst = vc + (((size_t)s * KVH + kvh) * cap + pos) * hd + 2 * p;
    dst[0] = from_f<TC>(a);
    dst[1] = from_f<TC>(b);
    return;
  }
  const float2 cs = rope[(size_t)pos * half + p];  // (cos, sin)
  const float ra = a * cs.x - b * cs.y;
  const float rb = b * cs.x + a * cs.y;
  if (slot < H) {
    TA* dst = q_out + (row * H + slot) * hd + 2 * p;
    dst[0] = from_f<TA>(ra);
    dst[1] = from_f<TA>(rb);
  } else {
    const int kvh = slot - H;
    TC* dst = kc + (((size_t)s * KVH + kvh) * cap + pos) * hd + 2 * p;
    dst[0] = from_f<TC>(ra);
    dst[1] = from_f<TC>(rb);
  }
}

// Gumbel-max sampling / greedy argmax over one logits row per workgroup, plus
// the chosen token's log-prob. Ties resolve to the lowest index (Burn argmax /
// the host sampler's reverse index order, generate.rs:144-152).
constexpr int kSampleThreads = 1024;

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(const float* __restrict__ logits,
                                                     int64_t ld, int vocab, float inv_temp,
                                                     uint64_t seed, int64_t step,
                                                     int32_t* __restrict__ tok, int64_t tok_stride,
                                                     float* __restrict__ lp, int64_t lp_stride,
                                                     int32_t* __restrict__ next_ids) {
  constexpr int NW = kSampleThreads / kWave;
  __shared__ float s_best[NW];
  __shared__ int s_idx[NW];
  __shared__ float s_m[NW], s_s[NW];
  const int64_t r = blockIdx.x;
  const float* row = logits + r * ld;
  float m = -INFINITY, s = 0.f, best = -INFINITY;
  int bidx = 0x7fffffff;
  // rng_key(seed, r, c) = mix64(row_key ^ c * K2): the per-row half is hoisted.
  const uint64_t row_key = mix64(seed + 0x9e3779b97f4a7c15ull * ((uint64_t)r + 1));
  const uint64_t cbase = (uint64_t)step * (uint64_t)vocab;
  constexpr uint64_t kK2 = 0xd1b54a32d192ed03ull;
  // hc = (cbase + v) * K2 (mod 2^64), the counter half of rng_key
  auto visit_h = [&](float x, int v, uint64_t hc) {
    if (x > m) { s = s * __expf(m - x) + 1.f; m = x; } else { s += __expf(x - m); }
    float key = x;
    if (inv_temp > 0.f) {
      const float u = u01(mix64(row_key ^ hc));
      key = x * inv_temp - logf(-logf(u));
    }
    if (key > best) { best = key; bidx = v; }  // v increases per thread: first max kept
  };
  auto visit = [&](float x, int v) { visit_h(x, v, (cbase + (uint64_t)v) * kK2); };
  // four consecutive elements: one 64-bit multiply for the first counter, the
  // next three K2 apart (the same values mod 2^64; the hash is VALU-bound on
  // its 64-bit multiplies)
  auto visit4 = [&](const float4& a, int v) {
    const uint64_t h0 = (cbase + (uint64_t)v) * kK2;
    visit_h(a.x, v, h0);
    visit_h(a.y, v + 1, h0 + kK2);
    visit_h(a.z, v + 2, h0 + 2 * kK2);
    visit_h(a.w, v + 3, h0 + 3 * kK2);
  };
  if (vocab % 4 == 0 && ld % 4 == 0 && reinterpret_cast<uintptr_t>(logits) % 16 == 0) {
    // 16-byte loads, four of them in flight per thread: thread t takes float4s
    // t, t + T, t + 2T, ... (T threads), so its elements still come in
    // increasing order. One element per load left the row's 256 KB waiting on
    // one load per thread at a time (40 us at config[2]'s 256 x 65536).
    const float4* row4 = reinterpret_cast<const float4*>(row);
    const int n4 = vocab / 4;
    int i = threadIdx.x;
    for (; i + 3 * kSampleThreads < n4; i += 4 * kSampleThreads) {
      float4 a[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = row4[i + u * kSampleThreads];
#pragma unroll
      for (int u = 0; u < 4; ++u) visit4(a[u], 4 * (i + u * kSampleThreads));
    }
    for (; i < n4; i += kSampleThreads) visit4(row4[i], 4 * i);
  } else {
    for (int v = threadIdx.x; v < vocab; v += kSampleThreads) visit(row[v], v);
  }
  // wave reduce (max with lowest index on ties)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ob = __shfl_xor(best, o, kWave);
    const int oi = __shfl_xor(bidx, o, kWave);
    if (ob > best || (ob == best && oi < bidx)) { best = ob; bidx = oi; }
    const float om = __shfl_xor(m, o, kWave), os = __shfl_xor(s, o, kWave);
    lse_merge(m, s, om, os);
  }
  const int w = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) { s_best[w] = best; s_idx[w] = bidx; s_m[w] = m; s_s[w] = s; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < NW; ++k) {
      if (s_best[k] > best || (s_best[k] == best && s_idx[k] < bidx)) { best = s_best[k]; bidx = s_idx[k]; }
      lse_merge(m, s, s_m[k], s_s[k]);
    }
    if (bidx >= vocab) bidx = 0;  // all-NaN row: deterministic fallback
    tok[r * tok_stride] = bidx;
    if (next_ids) next_ids[r] = bidx;
    if (lp) lp[r * lp_stride] = row[bidx] - (m + __logf(s));
  }
}

}  // namespace
}  // namespace sm

using namespace sm;

extern "C" int sm_embed(const void* table, int dtype, const int32_t* ids, int64_t rows, int64_t d,
                        int64_t vocab, float scale, float* x, void* stream) {
  SM_REQUIRE(table && ids && x, "sm_embed: null buffer");
  SM_REQUIRE(rows >= 0 && d > 0 && vocab > 0, "sm_embed: bad shape");
  if (rows == 0) return SM_OK;
  if (dtype == SM_BF16)
    embed_kernel<uint16_t><<<(unsigned)rows, 256, 0, as_stream(stream)>>>(
        (const uint16_t*)table, ids, rows, (int)d, (int)vocab, scale, x);
  else if (dtype == SM_F32)
    embed_kernel<float><<<(unsigned)rows, 256, 0, as_stream(stream)>>>(
        (const float*)table, ids, rows, (int)d, (int)vocab, scale, x);
  else SM_REQUIRE(false, "sm_embed: dtype must be SM_BF16 or SM_F32");
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_rmsnorm(const float* x, const float* gamma, int64_t rows, int64_t d, float eps,
                          void* y, int out_dtype, void* stream) {
  SM_REQUIRE(x && gamma && y, "sm_rmsnorm: null buffer");
  SM_REQUIRE(rows >= 0 && d > 0, "sm_rmsnorm: bad shape");
  SM_REQUIRE(out_dtype == SM_BF16 || out_dtype == SM_F16 || out_dtype == SM_F16X2 ||
                 out_dtype == SM_F32,
             "sm_rmsnorm: out_dtype must be SM_F32, SM_BF16, SM_F16 or SM_F16X2");
  if (rows == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(gamma) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(y) % 16 == 0;
  const int v = (d % 256 == 0 && aligned) ? (int)(d / 256) : 0;
  if (v == 3 || v == 4 || v == 8 || v == 12 || v == 16) {
    const unsigned blocks = (unsigned)ceil_div(rows, 4);
#define SM_RMSW(TO, PAIR, V) \
  rmsnorm_wave_kernel<TO, PAIR, V><<<blocks, 256, 0, st>>>(x, gamma, rows, eps, (TO*)y)
#define SM_RMSW_V(TO, PAIR)            \
  do {                                 \
    if (v == 3) SM_RMSW(TO, PAIR, 3);  \
    else if (v == 4) SM_RMSW(TO, PAIR, 4);   \
    else if (v == 8) SM_RMSW(TO, PAIR, 8);   \
    else if (v == 12) SM_RMSW(TO, PAIR, 12); \
    else SM_RMSW(TO, PAIR, 16);        \
  } while (0)
    if (out_dtype == SM_BF16) SM_RMSW_V(uint16_t, false);
    else if (out_dtype == SM_F16) SM_RMSW_V(_Float16, false);
    else if (out_dtype == SM_F16X2) SM_RMSW_V(_Float16, true);
    else SM_RMSW_V(float, false);
#undef SM_RMSW_V
#undef SM_RMSW
  } else if (out_dtype == SM_BF16)
    rmsnorm_kernel<uint16_t><<<(unsigned)rows, 256, 0, st>>>(x, gamma, (int)d, eps, (uint16_t*)y);
  else if (out_dtype == SM_F16)
    rmsnorm_kernel<_Float16><<<(unsigned)rows, 256, 0, st>>>(x, gamma, (int)d, eps, (_Float16*)y);
  else if (out_dtype == SM_F16X2)
    rmsnorm_kernel<_Float16, true><<<(unsigned)rows, 256, 0, st>>>(x, gamma, (int)d, eps,
                                                                  (_Float16*)y);
  else
    rmsnorm_kernel<float><<<(unsigned)rows, 256, 0, st>>>(x, gamma, (int)d, eps, (float*)y);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_rope_append(const float* qkv, const float* rope_table, const int32_t* pos0,
                              int64_t S, int64_t L, int64_t H, int64_t KVH, int64_t head_dim,
                              int64_t cap, void* q_out, int q_dtype, void* kcache, void* vcache,
                              int cache_dtype, void* stream) {
  SM_REQUIRE(qkv && rope_table && pos0 && q_out && kcache && vcache, "sm_rope_append: null buffer");
  SM_REQUIRE(S >= 0 && L >= 0 && H > 0 && KVH > 0 && head_dim > 0 && head_dim % 2 == 0 && cap > 0,
             "sm_rope_append: bad shape");
  const int64_t rows = S * L;
  const int64_t n = rows * (H + 2 * KVH) * (head_dim / 2);
  if (n == 0) return SM_OK;
  const unsigned blocks = (unsigned)ceil_div(n, 256);
  hipStream_t st = as_stream(stream);
  const float2* rt = reinterpret_cast<const float2*>(rope_table);
#define SM_ROPE(TA, TC)                                                                         \
  rope_append_kernel<TA, TC><<<blocks, 256, 0, st>>>(qkv, rt, pos0, (int)L, (int)H, (int)KVH,  \
                                                     (int)head_dim, (int)cap, rows, (TA*)q_out, \
                                                     (TC*)kcache, (TC*)vcache)
  if (q_dtype == SM_BF16 && cache_dtype == SM_BF16) SM_ROPE(uint16_t, uint16_t);
  else if (q_dtype == SM_F32 && cache_dtype == SM_F32) SM_ROPE(float, float);
  else if (q_dtype == SM_F32 && cache_dtype == SM_BF16) SM_ROPE(float, uint16_t);
  else if (q_dtype == SM_F16 && cache_dtype == SM_F16) SM_ROPE(_Float16, _Float16);
  else SM_REQUIRE(false, "sm_rope_append: unsupported dtype combination");
#undef SM_ROPE
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_sample(const float* logits, int64_t rows, int64_t ld, int64_t vocab,
                         float temperature, uint64_t seed, int64_t step, int32_t* tokens,
                         int64_t tok_stride, float* logprobs, int64_t lp_stride,
                         int32_t* next_ids, void* stream) {
  SM_REQUIRE(logits && tokens, "sm_sample: null buffer");
  SM_REQUIRE(rows >= 0 && vocab > 0 && vocab <= ld, "sm_sample: bad shape");
  SM_REQUIRE(!std::isnan(temperature), "temperature must not be NaN");
  if (rows == 0) return SM_OK;
  const float inv_temp = temperature > 0.f ? 1.f / temperature : 0.f;
  sample_kernel<<<(unsigned)rows, kSampleThreads, 0, as_stream(stream)>>>(
      logits, ld, (int)vocab, inv_temp, seed, step, tokens, tok_stride, logprobs, lp_stride,
      next_ids);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

namespace sm {
namespace {
__global__ void completion_mask_kernel(const int32_t* __restrict__ lengths, int64_t S, int64_t N,
                                       float* __restrict__ mask) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < S * N) mask[i] = (i % N) < (int64_t)lengths[i / N] ? 1.f : 0.f;
}
}  // namespace
}  // namespace sm

extern "C" int sm_completion_mask(const int32_t* lengths, int64_t S, int64_t N, float* mask,
                                  void* stream) {
  using namespace sm;
  SM_REQUIRE(lengths && mask, "sm_completion_mask: null buffer");
  SM_REQUIRE(S >= 0 && N > 0, "sm_completion_mask: bad shape");
  if (S == 0) return SM_OK;
  completion_mask_kernel<<<(unsigned)ceil_div(S * N, 256), 256, 0, as_stream(stream)>>>(
      lengths, S, N, mask);
  SM_LAUNCH_CHECK();
  return SM_OK;
}
