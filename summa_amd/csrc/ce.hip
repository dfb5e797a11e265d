// Fused row-wise log-softmax / cross-entropy / token log-prob (kernel 3).
//
// Semantics follow the reference row kernels
//   ce_row_statistics  summa-llm/src/model/linear_cross_entropy/gpu.rs:29-114
//   ce_row_gradient    summa-llm/src/model/linear_cross_entropy/gpu.rs:123-158
// and the portable oracle linear_cross_entropy/reference.rs:21-92: per row an
// online (max, sum exp) over the logical vocabulary, lp = x_t - max - ln(sum),
// grad = (softmax - onehot) * scale, padded columns never read and written as
// exact zeros.
//
// MI355X design. The op is HBM-bound (≈1 flop per byte), so everything is
// about streaming each row once with 16-byte loads:
//   * lp / loss only: one 256-thread workgroup per row, 4 x 16 B loads in
//     flight per lane, online max/sum in registers, wave shuffles + LDS merge.
//     Traffic = one read of the logits.
//   * lp + grad in place: one 512-thread workgroup per row streams the row
//     twice: a statistics pass with ordinary (cached) loads, then a gradient
//     pass whose loads and stores are nontemporal (last use), 8 vectors per
//     lane in flight. The second read of a row (256 KB at config[3]) misses
//     L2: the L2-miss read counter shows 1.76x the algorithmic read, served by
//     the 256 MB MALL or by HBM. Config[3] (bf16 65536 x 131072): 7.2 ms for
//     34 GB of algorithmic traffic; a plain elementwise in-place pass over the
//     same bytes (one read, one write, no statistics pass) runs at 5.9 TB/s.
//     Plain or mixed load / store kinds in the second pass: 7.4-7.6 ms; 1024
//     threads x 4 vectors: 7.3-7.4 ms. Keeping each row in VGPRs
//     (read once, write once) was 9.9 ms: a 1024-thread workgroup holding
//     256 KB in registers fits once per CU, so its read, reduce and write
//     phases never overlap with another row's. Keeping only the row's last
//     1/8 to 1/2 in registers (those gradients written without a second
//     read, the rest re-read newest first) was 7.3-8.6 ms: the registers
//     cost rows in flight per CU, and with them more than the re-reads.
#include <cfloat>
#include <cmath>

#include "common.hpp"

namespace sm {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Elements of a 16-byte vector for each input dtype.
template <bool BF16> struct Elem;
template <> struct Elem<true> { static constexpr int kVec = 8; static constexpr int kSize = 2; };
template <> struct Elem<false> { static constexpr int kVec = 4; static constexpr int kSize = 4; };

template <bool BF16>
__device__ inline void unpack(const u32x4& v, float (&x)[Elem<BF16>::kVec]) {
  if constexpr (BF16) {
    x[0] = bf16lo(v.x); x[1] = bf16hi(v.x); x[2] = bf16lo(v.y); x[3] = bf16hi(v.y);
    x[4] = bf16lo(v.z); x[5] = bf16hi(v.z); x[6] = bf16lo(v.w); x[7] = bf16hi(v.w);
  } else {
    x[0] = __uint_as_float(v.x); x[1] = __uint_as_float(v.y);
    x[2] = __uint_as_float(v.z); x[3] = __uint_as_float(v.w);
  }
}

template <bool BF16>
__device__ inline float load_scalar(const void* p, int64_t i) {
  if constexpr (BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return static_cast<const float*>(p)[i];
}

template <bool BF16>
__device__ inline void store_scalar(void* p, int64_t i, float v) {
  if constexpr (BF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  else static_cast<float*>(p)[i] = v;
}

// Online update of a running (m, s) in the log2 domain: s = sum 2^(x*log2e - m2)
// where m2 = m*log2e. Processes one vector of values.
template <int N>
__device__ inline void online_update(const float (&x)[N], float& m, float& s) {
  float lm = x[0];
#pragma unroll
  for (int i = 1; i < N; ++i) lm = fmaxf(lm, x[i]);
  if (lm > m) {
    s *= exp2f((m - lm) * kLog2e);
    m = lm;
  }
  const float nm = -m * kLog2e;
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) acc += exp2f(fmaf(x[i], kLog2e, nm));
  s += acc;
}

// Block-wide merge of per-thread (m, s); every thread receives the result.
template <int THREADS>
__device__ inline void block_lse(float& m, float& s) {
  __shared__ float sm_m[THREADS / kWave];
  __shared__ float sm_s[THREADS / kWave];
  wave_lse(m, s);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) { sm_m[wave] = m; sm_s[wave] = s; }
  __syncthreads();
  m = sm_m[0];
  s = sm_s[0];
#pragma unroll
  for (int w = 1; w < THREADS / kWave; ++w) lse_merge(m, s, sm_m[w], sm_s[w]);
}

// Statistics of one row by streaming reads (used by the lp-only kernel and by
// the first pass of the two-read gradient kernel).
template <int THREADS, bool BF16, bool VEC>
__device__ inline void row_stats_stream(const void* row_ptr, int64_t vl, float& m, float& s) {
  m = -INFINITY;
  s = 0.f;
  constexpr int kV = Elem<BF16>::kVec;
  int64_t done = 0;
  if constexpr (VEC) {
    constexpr int U = 4;
    const u32x4* vp = static_cast<const u32x4*>(row_ptr);
    const int64_t nvec = vl / kV;
    for (int64_t v0 = threadIdx.x; v0 < nvec; v0 += (int64_t)THREADS * U) {
      u32x4 buf[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t idx = v0 + (int64_t)u * THREADS;
        if (idx < nvec) buf[u] = __builtin_nontemporal_load(&vp[idx]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t idx = v0 + (int64_t)u * THREADS;
        if (idx < nvec) {
          float x[kV];
          unpack<BF16>(buf[u], x);
          online_update(x, m, s);
        }
      }
    }
    done = nvec * kV;
  }
  for (int64_t c = done + threadIdx.x; c < vl; c += THREADS) {
    float x[1] = {load_scalar<BF16>(row_ptr, c)};
    online_update(x, m, s);
  }
  block_lse<THREADS>(m, s);
}

// lp / lse only: one workgroup per row, one read of the row.
template <int THREADS, bool BF16, bool VEC>
__global__ __launch_bounds__(THREADS) void ce_lp_kernel(const void* __restrict__ logits,
                                                        const int32_t* __restrict__ targets,
                                                        int64_t ld, int64_t vl,
                                                        float* __restrict__ lp,
                                                        float* __restrict__ lse_out) {
  const int64_t row = blockIdx.x;
  const char* row_ptr = static_cast<const char*>(logits) + row * ld * Elem<BF16>::kSize;
  float m, s;
  row_stats_stream<THREADS, BF16, VEC>(row_ptr, vl, m, s);
  if (threadIdx.x == 0) {
    const float lse = m + __logf(s);
    if (lse_out) lse_out[row] = lse;
    if (lp) {
      const int32_t t = targets[row];
      lp[row] = (t >= 0 && t < vl) ? load_scalar<BF16>(row_ptr, t) - lse : NAN;
    }
  }
}

// The gradient of 8 (bf16) or 4 (f32) consecutive columns starting at
// column c0, packed for one 16-byte store: (softmax - onehot(t)) * scale,
// exact zeros at padded columns (>= vl).
template <bool BF16>
__device__ inline u32x4 grad_vec(const u32x4& v, int64_t c0, int64_t vl, int32_t t, float nl,
                                 float scale) {
  constexpr int kV = Elem<BF16>::kVec;
  float x[kV];
  unpack<BF16>(v, x);
  float g[kV];
#pragma unroll
  for (int e = 0; e < kV; ++e) {
    const int64_t col = c0 + e;
    float p = exp2f(fmaf(x[e], kLog2e, nl)) * scale;
    if (col == t) p -= scale;
    g[e] = (col < vl) ? p : 0.f;
  }
  u32x4 o;
  if constexpr (BF16) {
    o.x = pack_bf16x2(g[0], g[1]);
    o.y = pack_bf16x2(g[2], g[3]);
    o.z = pack_bf16x2(g[4], g[5]);
    o.w = pack_bf16x2(g[6], g[7]);
  } else {
    o.x = __float_as_uint(g[0]); o.y = __float_as_uint(g[1]);
    o.z = __float_as_uint(g[2]); o.w = __float_as_uint(g[3]);
  }
  return o;
}

// Gradient in place, 16-byte vectors (ld * size % 16 == 0, 16-byte aligned
// rows): a statistics pass over the logical columns with cached loads, then
// the gradient pass over the stored row with nontemporal loads and stores.
// Per thread the vectors are visited in the same order in both passes
// (idx = tid, tid + THREADS, ...), U of them in flight.
template <int THREADS, int U, bool BF16>
__global__ __launch_bounds__(THREADS) void ce_grad_stream_kernel(
    void* __restrict__ logits, const int32_t* __restrict__ targets, int64_t ld, int64_t vl,
    float* __restrict__ lp, float* __restrict__ lse_out, float grad_scale,
    const float* __restrict__ row_scale) {
  constexpr int kV = Elem<BF16>::kVec;
  const int64_t row = blockIdx.x;
  char* row_ptr = static_cast<char*>(logits) + row * ld * Elem<BF16>::kSize;
  u32x4* vp = reinterpret_cast<u32x4*>(row_ptr);
  const int64_t nvec = vl / kV;     // full vectors inside the logical vocab
  const int64_t nvec_st = ld / kV;  // vectors in the stored row
  const int32_t t = targets[row];
  __shared__ float target_logit;
  if (threadIdx.x == 0) target_logit = (t >= 0 && t < vl) ? load_scalar<BF16>(row_ptr, t) : NAN;
  float m = -INFINITY, s = 0.f;
  for (int64_t v0 = threadIdx.x; v0 < nvec; v0 += (int64_t)THREADS * U) {
    u32x4 buf[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t idx = v0 + (int64_t)u * THREADS;
      if (idx < nvec) buf[u] = vp[idx];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t idx = v0 + (int64_t)u * THREADS;
      if (idx < nvec) {
        float x[kV];
        unpack<BF16>(buf[u], x);
        online_update(x, m, s);
      }
    }
  }
  for (int64_t c = nvec * kV + threadIdx.x; c < vl; c += THREADS) {  // logical tail
    float x[1] = {load_scalar<BF16>(row_ptr, c)};
    online_update(x, m, s);
  }
  block_lse<THREADS>(m, s);  // contains a barrier after target_logit is set
  const float lse = m + __logf(s);
  if (threadIdx.x == 0) {
    if (lse_out) lse_out[row] = lse;
    if (lp) lp[row] = target_logit - lse;
  }
  const float scale = grad_scale * (row_scale ? row_scale[row] : 1.f);
  const float nl = -lse * kLog2e;
  for (int64_t v0 = threadIdx.x; v0 < nvec_st; v0 += (int64_t)THREADS * U) {
    u32x4 buf[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t idx = v0 + (int64_t)u * THREADS;
      if (idx < nvec_st) buf[u] = __builtin_nontemporal_load(&vp[idx]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t idx = v0 + (int64_t)u * THREADS;
      if (idx < nvec_st)
        __builtin_nontemporal_store(grad_vec<BF16>(buf[u], idx * kV, vl, t, nl, scale), &vp[idx]);
    }
  }
}

// Gradient in place for any row length: stats pass, then a read+write pass.
template <int THREADS, bool BF16, bool VEC>
__global__ __launch_bounds__(THREADS) void ce_grad_2pass_kernel(
    void* __restrict__ logits, const int32_t* __restrict__ targets, int64_t ld, int64_t vl,
    float* __restrict__ lp, float* __restrict__ lse_out, float grad_scale,
    const float* __restrict__ row_scale) {
  const int64_t row = blockIdx.x;
  char* row_ptr = static_cast<char*>(logits) + row * ld * Elem<BF16>::kSize;
  const int32_t t = targets[row];
  __shared__ float target_logit;
  if (threadIdx.x == 0) target_logit = (t >= 0 && t < vl) ? load_scalar<BF16>(row_ptr, t) : NAN;
  float m, s;
  row_stats_stream<THREADS, BF16, VEC>(row_ptr, vl, m, s);
  const float lse = m + __logf(s);
  if (threadIdx.x == 0) {
    if (lse_out) lse_out[row] = lse;
    if (lp) lp[row] = target_logit - lse;
  }
  const float scale = grad_scale * (row_scale ? row_scale[row] : 1.f);
  const float nl = -lse * kLog2e;
  for (int64_t c = threadIdx.x; c < ld; c += THREADS) {
    float g = 0.f;
    if (c < vl) {
      g = exp2f(fmaf(load_scalar<BF16>(row_ptr, c), kLog2e, nl)) * scale;
      if (c == t) g -= scale;
    }
    store_scalar<BF16>(row_ptr, c, g);
  }
}

// loss = -mean(lp), fixed-order f64 reduction in one workgroup.
__global__ __launch_bounds__(1024) void mean_neg_kernel(const float* __restrict__ lp, int64_t n,
                                                        float* __restrict__ loss) {
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

template <bool BF16>
int launch_ce(const void* logits, const int32_t* targets, int64_t rows, int64_t ld, int64_t vl,
              float* lp, float* lse, void* grad, float grad_scale, const float* row_scale,
              hipStream_t st) {
  const bool vec = (reinterpret_cast<uintptr_t>(logits) % 16 == 0) &&
                   ((ld * Elem<BF16>::kSize) % 16 == 0);
  const dim3 grid(static_cast<unsigned>(rows));
  if (!grad) {
    if (vec) ce_lp_kernel<256, BF16, true><<<grid, 256, 0, st>>>(logits, targets, ld, vl, lp, lse);
    else ce_lp_kernel<256, BF16, false><<<grid, 256, 0, st>>>(logits, targets, ld, vl, lp, lse);
    SM_LAUNCH_CHECK();
    return SM_OK;
  }
  if (vec) {
    ce_grad_stream_kernel<512, 8, BF16><<<grid, 512, 0, st>>>(grad, targets, ld, vl, lp, lse,
                                                               grad_scale, row_scale);
  } else {
    ce_grad_2pass_kernel<256, BF16, false><<<grid, 256, 0, st>>>(grad, targets, ld, vl, lp, lse,
                                                                 grad_scale, row_scale);
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace

}  // namespace sm

extern "C" int sm_ce_rows(const void* logits, int dtype, const int32_t* targets, int64_t rows,
                          int64_t stored_vocab, int64_t logical_vocab, float* token_logprob,
                          float* row_lse, void* grad, float grad_scale, const float* row_scale,
                          float* loss, void* stream) {
  using namespace sm;
  SM_REQUIRE(logits && targets, "sm_ce_rows: logits and targets are required");
  SM_REQUIRE(dtype == SM_BF16 || dtype == SM_F32, "sm_ce_rows: dtype must be SM_BF16 or SM_F32");
  SM_REQUIRE(rows >= 0 && rows <= 0x7fffffff, "sm_ce_rows: rows %lld out of range", (long long)rows);
  SM_REQUIRE(logical_vocab > 0 && logical_vocab <= stored_vocab,
             "logical vocabulary %lld must be in 1..=%lld", (long long)logical_vocab,
             (long long)stored_vocab);
  SM_REQUIRE(stored_vocab <= 0x7fffffff, "sm_ce_rows: vocabulary too large");
  SM_REQUIRE(!grad || grad == logits, "sm_ce_rows: grad must be NULL or alias logits (in place)");
  SM_REQUIRE(!loss || token_logprob, "sm_ce_rows: loss needs token_logprob");
  if (rows == 0) {
    SM_REQUIRE(!loss, "linear cross-entropy requires at least one token");
    return SM_OK;
  }
  hipStream_t st = as_stream(stream);
  int s = (dtype == SM_BF16)
              ? launch_ce<true>(logits, targets, rows, stored_vocab, logical_vocab, token_logprob,
                                row_lse, grad, grad_scale, row_scale, st)
              : launch_ce<false>(logits, targets, rows, stored_vocab, logical_vocab, token_logprob,
                                 row_lse, grad, grad_scale, row_scale, st);
  if (s != SM_OK) return s;
  if (loss) {
    mean_neg_kernel<<<1, 1024, 0, st>>>(token_logprob, rows, loss);
    SM_LAUNCH_CHECK();
  }
  return SM_OK;
}
