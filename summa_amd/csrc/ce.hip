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
//   * lp + grad in place, bf16 rows of 64k-128k columns (config[3]'s
//     131072): ce_grad_resident_kernel holds the row on chip (VGPRs + an LDS
//     stash), so it is read once and written once: 6.13 ms for 34.4 GB at
//     config[3], 0.70 of HBM, counters 1.00x the algorithmic bytes.
//   * lp + grad in place, other rows: one 512-thread workgroup per row
//     streams the row twice: a statistics pass with ordinary (cached) loads,
//     then a gradient pass whose loads and stores are nontemporal (last use),
//     8 vectors per lane in flight. The second read of a row misses L2 when
//     the row is long (256 KB at config[3]: 1.5x the algorithmic bytes beyond
//     L2, 7.2 ms). Measured there and not kept: plain or mixed load / store
//     kinds in the second pass (7.4-7.6 ms); 1024 threads x 4 vectors
//     (7.3-7.4 ms); the row in VGPRs of one 1024-thread workgroup, once per CU,
//     so its read, reduce and write phases never overlap another row's
//     (8.2-9.9 ms); only the row's last 1/8 to 1/2 in registers (7.3-8.6 ms).
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

// Gradient in place with the row held on chip: bf16 rows of at most
// 8 * 512 * (VR + VL) stored columns, 16-byte aligned. Each of the 512
// threads keeps VR 16-byte vectors of its row in VGPRs (vector u*512 + tid)
// and VL more in an LDS stash (vector (VR + w)*512 + tid, copied there by
// global_load_lds_dwordx4 without passing through registers), so the row is
// read from HBM once and written once. With the row resident the statistics
// need no online rescaling: the row max first (one workgroup reduction), then
// sum exp(x - max) (another), in a fixed order, so lse is deterministic (it
// differs from the streaming kernels' online order in the last bits; measured
// 1 % faster than one online pass here).
// 96 + 64 KB at VR = 24, VL = 8 (config[3]'s 131072 columns), 128 VGPRs:
// two workgroups per CU, so one row's reads overlap another row's writes.
// Loads and stores are nontemporal (each element is read once and written
// once): 6.24 against 6.28-6.57 ms with plain loads or stores. A persistent
// grid (two workgroups per CU walking the rows) measured 6.52 ms.
// The gradient away from the target column and the padding is
// 2^(x log2e - lse log2e + log2 |scale|) with the sign set on the bf16 bits
// (one exp, no multiply; within a few f32 ulps of softmax * scale before the
// bf16 rounding); elsewhere it is ce_grad_stream_kernel's arithmetic.
template <int VR, int VL, bool FULL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void
ce_grad_resident_kernel(void* __restrict__ logits, const int32_t* __restrict__ targets,
                        int64_t ld, int64_t vl, float* __restrict__ lp,
                        float* __restrict__ lse_out, float grad_scale,
                        const float* __restrict__ row_scale) {
  constexpr int T = 512, kV = 8, NW = T / kWave;
  __shared__ u32x4 stash[VL > 0 ? VL * T : 1];
  __shared__ float red_m[NW], red_s[NW];
  __shared__ float target_logit;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  // FULL: ld == vl == 512 * 8 * (VR + VL), every vector present, no masks
  const int nvec = FULL ? (VR + VL) * T : (int)(vl / kV);
  const int nvec_st = FULL ? (VR + VL) * T : (int)(ld / kV), vli = FULL ? nvec * kV : (int)vl;
  const int tl = tid;
  const int64_t row = blockIdx.x;
  const uint32_t lo16 = (uint32_t)tl * 16u;  // lane offset inside each 8 KB slice
  auto present = [&](int i, int n) { return FULL || i * T + tl < n; };
  char* row_ptr = static_cast<char*>(logits) + row * ld * 2;
  // vector i*512 + tid sits at slice(i) + lo16
  auto slice = [&](int i) { return row_ptr + (size_t)i * (T * 16); };
  const int32_t t = targets[row];
  if (tid == 0)
    target_logit =
        (t >= 0 && t < vl) ? bf16_to_f32(reinterpret_cast<const uint16_t*>(row_ptr)[t]) : NAN;
  // the stash copies first, then the register vectors: loads complete in
  // order, so the max pass can start on r[0] while the rest arrive
#if defined(__HIP_DEVICE_COMPILE__)  // (the host pass does not emit the launch stub otherwise)
#pragma unroll
  for (int w = 0; w < VL; ++w) {
    if (present(VR + w, nvec_st))  // aux 2: nontemporal, the row's only read
      __builtin_amdgcn_global_load_lds(
          slice(VR + w) + lo16,
          (__attribute__((address_space(3))) void*)&stash[w * T + wave * kWave], 16, 0, 2);
  }
#endif
  u32x4 r[VR];
#pragma unroll
  for (int u = 0; u < VR; ++u) {
    r[u] = present(u, nvec_st)
               ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(slice(u) + lo16))
               : u32x4{0u, 0u, 0u, 0u};
  }
  // ---- row max
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < VR; ++u) {
    if (present(u, nvec)) {
      float x[kV];
      unpack<true>(r[u], x);
#pragma unroll
      for (int e = 0; e < kV; ++e) mx = fmaxf(mx, x[e]);
    }
  }
  // the stash copies are done (each wave reads back only the slots it copied)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int w = 0; w < VL; ++w) {
    if (present(VR + w, nvec)) {
      float x[kV];
      unpack<true>(stash[w * T + tid], x);
#pragma unroll
      for (int e = 0; e < kV; ++e) mx = fmaxf(mx, x[e]);
    }
  }
  if (!FULL)
    for (int c = nvec * kV + tl; c < vli; c += T) mx = fmaxf(mx, load_scalar<true>(row_ptr, c));
  mx = wave_max(mx);
  if (lane == 0) red_m[wave] = mx;
  __syncthreads();
  float m = red_m[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) m = fmaxf(m, red_m[w]);
  // ---- sum of exp(x - max), in the log2 domain as online_update
  const float nm = -m * kLog2e;
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < VR; ++u) {
    asm volatile("" : "+v"(r[u]));  // unpack again: no unpacked row kept across passes
    if (present(u, nvec)) {
      float x[kV];
      unpack<true>(r[u], x);
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < kV; ++e) acc += __builtin_amdgcn_exp2f(fmaf(x[e], kLog2e, nm));
      sum += acc;
    }
  }
#pragma unroll
  for (int w = 0; w < VL; ++w) {
    if (present(VR + w, nvec)) {
      float x[kV];
      unpack<true>(stash[w * T + tid], x);
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < kV; ++e) acc += __builtin_amdgcn_exp2f(fmaf(x[e], kLog2e, nm));
      sum += acc;
    }
  }
  if (!FULL)
    for (int c = nvec * kV + tl; c < vli; c += T)
      sum += __builtin_amdgcn_exp2f(fmaf(load_scalar<true>(row_ptr, c), kLog2e, nm));
  sum = wave_sum(sum);
  if (lane == 0) red_s[wave] = sum;
  __syncthreads();
  float s = red_s[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) s += red_s[w];
  const float lse = m + __logf(s);
  if (tid == 0) {
    if (lse_out) lse_out[row] = lse;
    if (lp) lp[row] = target_logit - lse;
  }
  // ---- gradient: (softmax - onehot(t)) * scale, zeros past the logical vocab
  const float scale = grad_scale * (row_scale ? row_scale[row] : 1.f);
  const float nl = -lse * kLog2e;
  // away from the target and the padding: |scale| p = 2^(x log2e - lse log2e +
  // log2 |scale|), the sign of scale set on the packed bf16 words (no multiply)
  const float nls = nl + __log2f(fabsf(scale));
  const uint32_t sgn = scale < 0.f ? 0x80008000u : 0u;
  auto grad = [&](const u32x4& v, int c0) -> u32x4 {
    if (c0 + kV <= vli && (unsigned)(t - c0) >= (unsigned)kV) {  // no target, no padding
      float x[kV];
      unpack<true>(v, x);
      float g[kV];
#pragma unroll
      for (int e = 0; e < kV; ++e) g[e] = __builtin_amdgcn_exp2f(fmaf(x[e], kLog2e, nls));
      return u32x4{pack_bf16x2(g[0], g[1]) ^ sgn, pack_bf16x2(g[2], g[3]) ^ sgn,
                   pack_bf16x2(g[4], g[5]) ^ sgn, pack_bf16x2(g[6], g[7]) ^ sgn};
    }
    return grad_vec<true>(v, c0, vl, t, nl, scale);
  };
#pragma unroll
  for (int u = 0; u < VR; ++u) {
    asm volatile("" : "+v"(r[u]));
    uint32_t off = lo16;
    asm volatile("" : "+v"(off));  // the store address is formed here, not kept from the loads
    if (present(u, nvec_st))
      __builtin_nontemporal_store(grad(r[u], (u * T + tl) * kV),
                                  reinterpret_cast<u32x4*>(slice(u) + off));
  }
#pragma unroll
  for (int w = 0; w < VL; ++w) {
    uint32_t off = lo16;
    asm volatile("" : "+v"(off));
    if (present(VR + w, nvec_st))
      __builtin_nontemporal_store(grad(stash[w * T + tid], ((VR + w) * T + tl) * kV),
                                  reinterpret_cast<u32x4*>(slice(VR + w) + off));
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

// bf16 columns the resident gradient kernel holds (512 threads x 32 vectors)
constexpr int64_t kResidentCols = 512 * 32 * 8;

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
  if constexpr (BF16) {
    if (vec && ld > kResidentCols / 2 && ld <= kResidentCols) {
      if (ld == kResidentCols && vl == ld)
        ce_grad_resident_kernel<24, 8, true><<<grid, 512, 0, st>>>(grad, targets, ld, vl, lp, lse,
                                                                    grad_scale, row_scale);
      else
        ce_grad_resident_kernel<24, 8, false><<<grid, 512, 0, st>>>(grad, targets, ld, vl, lp,
                                                                     lse, grad_scale, row_scale);
      SM_LAUNCH_CHECK();
      return SM_OK;
    }
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
