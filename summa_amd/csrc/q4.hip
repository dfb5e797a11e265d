// Q4G128 quantized matmul (kernel 1: decode GEMV / small-M GEMM) and the
// device-side Q4G128 quantizer.
//
// Format (defined by this build as HQUANT format tag 4, alongside the
// reference's binary/ternary g128 codecs in summa-train/src/quantization.rs:
// 34-77, 416-423): weight W[N, K] (N = out features, K = in features,
// i.e. the transpose of Burn's [d_in, d_out] Linear layout) row-major,
// groups of 128 consecutive elements of the flattened tensor, one bf16 scale
// per group = bf16(absmax / 7), signed int4 two's-complement codes
// q = clamp(round_half_away(w / scale), -8, 7), two per byte, low nibble = even
// element. value = scale * q (exact in f32). The GPU kernels need K % 128 == 0
// so that a group never straddles two rows.
//
// y[m, n] = sum_k x[m, k] * value(n, k), x bf16, f32 accumulate. This is the
// matmul the reference's PackedTensor::matrix_vector states for one row of x
// (quantization.rs:630-654) and Linear::forward computes for a batch.
//
// MI355X design: v_mfma_f32_16x16x32_f16. The B operand (weights) goes from
// HBM straight into registers: lane (j = l%16, g = l/16) loads one 16-byte
// chunk = 32 consecutive k of weight row n0+j per 128-k group, and each of its
// four 32-bit words becomes the lane's 8 f16 B values of one MFMA step via the
// 0x6400 magic-exponent trick (x ^ 0x8 -> offset binary, OR into the f16
// mantissa, one packed subtract / fma) and one packed multiply by the group
// scale. q * scale is exact in f16 (<= 11 significant bits) as long as the
// scale is an f16 normal, which sm_q4_quantize checks. The A operand
// (activations, f16 or bf16 in HBM) is read by the lanes whose row is < M
// only, converted to f16 if needed and permuted to the same k order as the
// dequantised words. For
// tiny N the four waves of a workgroup split the K groups and merge their
// accumulators through LDS in a fixed order (deterministic).
#include <cmath>

#include "common.hpp"

namespace sm {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

enum Epi : int {
  EPI_STORE_F32 = 0,   // y (f32) = acc
  EPI_STORE_BF16 = 1,  // y (bf16) = acc
  EPI_ADD_F32 = 2,     // y (f32) += acc          (residual stream)
  EPI_SWIGLU_BF16 = 3, // y (bf16)[m, j] = silu(acc[m, j]) * acc[m, F + j]
  EPI_SWIGLU_F16 = 4   // same, f16 output
};

constexpr bool is_swiglu(int e) { return e == EPI_SWIGLU_BF16 || e == EPI_SWIGLU_F16; }

__device__ inline h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }

// 8 signed nibbles of `w` times scale `s` -> f16 in k order [0,4,1,5,2,6,3,7].
__device__ inline h8 dequant_word(uint32_t w, h2 s) {
  w ^= 0x88888888u;  // two's complement -> offset binary (u = q + 8)
  const uint32_t w2 = w >> 8;
  const h2 k1032 = {(_Float16)-1032.f, (_Float16)-1032.f};
  const h2 k72 = {(_Float16)-72.f, (_Float16)-72.f};
  const h2 k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  h2 a = as_h2((w & 0x000F000Fu) | 0x64006400u) + k1032;        // q0, q4
  h2 b = as_h2((w & 0x00F000F0u) | 0x64006400u) * k16 + k72;    // q1, q5
  h2 c = as_h2((w2 & 0x000F000Fu) | 0x64006400u) + k1032;       // q2, q6
  h2 d = as_h2((w2 & 0x00F000F0u) | 0x64006400u) * k16 + k72;   // q3, q7
  a *= s; b *= s; c *= s; d *= s;
  return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// 8 bf16 activations (one 16-byte load, k..k+7) -> f16 in k order [0,4,1,5,2,6,3,7].
__device__ inline h8 act_frag(u32x4 v) {
  return h8{(_Float16)bf16lo(v.x), (_Float16)bf16lo(v.z), (_Float16)bf16hi(v.x),
            (_Float16)bf16hi(v.z), (_Float16)bf16lo(v.y), (_Float16)bf16lo(v.w),
            (_Float16)bf16hi(v.y), (_Float16)bf16hi(v.w)};
}

// 8 f16 activations (k..k+7) -> k order [0,4,1,5,2,6,3,7].
__device__ inline h8 act_frag_f16(h8 v) {
  return h8{v[0], v[4], v[1], v[5], v[2], v[6], v[3], v[7]};
}

__device__ inline float silu(float g) { return g / (1.f + __expf(-g)); }

struct Q4Args {
  const uint8_t* codes;    // [N, K/2]
  const uint16_t* scales;  // [N, K/128] bf16
  const void* x;           // [M, ldx] bf16 or f16
  void* y;                 // [M, ldy]
  int M, N, K;             // N = weight rows (for SWIGLU: 2F)
  int ldx, ldy;
  int ncols;               // logical output columns (N, or F for SWIGLU)
};

// MT: 16-row M blocks per wave; NB: 16-column N blocks per wave;
// KSPLIT: 1 = the 4 waves tile N (WG tile 16MT x 64NB), 4 = the 4 waves split
// the K groups of one 16MT x 16NB tile.
template <int MT, int NB, int KSPLIT, int EPI, bool XF16>
__global__ __launch_bounds__(256) void q4_gemm_kernel(Q4Args a) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int m0 = blockIdx.y * (16 * MT);
  const int wave_cols = 16 * NB;
  const int tile_cols = (KSPLIT == 1) ? 4 * wave_cols : wave_cols;
  const int c0 = blockIdx.x * tile_cols + ((KSPLIT == 1) ? wave * wave_cols : 0);
  const int ngroups = a.K / 128;
  const int half_cols = is_swiglu(EPI) ? wave_cols / 2 : wave_cols;
  // Weight row read by this lane for block b.
  int brow[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (is_swiglu(EPI)) {
      // first NB/2 blocks: gate columns, last NB/2: value columns (same j)
      const int col = c0 / 2 + (b % (NB / 2)) * 16 + j;  // logical h column
      brow[b] = (col < a.ncols) ? ((b < NB / 2) ? col : a.ncols + col) : -1;
    } else {
      const int col = c0 + b * 16 + j;
      brow[b] = (col < a.N) ? col : -1;
    }
  }
  (void)half_cols;
  f4 acc[MT][NB];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[mt][b] = f4{0.f, 0.f, 0.f, 0.f};

  // U k-groups of weights are loaded before any of them is consumed, so each
  // lane keeps U*NB 16-byte loads in flight (the M=1 GEMV is pure latency x
  // bandwidth: these loads are all the work there is).
  constexpr int U = (MT <= 2) ? 4 : 2;
  const int kg0 = (KSPLIT == 1) ? 0 : wave;
  for (int kb0 = kg0; kb0 < ngroups; kb0 += KSPLIT * U) {
    u32x4 wv[U][NB];
    h2 sc[U][NB];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kg = kb0 + u * KSPLIT;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (brow[b] >= 0 && kg < ngroups) {
          const uint8_t* p = a.codes + (size_t)brow[b] * (a.K / 2) + kg * 64 + g * 16;
          wv[u][b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
          const _Float16 s = (_Float16)bf16_to_f32(a.scales[(size_t)brow[b] * ngroups + kg]);
          sc[u][b] = h2{s, s};
        } else {
          wv[u][b] = u32x4{0u, 0u, 0u, 0u};
          sc[u][b] = h2{(_Float16)0.f, (_Float16)0.f};
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kg = kb0 + u * KSPLIT;
      if (kg >= ngroups) break;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        h8 bf[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) bf[b] = dequant_word(wv[u][b][s], sc[u][b]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int row = m0 + mt * 16 + j;
          h8 af = h8{0, 0, 0, 0, 0, 0, 0, 0};
          if (row < a.M) {
            const size_t xo = (size_t)row * a.ldx + kg * 128 + g * 32 + s * 8;
            if constexpr (XF16)
              af = act_frag_f16(*reinterpret_cast<const h8*>(static_cast<const _Float16*>(a.x) + xo));
            else
              af = act_frag(*reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.x) + xo));
          }
#pragma unroll
          for (int b = 0; b < NB; ++b)
            acc[mt][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[b], acc[mt][b], 0, 0, 0);
        }
      }
    }
  }

  if constexpr (KSPLIT > 1) {
    __shared__ f4 red[KSPLIT - 1][MT * NB][kWave];
    if (wave > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int b = 0; b < NB; ++b) red[wave - 1][mt * NB + b][lane] = acc[mt][b];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < KSPLIT - 1; ++w)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[mt][b] += red[w][mt * NB + b][lane];
  }

  // Epilogue: lane holds rows 4*g + r (r = 0..3) of column j of every block.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + mt * 16 + 4 * g + r;
      if (row >= a.M) continue;
      if constexpr (is_swiglu(EPI)) {
#pragma unroll
        for (int b = 0; b < NB / 2; ++b) {
          const int col = c0 / 2 + b * 16 + j;
          if (col < a.ncols) {
            const float h = silu(acc[mt][b][r]) * acc[mt][b + NB / 2][r];
            if constexpr (EPI == EPI_SWIGLU_F16)
              static_cast<_Float16*>(a.y)[(size_t)row * a.ldy + col] = (_Float16)h;
            else
              static_cast<uint16_t*>(a.y)[(size_t)row * a.ldy + col] = f32_to_bf16(h);
          }
        }
      } else {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int col = c0 + b * 16 + j;
          if (col >= a.N) continue;
          const size_t o = (size_t)row * a.ldy + col;
          const float v = acc[mt][b][r];
          if constexpr (EPI == EPI_STORE_F32) static_cast<float*>(a.y)[o] = v;
          else if constexpr (EPI == EPI_STORE_BF16) static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(v);
          else static_cast<float*>(a.y)[o] += v;
        }
      }
    }
  }
}

template <int MT, int NB, int KSPLIT, bool XF16>
int launch_q4_x(const Q4Args& a, int epi, hipStream_t st) {
  static_assert(NB % 2 == 0, "SwiGLU pairs gate/value blocks");
  const int wave_cols = 16 * NB;
  const int tile_cols = (KSPLIT == 1) ? 4 * wave_cols : wave_cols;
  const int logical_cols = is_swiglu(epi) ? 2 * a.ncols : a.N;
  dim3 grid((unsigned)ceil_div(logical_cols, tile_cols), (unsigned)ceil_div(a.M, 16 * MT));
  switch (epi) {
#define SM_Q4_EPI(E) \
    case E: q4_gemm_kernel<MT, NB, KSPLIT, E, XF16><<<grid, 256, 0, st>>>(a); break;
    SM_Q4_EPI(EPI_STORE_F32)
    SM_Q4_EPI(EPI_STORE_BF16)
    SM_Q4_EPI(EPI_ADD_F32)
    SM_Q4_EPI(EPI_SWIGLU_BF16)
    SM_Q4_EPI(EPI_SWIGLU_F16)
#undef SM_Q4_EPI
    default: set_error("sm_q4_matmul: unknown epilogue %d", epi); return SM_ERR_INVALID;
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

template <int MT, int NB, int KSPLIT>
int launch_q4(const Q4Args& a, int epi, bool xf16, hipStream_t st) {
  return xf16 ? launch_q4_x<MT, NB, KSPLIT, true>(a, epi, st)
              : launch_q4_x<MT, NB, KSPLIT, false>(a, epi, st);
}

// Picks the tile shape. Up to 256 rows (decode batches, GEMV) every wave owns
// 16 rows so the grid has M/16 row tiles; bigger M (prefill / recompute) uses
// 128-row tiles. When the grid would have fewer than 512 workgroups the four
// waves of a workgroup split K instead of N (more workgroups, same work).
int dispatch_q4(const Q4Args& a, int epi, bool xf16, hipStream_t st) {
  const int64_t logical_cols = is_swiglu(epi) ? 2 * (int64_t)a.ncols : a.N;
  const bool ksplit_ok = a.K >= 4 * 128;
  if (a.M <= 256) {
    const int64_t wgs = ceil_div(logical_cols, 128) * ceil_div(a.M, 16);
    if (wgs < 512 && ksplit_ok) return launch_q4<1, 2, 4>(a, epi, xf16, st);
    return launch_q4<1, 2, 1>(a, epi, xf16, st);
  }
  const int64_t wgs = ceil_div(logical_cols, 128) * ceil_div(a.M, 128);
  if (wgs < 512 && ksplit_ok) return launch_q4<8, 2, 4>(a, epi, xf16, st);
  return launch_q4<8, 2, 1>(a, epi, xf16, st);
}

// ----------------------------------------------------------- quantizer ---
// One wave per 128-element group; lane l owns elements 2l, 2l+1 (one byte).
__device__ inline float round_half_away(float v) {
  return v >= 0.f ? floorf(v + 0.5f) : -floorf(-v + 0.5f);
}

template <typename T>
__device__ inline float ld_val(const T* p, int64_t i);
template <> __device__ inline float ld_val<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ inline float ld_val<uint16_t>(const uint16_t* p, int64_t i) {
  return bf16_to_f32(p[i]);
}

template <typename T>
__global__ __launch_bounds__(256) void q4_quantize_kernel(const T* __restrict__ w, int64_t n,
                                                          uint8_t* __restrict__ codes,
                                                          uint16_t* __restrict__ scales,
                                                          int32_t* __restrict__ bad_scales) {
  const int64_t grp = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t ngroups = (n + 127) / 128;
  if (grp >= ngroups) return;
  const int64_t i0 = grp * 128 + 2 * lane;
  const float v0 = (i0 < n) ? ld_val(w, i0) : 0.f;
  const float v1 = (i0 + 1 < n) ? ld_val(w, i0 + 1) : 0.f;
  const float amax = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
  const uint16_t sb = f32_to_bf16(amax / 7.0f);
  const float s = bf16_to_f32(sb);
  int q0 = 0, q1 = 0;
  if (s > 0.f) {
    q0 = (int)fminf(fmaxf(round_half_away(v0 / s), -8.f), 7.f);
    q1 = (int)fminf(fmaxf(round_half_away(v1 / s), -8.f), 7.f);
  }
  if (i0 >= n) q0 = 0;
  if (i0 + 1 >= n) q1 = 0;
  codes[grp * 64 + lane] = (uint8_t)((q0 & 0xf) | ((q1 & 0xf) << 4));
  if (lane == 0) {
    scales[grp] = sb;
    // q*scale must be exact in f16: scale 0 or an f16 normal with 8*scale finite.
    const bool ok = (s == 0.f) || (s >= 6.103515625e-05f && s * 8.f <= 65504.f);
    if (!ok && bad_scales) atomicAdd(bad_scales, 1);
  }
}

}  // namespace
}  // namespace sm

extern "C" int sm_q4_quantize(const void* w, int dtype, int64_t n, uint8_t* codes,
                              uint16_t* scales, int32_t* bad_scales, void* stream) {
  using namespace sm;
  SM_REQUIRE(w && codes && scales, "sm_q4_quantize: null buffer");
  SM_REQUIRE(dtype == SM_F32 || dtype == SM_BF16, "sm_q4_quantize: dtype must be f32 or bf16");
  SM_REQUIRE(n > 0, "packed tensor is empty");
  const int64_t groups = ceil_div(n, 128);
  const unsigned blocks = (unsigned)ceil_div(groups, 4);
  if (dtype == SM_F32)
    q4_quantize_kernel<float><<<blocks, 256, 0, as_stream(stream)>>>(
        static_cast<const float*>(w), n, codes, scales, bad_scales);
  else
    q4_quantize_kernel<uint16_t><<<blocks, 256, 0, as_stream(stream)>>>(
        static_cast<const uint16_t*>(w), n, codes, scales, bad_scales);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_q4_matmul(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                            const void* x, int x_dtype, int64_t M, int64_t ldx, void* y,
                            int64_t ldy, int epilogue, void* stream) {
  using namespace sm;
  SM_REQUIRE(codes && scales && x && y, "sm_q4_matmul: null buffer");
  SM_REQUIRE(K > 0 && K % 128 == 0, "sm_q4_matmul: K=%lld must be a positive multiple of 128",
             (long long)K);
  SM_REQUIRE(N > 0 && N <= 0x7fffffff && K <= 0x7fffffff, "sm_q4_matmul: bad N");
  SM_REQUIRE(M >= 0 && M <= 0x7fffffff, "sm_q4_matmul: bad M");
  SM_REQUIRE(ldx >= K && ldx % 8 == 0, "sm_q4_matmul: ldx must be >= K and a multiple of 8");
  SM_REQUIRE(reinterpret_cast<uintptr_t>(codes) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(x) % 16 == 0,
             "sm_q4_matmul: codes and x must be 16-byte aligned");
  SM_REQUIRE(epilogue >= EPI_STORE_F32 && epilogue <= EPI_SWIGLU_F16,
             "sm_q4_matmul: unknown epilogue %d", epilogue);
  SM_REQUIRE(x_dtype == SM_BF16 || x_dtype == SM_F16, "sm_q4_matmul: x must be bf16 or f16");
  const int64_t ncols = is_swiglu(epilogue) ? N / 2 : N;
  SM_REQUIRE(!is_swiglu(epilogue) || N % 2 == 0, "sm_q4_matmul: SwiGLU needs even N");
  SM_REQUIRE(ldy >= ncols, "sm_q4_matmul: ldy < output columns");
  if (M == 0) return SM_OK;
  Q4Args a{codes, scales, x, y, (int)M, (int)N, (int)K, (int)ldx, (int)ldy, (int)ncols};
  return dispatch_q4(a, epilogue, x_dtype == SM_F16, as_stream(stream));
}
