// Shared host/device helpers for the summa_amd HIP library (gfx950 only).
//
// Status convention of every exported entry point: 0 on success, a negative
// sm_status on failure, with a message retrievable via sm_last_error() from the
// calling thread. No entry point aborts or throws across the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/summa_amd.h"

namespace sm {

// ---------------------------------------------------------------- errors ---
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define SM_REQUIRE(cond, ...)                \
  do {                                       \
    if (!(cond)) {                           \
      ::sm::set_error(__VA_ARGS__);          \
      return SM_ERR_INVALID;                 \
    }                                        \
  } while (0)

#define SM_HIP(call)                                                         \
  do {                                                                       \
    hipError_t _e = (call);                                                  \
    if (_e != hipSuccess) {                                                  \
      ::sm::set_error("%s failed: %s (%s:%d)", #call, hipGetErrorString(_e), \
                      __FILE__, __LINE__);                                   \
      return SM_ERR_HIP;                                                     \
    }                                                                        \
  } while (0)

// Checks the launch that was just enqueued.
#define SM_LAUNCH_CHECK() SM_HIP(hipGetLastError())

#define SM_TRY(expr)              \
  do {                            \
    int _s = (expr);              \
    if (_s != SM_OK) return _s;   \
  } while (0)

// Native 16-byte vector (usable with the nontemporal load/store builtins).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------------ bf16 ---
// bf16 values travel as raw uint16_t bit patterns; conversions are the IEEE
// truncation of fp32 with round-to-nearest-even.
__host__ __device__ inline float bf16_to_f32(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
    return static_cast<uint16_t>((u >> 16) | 0x40u);  // quiet NaN
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Two fp32 values -> one packed bf16 pair (a in the low half), round to
// nearest even: a single v_cvt_pk_bf16_f32 on gfx950, which gives the same
// bits as f32_to_bf16 for every one of the 2^32 inputs (NaNs included;
// checked exhaustively on the device).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t pack_bf16x2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Low / high bf16 halves of a packed 32-bit word, as fp32.
__device__ inline float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// -------------------------------------------------------- wave reductions ---
constexpr int kWave = 64;

// Wave-wide reductions (call with the whole wave active). Within each row of
// 16 lanes four DPP steps combine lanes i^1, i^2 (quad_perm), 7-i (row half
// mirror) and 15-i (row mirror); each step is symmetric, so every lane of a
// row holds the same row value. The four row values are then read into scalar
// registers and combined in a fixed order, (r0 . r1) . (r2 . r3), so every lane
// returns the same bits. VALU work with no LDS round trips: the ds_bpermute
// butterfly this replaces cost six dependent LDS trips per reduction.
template <int CTRL>
__device__ inline float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ inline float lane_f32(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
constexpr int kDppXor1 = 0xB1;       // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;       // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppMirror>(v));
  return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

__device__ inline float wave_sum(float v) {
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppHalfMirror>(v);
  v += dpp_f32<kDppMirror>(v);
  return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

__device__ inline double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// Merge two online-softmax partials (max m, sum of exp(x - m) s). Empty
// partials carry (-inf, 0) and merge as exact zeros.
__device__ inline void lse_merge(float& m, float& s, float m2, float s2) {
  float mm = fmaxf(m, m2);
  float a = (s > 0.f) ? s * __expf(m - mm) : 0.f;
  float b = (s2 > 0.f) ? s2 * __expf(m2 - mm) : 0.f;
  m = mm;
  s = a + b;
}

__device__ inline void wave_lse(float& m, float& s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float m2 = __shfl_xor(m, o, kWave);
    float s2 = __shfl_xor(s, o, kWave);
    lse_merge(m, s, m2, s2);
  }
}

// ------------------------------------------------------------ counter RNG ---
// SplitMix64 finaliser over a (seed, stream, counter) key. Stateless, so any
// thread can draw the value for any (row, step, column) without coordination.
__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__host__ __device__ inline uint64_t rng_key(uint64_t seed, uint64_t stream, uint64_t counter) {
  return mix64(mix64(seed + 0x9e3779b97f4a7c15ull * (stream + 1)) ^ (counter * 0xd1b54a32d192ed03ull));
}

// Uniform in (0, 1): 24 random bits, offset by half a step so 0 and 1 never occur.
__host__ __device__ inline float u01(uint64_t bits) {
  return (static_cast<float>(bits >> 40) + 0.5f) * (1.0f / 16777216.0f);
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ------------------------------------------------- prepared Q4G128 layout ---
// Device weights use a tiled copy of the row-major Q4G128 codec: 16 weight
// rows x one 128-element group form a 1 KB tile (row r of the tile at byte
// 64*r), tiles ordered [row_block][group]. One wave instruction in which lane
// (r = lane%16, c = lane/16) loads 16 bytes at 64*r + 16*c reads the whole tile
// contiguously. Scales follow the same order: 16 bf16 per tile.
__host__ __device__ inline size_t q4t_code_offset(int64_t row, int64_t group, int64_t ngroups) {
  return ((size_t)(row >> 4) * ngroups + group) * 1024 + (size_t)(row & 15) * 64;
}
__host__ __device__ inline size_t q4t_scale_index(int64_t row, int64_t group, int64_t ngroups) {
  return ((size_t)(row >> 4) * ngroups + group) * 16 + (size_t)(row & 15);
}
__host__ __device__ inline int64_t q4t_rows(int64_t n) { return ceil_div(n, 16) * 16; }

// Inside the prepared layout each 32-bit word (8 consecutive k of one row)
// stores offset-binary nibbles u = q + 8, the even k in nibbles 0-3 and the
// odd k in nibbles 4-7, so that the magic-exponent unpack below yields the
// eight values in natural k order with no extra shuffles.
__host__ __device__ inline uint32_t q4_prepare_word(uint32_t w) {
  uint32_t out = 0;
  for (int k = 0; k < 8; ++k) {
    const uint32_t u = ((w >> (4 * k)) & 0xfu) ^ 0x8u;
    const int dst = (k & 1) ? 4 + (k >> 1) : (k >> 1);
    out |= u << (4 * dst);
  }
  return out;
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ inline h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }

// fp32 -> f16 pair (the SM_F16X2 activation format): hi = f16(x),
// lo = f16(x - hi), so hi + lo carries x to about 22 significant bits.
__device__ inline void split_f16(float x, _Float16& hi, _Float16& lo) {
  // Both halves must come from one rounded f32 value. Without the empty asm
  // the compiler may fold the multiply that produced x into the f16
  // conversions (v_fma_mix*), rounding hi from the f32 product for the store
  // but from the exact product for the subtraction: when the f32 rounding lands
  // on an f16 midpoint the pair is then off by one f16 ulp (~1 value in 8000).
  asm volatile("" : "+v"(x));
  hi = (_Float16)x;
  lo = (_Float16)(x - (float)hi);
}

// The RMSNorm of one row of D = 256 * V columns written as f16 pairs, with
// one workgroup per row: wave i holds float4 i * 64 + lane (v) and gamma (g).
// The squares meet in LDS (sq [V][64]) so that wave 0 sums them in the order
// of a one-wave-per-row norm (lane l over float4s l, 64 + l, ... then one wave
// reduction); then x / rms * gamma, split into hi | lo halves of the row.
// pair_out (optional): the four values as the pair holds them, hi + lo in f32
// (what a consumer of the pair row reads back).
template <int V>
__device__ inline void row_rmsnorm_pair(const float4& v, const float4& g, float eps,
                                        float4 (&sq)[V][64], float& rms_s, _Float16* row,
                                        float* pair_out = nullptr) {
  constexpr int D = 256 * V;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int c4 = wave * 64 + lane;
  sq[wave][lane] = v;
  __syncthreads();
  if (wave == 0) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float4 t = sq[i][lane];
      ss = fmaf(t.w, t.w, fmaf(t.z, t.z, fmaf(t.y, t.y, fmaf(t.x, t.x, ss))));
    }
    ss = wave_sum(ss);
    if (lane == 0) rms_s = sqrtf(ss / (float)D + eps);
  }
  __syncthreads();
  const float rms = rms_s;
  const float o[4] = {v.x / rms * g.x, v.y / rms * g.y, v.z / rms * g.z, v.w / rms * g.w};
  _Float16 hi[4], lo[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) split_f16(o[e], hi[e], lo[e]);
  *reinterpret_cast<h4*>(row + 4 * c4) = h4{hi[0], hi[1], hi[2], hi[3]};
  *reinterpret_cast<h4*>(row + D + 4 * c4) = h4{lo[0], lo[1], lo[2], lo[3]};
  if (pair_out) {
#pragma unroll
    for (int e = 0; e < 4; ++e) pair_out[e] = (float)hi[e] + (float)lo[e];
  }
}

// One prepared word -> its 8 codes q in natural k order as f16. Each 16-bit
// half becomes 1024 + u (or 1024 + 16u) by OR-ing the nibble into the
// mantissa of 0x6400; one packed add / fma removes the bias. 9 VALU ops: each
// mask-and-OR is one v_and_or_b32, which (VOP3 on this architecture) takes no
// literal and at most one scalar operand, so the 0x6400 magic is handed over in
// a vector register (an empty-effect v_mov the compiler hoists and shares);
// with both constants as literals it emitted a separate v_and and v_or (13.5
// VALU per word).
__device__ inline uint32_t q4_magic() {
  uint32_t m;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(m));
  return m;
}
__device__ inline h8 q4_unpack(uint32_t w) {
  const uint32_t magic = q4_magic();
  const uint32_t w2 = w >> 8;
  const h2 k1032 = {(_Float16)-1032.f, (_Float16)-1032.f};
  const h2 k72 = {(_Float16)-72.f, (_Float16)-72.f};
  const h2 k16 = {(_Float16)0.0625f, (_Float16)0.0625f};
  const h2 a = as_h2((w & 0x000F000Fu) | magic) + k1032;       // k0, k1
  const h2 b = as_h2((w & 0x00F000F0u) | magic) * k16 + k72;   // k2, k3
  const h2 c = as_h2((w2 & 0x000F000Fu) | magic) + k1032;      // k4, k5
  const h2 d = as_h2((w2 & 0x00F000F0u) | magic) * k16 + k72;  // k6, k7
  return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Same, times the group scale: q * scale is exact in f16 while the scale is an
// f16 normal (<= 11 significant bits), which the quantizer checks.
__device__ inline h8 q4_unpack_scaled(uint32_t w, _Float16 s) {
  h8 v = q4_unpack(w);
  return v * s;
}

}  // namespace sm
