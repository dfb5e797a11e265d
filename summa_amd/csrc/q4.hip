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
// MI355X design: v_mfma_f32_16x16x32_f16. The kernels read the prepared tiled
// copy of the codec (sm_q4_pack; common.hpp q4t_*), in which one 16-row x
// 128-group MFMA block is a contiguous 1 KB: lane (j = l%16, g = l/16) loads
// the 16-byte chunk = 32 consecutive k of weight row n0+j, so each wave load
// instruction streams 1 KB contiguously (the row-major codec would make it 16
// 64-byte pieces 1 KB apart). The prepared words hold offset-binary nibbles in
// an order that unpacks to natural k order, so each of the chunk's four 32-bit
// words becomes the lane's 8 f16 B values of one MFMA step in 9 VALU ops (0x6400
// magic exponent, common.hpp q4_unpack), and f16 activations feed the A operand
// with no conversion at all. The small-M kernel accumulates each group's four
// k-steps unscaled and applies the group scale with one FMA per output; the
// large-M kernel folds the scale into B (exact in f16 for an f16-normal scale,
// which sm_q4_quantize checks). Lanes of rows >= M read a clamped valid row
// and feed only output rows that are not stored. For
// tiny N the four waves of a workgroup split the K groups and merge their
// accumulators through LDS in a fixed order (deterministic).
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "moe_plan.hpp"
#include "q4_internal.hpp"

namespace sm {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

enum Epi : int {
  EPI_STORE_F32 = 0,   // y (f32) = acc
  EPI_STORE_BF16 = 1,  // y (bf16) = acc
  EPI_ADD_F32 = 2,     // y (f32) += acc          (residual stream)
  EPI_SWIGLU_BF16 = 3, // y (bf16)[m, j] = silu(acc[m, j]) * acc[m, F + j]
  EPI_SWIGLU_F16 = 4,  // same, f16 output
  EPI_SWIGLU_F16X2 = 5 // same, f16 pair (hi at [m, j], lo at [m, F + j])
};

constexpr bool is_swiglu(int e) { return e >= EPI_SWIGLU_BF16 && e <= EPI_SWIGLU_F16X2; }

// Activation input modes (template parameter XT of the kernels).
enum XMode : int { X_BF16 = 0, X_F16 = 1, X_F16X2 = 2 };

inline int xmode_of(int dtype) {
  return dtype == SM_BF16 ? X_BF16 : dtype == SM_F16 ? X_F16 : dtype == SM_F16X2 ? X_F16X2 : -1;
}

// 8 bf16 activations (one 16-byte load, k..k+7) -> f16, natural order.
__device__ inline h8 act_frag(u32x4 v) {
  return h8{(_Float16)bf16lo(v.x), (_Float16)bf16hi(v.x), (_Float16)bf16lo(v.y),
            (_Float16)bf16hi(v.y), (_Float16)bf16lo(v.z), (_Float16)bf16hi(v.z),
            (_Float16)bf16lo(v.w), (_Float16)bf16hi(v.w)};
}

__device__ inline float silu(float g) { return g / (1.f + __expf(-g)); }

struct Q4Args {
  const uint8_t* codes;    // [N, K/2]
  const uint16_t* scales;  // [N, K/128] bf16
  const void* x;           // [M, ldx] bf16, f16 or f16 pairs (lo at +K)
  void* y;                 // [M, ldy]
  int M, N, K;             // N = weight rows (for SWIGLU: 2F)
  int ldx, ldy;
  int ncols;               // logical output columns (N, or F for SWIGLU)
  // Grouped (MoE) mode when tiles != nullptr: workgroup row tile y is tile
  // (expert e, first row r) of the route plan; its rows are sorted positions
  // goff[e] + r .. goff[e+1]-1, the A row of position p is rowidx[p] (or p),
  // and expert e's weights start at codes + e*cstride, scales + e*sstride.
  const int32_t* tiles = nullptr;
  const int32_t* ntiles = nullptr;
  const int32_t* goff = nullptr;
  const int32_t* rowidx = nullptr;
  size_t cstride = 0, sstride = 0;
  // qkv projection + RoPE + KV-cache append (q4_grouped_lds_kernel EPI 6,
  // dense mode): row = s*rope_L + i sits at position pos0[s] + i; columns are
  // [q | k | v] heads of hd (as q4_gemm_bl.hip's EPI 6)
  const float2* rope = nullptr;
  const int32_t* pos0 = nullptr;
  int rope_L = 0, cap = 0, H = 0, KVH = 0, hd = 0;
  _Float16 *q_out = nullptr, *kc = nullptr, *vc = nullptr;
  // split-K (q4_grouped_lds_kernel dense mode): blockIdx.z = split z covers K
  // groups [z*gper, min(K/128, (z+1)*gper)) and writes its f32 partial tile to
  // part[z][row][logical column]; splitk_reduce sums the splits in order
  float* part = nullptr;
  int gper = 0;
};

// One workgroup = 16 rows (M tile) x its column tile. NB: 16-column blocks per
// wave; KSPLIT: 1 = the 4 waves tile N (workgroup tile 16 x 64NB), 4 = the 4
// waves split the K groups of one 16 x 16NB tile and merge in LDS.
// Per wave, kU K groups of weights are requested before any is consumed, and
// the activation fragments of the next group are fetched while the current
// one is multiplied. (For the narrow M=1 GEMV 4 groups measured best: with
// one 16-column block per wave there are enough waves in flight already.)

template <int NB, int KSPLIT, int EPI, int XT, int kU>
__global__ __launch_bounds__(256) void q4_gemm_kernel(Q4Args a) {
  constexpr int NA = (XT == X_F16X2) ? 2 : 1;  // A fragments per k-step (hi, lo)
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  int m0 = blockIdx.y * 16;
  int mlim = a.M;  // rows [m0, mlim) are valid for this workgroup
  const uint8_t* codes = a.codes;
  const uint16_t* scales = a.scales;
  if (a.tiles) {
    if ((int)blockIdx.y >= a.ntiles[0]) return;  // uniform per workgroup
    const int e = a.tiles[2 * blockIdx.y];
    m0 = a.goff[e] + a.tiles[2 * blockIdx.y + 1];
    mlim = a.goff[e + 1];
    codes += (size_t)e * a.cstride;
    scales += (size_t)e * a.sstride;
  }
  const int wave_cols = 16 * NB;
  const int tile_cols = (KSPLIT == 1) ? 4 * wave_cols : wave_cols;
  const int c0 = blockIdx.x * tile_cols + ((KSPLIT == 1) ? wave * wave_cols : 0);
  const int ngroups = a.K / 128;
  // Weight row read by this lane for block b.
  int brow[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if constexpr (is_swiglu(EPI)) {
      // first NB/2 blocks: gate columns, last NB/2: value columns (same j)
      const int col = c0 / 2 + (b % (NB / 2)) * 16 + j;  // logical h column
      brow[b] = (col < a.ncols) ? ((b < NB / 2) ? col : a.ncols + col) : -1;
    } else {
      const int col = c0 + b * 16 + j;
      brow[b] = (col < a.N) ? col : -1;
    }
  }
  // All loads below are branch-free (clamped addresses, zeroed afterwards):
  // loads inside divergent branches make the compiler wait on each one, which
  // serialises the round trips this kernel exists to overlap.
  const int prow = min(m0 + j, mlim - 1);  // activation row this lane feeds to the A operand
  const int arow = a.rowidx ? a.rowidx[prow] : prow;
  auto load_act = [&](int kg, h8 (&af)[NA][4]) {
    const int kc = min(kg, ngroups - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const size_t xo = (size_t)arow * a.ldx + kc * 128 + g * 32 + s * 8;
      if constexpr (XT == X_BF16) {
        af[0][s] = act_frag(*reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.x) + xo));
      } else {
        af[0][s] = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(a.x) + xo);
        if constexpr (NA == 2)
          af[1][s] = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(a.x) + xo + a.K);
      }
    }
  };
  int brow_c[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) brow_c[b] = brow[b] >= 0 ? brow[b] : 0;

  f4 acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = f4{0.f, 0.f, 0.f, 0.f};

  const int kg0 = (KSPLIT == 1) ? 0 : wave;
  h8 an[NA][4];
  load_act(kg0, an);
  for (int kb0 = kg0; kb0 < ngroups; kb0 += KSPLIT * kU) {
    u32x4 wv[kU][NB];
    uint16_t sraw[kU][NB];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int kc = min(kb0 + u * KSPLIT, ngroups - 1);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        wv[u][b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            codes + q4t_code_offset(brow_c[b], kc, ngroups) + g * 16));
        sraw[u][b] = scales[q4t_scale_index(brow_c[b], kc, ngroups)];
      }
    }
    // keep the whole batch of loads ahead of the math (the scheduler would
    // otherwise sink each load next to its first use)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int kg = kb0 + u * KSPLIT;
      if (kg >= ngroups) break;
      // Lanes of rows past mlim hold a clamped valid row: they only feed MFMA
      // output rows that the epilogue never stores (each D row depends on its
      // A row alone), so no zeroing is needed.
      h8 af[NA][4];
#pragma unroll
      for (int h = 0; h < NA; ++h)
#pragma unroll
        for (int s = 0; s < 4; ++s) af[h][s] = an[h][s];
      load_act(kg + KSPLIT, an);  // next group's activations, in flight during this one
      // Per block: the group's 4 k-steps accumulate unscaled codes, then one
      // FMA per output applies the group scale (cheaper than scaling B). f16
      // pairs take a second MFMA on the same unpacked codes for the lo half.
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        f4 t = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const h8 bq = q4_unpack(wv[u][b][s]);
          t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[0][s], bq, t, 0, 0, 0);
          if constexpr (NA == 2) t = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[1][s], bq, t, 0, 0, 0);
        }
        const float sc = brow[b] >= 0 ? bf16_to_f32(sraw[u][b]) : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[b][r] = fmaf(t[r], sc, acc[b][r]);
      }
    }
  }

  if constexpr (KSPLIT > 1) {
    __shared__ f4 red[KSPLIT - 1][NB][kWave];
    if (wave > 0) {
#pragma unroll
      for (int b = 0; b < NB; ++b) red[wave - 1][b][lane] = acc[b];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < KSPLIT - 1; ++w)
#pragma unroll
      for (int b = 0; b < NB; ++b) acc[b] += red[w][b][lane];
  }

  // Epilogue: lane holds rows 4*g + r (r = 0..3) of column j of every block.
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = m0 + 4 * g + r;
    if (row >= mlim) continue;
    if constexpr (is_swiglu(EPI)) {
#pragma unroll
      for (int b = 0; b < NB / 2; ++b) {
        const int col = c0 / 2 + b * 16 + j;
        if (col < a.ncols) {
          const float h = silu(acc[b][r]) * acc[b + NB / 2][r];
          if constexpr (EPI == EPI_SWIGLU_F16X2) {
            _Float16 hi, lo;
            split_f16(h, hi, lo);
            static_cast<_Float16*>(a.y)[(size_t)row * a.ldy + col] = hi;
            static_cast<_Float16*>(a.y)[(size_t)row * a.ldy + a.ncols + col] = lo;
          } else if constexpr (EPI == EPI_SWIGLU_F16)
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
        const float v = acc[b][r];
        if constexpr (EPI == EPI_STORE_F32) static_cast<float*>(a.y)[o] = v;
        else if constexpr (EPI == EPI_STORE_BF16) static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(v);
        else static_cast<float*>(a.y)[o] += v;
      }
    }
  }
}

// Grouped (MoE) decode: the route plan's 16-row tiles with few rows each and
// wide expert matrices. One workgroup = 8 waves x 16*NB columns of one plan
// tile. q4_gemm_kernel's four waves each load the tile's activation rows
// themselves, so at decode size those loads are 2/3 of the memory
// instructions and the texture addresser, not HBM, sets the pace (~1.6 TB/s of
// expert weights at config[4]). Here every K group's activation tile (16 rows x
// 128 k, both halves of f16 pairs) is loaded once per workgroup, one 16-byte
// chunk per thread, into one of two LDS buffers (one barrier per group), and
// each wave reads its A fragments from LDS; weight groups stay register-direct
// and double-buffered. Per block and group the MFMA sequence and the scale
// FMA are q4_gemm_kernel's, so the results are identical.
// Dense mode (tiles == nullptr): row tile y = rows 16y .. 16y+15 of M. Measured
// faster than the batch kernel for decode batches (M <= 256) with K <= 2048 and
// 2k-8k output columns (config[2] qkv 27 -> 18 us, o 19 -> 16 us; config[1]
// qkv 12 -> 10 us): its 64 x 64 tiles re-read every activation row once per
// 64 columns, here once per 256. EPI 2 adds into y; EPI 6 is the qkv
// projection with RoPE and the KV-cache append (q4_gemm_bl.hip's EPI 6).
template <int NB, int EPI, int XT>
__global__ __launch_bounds__(512) void q4_grouped_lds_kernel(Q4Args a) {
  constexpr int NA = (XT == X_F16X2) ? 2 : 1;
  constexpr int AP = NA * 128 + 8;      // LDS row (f16): hi | lo | pad
  constexpr int STG = 16 * NA * 16;     // 16-byte chunks per group tile
  __shared__ __attribute__((aligned(16))) _Float16 As[2][16 * AP];
  int m0, mlim = a.M;
  const uint8_t* codes = a.codes;
  const uint16_t* scales = a.scales;
  if (a.tiles) {
    if ((int)blockIdx.y >= a.ntiles[0]) return;  // uniform per workgroup
    const int e = a.tiles[2 * blockIdx.y];
    m0 = a.goff[e] + a.tiles[2 * blockIdx.y + 1];
    mlim = a.goff[e + 1];
    codes += (size_t)e * a.cstride;
    scales += (size_t)e * a.sstride;
  } else {
    m0 = (int)blockIdx.y * 16;
  }
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int c0 = (int)blockIdx.x * 8 * 16 * NB + wave * 16 * NB;
  const int ngroups = a.K / 128;
  const int g0 = a.part ? (int)blockIdx.z * a.gper : 0;  // host: g0 < g1
  const int g1 = a.part ? min(ngroups, g0 + a.gper) : ngroups;
  int brow[NB], brow_c[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if constexpr (is_swiglu(EPI)) {
      const int col = c0 / 2 + (b % (NB / 2)) * 16 + j;
      brow[b] = (col < a.ncols) ? ((b < NB / 2) ? col : a.ncols + col) : -1;
    } else {
      const int col = c0 + b * 16 + j;
      brow[b] = (col < a.N) ? col : -1;
    }
    brow_c[b] = brow[b] >= 0 ? brow[b] : 0;
  }
  // staging: thread t < STG copies chunk c of half h of tile row `srow`
  const int t = threadIdx.x;
  const bool stager = t < STG;
  const int srow = t / (NA * 16), sh = (t / 16) % NA, sc16 = t % 16;
  const int sprow = min(m0 + srow, mlim - 1);  // rows past the tile repeat a valid row
  const int sarow = a.rowidx ? a.rowidx[sprow] : sprow;
  const size_t sxo = (size_t)sarow * a.ldx + (size_t)sh * a.K + sc16 * 8;
  const int sdst = srow * AP + sh * 128 + sc16 * 8;
  auto aload = [&](int kg) {
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (stager) {
      const size_t xo = sxo + (size_t)min(kg, g1 - 1) * 128;
      if constexpr (XT == X_BF16) {
        const h8 f = act_frag(*reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.x) + xo));
        v = __builtin_bit_cast(u32x4, f);
      } else {
        v = *reinterpret_cast<const u32x4*>(static_cast<const _Float16*>(a.x) + xo);
      }
    }
    return v;
  };
  auto astore = [&](int buf, const u32x4& v) {
    if (stager) *reinterpret_cast<u32x4*>(&As[buf][sdst]) = v;
  };
  auto wload = [&](int kg, u32x4 (&w)[NB], uint16_t (&sr)[NB]) {
    const int kc = min(kg, g1 - 1);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      w[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          codes + q4t_code_offset(brow_c[b], kc, ngroups) + g * 16));
      sr[b] = scales[q4t_scale_index(brow_c[b], kc, ngroups)];
    }
  };
  f4 acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = f4{0.f, 0.f, 0.f, 0.f};
  // EPI 2 / 6 operands that do not depend on the product, loaded before the
  // main loop so their latency hides behind it: y for the residual add; the
  // positions and (cos, sin) pairs for RoPE (even lanes own pairs (e, e+1))
  float yv[NB][4];
  int slot_b[NB], e_b[NB], srow_q[4], prow_q[4];
  float2 csr[4][NB];
  if constexpr (EPI == EPI_ADD_F32) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = min(m0 + 4 * g + r, mlim - 1), col = min(c0 + b * 16 + j, a.N - 1);
        yv[b][r] = static_cast<const float*>(a.y)[(size_t)row * a.ldy + col];
      }
  }
  if constexpr (EPI == 6) {
    const int hd_shift = __builtin_ctz(a.hd);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int col = c0 + b * 16 + j;
      slot_b[b] = col < a.N ? (col >> hd_shift) : -1;
      e_b[b] = col & (a.hd - 1);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + 4 * g + r;
      const int rc = min(row, mlim - 1);
      const int sq = (a.rope_L == 1) ? rc : rc / a.rope_L;
      const int pos = a.pos0[sq] + (rc - sq * a.rope_L);
      srow_q[r] = sq;
      prow_q[r] = (row < mlim && pos >= 0 && pos < a.cap) ? pos : -1;
      const float2* rrow = a.rope + (size_t)max(prow_q[r], 0) * (a.hd / 2);
#pragma unroll
      for (int b = 0; b < NB; ++b) csr[r][b] = rrow[e_b[b] >> 1];
    }
  }
  auto group = [&](int kg, const u32x4 (&w)[NB], const uint16_t (&sr)[NB]) {
    const _Float16* ab = &As[(kg - g0) & 1][j * AP + g * 32];
    h8 af[NA][4];
#pragma unroll
    for (int h = 0; h < NA; ++h)
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) af[h][s4] = *reinterpret_cast<const h8*>(ab + h * 128 + s4 * 8);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      f4 tt = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4) {
        const h8 bq = q4_unpack(w[b][s4]);
        tt = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[0][s4], bq, tt, 0, 0, 0);
        if constexpr (NA == 2) tt = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[1][s4], bq, tt, 0, 0, 0);
      }
      const float scl = brow[b] >= 0 ? bf16_to_f32(sr[b]) : 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[b][r] = fmaf(tt[r], scl, acc[b][r]);
    }
  };
  // prologue: group 0's activations in LDS, weight groups 0 (and 1 below) in flight
  u32x4 w0[NB], w1[NB];
  uint16_t s0[NB], s1[NB];
  u32x4 av = aload(g0);
  wload(g0, w0, s0);
  astore(0, av);
  // step kg: issue group kg+1's activations and weights, barrier (group kg's
  // tile is in LDS), math of group kg, then group kg+1's tile into the other
  // buffer (last read in step kg-1, before this step's barrier); buffers by
  // kg - g0
  for (int kg = g0; kg < g1; kg += 2) {
    av = aload(kg + 1);
    wload(kg + 1, w1, s1);
    __syncthreads();
    group(kg, w0, s0);
    astore((kg + 1 - g0) & 1, av);
    if (kg + 1 >= g1) break;
    av = aload(kg + 2);
    wload(kg + 2, w0, s0);
    __syncthreads();
    group(kg + 1, w1, s1);
    astore((kg - g0) & 1, av);
  }
  if (a.part) {  // split-K partial tile, logical columns (uniform branch)
    const int lc_total = is_swiglu(EPI) ? 2 * a.ncols : a.N;
    float* pp = a.part + (size_t)blockIdx.z * a.M * lc_total;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + 4 * g + r;
      if (row >= mlim) continue;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        int lc;
        if constexpr (is_swiglu(EPI)) {
          const int hcol = c0 / 2 + (b % (NB / 2)) * 16 + j;
          if (hcol >= a.ncols) continue;
          lc = (b < NB / 2) ? hcol : a.ncols + hcol;
        } else {
          lc = c0 + b * 16 + j;
          if (lc >= a.N) continue;
        }
        pp[(size_t)row * lc_total + lc] = acc[b][r];
      }
    }
    return;
  }
  // epilogue (rows 4g + r, as q4_gemm_kernel)
  if constexpr (EPI == 6) {
    // RoPE pairs (2p, 2p+1) are adjacent columns, i.e. lanes j and j^1 of the
    // same rows: swap partners before any lane-dependent branch
    f4 partner[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) partner[b][r] = __shfl_xor(acc[b][r], 1, kWave);
    if ((j & 1) != 0) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pos = prow_q[r];
      if (pos < 0) continue;
      const int row = m0 + 4 * g + r, sq = srow_q[r];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int slot = slot_b[b], e = e_b[b];
        if (slot < 0) continue;
        const float va = acc[b][r], vb = partner[b][r];  // columns e, e+1
        h2 out;
        _Float16* dst;
        if (slot >= a.H + a.KVH) {  // value: no rotation
          out = h2{(_Float16)va, (_Float16)vb};
          dst = a.vc + (((size_t)sq * a.KVH + (slot - a.H - a.KVH)) * a.cap + pos) * a.hd + e;
        } else {
          const float2 c = csr[r][b];
          out = h2{(_Float16)(va * c.x - vb * c.y), (_Float16)(vb * c.x + va * c.y)};
          dst = (slot < a.H) ? a.q_out + ((size_t)row * a.H + slot) * a.hd + e
                             : a.kc + (((size_t)sq * a.KVH + (slot - a.H)) * a.cap + pos) * a.hd + e;
        }
        *reinterpret_cast<h2*>(dst) = out;
      }
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = m0 + 4 * g + r;
    if (row >= mlim) continue;
    if constexpr (is_swiglu(EPI)) {
#pragma unroll
      for (int b = 0; b < NB / 2; ++b) {
        const int col = c0 / 2 + b * 16 + j;
        if (col < a.ncols) {
          const float hv = silu(acc[b][r]) * acc[b + NB / 2][r];
          if constexpr (EPI == EPI_SWIGLU_F16X2) {
            _Float16 hi, lo;
            split_f16(hv, hi, lo);
            static_cast<_Float16*>(a.y)[(size_t)row * a.ldy + col] = hi;
            static_cast<_Float16*>(a.y)[(size_t)row * a.ldy + a.ncols + col] = lo;
          } else if constexpr (EPI == EPI_SWIGLU_F16)
            static_cast<_Float16*>(a.y)[(size_t)row * a.ldy + col] = (_Float16)hv;
          else
            static_cast<uint16_t*>(a.y)[(size_t)row * a.ldy + col] = f32_to_bf16(hv);
        }
      }
    } else {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int col = c0 + b * 16 + j;
        if (col >= a.N) continue;
        const size_t o = (size_t)row * a.ldy + col;
        if constexpr (EPI == EPI_STORE_F32) static_cast<float*>(a.y)[o] = acc[b][r];
        else if constexpr (EPI == EPI_ADD_F32) static_cast<float*>(a.y)[o] = yv[b][r] + acc[b][r];
        else static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(acc[b][r]);
      }
    }
  }
}

// Dense decode batches with thick waves: q4_grouped_lds_kernel's scheme (each
// K group's activation tile staged once per workgroup into LDS; weight codes
// register-direct per wave, dequantised in the wave; per group and 16 x 16
// block the four k-steps accumulated unscaled, then one scale FMA, so the
// results are that kernel's bits) with MT 16-row blocks per wave and W waves
// of NB 16-column blocks per workgroup. Every dequantised B fragment feeds
// MT x (1 or 2) MFMAs and every A fragment read from LDS NB of them, where
// the 16-row form pays one LDS read and one dequantisation per two MFMAs.
template <int W, int MT, int NB, int EPI, int XT>
__global__ __launch_bounds__(W * 64) void q4_thick_kernel(Q4Args a) {
  constexpr int NA = (XT == X_F16X2) ? 2 : 1;
  constexpr int T = W * 64, TM = 16 * MT;
  constexpr int AP = NA * 128 + 8;            // LDS row (f16): hi | lo | pad
  constexpr int STG = TM * NA * 16;           // 16-byte chunks per group tile
  constexpr int SPT = (STG + T - 1) / T;      // chunks per thread
  __shared__ __attribute__((aligned(16))) _Float16 As[2][TM * AP];
  const int m0 = (int)blockIdx.y * TM, mlim = a.M;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int c0 = (int)blockIdx.x * W * 16 * NB + wave * 16 * NB;
  const int ngroups = a.K / 128;
  const int g0 = a.part ? (int)blockIdx.z * a.gper : 0;  // host: g0 < g1
  const int g1 = a.part ? min(ngroups, g0 + a.gper) : ngroups;
  int brow[NB], brow_c[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if constexpr (is_swiglu(EPI)) {
      const int col = c0 / 2 + (b % (NB / 2)) * 16 + j;
      brow[b] = (col < a.ncols) ? ((b < NB / 2) ? col : a.ncols + col) : -1;
    } else {
      const int col = c0 + b * 16 + j;
      brow[b] = (col < a.N) ? col : -1;
    }
    brow_c[b] = brow[b] >= 0 ? brow[b] : 0;
  }
  // staging: chunk c = t + i*T copies 16 bytes of half (c / 16) % NA of tile
  // row c / (16 NA); rows past M repeat a valid row
  const int t = threadIdx.x;
  size_t sxo[SPT];
  int sdst[SPT];
#pragma unroll
  for (int i = 0; i < SPT; ++i) {
    const int c = min(t + i * T, STG - 1);
    const int srow = c / (NA * 16), sh = (c / 16) % NA, sc16 = c % 16;
    const int sprow = min(m0 + srow, mlim - 1);
    sxo[i] = (size_t)sprow * a.ldx + (size_t)sh * a.K + sc16 * 8;
    sdst[i] = srow * AP + sh * 128 + sc16 * 8;
  }
  auto aload = [&](int kg, u32x4 (&v)[SPT]) {
    const size_t ko = (size_t)min(kg, g1 - 1) * 128;
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      if (STG % T == 0 || t + i * T < STG) {
        if constexpr (XT == X_BF16) {
          const h8 f = act_frag(
              *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.x) + sxo[i] + ko));
          v[i] = __builtin_bit_cast(u32x4, f);
        } else {
          v[i] = *reinterpret_cast<const u32x4*>(static_cast<const _Float16*>(a.x) + sxo[i] + ko);
        }
      }
    }
  };
  auto astore = [&](int buf, const u32x4 (&v)[SPT]) {
#pragma unroll
    for (int i = 0; i < SPT; ++i)
      if (STG % T == 0 || t + i * T < STG) *reinterpret_cast<u32x4*>(&As[buf][sdst[i]]) = v[i];
  };
  auto wload = [&](int kg, u32x4 (&w)[NB], uint16_t (&sr)[NB]) {
    const int kc = min(kg, g1 - 1);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      w[b] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          a.codes + q4t_code_offset(brow_c[b], kc, ngroups) + g * 16));
      sr[b] = a.scales[q4t_scale_index(brow_c[b], kc, ngroups)];
    }
  };
  f4 acc[MT][NB];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[mt][b] = f4{0.f, 0.f, 0.f, 0.f};
  auto group = [&](int kg, const u32x4 (&w)[NB], const uint16_t (&sr)[NB]) {
    const _Float16* ab = &As[(kg - g0) & 1][j * AP + g * 32];
    f4 tt[MT][NB];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int b = 0; b < NB; ++b) tt[mt][b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      h8 af[MT][NA];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int h = 0; h < NA; ++h)
          af[mt][h] = *reinterpret_cast<const h8*>(ab + mt * 16 * AP + h * 128 + s4 * 8);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const h8 bq = q4_unpack(w[b][s4]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          tt[mt][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mt][0], bq, tt[mt][b], 0, 0, 0);
          if constexpr (NA == 2)
            tt[mt][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mt][1], bq, tt[mt][b], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float scl = brow[b] >= 0 ? bf16_to_f32(sr[b]) : 0.f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mt][b][r] = fmaf(tt[mt][b][r], scl, acc[mt][b][r]);
    }
  };
  // the two-stage loop of q4_grouped_lds_kernel
  u32x4 w0[NB], w1[NB];
  uint16_t s0[NB], s1[NB];
  u32x4 av[SPT];
  aload(g0, av);
  wload(g0, w0, s0);
  astore(0, av);
  for (int kg = g0; kg < g1; kg += 2) {
    aload(kg + 1, av);
    wload(kg + 1, w1, s1);
    __syncthreads();
    group(kg, w0, s0);
    astore((kg + 1 - g0) & 1, av);
    if (kg + 1 >= g1) break;
    aload(kg + 2, av);
    wload(kg + 2, w0, s0);
    __syncthreads();
    group(kg + 1, w1, s1);
    astore((kg - g0) & 1, av);
  }
  // ---- epilogue: lane holds rows m0 + 16 mt + 4g + r of column j of each block
  if (a.part) {  // split-K partial tile, logical columns (uniform branch)
    const int lc_total = is_swiglu(EPI) ? 2 * a.ncols : a.N;
    float* pp = a.part + (size_t)blockIdx.z * a.M * lc_total;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + mt * 16 + 4 * g + r;
        if (row >= mlim) continue;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          int lc;
          if constexpr (is_swiglu(EPI)) {
            const int hcol = c0 / 2 + (b % (NB / 2)) * 16 + j;
            if (hcol >= a.ncols) continue;
            lc = (b < NB / 2) ? hcol : a.ncols + hcol;
          } else {
            lc = c0 + b * 16 + j;
            if (lc >= a.N) continue;
          }
          pp[(size_t)row * lc_total + lc] = acc[mt][b][r];
        }
      }
    return;
  }
  if constexpr (EPI == 6) {
    // RoPE pairs (2p, 2p+1) are adjacent columns, i.e. lanes j and j^1 of the
    // same rows: swap partners before any lane-dependent branch
    f4 partner[MT][NB];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) partner[mt][b][r] = __shfl_xor(acc[mt][b][r], 1, kWave);
    if ((j & 1) != 0) return;
    const int hd_shift = __builtin_ctz(a.hd);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + mt * 16 + 4 * g + r;
        const int rc = min(row, mlim - 1);
        const int sq = (a.rope_L == 1) ? rc : rc / a.rope_L;
        const int pos = a.pos0[sq] + (rc - sq * a.rope_L);
        if (row >= mlim || pos < 0 || pos >= a.cap) continue;
        const float2* rrow = a.rope + (size_t)pos * (a.hd / 2);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int col = c0 + b * 16 + j;
          if (col >= a.N) continue;
          const int slot = col >> hd_shift, e = col & (a.hd - 1);
          const float va = acc[mt][b][r], vb = partner[mt][b][r];  // columns e, e+1
          h2 out;
          _Float16* dst;
          if (slot >= a.H + a.KVH) {  // value: no rotation
            out = h2{(_Float16)va, (_Float16)vb};
            dst = a.vc + (((size_t)sq * a.KVH + (slot - a.H - a.KVH)) * a.cap + pos) * a.hd + e;
          } else {
            const float2 cs = rrow[e >> 1];
            out = h2{(_Float16)(va * cs.x - vb * cs.y), (_Float16)(vb * cs.x + va * cs.y)};
            dst = (slot < a.H) ? a.q_out + ((size_t)row * a.H + slot) * a.hd + e
                               : a.kc + (((size_t)sq * a.KVH + (slot - a.H)) * a.cap + pos) * a.hd + e;
          }
          *reinterpret_cast<h2*>(dst) = out;
        }
      }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + mt * 16 + 4 * g + r;
      if (row >= mlim) continue;
      if constexpr (is_swiglu(EPI)) {
#pragma unroll
        for (int b = 0; b < NB / 2; ++b) {
          const int col = c0 / 2 + b * 16 + j;
          if (col < a.ncols) {
            const float hv = silu(acc[mt][b][r]) * acc[mt][b + NB / 2][r];
            if constexpr (EPI == EPI_SWIGLU_F16X2) {
              _Float16 hi, lo;
              split_f16(hv, hi, lo);
              static_cast<_Float16*>(a.y)[(size_t)row * a.ldy + col] = hi;
              static_cast<_Float16*>(a.y)[(size_t)row * a.ldy + a.ncols + col] = lo;
            } else if constexpr (EPI == EPI_SWIGLU_F16) {
              static_cast<_Float16*>(a.y)[(size_t)row * a.ldy + col] = (_Float16)hv;
            } else {
              static_cast<uint16_t*>(a.y)[(size_t)row * a.ldy + col] = f32_to_bf16(hv);
            }
          }
        }
      } else {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int col = c0 + b * 16 + j;
          if (col >= a.N) continue;
          const size_t o = (size_t)row * a.ldy + col;
          if constexpr (EPI == EPI_STORE_F32) static_cast<float*>(a.y)[o] = acc[mt][b][r];
          else if constexpr (EPI == EPI_ADD_F32) static_cast<float*>(a.y)[o] += acc[mt][b][r];
          else static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(acc[mt][b][r]);
        }
      }
    }
}

template <int W, int MT, int NB, int XT>
int launch_thick(const Q4Args& a, int epi, hipStream_t st, int ks) {
  const int logical_cols = is_swiglu(epi) ? 2 * a.ncols : a.N;
  const dim3 grid((unsigned)ceil_div(logical_cols, W * 16 * NB), (unsigned)ceil_div(a.M, 16 * MT),
                  (unsigned)ks);
  switch (epi) {  // the SwiGLU FFN-in is the shape it is used for (use_thick)
#define SM_TK(E) \
    case E: q4_thick_kernel<W, MT, NB, E, XT><<<grid, W * 64, 0, st>>>(a); break;
    SM_TK(EPI_SWIGLU_BF16)
    SM_TK(EPI_SWIGLU_F16)
    SM_TK(EPI_SWIGLU_F16X2)
    SM_TK(EPI_ADD_F32)
#undef SM_TK
    default: set_error("sm_q4_matmul: thick kernel for epilogue %d", epi); return SM_ERR_INVALID;
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

// The decode FFN-in at 128 < M <= 256 with more than 8192 gate + value columns
// (config[2]: M 256, 2 x 5632): 4 waves of 2 x 2 blocks (32 x 128 tiles).
// Measured against the batch kernel (42.3 us) on that shape, 16-column wave
// tiles: 33.7 us; 8 waves 34.5; 64-row tiles 40.3; 4 column blocks 38.5; the
// 16-row form 38.8. The qkv projection measured no faster in this form
// (15.6 -> 16-25 us); the residual projections take it in K splits
// (thick_add_rmsnorm_splits).
inline bool use_thick(int64_t M, int64_t logical_cols, int epi, int xt) {
  return is_swiglu(epi) && (xt == X_F16X2 || xt == X_F16) && M > 128 && M <= 256 &&
         logical_cols > 8192;
}

// Dense decode shapes that the LDS-shared kernel serves faster (measured).
inline bool use_dense_lds(int64_t M, int64_t K, int64_t logical_cols, int xt) {
  return (xt == X_F16X2 || xt == X_F16) && M > 32 && M <= 256 && K <= 2048 &&
         logical_cols >= 2048 && logical_cols <= 8192;
}

// Decode shapes outside that window (long K, or narrow N) with a split-K
// workspace: the same kernel over K ranges, partials reduced in order.
inline bool use_dense_lds_split(int64_t M, int64_t K, int64_t logical_cols, int xt) {
  return (xt == X_F16X2 || xt == X_F16) && M > 32 && M <= 256 && K >= 6 * 128 &&
         (K > 2048 || logical_cols < 2048) && logical_cols <= 8192;
}

// SwiGLU tiles pair gate and value blocks, so they need an even NB
template <int NB, int E, int XT>
void launch_gl(dim3 grid, hipStream_t st, const Q4Args& a) {
  if constexpr (!is_swiglu(E) || NB % 2 == 0) q4_grouped_lds_kernel<NB, E, XT><<<grid, 512, 0, st>>>(a);
}

template <int XT, int NB>
int launch_grouped_lds_nb(const Q4Args& a, int epi, hipStream_t st, int64_t row_tiles, int ks,
                          bool reduce = true) {
  const int logical_cols = is_swiglu(epi) ? 2 * a.ncols : a.N;
  const dim3 grid((unsigned)ceil_div(logical_cols, 8 * 16 * NB), (unsigned)row_tiles, (unsigned)ks);
  switch (epi) {
#define SM_GL(E) \
    case E: launch_gl<NB, E, XT>(grid, st, a); break;
    SM_GL(EPI_STORE_F32)
    SM_GL(EPI_STORE_BF16)
    SM_GL(EPI_ADD_F32)
    SM_GL(6)
    SM_GL(EPI_SWIGLU_BF16)
    SM_GL(EPI_SWIGLU_F16)
    SM_GL(EPI_SWIGLU_F16X2)
#undef SM_GL
    default: set_error("sm_q4_grouped_matmul: unknown epilogue %d", epi); return SM_ERR_INVALID;
  }
  SM_LAUNCH_CHECK();
  if (ks > 1 && reduce) return splitk_reduce(a.part, ks, a.M, a.N, a.ncols, a.y, a.ldy, epi, st);
  return SM_OK;
}

// 256 columns per workgroup: measured against 512 at config[4] decode
// (FFN-in 30 vs 32 us, down 17 vs 24 us: the narrower tile gives the down
// projection's 2048 columns enough workgroups). Dense non-SwiGLU launches of
// at most 128 rows take 128 columns (one 16-column block per wave; the same
// bits): config[1] rollout 213.4 -> 206.8 ms, config[4] 844 -> 837 ms, while
// config[2]'s 256-row decode is 0.8 % slower that way and keeps 256. The
// qkv projection with its RoPE epilogue keeps 256 columns from K 2048 on
// (config[4]: 17.3 -> 16.1 us per call; at config[1]'s K 768 the narrow
// tile stays faster, 9.3 against 11.6 us).
template <int XT>
int launch_grouped_lds(const Q4Args& a, int epi, hipStream_t st, int64_t row_tiles, int ks = 1,
                       bool reduce = true) {

  if (!a.tiles && !is_swiglu(epi) && a.M <= 128 && !(epi == 6 && a.K >= 2048))
    return launch_grouped_lds_nb<XT, 1>(a, epi, st, row_tiles, ks, reduce);
  return launch_grouped_lds_nb<XT, 2>(a, epi, st, row_tiles, ks, reduce);
}

// M = 1 (one sequence's decode step; the LM head at batch 1). One wave owns a
// 16-row block of W; KS = 1: four blocks per workgroup, each wave over all of
// K; KS = 4: one block per workgroup, wave w over the K groups w, w + 4, ...,
// merged in LDS in wave order (for N too small to fill the GPU otherwise). The activation
// row is staged in LDS once per workgroup, after the first weight group has
// been requested, and feeds every A row of the MFMA (so every D row is the
// result and no lane is masked). With K split over the waves each wave copies
// only its own groups of the row and waits on no other wave (measured with
// every group of a wave requested up front: 3072 x 2048 3.0 -> 2.7 us,
// 4096 x 4096 4.4 -> 3.65 us, LM head 12.9 -> 12.7 us). Weight groups are double-buffered in
// registers, which leaves the weight stream alone on the vector-memory
// counter: activation loads interleaved with it made every wait drain the
// next group's weights too. The arithmetic per group is that of
// q4_gemm_kernel (codes x activations over 4 k-steps, then one FMA with the
// group scale), so the two kernels give the same bits.
template <int NA, int EPI, int KS, int ALL = 0>
__global__ __launch_bounds__(256) void q4_gemv1_kernel(Q4Args a) {
  extern __shared__ _Float16 xs[];  // NA * K activations (hi, then lo)
  __shared__ float red[KS][4][16];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  constexpr int BPW = 4 / KS;  // row blocks per workgroup
  const int blk = wave % BPW, part = wave / BPW;
  const int nrb = (a.N + 15) / 16;
  const int rb_raw = (int)blockIdx.x * BPW + blk;
  const int rb = min(rb_raw, nrb - 1);  // tail waves re-read the last block, store nothing
  const int ng = a.K / 128;
  const uint8_t* cb = a.codes + q4t_code_offset((int64_t)rb * 16 + j, 0, ng) + g * 16;
  const uint16_t* sb = a.scales + q4t_scale_index((int64_t)rb * 16 + j, 0, ng);
  auto load = [&](int kc, u32x4& w, uint16_t& sc) {
    kc = min(kc, ng - 1);
    w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(cb + (size_t)kc * 1024));
    sc = sb[kc * 16];
  };
  u32x4 w0, w1, wa[ALL > 0 ? ALL : 1];
  uint16_t s0, s1, sa[ALL > 0 ? ALL : 1];
  const _Float16* x = static_cast<const _Float16*>(a.x);
  // With every group requested up front, this wave's activation chunks are
  // requested first: loads complete in issue order, so the copy into LDS then
  // waits for them alone and the math starts as the first weight group lands.
  constexpr int XN = NA * (ALL > 0 ? ALL : 1) * 16, XC = (XN + kWave - 1) / kWave;
  h8 xr[XC];
  int xoff[XC];
  if constexpr (ALL > 0 && KS == 4) {
#pragma unroll
    for (int u = 0; u < XC; ++u) {
      const int c = lane + u * kWave;
      const int h = c / (ALL * 16), i = (c / 16) % ALL, ch = c % 16;
      xoff[u] = h * a.K + (part + 4 * i) * 128 + ch * 8;
      if (c < XN) xr[u] = *reinterpret_cast<const h8*>(x + xoff[u]);
    }
  }
  if constexpr (ALL > 0) {
#pragma unroll
    for (int i = 0; i < ALL; ++i) load(part + i * KS, wa[i], sa[i]);
  } else {
    load(part, w0, s0);
  }
  if constexpr (KS == 4) {
    // each wave copies only its own K groups (part + 4i) of the activation row
    // into their places in LDS; no workgroup barrier before the math
    if constexpr (ALL > 0) {
#pragma unroll
      for (int u = 0; u < XC; ++u)
        if (lane + u * kWave < XN) *reinterpret_cast<h8*>(xs + xoff[u]) = xr[u];
    } else {
      const int mine = (ng - part + 3) / 4;
      for (int c = lane; c < NA * mine * 16; c += kWave) {
        const int h = c / (mine * 16), i = (c / 16) % mine, ch = c % 16;
        const int off = h * a.K + (part + 4 * i) * 128 + ch * 8;
        *reinterpret_cast<h8*>(xs + off) = *reinterpret_cast<const h8*>(x + off);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    for (int i = threadIdx.x * 8; i < NA * a.K; i += 256 * 8)
      *reinterpret_cast<h8*>(xs + i) = *reinterpret_cast<const h8*>(x + i);
    __syncthreads();
  }
  float acc = 0.f;
  auto group = [&](int kg, const u32x4& w, uint16_t sc) {
    f4 t = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const h8 bq = q4_unpack(w[q]);
      const h8 ah = *reinterpret_cast<const h8*>(xs + kg * 128 + g * 32 + q * 8);
      t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq, t, 0, 0, 0);
      if constexpr (NA == 2) {
        const h8 al = *reinterpret_cast<const h8*>(xs + a.K + kg * 128 + g * 32 + q * 8);
        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq, t, 0, 0, 0);
      }
    }
    acc = fmaf(t[0], bf16_to_f32(sc), acc);
  };
  if constexpr (ALL > 0) {
#pragma unroll
    for (int i = 0; i < ALL; ++i) group(part + i * KS, wa[i], sa[i]);
  } else {
    for (int kb = part; kb < ng; kb += 2 * KS) {
      load(kb + KS, w1, s1);
      group(kb, w0, s0);
      if (kb + KS >= ng) break;
      load(kb + 2 * KS, w0, s0);
      group(kb + KS, w1, s1);
    }
  }
  if constexpr (KS > 1) {
    if (g == 0) red[part][blk][j] = acc;
    __syncthreads();
    if (part != 0) return;
    acc = red[0][blk][j];
#pragma unroll
    for (int p = 1; p < KS; ++p) acc += red[p][blk][j];
  }
  const int col = rb * 16 + j;
  if (g != 0 || rb_raw >= nrb || col >= a.N) return;
  if constexpr (EPI == EPI_STORE_F32) static_cast<float*>(a.y)[col] = acc;
  else if constexpr (EPI == EPI_STORE_BF16) static_cast<uint16_t*>(a.y)[col] = f32_to_bf16(acc);
  else static_cast<float*>(a.y)[col] += acc;
}

// The K-split variant runs where the tile kernel's narrow GEMV splits K (fewer
// than 512 of its 64-column workgroups; the same choice keeps the two kernels'
// bits equal) and for rows of 2048 or more: measured on the config[2] LM head
// (N = 65536, K = 2048), four waves per 16-row block over a quarter of K each
// take 13.6 us per launch against 14.2 us for one wave over all of K (N = 32768,
// K = 2048: 9.1 against 9.9 us; at K = 1024 the split gains nothing). The
// tile kernel keeps 512 there: split, its M = 2..16 calls run 1.2-1.6x slower.
// Where each wave owns 4, 8 or 11 groups (K = 2048, 4096, 5632) it requests
// them all before staging the activation row (ALL): 13.0 us on the LM head,
// 6.5 -> 4.6 us at 2048 x 5632, 5.6 -> 4.3 us at 4096 x 4096. Walking several
// row blocks per workgroup with the next block's weights in flight (2, 4 or 8
// blocks) measured 13.7-14.3 us on the LM head, so each workgroup owns one.
template <int NA, int EPI>
int launch_gemv1(const Q4Args& a, hipStream_t st) {
  const int64_t nrb = ceil_div(a.N, 16);
  const size_t lds = (size_t)NA * a.K * 2;
  const int64_t ng = a.K / 128;
  if (ng == 16)  // 4, 8 or 11 K groups per wave, all requested at once
    q4_gemv1_kernel<NA, EPI, 4, 4><<<(unsigned)nrb, 256, lds, st>>>(a);
  else if (ng == 32)
    q4_gemv1_kernel<NA, EPI, 4, 8><<<(unsigned)nrb, 256, lds, st>>>(a);
  else if (ng == 44)
    q4_gemv1_kernel<NA, EPI, 4, 11><<<(unsigned)nrb, 256, lds, st>>>(a);
  else if ((ceil_div(a.N, 64) < 512 || a.K >= 2048) && a.K >= 4 * 128)
    q4_gemv1_kernel<NA, EPI, 4><<<(unsigned)nrb, 256, lds, st>>>(a);
  else
    q4_gemv1_kernel<NA, EPI, 1><<<(unsigned)ceil_div(nrb, 4), 256, lds, st>>>(a);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

int launch_gemv1_x(const Q4Args& a, int epi, int xt, hipStream_t st) {
#define SM_G1(NA)                                                        \
  switch (epi) {                                                         \
    case EPI_STORE_F32: return launch_gemv1<NA, EPI_STORE_F32>(a, st);   \
    case EPI_STORE_BF16: return launch_gemv1<NA, EPI_STORE_BF16>(a, st); \
    default: return launch_gemv1<NA, EPI_ADD_F32>(a, st);                \
  }
  if (xt == X_F16X2) SM_G1(2)
  SM_G1(1)
#undef SM_G1
}

template <int NB, int KSPLIT, int XT, int KU = 8>
int launch_q4_x(const Q4Args& a, int epi, hipStream_t st, int64_t row_tiles) {
  const int wave_cols = 16 * NB;
  const int tile_cols = (KSPLIT == 1) ? 4 * wave_cols : wave_cols;
  const int logical_cols = is_swiglu(epi) ? 2 * a.ncols : a.N;
  dim3 grid((unsigned)ceil_div(logical_cols, tile_cols), (unsigned)row_tiles);
  switch (epi) {
#define SM_Q4_EPI(E) \
    case E: q4_gemm_kernel<NB, KSPLIT, E, XT, KU><<<grid, 256, 0, st>>>(a); break;
    SM_Q4_EPI(EPI_STORE_F32)
    SM_Q4_EPI(EPI_STORE_BF16)
    SM_Q4_EPI(EPI_ADD_F32)
#undef SM_Q4_EPI
    case EPI_SWIGLU_BF16:
    case EPI_SWIGLU_F16:
    case EPI_SWIGLU_F16X2:
      if constexpr (NB % 2 == 0) {
        if (epi == EPI_SWIGLU_F16X2)
          q4_gemm_kernel<NB, KSPLIT, EPI_SWIGLU_F16X2, XT, KU><<<grid, 256, 0, st>>>(a);
        else if (epi == EPI_SWIGLU_F16)
          q4_gemm_kernel<NB, KSPLIT, EPI_SWIGLU_F16, XT, KU><<<grid, 256, 0, st>>>(a);
        else
          q4_gemm_kernel<NB, KSPLIT, EPI_SWIGLU_BF16, XT, KU><<<grid, 256, 0, st>>>(a);
        break;
      } else {
        set_error("internal: SwiGLU needs an even number of column blocks");
        return SM_ERR_INVALID;
      }
    default: set_error("sm_q4_matmul: unknown epilogue %d", epi); return SM_ERR_INVALID;
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

template <int NB, int KSPLIT, int KU = 8>
int launch_q4(const Q4Args& a, int epi, int xt, hipStream_t st, int64_t row_tiles) {
  switch (xt) {
    case X_BF16: return launch_q4_x<NB, KSPLIT, X_BF16, KU>(a, epi, st, row_tiles);
    case X_F16: return launch_q4_x<NB, KSPLIT, X_F16, KU>(a, epi, st, row_tiles);
    default: return launch_q4_x<NB, KSPLIT, X_F16X2, KU>(a, epi, st, row_tiles);
  }
}

}  // namespace



namespace {

// Picks the kernel. More than 32 rows (decode batches, prefill, recompute):
// q4_gemm_bl.hip, which dequantises each weight once per workgroup into LDS
// (and, given a workspace, splits K when its grid is small), unless its grid
// would have fewer than 64 workgroups (a narrow N at decode batch size), where
// the in-workgroup K-split of the kernel above was measured faster. Otherwise (GEMV-like, HBM-bound): the
// register-direct kernel above with 16-row wave tiles (M/16 row tiles); when
// that grid would have fewer than 512 workgroups the four waves of a
// workgroup split K instead of N.
int dispatch_q4(const Q4Args& a, int epi, int xt, hipStream_t st, void* ws, int64_t ws_bytes) {
  // one activation row in f16 (or pairs) with a plain epilogue: the M = 1 GEMV
  if (a.M == 1 && !a.tiles && !a.rowidx && xt != X_BF16 && epi <= EPI_ADD_F32 &&
      (int64_t)(xt == X_F16X2 ? 2 : 1) * a.K * 2 <= 65536)
    return launch_gemv1_x(a, epi, xt, st);
  const int64_t logical_cols = is_swiglu(epi) ? 2 * (int64_t)a.ncols : a.N;
  const bool ksplit_ok = a.K >= 4 * 128;
  const int64_t bl_wgs = ceil_div(a.M, 64) * ceil_div(logical_cols, 64);
  if (a.M <= 32 || (a.M <= 256 && bl_wgs < 64)) {
    const int64_t rt = ceil_div(a.M, 16);
    // GEMV-like M: 16-column wave tiles double the workgroup count (SwiGLU
    // needs gate/value block pairs, so it keeps 32).
    const bool narrow = a.M <= 16 && !is_swiglu(epi);
    const int64_t wgs = ceil_div(logical_cols, narrow ? 64 : 128) * rt;
    if (narrow) {
      if (wgs < 512 && ksplit_ok) return launch_q4<1, 4>(a, epi, xt, st, rt);
      return launch_q4<1, 1, 4>(a, epi, xt, st, rt);  // measured best batch depth for GEMV
    }
    if (wgs < 512 && ksplit_ok) return launch_q4<2, 4>(a, epi, xt, st, rt);
    return launch_q4<2, 1>(a, epi, xt, st, rt);
  }
  if (!a.tiles && !a.rowidx && use_thick(a.M, logical_cols, epi, xt)) {
    if (xt == X_F16X2) return launch_thick<4, 2, 2, X_F16X2>(a, epi, st, 1);
    return launch_thick<4, 2, 2, X_F16>(a, epi, st, 1);
  }
  if (!a.tiles && !a.rowidx && use_dense_lds(a.M, a.K, logical_cols, xt)) {
    if (xt == X_F16X2) return launch_grouped_lds<X_F16X2>(a, epi, st, ceil_div(a.M, 16));
    return launch_grouped_lds<X_F16>(a, epi, st, ceil_div(a.M, 16));
  }
  if (!a.tiles && !a.rowidx && ws && use_dense_lds_split(a.M, a.K, logical_cols, xt)) {
    // K split over workgroups: >= 3 groups per split, up to ~512 workgroups
    const int64_t rt = ceil_div(a.M, 16), base = ceil_div(logical_cols, 256) * rt;
    const int ng = a.K / 128;
    int ks = (int)std::min<int64_t>(ng / 3, std::max<int64_t>(1, 512 / base));
    const int64_t lc_total = logical_cols;
    while (ks > 1 && (int64_t)ks * a.M * lc_total * 4 > ws_bytes) --ks;
    if (ks > 1) {
      Q4Args b = a;
      b.gper = (int)ceil_div(ng, ks);
      ks = (int)ceil_div(ng, b.gper);  // every split non-empty
      b.part = static_cast<float*>(ws);
      if (xt == X_F16X2) return launch_grouped_lds<X_F16X2>(b, epi, st, rt, ks);
      return launch_grouped_lds<X_F16>(b, epi, st, rt, ks);
    }
  }
  return q4_gemm_bl(a.codes, a.scales, a.N, a.K, a.x, xt, a.M, a.ldx, a.y, a.ldy, epi, a.ncols,
                    st, nullptr, nullptr, 0, nullptr, nullptr, 0, 0, ws, ws_bytes, nullptr);
}

// Split-K partials of a residual projection, summed in split order and added
// to the residual (splitk_reduce_kernel's EPI_ADD_F32 arithmetic), then the
// next RMSNorm of the updated rows written as f16 pairs, with
// rmsnorm_wave_kernel's arithmetic: lane l's sum of squares runs over float4s
// l, 64 + l, ... of the row in that order, then one wave reduction, and
// x / rms * gamma. One workgroup per row, wave i owning float4s i*64 + l; KS
// (the split count, 0 = given at run time) is a template parameter so every
// lane issues all its partial, residual and gamma loads at once. The squares
// meet in LDS so that wave 0 sums them in the one-wave order. Replaces the
// reduce launch and the norm launch with one.
//
// With a router (ROUTER, the MoE layers' FFN norm): the row's router logits
// sum_c h[c] * wr[e, c] (SparseMoe::forward's fp32 router, ffn.rs:489-490)
// over h as its f16 pair holds it (hi + lo, what the router kernel reads):
// each lane multiplies its four columns by every expert's weights (all of
// them requested at once), a wave sums the lanes, and the V wave sums are
// added in wave order. Wave 0 then takes the row's top-2 as the sequential
// strict '>' scan would (top2_indices_kernel, moe_topk.rs:74-104: the
// lowest index among equal maxima; NaN never wins; an all -inf / NaN row
// keeps the scan's initial index 0) and the softmax over the pair (ffn.rs:514),
// into top_idx / top_w [rows, 2]; logits [rows, E] optional. This replaces
// the router launch of a decode step.
constexpr int kRouterMaxExperts = 64;

template <int V, int KS, bool ROUTER = false>
__global__ __launch_bounds__(64 * V) void splitk_add_rmsnorm_kernel(
    const float* __restrict__ part, int ks, int64_t rows, float* __restrict__ resid,
    const float* __restrict__ gamma, float eps, _Float16* __restrict__ h,
    const float* __restrict__ wr = nullptr, int E = 0, float* __restrict__ logits = nullptr,
    int32_t* __restrict__ top_idx = nullptr, float* __restrict__ top_w = nullptr) {
  constexpr int D = 256 * V;
  __shared__ float4 sq[V][64];
  __shared__ float rms_s;
  __shared__ float red[V][kRouterMaxExperts];
  const int64_t r = blockIdx.x;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int c4 = wave * kWave + lane;
  const size_t split4 = (size_t)rows * (D / 4);
  const float4* pr = reinterpret_cast<const float4*>(part) + r * (D / 4) + c4;
  float4* xr = reinterpret_cast<float4*>(resid + r * D) + c4;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if constexpr (KS > 0) {
    float4 p[KS];
#pragma unroll
    for (int k = 0; k < KS; ++k) p[k] = pr[k * split4];
#pragma unroll
    for (int k = 0; k < KS; ++k) {
      acc.x += p[k].x; acc.y += p[k].y; acc.z += p[k].z; acc.w += p[k].w;
    }
  } else {
    for (int k = 0; k < ks; ++k) {
      const float4 p = pr[k * split4];
      acc.x += p.x; acc.y += p.y; acc.z += p.z; acc.w += p.w;
    }
  }
  const float4 x = *xr;
  const float4 gm = reinterpret_cast<const float4*>(gamma)[c4];
  const float4 v = make_float4(x.x + acc.x, x.y + acc.y, x.z + acc.z, x.w + acc.w);
  *xr = v;
  float hv[4];
  row_rmsnorm_pair<V>(v, gm, eps, sq, rms_s, h + r * 2 * D, hv);
  if constexpr (!ROUTER) return;
  // every expert's weights for this lane's columns requested at once (32
  // experts per round; rows past E re-read the last expert, unused), so the
  // router costs one L2 round trip per 32 experts
  constexpr int EB = 32;
  for (int e0 = 0; e0 < E; e0 += EB) {
    float4 w[EB];
#pragma unroll
    for (int u = 0; u < EB; ++u)
      w[u] = reinterpret_cast<const float4*>(wr + (size_t)min(e0 + u, E - 1) * D)[c4];
#pragma unroll
    for (int u = 0; u < EB; ++u) {
      float p = hv[0] * w[u].x;
      p = fmaf(hv[1], w[u].y, p);
      p = fmaf(hv[2], w[u].z, p);
      p = fmaf(hv[3], w[u].w, p);
      p = wave_sum(p);
      if (lane == 0 && e0 + u < E) red[wave][e0 + u] = p;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float lv = -INFINITY;
  if (lane < E) {
    lv = 0.f;
#pragma unroll
    for (int w = 0; w < V; ++w) lv += red[w][lane];
    if (logits) logits[r * E + lane] = lv;
  }
  const float key = (lv == lv) ? lv : -INFINITY;  // NaN never wins a '>'
  const float v0 = wave_max(key);
  int i0 = __ffsll((unsigned long long)__ballot(lane < E && key == v0)) - 1;
  if (v0 == -INFINITY) i0 = 0;
  const float key1 = (lane == i0) ? -INFINITY : key;
  const float v1 = wave_max(key1);
  int i1 = __ffsll((unsigned long long)__ballot(lane < E && lane != i0 && key1 == v1)) - 1;
  if (v1 == -INFINITY) i1 = 0;
  if (lane == 0) {
    const float e1 = expf(v1 - v0);  // softmax over [v0, v1] (v0 >= v1)
    top_idx[r * 2] = i0;
    top_idx[r * 2 + 1] = i1;
    top_w[r * 2] = 1.f / (1.f + e1);
    top_w[r * 2 + 1] = e1 / (1.f + e1);
  }
}

// K splits of the fused residual projection + RMSNorm, or 0 when the fused
// form does not apply (dispatch_q4 would not pick the LDS-staged decode kernel
// for this shape, the width is not one the row-in-registers norm handles, or
// the workspace cannot hold two splits). The split count follows dispatch_q4's
// rule for the LDS-staged kernel over K ranges (>= 3 groups per split, up to
// ~512 workgroups), so a projection it already splits keeps its partials.
int add_rmsnorm_splits(int64_t M, int64_t N, int64_t K, int xt, int64_t ws_bytes) {
  if (xt != X_F16X2 && xt != X_F16) return 0;
  if (N % 256 != 0) return 0;
  const int64_t v = N / 256;
  if (v != 3 && v != 4 && v != 8 && v != 12 && v != 16) return 0;
  // decode batch sizes with the LDS-staged kernel's shapes; for narrow N
  // (fewer than 64 batch-kernel workgroups) dispatch_q4 would take the
  // in-workgroup K-split kernel instead, 1-3 us faster per call at config[1],
  // but the fused form saves a ~4.5 us norm launch
  if (M <= 32 || M > 256) return 0;
  if (!use_dense_lds(M, K, N, xt) && !use_dense_lds_split(M, K, N, xt)) return 0;
  const int ng = (int)(K / 128);
  const int64_t base = ceil_div(N, 256) * ceil_div(M, 16);
  int ks = (int)std::min<int64_t>(ng / 3, std::max<int64_t>(1, 512 / base));
  while (ks > 1 && (int64_t)ks * M * N * 4 > ws_bytes) --ks;
  if (ks < 2) return 0;
  const int gper = (int)ceil_div(ng, ks);
  return (int)ceil_div(ng, gper);  // every split non-empty
}

// The residual projections of the fused add + RMSNorm at 128 < M <= 256
// (config[2], M 256, N 2048): the thick-wave kernel over K splits sized for
// about 512 workgroups, 16-row wave tiles for K <= 2048 and 32-row ones past
// it. Measured, GEMM + split reduction: o (K 2048) 13.3 + 4.5 us with the
// grouped kernel in 4 splits -> 11.4 + 4.3 us in 2 (16-row tiles; 4 splits
// 12.9, 32-row tiles 13.5); down (K 8192) 20.4 + 5.0 -> 19.9 + 4.6 us in 4
// (32-row tiles; 16-row tiles 21.2, 2 and 8 splits 24.9 and 21.3). Returns
// the split count (0: keep the grouped kernel) and the tile height in mt.
int thick_add_rmsnorm_splits(int64_t M, int64_t N, int64_t K, int64_t ws_bytes, int& mt) {
  if (M <= 128 || M > 256 || N < 2048) return 0;
  mt = (K > 2048) ? 2 : 1;
  const int ng = (int)(K / 128);
  const int64_t base = ceil_div(N, 4 * 16 * 2) * ceil_div(M, 16 * mt);
  int ks = (int)std::min<int64_t>(ng / 3, std::max<int64_t>(1, 512 / base));
  while (ks > 1 && (int64_t)ks * M * N * 4 > ws_bytes) --ks;
  if (ks < 2) return 0;
  const int gper = (int)ceil_div(ng, ks);
  return (int)ceil_div(ng, gper);
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

// Row-major codec -> prepared tiled layout; one thread per 16-byte chunk.
// Rows n..q4t_rows(N) beyond N are zero (padding of the last row block).
__global__ void q4_pack_kernel(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
                               int64_t N, int64_t K, uint8_t* __restrict__ tcodes,
                               uint16_t* __restrict__ tscales) {
  const int64_t ngroups = K / 128;
  const int64_t rows = q4t_rows(N);
  const int64_t chunk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // 16-byte chunk
  if (chunk >= rows * ngroups * 4) return;
  const int c = chunk % 4;
  const int64_t kg = (chunk / 4) % ngroups;
  const int64_t row = chunk / (4 * ngroups);
  u32x4 v = u32x4{0u, 0u, 0u, 0u};
  if (row < N) {
    v = *reinterpret_cast<const u32x4*>(codes + row * (K / 2) + kg * 64 + c * 16);
    v = u32x4{q4_prepare_word(v.x), q4_prepare_word(v.y), q4_prepare_word(v.z),
              q4_prepare_word(v.w)};
  }
  *reinterpret_cast<u32x4*>(tcodes + q4t_code_offset(row, kg, ngroups) + c * 16) = v;
  if (c == 0) tscales[q4t_scale_index(row, kg, ngroups)] = (row < N) ? scales[row * ngroups + kg] : 0;
}

}  // namespace
}  // namespace sm

extern "C" int sm_q4_pack(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                          uint8_t* tiled_codes, uint16_t* tiled_scales, void* stream) {
  using namespace sm;
  SM_REQUIRE(codes && scales && tiled_codes && tiled_scales, "sm_q4_pack: null buffer");
  SM_REQUIRE(N > 0 && K > 0 && K % 128 == 0, "sm_q4_pack: K=%lld must be a positive multiple of 128",
             (long long)K);
  SM_REQUIRE(reinterpret_cast<uintptr_t>(codes) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(tiled_codes) % 16 == 0,
             "sm_q4_pack: code buffers must be 16-byte aligned");
  const int64_t chunks = q4t_rows(N) * (K / 128) * 4;
  q4_pack_kernel<<<(unsigned)ceil_div(chunks, 256), 256, 0, as_stream(stream)>>>(
      codes, scales, N, K, tiled_codes, tiled_scales);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

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

extern "C" int64_t sm_q4_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K, int epilogue) {
  (void)K;
  if (M <= 32 || M > 0x7fffffff || N <= 0) return 0;
  const int64_t cols = (epilogue >= sm::EPI_SWIGLU_BF16) ? 2 * (N / 2) : N;
  return sm::bl_counter_bytes() + 8 * M * cols * (int64_t)sizeof(float);
}

extern "C" int sm_q4_matmul(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                            const void* x, int x_dtype, int64_t M, int64_t ldx, void* y,
                            int64_t ldy, int epilogue, void* stream) {
  return sm_q4_matmul_ws(codes, scales, N, K, x, x_dtype, M, ldx, y, ldy, epilogue, nullptr, 0,
                         stream);
}

extern "C" int sm_q4_matmul_ws(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                               const void* x, int x_dtype, int64_t M, int64_t ldx, void* y,
                               int64_t ldy, int epilogue, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  using namespace sm;
  SM_REQUIRE(codes && scales && x && y, "sm_q4_matmul: null buffer");
  SM_REQUIRE(workspace_bytes >= 0 && (workspace || workspace_bytes == 0) &&
                 reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
             "sm_q4_matmul: bad workspace");
  SM_REQUIRE(K > 0 && K % 128 == 0, "sm_q4_matmul: K=%lld must be a positive multiple of 128",
             (long long)K);
  SM_REQUIRE(N > 0 && N <= 0x7fffffff && K <= 0x7fffffff, "sm_q4_matmul: bad N");
  SM_REQUIRE(M >= 0 && M <= 0x7fffffff, "sm_q4_matmul: bad M");
  const int xt = xmode_of(x_dtype);
  SM_REQUIRE(xt >= 0, "sm_q4_matmul: x must be bf16, f16 or f16 pairs");
  const int64_t xw = (xt == X_F16X2) ? 2 * K : K;  // f16 elements per x row
  SM_REQUIRE(ldx >= xw && ldx % 8 == 0 && ldx <= 0x7fffffff,
             "sm_q4_matmul: ldx must be >= %lld and a multiple of 8", (long long)xw);
  SM_REQUIRE(reinterpret_cast<uintptr_t>(codes) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(x) % 16 == 0,
             "sm_q4_matmul: codes and x must be 16-byte aligned");
  SM_REQUIRE(epilogue >= EPI_STORE_F32 && epilogue <= EPI_SWIGLU_F16X2,
             "sm_q4_matmul: unknown epilogue %d", epilogue);
  const int64_t ncols = is_swiglu(epilogue) ? N / 2 : N;
  SM_REQUIRE(!is_swiglu(epilogue) || N % 2 == 0, "sm_q4_matmul: SwiGLU needs even N");
  const int64_t yw = (epilogue == EPI_SWIGLU_F16X2) ? 2 * ncols : ncols;
  SM_REQUIRE(ldy >= yw && ldy <= 0x7fffffff, "sm_q4_matmul: ldy < output row width");
  if (M == 0) return SM_OK;
  Q4Args a{codes, scales, x, y, (int)M, (int)N, (int)K, (int)ldx, (int)ldy, (int)ncols};
  return dispatch_q4(a, epilogue, xt, as_stream(stream), workspace, workspace_bytes);
}

extern "C" int sm_rmsnorm(const float* x, const float* gamma, int64_t rows, int64_t d, float eps,
                          void* y, int out_dtype, void* stream);

extern "C" int sm_moe_router_top2(const void* h, int h_dtype, const float* w_router,
                                  int64_t tokens, int64_t d, int64_t experts, float* logits_out,
                                  int32_t* top_idx, float* top_w, void* stream);

namespace sm {
namespace {

// sm_q4_matmul_add_rmsnorm, and with wr the router logits of the normed rows
// (sm_q4_matmul_add_rmsnorm_router).
int matmul_add_rmsnorm(const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K,
                       const void* x, int x_dtype, int64_t M, int64_t ldx, float* resid,
                       const float* gamma, float eps, void* h_out, void* workspace,
                       int64_t workspace_bytes, const float* wr, int64_t E, float* logits,
                       int32_t* top_idx, float* top_w, void* stream) {
  const int xt = xmode_of(x_dtype);
  int ks = (xt >= 0 && workspace && reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(resid) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(gamma) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(h_out) % 8 == 0 &&
                  (!wr || reinterpret_cast<uintptr_t>(wr) % 16 == 0) && M <= 0x7fffffff &&
                  N <= 0x7fffffff && K > 0 && K % 128 == 0)
                     ? add_rmsnorm_splits(M, N, K, xt, workspace_bytes) : 0;
  hipStream_t st = as_stream(stream);
  if (ks == 0) {  // the two-step form: residual projection, then the norm (and router)
    SM_TRY(sm_q4_matmul_ws(codes, scales, N, K, x, x_dtype, M, ldx, resid, N, EPI_ADD_F32,
                           workspace, workspace_bytes, stream));
    SM_TRY(sm_rmsnorm(resid, gamma, M, N, eps, h_out, SM_F16X2, stream));
    return wr ? sm_moe_router_top2(h_out, SM_F16X2, wr, M, N, E, logits, top_idx, top_w, stream)
              : SM_OK;
  }
  SM_REQUIRE(codes && scales && x && ldx >= (xt == X_F16X2 ? 2 * K : K) && ldx % 8 == 0 &&
                 reinterpret_cast<uintptr_t>(codes) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(x) % 16 == 0,
             "sm_q4_matmul_add_rmsnorm: bad matmul operands");
  Q4Args a{codes, scales, x, resid, (int)M, (int)N, (int)K, (int)ldx, (int)N, (int)N};
  const int ng = (int)(K / 128);
  a.part = static_cast<float*>(workspace);
  int mt = 0;
  if (const int tks = thick_add_rmsnorm_splits(M, N, K, workspace_bytes, mt)) {
    ks = tks;
    a.gper = (int)ceil_div(ng, ks);
    if (xt == X_F16X2)
      SM_TRY((mt == 1 ? launch_thick<4, 1, 2, X_F16X2>(a, EPI_ADD_F32, st, ks)
                      : launch_thick<4, 2, 2, X_F16X2>(a, EPI_ADD_F32, st, ks)));
    else
      SM_TRY((mt == 1 ? launch_thick<4, 1, 2, X_F16>(a, EPI_ADD_F32, st, ks)
                      : launch_thick<4, 2, 2, X_F16>(a, EPI_ADD_F32, st, ks)));
  } else {
    a.gper = (int)ceil_div(ng, ks);
    const int64_t rt = ceil_div(M, 16);
    if (xt == X_F16X2) SM_TRY(launch_grouped_lds<X_F16X2>(a, EPI_ADD_F32, st, rt, ks, false));
    else SM_TRY(launch_grouped_lds<X_F16>(a, EPI_ADD_F32, st, rt, ks, false));
  }
  const unsigned blocks = (unsigned)M;
  _Float16* h = static_cast<_Float16*>(h_out);
#define SM_ARK(V, KS)                                                                       \
  do {                                                                                      \
    if (wr)                                                                                 \
      splitk_add_rmsnorm_kernel<V, KS, true><<<blocks, 64 * V, 0, st>>>(                    \
          a.part, ks, M, resid, gamma, eps, h, wr, (int)E, logits, top_idx, top_w);         \
    else                                                                                    \
      splitk_add_rmsnorm_kernel<V, KS><<<blocks, 64 * V, 0, st>>>(a.part, ks, M, resid,     \
                                                                  gamma, eps, h);           \
  } while (0)
#define SM_ARN(V)                                                \
    case V:                                                      \
      if (ks == 2) SM_ARK(V, 2);                                 \
      else if (ks == 3) SM_ARK(V, 3);                            \
      else if (ks == 4) SM_ARK(V, 4);                            \
      else if (ks == 6) SM_ARK(V, 6);                            \
      else if (ks == 8) SM_ARK(V, 8);                            \
      else SM_ARK(V, 0);                                         \
      break;
  switch (N / 256) {
    SM_ARN(3)
    SM_ARN(4)
    SM_ARN(8)
    SM_ARN(12)
    SM_ARN(16)
    default: set_error("sm_q4_matmul_add_rmsnorm: width %lld", (long long)N); return SM_ERR_INVALID;
  }
#undef SM_ARN
#undef SM_ARK
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace
}  // namespace sm

extern "C" int sm_q4_matmul_add_rmsnorm(const uint8_t* codes, const uint16_t* scales, int64_t N,
                                        int64_t K, const void* x, int x_dtype, int64_t M,
                                        int64_t ldx, float* resid, const float* gamma, float eps,
                                        void* h_out, void* workspace, int64_t workspace_bytes,
                                        void* stream) {
  using namespace sm;
  SM_REQUIRE(resid && gamma && h_out, "sm_q4_matmul_add_rmsnorm: null buffer");
  return matmul_add_rmsnorm(codes, scales, N, K, x, x_dtype, M, ldx, resid, gamma, eps, h_out,
                            workspace, workspace_bytes, nullptr, 0, nullptr, nullptr, nullptr,
                            stream);
}

extern "C" int sm_q4_matmul_add_rmsnorm_router(
    const uint8_t* codes, const uint16_t* scales, int64_t N, int64_t K, const void* x,
    int x_dtype, int64_t M, int64_t ldx, float* resid, const float* gamma, float eps, void* h_out,
    const float* w_router, int64_t experts, float* router_logits, int32_t* top_idx,
    float* top_w, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace sm;
  SM_REQUIRE(resid && gamma && h_out && w_router && top_idx && top_w,
             "sm_q4_matmul_add_rmsnorm_router: null buffer");
  SM_REQUIRE(experts >= 2 && experts <= kRouterMaxExperts,
             "sm_q4_matmul_add_rmsnorm_router: experts must be in 2..=%d", kRouterMaxExperts);
  return matmul_add_rmsnorm(codes, scales, N, K, x, x_dtype, M, ldx, resid, gamma, eps, h_out,
                            workspace, workspace_bytes, w_router, experts, router_logits, top_idx,
                            top_w, stream);
}

extern "C" int sm_q4_grouped_matmul(const uint8_t* codes, const uint16_t* scales, int64_t experts,
                                    int64_t N, int64_t K, const void* x, int x_dtype, int64_t ldx,
                                    int gather, const int32_t* plan, int64_t tokens, int64_t top_k,
                                    void* y, int64_t ldy, int epilogue, void* stream) {
  using namespace sm;
  SM_REQUIRE(codes && scales && x && plan && y, "sm_q4_grouped_matmul: null buffer");
  SM_REQUIRE(experts >= 1 && K > 0 && K % 128 == 0 && N > 0,
             "sm_q4_grouped_matmul: K must be a positive multiple of 128");
  const int xt = xmode_of(x_dtype);
  SM_REQUIRE(xt >= 0, "sm_q4_grouped_matmul: x must be bf16, f16 or f16 pairs");
  SM_REQUIRE(epilogue >= EPI_STORE_F32 && epilogue <= EPI_SWIGLU_F16X2 && epilogue != EPI_ADD_F32,
             "sm_q4_grouped_matmul: epilogue must store (f32/bf16) or SwiGLU");
  const int64_t xw = (xt == X_F16X2) ? 2 * K : K;
  SM_REQUIRE(ldx >= xw && ldx % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0,
             "sm_q4_grouped_matmul: x must be 16-byte aligned rows of >= %lld elements",
             (long long)xw);
  SM_REQUIRE(!is_swiglu(epilogue) || N % 2 == 0, "sm_q4_grouped_matmul: SwiGLU needs even N");
  const int64_t routes = tokens * top_k;
  const int64_t ncols = is_swiglu(epilogue) ? N / 2 : N;
  SM_REQUIRE(ldy >= ((epilogue == EPI_SWIGLU_F16X2) ? 2 * ncols : ncols),
             "sm_q4_grouped_matmul: ldy < output row width");
  if (routes == 0) return SM_OK;
  PlanView pv = plan_view(const_cast<int32_t*>(plan), routes, experts);
  const size_t cstride = (size_t)q4t_rows(N) * (K / 2), sstride = (size_t)q4t_rows(N) * (K / 128);
  const int32_t* rowidx = gather ? pv.src_rows : nullptr;
  hipStream_t st = as_stream(stream);
  if (routes <= 4096) {
    Q4Args a{codes, scales, x, y, (int)routes, (int)N, (int)K, (int)ldx, (int)ldy, (int)ncols};
    a.tiles = pv.tiles16;
    a.ntiles = pv.ntiles16;
    a.goff = pv.offsets;
    a.rowidx = rowidx;
    a.cstride = cstride;
    a.sstride = sstride;
    const int64_t rt = moe_max_tiles(routes, experts, 16);
    if (xt == X_F16X2) return launch_grouped_lds<X_F16X2>(a, epilogue, st, rt);
    if (xt == X_F16) return launch_grouped_lds<X_F16>(a, epilogue, st, rt);
    if (is_swiglu(epilogue) || K < 4 * 128) return launch_q4<2, 1>(a, epilogue, xt, st, rt);
    return launch_q4<2, 4>(a, epilogue, xt, st, rt);
  }
  return q4_gemm_bl(codes, scales, (int)N, (int)K, x, xt, (int)routes, (int)ldx, y, (int)ldy,
                    epilogue, (int)ncols, st, pv.tiles128, pv.ntiles128,
                    moe_max_tiles(routes, experts, 128), pv.offsets, rowidx, cstride, sstride,
                    nullptr, 0, nullptr);
}

extern "C" int sm_q4_qkv_rope(const uint8_t* codes, const uint16_t* scales, int64_t H,
                              int64_t KVH, int64_t head_dim, int64_t K, const void* x,
                              int x_dtype, int64_t S, int64_t L, int64_t ldx,
                              const float* rope_table, const int32_t* pos0, int64_t cap,
                              void* q_out, void* kcache, void* vcache, int cache_dtype,
                              void* stream) {
  using namespace sm;
  SM_REQUIRE(codes && scales && x && rope_table && pos0 && q_out && kcache && vcache,
             "sm_q4_qkv_rope: null buffer");
  SM_REQUIRE(cache_dtype == SM_F16, "sm_q4_qkv_rope: the fused path writes f16 q / cache");
  SM_REQUIRE(H > 0 && KVH > 0 && head_dim >= 16 && (head_dim & (head_dim - 1)) == 0 && cap > 0 &&
                 S >= 0 && L > 0 && S * L <= 0x7fffffff,
             "sm_q4_qkv_rope: bad shape (head_dim a power of two >= 16)");
  SM_REQUIRE(K > 0 && K % 128 == 0, "sm_q4_qkv_rope: K must be a positive multiple of 128");
  const int xt = xmode_of(x_dtype);
  SM_REQUIRE(xt >= 0, "sm_q4_qkv_rope: x must be bf16, f16 or f16 pairs");
  const int64_t xw = (xt == X_F16X2) ? 2 * K : K;
  SM_REQUIRE(ldx >= xw && ldx % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(codes) % 16 == 0,
             "sm_q4_qkv_rope: x rows must be 16-byte aligned, >= %lld elements", (long long)xw);
  const int64_t N = (H + 2 * KVH) * head_dim;
  if (S == 0) return SM_OK;
  if (use_dense_lds(S * L, K, N, xt)) {
    Q4Args a{codes, scales, x, nullptr, (int)(S * L), (int)N, (int)K, (int)ldx, 0, (int)N};
    a.rope = reinterpret_cast<const float2*>(rope_table);
    a.pos0 = pos0;
    a.rope_L = (int)L;
    a.cap = (int)cap;
    a.H = (int)H;
    a.KVH = (int)KVH;
    a.hd = (int)head_dim;
    a.q_out = static_cast<_Float16*>(q_out);
    a.kc = static_cast<_Float16*>(kcache);
    a.vc = static_cast<_Float16*>(vcache);
    const int64_t rt = ceil_div(S * L, 16);
    if (xt == X_F16X2) return launch_grouped_lds<X_F16X2>(a, 6, as_stream(stream), rt);
    return launch_grouped_lds<X_F16>(a, 6, as_stream(stream), rt);
  }
  QkvRope qr{rope_table, pos0, (int)L, (int)cap, (int)H, (int)KVH, (int)head_dim,
             q_out, kcache, vcache};
  return q4_gemm_bl(codes, scales, (int)N, (int)K, x, xt, (int)(S * L), (int)ldx, nullptr, 0, 6,
                    (int)N, as_stream(stream), nullptr, nullptr, 0, nullptr, nullptr, 0, 0,
                    nullptr, 0, &qr);
}
