// Large-M Q4G128 GEMM for prefill and log-prob recompute (kernel 5: the
// MFMA-bound dense GEMMs of the recompute, Transformer::forward_selected_logits
// -> matmul::linear, summa-llm/src/model/transformer.rs:742-822, matmul.rs:57-66,
// here over this build's Q4G128 weights; same epilogues as q4.hip).
//
// Tiling (gfx950, v_mfma_f32_16x16x32_f16):
//   workgroup 256 threads = 2 x 2 waves, tile 256 (M) x 128 (N), K step = one
//   128-wide quantisation group;
//   wave tile 128 x 64 = 8 x 4 MFMA blocks (32 accumulator VGPR quads);
//   A (activations) is staged per K group in LDS (256 x 128 f16, rows padded
//   to 272 B so the 16 rows a ds_read_b128 touches hit distinct banks);
//   B (weights, prepared tiled layout: one contiguous 1 KB per 16 rows x
//   group) goes from HBM straight into registers: per group each lane
//   loads one 16-byte chunk per 16-column block and unpacks word s for
//   k-step s (common.hpp q4_unpack), scaled by the group scale (exact in f16).
// Dequantisation costs ~3.5/MT VALU cycles per MFMA cycle; with MT = 8 it is
// under half the MFMA time, so the kernel is MFMA/LDS bound.
// Tile order is XCD-aware: workgroup w runs on XCD w % 8, and the 8 workgroups
// of consecutive w share an N tile but take 8 different M tiles, while each
// XCD sweeps all N tiles of its M tile back to back, so an A tile stays in that
// XCD's L2 for the whole sweep and the (small) weight matrix in MALL/L2.
#include <cmath>

#include "common.hpp"

namespace sm {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kTM = 256, kTN = 128;  // workgroup tile
constexpr int kMT = 8, kNB = 4;      // wave tile in 16x16 blocks
constexpr int kAP = 128 + 8;         // padded LDS row (f16 elements)

__device__ inline float silu(float g) { return g / (1.f + __expf(-g)); }

struct Args {
  const uint8_t* codes;
  const uint16_t* scales;
  const void* x;
  void* y;
  int M, N, K, ldx, ldy, ncols;
  int mtiles8, ntiles;  // M tiles rounded up to a multiple of 8; N tiles
  // grouped (MoE) mode when tiles != nullptr (see Q4Args in q4.hip)
  const int32_t* tiles;
  const int32_t* ntiles_dev;
  const int32_t* goff;
  const int32_t* rowidx;
  size_t cstride, sstride;
};

// EPI: 0 store f32, 1 store bf16, 2 add f32, 3 swiglu bf16, 4 swiglu f16,
// 5 swiglu f16 pair. XT: 0 bf16 x, 1 f16 x, 2 f16-pair x (hi and lo tiles are
// both staged; each k-step issues the MFMA twice on the same B fragment).
template <int EPI, int XT>
__global__ __launch_bounds__(256, 1) void q4_gemm_lds_kernel(Args a) {
  constexpr bool SWIGLU = (EPI == 3 || EPI == 4 || EPI == 5);
  constexpr int NA = (XT == 2) ? 2 : 1;
  __shared__ __attribute__((aligned(16))) _Float16 As[NA][kTM * kAP];

  int tn, m_base, mlim = a.M;
  const uint8_t* codes = a.codes;
  const uint16_t* scales = a.scales;
  if (a.tiles) {
    // grouped: workgroup = (route-plan tile, N tile)
    tn = blockIdx.x % a.ntiles;
    const int ti = blockIdx.x / a.ntiles;
    if (ti >= a.ntiles_dev[0]) return;  // uniform per workgroup
    const int e = a.tiles[2 * ti];
    m_base = a.goff[e] + a.tiles[2 * ti + 1];
    mlim = a.goff[e + 1];
    codes += (size_t)e * a.cstride;
    scales += (size_t)e * a.sstride;
  } else {
    // XCD-aware tile order (see header).
    const int w = blockIdx.x;
    const int xcd = w % 8, q = w / 8;
    tn = q % a.ntiles;
    const int tm = (q / a.ntiles) * 8 + xcd;
    m_base = tm * kTM;
    if (m_base >= a.M) return;  // padding tile (uniform per workgroup)
  }

  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int wm = wave / 2, wn = wave % 2;  // 2 x 2 waves
  const int ngroups = a.K / 128;

  // B row of each of the wave's 4 column blocks.
  int brow[kNB];
#pragma unroll
  for (int b = 0; b < kNB; ++b) {
    if constexpr (SWIGLU) {
      // blocks 0,1: gate columns; 2,3: value columns of the same h columns
      const int hcol = tn * (kTN / 2) + wn * 32 + (b % 2) * 16 + j;
      brow[b] = (hcol < a.ncols) ? (b < 2 ? hcol : a.ncols + hcol) : -1;
    } else {
      const int col = tn * kTN + wn * 64 + b * 16 + j;
      brow[b] = (col < a.N) ? col : -1;
    }
  }

  f4 acc[kMT][kNB];
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int b = 0; b < kNB; ++b) acc[mt][b] = f4{0.f, 0.f, 0.f, 0.f};

  for (int kg = 0; kg < ngroups; ++kg) {
    // weights of this group (issued before the barrier so they overlap it)
    // branch-free loads (clamped row, scale zeroed later) so they all issue
    // back to back
    u32x4 wv[kNB];
    uint16_t sraw[kNB];
#pragma unroll
    for (int b = 0; b < kNB; ++b) {
      const int rr = brow[b] >= 0 ? brow[b] : 0;
      wv[b] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(codes + q4t_code_offset(rr, kg, ngroups) + g * 16));
      sraw[b] = scales[q4t_scale_index(rr, kg, ngroups)];
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();  // previous group's A fully consumed
    // stage A[m_base .. +256][kg*128 .. +128] as permuted f16 chunks
#pragma unroll 2
    for (int c = threadIdx.x; c < kTM * 16; c += 256) {
      const int r = c / 16, ch = c % 16;
      const int prow = min(m_base + r, mlim - 1);
      const int row = a.rowidx ? a.rowidx[prow] : prow;
      const size_t xo = (size_t)row * a.ldx + kg * 128 + ch * 8;
      const bool live = m_base + r < mlim;
      h8 v;
      if constexpr (XT != 0) {
        v = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(a.x) + xo);
      } else {
        const u32x4 u = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.x) + xo);
        v = h8{(_Float16)bf16lo(u.x), (_Float16)bf16hi(u.x), (_Float16)bf16lo(u.y),
               (_Float16)bf16hi(u.y), (_Float16)bf16lo(u.z), (_Float16)bf16hi(u.z),
               (_Float16)bf16lo(u.w), (_Float16)bf16hi(u.w)};
      }
      if (!live) v = h8{0, 0, 0, 0, 0, 0, 0, 0};
      *reinterpret_cast<h8*>(&As[0][r * kAP + ch * 8]) = v;
      if constexpr (NA == 2) {
        h8 lo = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(a.x) + xo + a.K);
        if (!live) lo = h8{0, 0, 0, 0, 0, 0, 0, 0};
        *reinterpret_cast<h8*>(&As[1][r * kAP + ch * 8]) = lo;
      }
    }
    __syncthreads();
    _Float16 sc[kNB];
#pragma unroll
    for (int b = 0; b < kNB; ++b) sc[b] = brow[b] >= 0 ? (_Float16)bf16_to_f32(sraw[b]) : (_Float16)0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      h8 bf[kNB];
#pragma unroll
      for (int b = 0; b < kNB; ++b) bf[b] = q4_unpack_scaled(wv[b][s], sc[b]);
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt) {
        const int r = wm * 128 + mt * 16 + j;
        const h8 af = *reinterpret_cast<const h8*>(&As[0][r * kAP + g * 32 + s * 8]);
#pragma unroll
        for (int b = 0; b < kNB; ++b)
          acc[mt][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[b], acc[mt][b], 0, 0, 0);
        if constexpr (NA == 2) {
          const h8 al = *reinterpret_cast<const h8*>(&As[1][r * kAP + g * 32 + s * 8]);
#pragma unroll
          for (int b = 0; b < kNB; ++b)
            acc[mt][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bf[b], acc[mt][b], 0, 0, 0);
        }
      }
    }
  }

  // epilogue: lane holds rows 4g + r of column j in every block
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m_base + wm * 128 + mt * 16 + 4 * g + r;
      if (row >= mlim) continue;
      if constexpr (SWIGLU) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const int hcol = tn * (kTN / 2) + wn * 32 + b * 16 + j;
          if (hcol >= a.ncols) continue;
          const float h = silu(acc[mt][b][r]) * acc[mt][b + 2][r];
          const size_t o = (size_t)row * a.ldy + hcol;
          if constexpr (EPI == 5) {
            _Float16 hi, lo;
            split_f16(h, hi, lo);
            static_cast<_Float16*>(a.y)[o] = hi;
            static_cast<_Float16*>(a.y)[o + a.ncols] = lo;
          } else if constexpr (EPI == 4) {
            static_cast<_Float16*>(a.y)[o] = (_Float16)h;
          } else {
            static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(h);
          }
        }
      } else {
#pragma unroll
        for (int b = 0; b < kNB; ++b) {
          const int col = tn * kTN + wn * 64 + b * 16 + j;
          if (col >= a.N) continue;
          const size_t o = (size_t)row * a.ldy + col;
          const float v = acc[mt][b][r];
          if constexpr (EPI == 0) static_cast<float*>(a.y)[o] = v;
          else if constexpr (EPI == 1) static_cast<uint16_t*>(a.y)[o] = f32_to_bf16(v);
          else static_cast<float*>(a.y)[o] += v;
        }
      }
    }
  }
}

}  // namespace

// Called by sm_q4_matmul for M > 256 (argument checks done there).
int q4_gemm_lds(const uint8_t* codes, const uint16_t* scales, int N, int K, const void* x,
                int xt, int M, int ldx, void* y, int ldy, int epi, int ncols, hipStream_t st,
                const int32_t* tiles, const int32_t* ntiles, int64_t max_tiles,
                const int32_t* goff, const int32_t* rowidx, size_t cstride, size_t sstride) {
  Args a{codes, scales, x, y, M, N, K, ldx, ldy, ncols, 0, 0,
         tiles, ntiles, goff, rowidx, cstride, sstride};
  const int logical_cols = (epi >= 3) ? 2 * ncols : N;
  a.ntiles = (int)ceil_div(logical_cols, kTN);
  a.mtiles8 = (int)ceil_div(ceil_div(M, kTM), 8) * 8;
  const int64_t blocks = (int64_t)(tiles ? max_tiles : a.mtiles8) * a.ntiles;
  if (blocks > 0x7fffffff) {
    set_error("sm_q4_matmul: problem too large");
    return SM_ERR_UNSUPPORTED;
  }
  const dim3 grid((unsigned)blocks);
#define SM_LDS(E)                                                                    \
  do {                                                                               \
    if (xt == 2) q4_gemm_lds_kernel<E, 2><<<grid, 256, 0, st>>>(a);                  \
    else if (xt == 1) q4_gemm_lds_kernel<E, 1><<<grid, 256, 0, st>>>(a);             \
    else q4_gemm_lds_kernel<E, 0><<<grid, 256, 0, st>>>(a);                          \
  } while (0)
  switch (epi) {
    case 0: SM_LDS(0); break;
    case 1: SM_LDS(1); break;
    case 2: SM_LDS(2); break;
    case 3: SM_LDS(3); break;
    case 4: SM_LDS(4); break;
    case 5: SM_LDS(5); break;
    default: set_error("sm_q4_matmul: unknown epilogue %d", epi); return SM_ERR_INVALID;
  }
#undef SM_LDS
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace sm
