// Q4G128 GEMM for large M (prefill and the log-prob recompute): the same
// contract, epilogues and bits as q4_gemm_bl.hip's kernel, with a 256 x 256
// workgroup tile that halves the activation re-reads of its 128-column tiles.
// (Linear::forward over a quantized weight, summa-llm/src/model/matmul.rs:57-66,
// transformer.rs:742-822.)
//
// Design (gfx950, v_mfma_f32_16x16x32_f16):
//   workgroup = 8 waves (two per SIMD) in a 4 x 2 grid, each wave 64 rows x
//   128 columns (4 x 8 MFMA tiles, the accumulators in AGPRs); one pipeline
//   stage = 32 k (one MFMA k-step). Both operands go through LDS, two stages
//   deep: activations (f16, or the hi and lo planes of f16 pairs) as 256 rows
//   x 32 k, and weights dequantised once per workgroup (scaled f16, exact for
//   an f16-normal scale) as 256 columns x 32 k, in 64-byte rows whose 16-byte
//   chunks are XOR-swizzled by row so fragment reads are free of bank conflicts.
//   Global loads for stage s+2 and the LDS writes of stage s+1 are placed
//   between the MFMA groups of stage s (scheduling fences pin the order; left
//   to itself the compiler put all staging work before the MFMAs, leaving the
//   matrix cores idle while the eight waves, in step after each barrier,
//   staged together). One barrier per stage.
// Per 32-k stage and wave: 16 fragment reads (8 with plain f16) feed 64 MFMAs
// (32), every weight fragment serving 4 row blocks and every activation
// fragment 8 column blocks. The accumulation order per output (k-steps in
// order, hi before lo) is that of q4_gemm_bl_kernel, so both kernels produce
// identical results and callers may pick either by shape.
// Measured (MI355X, f16 pairs): 550-565 TF/s algorithmic on the config[2]
// recompute shapes against 400-457 TF/s for the 128 x 128 kernel.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "q4_internal.hpp"

namespace sm {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWM = 256, kWN = 256, kWK = 32;
constexpr int kWP = 32;  // LDS row: 32 k (64 bytes), 16-byte chunks swizzled
// Chunk c of row r sits at chunk c ^ ((r >> 1) & 3): the 16-byte fragment reads
// of a wave (16 rows x 4 chunks) then touch every bank group once per pass.
// Measured on MI355X (one 512-thread workgroup per CU, 16 fragment reads per
// wave): 357 ns per stage, against 598 ns with 80-byte padded rows.
__device__ inline int wsw(int row, int chunk) { return row * kWP + ((chunk ^ ((row >> 1) & 3)) << 3); }

__device__ inline float silu_w(float g) { return g / (1.f + __expf(-g)); }

struct WideArgs {
  const uint8_t* codes;
  const uint16_t* scales;
  const _Float16* x;
  void* y;
  int M, N, K, ldx, ldy, ncols;
  int mtiles, mtiles8, ntiles;
  // EPI 6 (qkv projection + RoPE + KV-cache append), as in q4_gemm_bl.hip
  const float2* rope;
  const int32_t* pos0;
  int rope_L, cap, H, KVH, hd;
  _Float16* q_out;
  _Float16* kc;
  _Float16* vc;
};

// EPI: 0 store f32, 1 store bf16, 2 add f32, 3 swiglu bf16, 4 swiglu f16,
// 5 swiglu f16 pair, 6 qkv + RoPE + cache append (f16). NA: 1 f16 x, 2 pairs.
template <int NA, int EPI>
__global__ __launch_bounds__(512, 1) void q4_gemm_wide_kernel(WideArgs a) {
  constexpr bool SWIGLU = (EPI >= 3 && EPI <= 5);
  constexpr int MT = 4, NB = 8;  // 16-row / 16-column blocks per wave
  __shared__ __attribute__((aligned(16))) _Float16 As[2][NA][kWM * kWP];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][kWN * kWP];

  // ---- tile: XCD-aware when there are >= 8 row tiles (workgroups w..w+7,
  //      one per XCD, take 8 row tiles of one column tile; each XCD sweeps
  //      the column tiles of its row tile back to back)
  int tn, tm;
  if (a.mtiles >= 8) {
    const int w = blockIdx.x, xcd = w % 8, q = w / 8;
    tn = q % a.ntiles;
    tm = (q / a.ntiles) * 8 + xcd;
    if (tm >= a.mtiles) return;  // padding tile (uniform per workgroup)
  } else {
    tn = blockIdx.x % a.ntiles;
    tm = blockIdx.x / a.ntiles;
  }
  const int m0 = tm * kWM;
  const int t = threadIdx.x, wave = t / kWave, lane = t % kWave;
  const int j = lane % 16, g = lane / 16;
  const int wr = wave / 2, wc = wave % 2;
  const int ngroups = a.K / 128, nst = a.K / kWK;

  // ---- staging assignments. Activations: 16-byte chunk c = i*512 + t of the
  //      256 x 32 stage is row c/4, k 8*(c%4). Weights: thread t dequantises
  //      half (16 k) of LDS column t/2.
  int aoff[2];
  const _Float16* xa[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = i * 512 + t;
    aoff[i] = wsw(c / 4, c % 4);
    xa[i] = a.x + (size_t)min(m0 + c / 4, a.M - 1) * a.ldx + (c % 4) * 8;
  }
  const int bcol = t / 2, bhalf = t & 1;
  int wrow;  // weight row staged into LDS column bcol (-1: zero column)
  {
    const int wcx = bcol / 128, bb = (bcol % 128) / 16, jj = bcol % 16;
    if constexpr (SWIGLU) {
      // wave column half wcx: blocks 0-3 gate, 4-7 value of the same h columns
      const int hcol = tn * (kWN / 2) + wcx * 64 + (bb % 4) * 16 + jj;
      wrow = hcol < a.ncols ? (bb < 4 ? hcol : a.ncols + hcol) : -1;
    } else {
      const int col = tn * kWN + bcol;
      wrow = col < a.N ? col : -1;
    }
  }
  const uint8_t* cbase = a.codes + q4t_code_offset(max(wrow, 0), 0, ngroups) + bhalf * 8;
  const uint16_t* sbase = a.scales + q4t_scale_index(max(wrow, 0), 0, ngroups);
  const int boff0 = wsw(bcol, bhalf * 2), boff1 = wsw(bcol, bhalf * 2 + 1);

  u32x4 ra[NA][2];
  u32x2 rb;
  uint16_t rs;
  auto gload_a = [&](int s) {
    const int k0 = min(s, nst - 1) * kWK;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      ra[0][i] = *reinterpret_cast<const u32x4*>(xa[i] + k0);
      if constexpr (NA == 2) ra[1][i] = *reinterpret_cast<const u32x4*>(xa[i] + k0 + a.K);
    }
  };
  auto gload_b = [&](int s) {
    const int s2 = min(s, nst - 1);
    const int kg = s2 >> 2, kq = s2 & 3;  // group, 32-k quarter of the group
    rb = __builtin_nontemporal_load(
        reinterpret_cast<const u32x2*>(cbase + (size_t)kg * 1024 + kq * 16));
    rs = sbase[kg * 16];
  };
  auto store_a = [&](int buf, int h) {
#pragma unroll
    for (int i = 0; i < 2; ++i) *reinterpret_cast<u32x4*>(&As[buf][h][aoff[i]]) = ra[h][i];
  };
  auto store_b = [&](int buf, int w) {
    const _Float16 sc = wrow >= 0 ? (_Float16)bf16_to_f32(rs) : (_Float16)0.f;
    *reinterpret_cast<h8*>(&Bs[buf][w ? boff1 : boff0]) = q4_unpack_scaled(rb[w], sc);
  };

  f4 acc[MT][NB];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[mt][b] = f4{0.f, 0.f, 0.f, 0.f};

  gload_a(0);
  gload_b(0);
  store_a(0, 0);
  if constexpr (NA == 2) store_a(0, 1);
  store_b(0, 0);
  store_b(0, 1);
  gload_a(1);
  gload_b(1);
  __syncthreads();
  for (int s = 0; s < nst; ++s) {
    const int buf = s & 1, nb = buf ^ 1;
    h8 fa[NA][MT], fb[NB];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      fa[0][mt] = *reinterpret_cast<const h8*>(&As[buf][0][wsw(wr * 64 + mt * 16 + j, g)]);
#pragma unroll
    for (int b = 0; b < NB; ++b)
      fb[b] = *reinterpret_cast<const h8*>(&Bs[buf][wsw(wc * 128 + b * 16 + j, g)]);
    if constexpr (NA == 2) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        fa[1][mt] =
            *reinterpret_cast<const h8*>(&As[buf][1][wsw(wr * 64 + mt * 16 + j, g)]);
    }
    auto mm = [&](int h, int b) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[h][mt], fb[b], acc[mt][b], 0, 0, 0);
    };
    // The stage s+1 writes go to the other buffer, last read in stage s-1
    // (before the previous barrier); on the last stage they fill a buffer
    // nobody reads, which keeps the loop body free of branches.
    __builtin_amdgcn_sched_barrier(0);
    mm(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    store_a(nb, 0);
    __builtin_amdgcn_sched_barrier(0);
    mm(0, 1);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NA == 2) store_a(nb, 1);
    __builtin_amdgcn_sched_barrier(0);
    mm(0, 2);
    __builtin_amdgcn_sched_barrier(0);
    store_b(nb, 0);
    __builtin_amdgcn_sched_barrier(0);
    mm(0, 3);
    __builtin_amdgcn_sched_barrier(0);
    store_b(nb, 1);
    __builtin_amdgcn_sched_barrier(0);
    mm(0, 4);
    __builtin_amdgcn_sched_barrier(0);
    gload_a(s + 2);
    __builtin_amdgcn_sched_barrier(0);
    mm(0, 5);
    __builtin_amdgcn_sched_barrier(0);
    gload_b(s + 2);
    __builtin_amdgcn_sched_barrier(0);
    mm(0, 6);
    mm(0, 7);
    if constexpr (NA == 2) {
#pragma unroll
      for (int b = 0; b < NB; ++b) mm(1, b);
    }
    __syncthreads();
  }

  // ---- epilogue: lane holds rows 4g + r of column j in every block
  if constexpr (EPI == 6) {
    // RoPE pairs (2p, 2p+1) are adjacent columns, i.e. lanes j and j^1: every
    // lane takes part in the swap, even lanes store the rotated pair. Row
    // positions are computed here (once per tile, after the long K loop).
    const int hd_shift = __builtin_ctz(a.hd);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wr * 64 + mt * 16 + 4 * g + r;
        const int rc = min(row, a.M - 1);
        const int sq = (a.rope_L == 1) ? rc : rc / a.rope_L;
        const int pos = a.pos0[sq] + (rc - sq * a.rope_L);
        const bool ok = row < a.M && pos >= 0 && pos < a.cap;
        const float2* rrow = a.rope + (size_t)(ok ? pos : 0) * (a.hd / 2);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const float va = acc[mt][b][r];
          const float vb = __shfl_xor(va, 1, kWave);  // column e + 1
          const int col = tn * kWN + wc * 128 + b * 16 + j;
          if (!ok || (j & 1) || col >= a.N) continue;
          const int slot = col >> hd_shift, e = col & (a.hd - 1);
          h2 out;
          _Float16* dst;
          if (slot >= a.H + a.KVH) {  // value: no rotation
            out = h2{(_Float16)va, (_Float16)vb};
            dst = a.vc + (((size_t)sq * a.KVH + (slot - a.H - a.KVH)) * a.cap + pos) * a.hd + e;
          } else {
            const float2 c = rrow[e >> 1];
            out = h2{(_Float16)(va * c.x - vb * c.y), (_Float16)(vb * c.x + va * c.y)};
            dst = (slot < a.H)
                      ? a.q_out + ((size_t)row * a.H + slot) * a.hd + e
                      : a.kc + (((size_t)sq * a.KVH + (slot - a.H)) * a.cap + pos) * a.hd + e;
          }
          *reinterpret_cast<h2*>(dst) = out;
        }
      }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m0 + wr * 64 + mt * 16 + 4 * g + r;
      if (row >= a.M) continue;
      if constexpr (SWIGLU) {
#pragma unroll
        for (int b = 0; b < NB / 2; ++b) {
          const int hcol = tn * (kWN / 2) + wc * 64 + b * 16 + j;
          if (hcol >= a.ncols) continue;
          const float h = silu_w(acc[mt][b][r]) * acc[mt][b + NB / 2][r];
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
        for (int b = 0; b < NB; ++b) {
          const int col = tn * kWN + wc * 128 + b * 16 + j;
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

template <int NA>
int launch_wide(const WideArgs& a, int epi, unsigned grid, hipStream_t st) {
  switch (epi) {
#define SM_WIDE(E) \
    case E: q4_gemm_wide_kernel<NA, E><<<grid, 512, 0, st>>>(a); break;
    SM_WIDE(0)
    SM_WIDE(1)
    SM_WIDE(2)
    SM_WIDE(3)
    SM_WIDE(4)
    SM_WIDE(5)
    SM_WIDE(6)
#undef SM_WIDE
    default: set_error("sm_q4_matmul: unknown epilogue %d", epi); return SM_ERR_INVALID;
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace

int64_t q4_wide_tiles(int M, int N, int ncols, int epi) {
  const bool swiglu = epi >= 3 && epi <= 5;
  const int64_t logical_cols = swiglu ? 2 * (int64_t)ncols : N;
  return ceil_div(M, kWM) * ceil_div(logical_cols, kWN);
}

int q4_gemm_wide(const uint8_t* codes, const uint16_t* scales, int N, int K, const void* x,
                 int xt, int M, int ldx, void* y, int ldy, int epi, int ncols, hipStream_t st,
                 const QkvRope* qr) {
  WideArgs a{};
  a.codes = codes;
  a.scales = scales;
  a.x = static_cast<const _Float16*>(x);
  a.y = y;
  a.M = M;
  a.N = N;
  a.K = K;
  a.ldx = ldx;
  a.ldy = ldy;
  a.ncols = ncols;
  if (epi == 6) {
    a.rope = reinterpret_cast<const float2*>(qr->rope);
    a.pos0 = qr->pos0;
    a.rope_L = qr->L;
    a.cap = qr->cap;
    a.H = qr->H;
    a.KVH = qr->KVH;
    a.hd = qr->hd;
    a.q_out = static_cast<_Float16*>(qr->q_out);
    a.kc = static_cast<_Float16*>(qr->kc);
    a.vc = static_cast<_Float16*>(qr->vc);
  }
  const bool swiglu = epi >= 3 && epi <= 5;
  const int64_t logical_cols = swiglu ? 2 * (int64_t)ncols : N;
  const int64_t mtiles = ceil_div(M, kWM);
  a.mtiles = (int)mtiles;
  a.ntiles = (int)ceil_div(logical_cols, kWN);
  a.mtiles8 = (int)(mtiles >= 8 ? ceil_div(mtiles, 8) * 8 : mtiles);
  const int64_t blocks = (int64_t)a.mtiles8 * a.ntiles;
  if (blocks > 0x7fffffff) {
    set_error("sm_q4_matmul: problem too large");
    return SM_ERR_UNSUPPORTED;
  }
  return xt == 2 ? launch_wide<2>(a, epi, (unsigned)blocks, st)
                 : launch_wide<1>(a, epi, (unsigned)blocks, st);
}

}  // namespace sm
