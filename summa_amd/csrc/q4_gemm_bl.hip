// Q4G128 GEMM for M > 32 rows: decode batches (M = rollouts), prefill and the
// log-prob recompute (kernels 1 and 5 at batch size; same contract and
// epilogues as q4.hip: Linear::forward over a quantized weight,
// summa-llm/src/model/matmul.rs:57-66, transformer.rs:742-822).
//
// Design (gfx950, v_mfma_f32_16x16x32_f16), "weights in LDS, activations in
// registers":
//   workgroup = 4 waves, tile TM = 4*WR rows x TN columns, K step = one
//   128-wide quantisation group. Each weight group tile (TN rows of W x 128 k)
//   is read once per workgroup from the prepared layout (1 KB per 16 rows,
//   one 16-byte load per thread and 16 rows), dequantised once (scaled f16,
//   exact for an f16-normal scale) into an LDS buffer [TN][128] shared by
//   the four waves; buffers alternate per group, so one barrier per group
//   separates writing group g+1 from reading group g.
//   Each wave owns WR distinct rows: its A fragments (16 rows x 32 k, one
//   16-byte load per lane, two for f16 pairs) go straight from global memory
//   into registers, prefetched one group ahead; no A staging, no sharing.
//   Each B fragment read from LDS feeds WR/16 (x2 for pairs) MFMAs.
// The dequantisation is done once per workgroup instead of once per 16 rows
// (q4.hip's small-M kernel), so batch GEMMs are MFMA-bound rather than
// VALU-bound. Tile order is XCD-aware when there are >= 8 row tiles: the 8
// workgroups w..w+7 (one per XCD) take 8 different row tiles of one column
// tile, and each XCD sweeps the column tiles of its row tile back to back,
// keeping that row tile's activations in the XCD's L2.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "q4_internal.hpp"

namespace sm {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kBP = 128;  // LDS row of one weight row's group (f16), 16 chunks of 16 bytes
// Chunk c of row r sits at chunk c ^ (r & 15): the fragment reads of a wave
// (16 rows, one chunk column each) spread over every bank group. Measured on
// MI355X (two 256-thread workgroups per CU, 32 fragment reads per wave and
// group): 575 ns per group against 1069 ns with 272-byte padded rows; the
// staging stores cost the same.
__device__ inline int bsw(int row, int chunk) { return row * kBP + ((chunk ^ (row & 15)) << 3); }

__device__ inline float silu(float g) { return g / (1.f + __expf(-g)); }

struct BLArgs {
  const uint8_t* codes;
  const uint16_t* scales;
  const void* x;
  void* y;
  int M, N, K, ldx, ldy, ncols;
  int mtiles, mtiles8, ntiles;  // row tiles, rounded up to 8; column tiles
  // grouped (MoE) mode when tiles != nullptr: workgroup = (plan tile, column
  // tile); a plan tile is (expert e, first row r) over sorted positions
  // goff[e] + r .. goff[e+1]-1; A row of position p = rowidx[p] (or p).
  const int32_t* tiles;
  const int32_t* ntiles_dev;
  const int32_t* goff;
  const int32_t* rowidx;
  size_t cstride, sstride;
  // split-K (dense mode only): blockIdx.y = split kz covers groups
  // [kz*gper, min(K/128, (kz+1)*gper)) and writes its f32 partial tile to
  // part[kz][row][logical column]; splitk_reduce_kernel sums the splits in
  // split order and applies the epilogue.
  float* part;
  int gper;
  // EPI 6 (qkv projection + RoPE + KV-cache append): row = s*rope_L + i sits
  // at position pos0[s] + i; columns are [q | k | v] heads of hd.
  const float2* rope;  // [max_pos][hd/2] (cos, sin)
  const int32_t* pos0;
  int rope_L, cap, H, KVH, hd;
  _Float16* q_out;  // [M][H][hd]
  _Float16* kc;     // [S][KVH][cap][hd]
  _Float16* vc;
};

// EPI: 0 store f32, 1 store bf16, 2 add f32, 3 swiglu bf16, 4 swiglu f16,
// 5 swiglu f16 pair, 6 qkv + RoPE + cache append (f16). XT: 0 bf16 x, 1 f16 x,
// 2 f16-pair x.
template <int WR, int TN, int EPI, int XT>
__global__ __launch_bounds__(256, 2) void q4_gemm_bl_kernel(BLArgs a) {
  constexpr bool SWIGLU = (EPI >= 3 && EPI <= 5);
  constexpr int NA = (XT == 2) ? 2 : 1;  // A fragments per k-step (hi, lo)
  constexpr int MT = WR / 16;            // 16-row blocks per wave
  constexpr int NBK = TN / 16;           // 16-column blocks per workgroup
  constexpr int CPT = TN / 64;           // 16-byte code chunks per thread per group
  static_assert(CPT >= 1 && (!SWIGLU || NBK % 2 == 0), "tile shape");
  __shared__ __attribute__((aligned(16))) _Float16 Bs[2][TN * kBP];

  // ---- which tile
  int tn, m_base, mlim = a.M;
  const uint8_t* codes = a.codes;
  const uint16_t* scales = a.scales;
  if (a.tiles) {
    tn = blockIdx.x % a.ntiles;
    const int ti = blockIdx.x / a.ntiles;
    if (ti >= a.ntiles_dev[0]) return;  // uniform per workgroup
    const int e = a.tiles[2 * ti];
    m_base = a.goff[e] + a.tiles[2 * ti + 1];
    mlim = a.goff[e + 1];
    codes += (size_t)e * a.cstride;
    scales += (size_t)e * a.sstride;
  } else if (a.mtiles >= 8) {
    const int w = blockIdx.x;
    const int xcd = w % 8, q = w / 8;
    tn = q % a.ntiles;
    const int tm = (q / a.ntiles) * 8 + xcd;
    if (tm >= a.mtiles) return;  // padding tile (uniform per workgroup)
    m_base = tm * 4 * WR;
  } else {
    tn = blockIdx.x % a.ntiles;
    m_base = (blockIdx.x / a.ntiles) * 4 * WR;
  }
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int ngroups = a.K / 128;
  const int g0 = blockIdx.y * a.gper;
  const int g1 = min(ngroups, g0 + a.gper);  // host guarantees g0 < g1

  // ---- weight rows this thread stages: chunk c = i*256 + t covers tile
  //      c/64 (16 LDS rows), LDS row (c/64)*16 + c%16, k 32*((c%64)/16) + 0..31
  int wrow[CPT], lrow[CPT], kq[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = i * 256 + threadIdx.x;
    const int lr = (c / 64) * 16 + (c % 16);  // LDS row = column of this tile
    lrow[i] = lr;
    kq[i] = ((c % 64) / 16) * 32;
    int n;
    if constexpr (SWIGLU) {
      // LDS rows [0, TN/2): gate columns, [TN/2, TN): value columns, same h cols
      const int hcol = tn * (TN / 2) + (lr % (TN / 2));
      n = (hcol < a.ncols) ? ((lr < TN / 2) ? hcol : a.ncols + hcol) : -1;
    } else {
      const int col = tn * TN + lr;
      n = (col < a.N) ? col : -1;
    }
    wrow[i] = n;
  }
  auto load_codes = [&](int kg, u32x4 (&cw)[CPT], uint16_t (&cs)[CPT]) {
    const int kc = min(kg, g1 - 1);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int n = wrow[i] >= 0 ? wrow[i] : 0;
      cw[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(codes + q4t_code_offset(n, kc, ngroups) + kq[i] / 2));
      cs[i] = scales[q4t_scale_index(n, kc, ngroups)];
    }
  };
  auto stage = [&](int buf, const u32x4 (&cw)[CPT], const uint16_t (&cs)[CPT]) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const _Float16 sc = wrow[i] >= 0 ? (_Float16)bf16_to_f32(cs[i]) : (_Float16)0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        *reinterpret_cast<h8*>(&Bs[buf][bsw(lrow[i], kq[i] / 8 + w)]) =
            q4_unpack_scaled(cw[i][w], sc);
    }
  };

  // ---- A fragments of this wave: rows m_base + wave*WR + mt*16 + j. Rows at
  //      or past mlim read a clamped valid row: they only feed output rows
  //      that the epilogue never stores.
  int arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int pc = min(m_base + wave * WR + mt * 16 + j, mlim - 1);
    arow[mt] = a.rowidx ? a.rowidx[pc] : pc;
  }
  auto load_a = [&](int kg, h8 (&af)[MT][4][NA]) {
    const int kc = min(kg, g1 - 1);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const size_t xo = (size_t)arow[mt] * a.ldx + kc * 128 + s * 32 + g * 8;
        if constexpr (XT == 0) {
          const u32x4 u = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.x) + xo);
          af[mt][s][0] = h8{(_Float16)bf16lo(u.x), (_Float16)bf16hi(u.x), (_Float16)bf16lo(u.y),
                            (_Float16)bf16hi(u.y), (_Float16)bf16lo(u.z), (_Float16)bf16hi(u.z),
                            (_Float16)bf16lo(u.w), (_Float16)bf16hi(u.w)};
        } else {
          af[mt][s][0] = *reinterpret_cast<const h8*>(static_cast<const _Float16*>(a.x) + xo);
          if constexpr (NA == 2)
            af[mt][s][1] =
                *reinterpret_cast<const h8*>(static_cast<const _Float16*>(a.x) + xo + a.K);
        }
      }
  };

  // EPI 6: the epilogue's positions and RoPE factors do not depend on the
  // product: load them before the main loop so their latency is hidden behind
  // it. Even lanes own pairs (e, e+1).
  int slot_b[NBK], e_b[NBK];
  int srow[MT][4], prow[MT][4];
  float2 cs[MT][4][NBK];
  if constexpr (EPI == 6) {
    const int hd_shift = __builtin_ctz(a.hd);
#pragma unroll
    for (int b = 0; b < NBK; ++b) {
      const int col = tn * TN + b * 16 + j;
      slot_b[b] = col < a.N ? (col >> hd_shift) : -1;
      e_b[b] = col & (a.hd - 1);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m_base + wave * WR + mt * 16 + 4 * g + r;
        const int rc = min(row, mlim - 1);
        const int sq = (a.rope_L == 1) ? rc : rc / a.rope_L;
        const int pos = a.pos0[sq] + (rc - sq * a.rope_L);
        srow[mt][r] = sq;
        prow[mt][r] = (row < mlim && pos >= 0 && pos < a.cap) ? pos : -1;
      }
  }
  // (cos, sin) pairs: loaded here for one row block per wave, their loads
  // completing during the main loop; 32-row waves load them in the epilogue
  // (registers)
  auto load_rope = [&]() {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float2* rrow = a.rope + (size_t)max(prow[mt][r], 0) * (a.hd / 2);
#pragma unroll
        for (int b = 0; b < NBK; ++b) cs[mt][r][b] = rrow[e_b[b] >> 1];
      }
  };
  if constexpr (EPI == 6 && MT == 1) load_rope();

  f4 acc[MT][NBK];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int b = 0; b < NBK; ++b) acc[mt][b] = f4{0.f, 0.f, 0.f, 0.f};

  // One group: prefetch group kg+1 (weights and activations), run the MFMAs
  // of group kg from LDS buffer kg&1 and registers `acur`, then stage group
  // kg+1 into the other buffer. Per k-step all B fragments are read first and
  // the lo MFMAs follow all hi MFMAs, so dependent MFMAs on one accumulator
  // are MT*NBK instructions apart.
  auto group = [&](int kg, const h8 (&acur)[MT][4][NA], h8 (&anext)[MT][4][NA]) {
    const int buf = (kg - g0) & 1;
    u32x4 cw[CPT];
    uint16_t cs[CPT];
    load_codes(kg + 1, cw, cs);
    load_a(kg + 1, anext);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      h8 bf[NBK];
#pragma unroll
      for (int b = 0; b < NBK; ++b)
        bf[b] = *reinterpret_cast<const h8*>(&Bs[buf][bsw(b * 16 + j, s * 4 + g)]);
#pragma unroll
      for (int h = 0; h < NA; ++h)
#pragma unroll
        for (int b = 0; b < NBK; ++b)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[mt][b] =
                __builtin_amdgcn_mfma_f32_16x16x32_f16(acur[mt][s][h], bf[b], acc[mt][b], 0, 0, 0);
    }
    if (kg + 1 < g1) stage(buf ^ 1, cw, cs);
    __syncthreads();
  };

  // prologue: group 0 staged, its A in registers; then ping-pong A buffers
  h8 a0[MT][4][NA], a1[MT][4][NA];
  {
    u32x4 cw[CPT];
    uint16_t cs[CPT];
    load_codes(g0, cw, cs);
    load_a(g0, a0);
    stage(0, cw, cs);
  }
  __syncthreads();
  for (int kg = g0; kg < g1; kg += 2) {
    group(kg, a0, a1);
    if (kg + 1 < g1) group(kg + 1, a1, a0);
  }

  // ---- epilogue: lane holds rows 4g + r of column j in every block
  if constexpr (EPI == 6) {
    // RoPE pairs (2p, 2p+1) are adjacent columns, i.e. lanes j and j^1 of the
    // same rows: swap partners before any lane-dependent branch
    f4 partner[MT][NBK];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int b = 0; b < NBK; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) partner[mt][b][r] = __shfl_xor(acc[mt][b][r], 1, kWave);
    if constexpr (MT > 1) load_rope();
    if ((j & 1) == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int pos = prow[mt][r];
          if (pos < 0) continue;
          const int row = m_base + wave * WR + mt * 16 + 4 * g + r, sq = srow[mt][r];
#pragma unroll
          for (int b = 0; b < NBK; ++b) {
            const int slot = slot_b[b], e = e_b[b];
            if (slot < 0) continue;
            const float va = acc[mt][b][r], vb = partner[mt][b][r];  // columns e, e+1
            h2 out;
            _Float16* dst;
            if (slot >= a.H + a.KVH) {  // value: no rotation
              out = h2{(_Float16)va, (_Float16)vb};
              dst = a.vc + (((size_t)sq * a.KVH + (slot - a.H - a.KVH)) * a.cap + pos) * a.hd + e;
            } else {
              const float2 c = cs[mt][r][b];
              out = h2{(_Float16)(va * c.x - vb * c.y), (_Float16)(vb * c.x + va * c.y)};
              dst = (slot < a.H)
                        ? a.q_out + ((size_t)row * a.H + slot) * a.hd + e
                        : a.kc + (((size_t)sq * a.KVH + (slot - a.H)) * a.cap + pos) * a.hd + e;
            }
            *reinterpret_cast<h2*>(dst) = out;
          }
        }
    }
    return;
  }
  if (a.part) {  // split-K (uniform branch): partial tile, logical columns
    const int lc_total = SWIGLU ? 2 * a.ncols : a.N;
    float* pp = a.part + (size_t)blockIdx.y * a.M * lc_total;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m_base + wave * WR + mt * 16 + 4 * g + r;
        if (row >= mlim) continue;
#pragma unroll
        for (int b = 0; b < NBK; ++b) {
          int lc;
          if constexpr (SWIGLU) {
            const int hcol = tn * (TN / 2) + (b % (NBK / 2)) * 16 + j;
            if (hcol >= a.ncols) continue;
            lc = (b < NBK / 2) ? hcol : a.ncols + hcol;
          } else {
            lc = tn * TN + b * 16 + j;
            if (lc >= a.N) continue;
          }
          pp[(size_t)row * lc_total + lc] = acc[mt][b][r];
        }
      }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = m_base + wave * WR + mt * 16 + 4 * g + r;
      if (row >= mlim) continue;
      if constexpr (SWIGLU) {
#pragma unroll
        for (int b = 0; b < NBK / 2; ++b) {
          const int hcol = tn * (TN / 2) + b * 16 + j;
          if (hcol >= a.ncols) continue;
          const float h = silu(acc[mt][b][r]) * acc[mt][b + NBK / 2][r];
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
        for (int b = 0; b < NBK; ++b) {
          const int col = tn * TN + b * 16 + j;
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

// Sums the split-K partials in split order and applies the epilogue.
template <int EPI>
__global__ void splitk_reduce_kernel(const float* __restrict__ part, int ks, int M, int N,
                                     int ncols, void* __restrict__ y, int ldy) {
  constexpr bool SWIGLU = (EPI >= 3);
  const int lc_total = SWIGLU ? 2 * ncols : N;
  const int width = SWIGLU ? ncols : N;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * width) return;
  const int row = (int)(i / width), c = (int)(i % width);
  const size_t split = (size_t)M * lc_total;
  const float* p = part + (size_t)row * lc_total + c;
  float v = 0.f;
  for (int k = 0; k < ks; ++k) v += p[k * split];
  const size_t o = (size_t)row * ldy + c;
  if constexpr (SWIGLU) {
    float u = 0.f;
    for (int k = 0; k < ks; ++k) u += p[k * split + ncols];
    const float h = silu(v) * u;
    if constexpr (EPI == 5) {
      _Float16 hi, lo;
      split_f16(h, hi, lo);
      static_cast<_Float16*>(y)[o] = hi;
      static_cast<_Float16*>(y)[o + ncols] = lo;
    } else if constexpr (EPI == 4) {
      static_cast<_Float16*>(y)[o] = (_Float16)h;
    } else {
      static_cast<uint16_t*>(y)[o] = f32_to_bf16(h);
    }
  } else if constexpr (EPI == 0) {
    static_cast<float*>(y)[o] = v;
  } else if constexpr (EPI == 1) {
    static_cast<uint16_t*>(y)[o] = f32_to_bf16(v);
  } else {
    static_cast<float*>(y)[o] += v;
  }
}

template <int WR, int TN, int XT>
int launch_bl(const BLArgs& a, int epi, dim3 grid, hipStream_t st) {
  switch (epi) {
#define SM_BL(E) \
    case E: q4_gemm_bl_kernel<WR, TN, E, XT><<<grid, 256, 0, st>>>(a); break;
    SM_BL(0)
    SM_BL(1)
    SM_BL(2)
    SM_BL(3)
    SM_BL(4)
    SM_BL(5)
    SM_BL(6)
#undef SM_BL
    default: set_error("sm_q4_matmul: unknown epilogue %d", epi); return SM_ERR_INVALID;
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

template <int WR, int TN>
int launch_bl_x(const BLArgs& a, int epi, int xt, dim3 grid, hipStream_t st) {
  if (xt == 2) return launch_bl<WR, TN, 2>(a, epi, grid, st);
  if (xt == 1) return launch_bl<WR, TN, 1>(a, epi, grid, st);
  return launch_bl<WR, TN, 0>(a, epi, grid, st);
}

}  // namespace

// Split-K workspace: the fp32 partials [splits][M][cols].
int64_t bl_counter_bytes() { return 0; }

constexpr int64_t kWideMinTiles = 128;

// Batch-M Q4 matmul (argument checks done by the callers in q4.hip).
// Dense mode (tiles == nullptr): rows 0..M-1. Grouped mode: the route plan's
// 128-row tile list (max_tiles entries at most). With a workspace (ws,
// ws_bytes) a dense call whose grid would underfill the chip splits K over up
// to 8 workgroups per tile; a second kernel sums the splits in order.
int q4_gemm_bl(const uint8_t* codes, const uint16_t* scales, int N, int K, const void* x, int xt,
               int M, int ldx, void* y, int ldy, int epi, int ncols, hipStream_t st,
               const int32_t* tiles, const int32_t* ntiles, int64_t max_tiles,
               const int32_t* goff, const int32_t* rowidx, size_t cstride, size_t sstride,
               void* ws, int64_t ws_bytes, const QkvRope* qr) {
  // Large dense problems with f16 / f16-pair activations: the 256 x 256 tile
  // kernel (same results), once it has at least half a wave of workgroups
  // (one per CU) and its row tiles are at least 3/4 full; measured faster
  // there (at M = 128 the half-empty tiles made the LM head 2x slower).
  const int64_t wide_rows = ceil_div(M, 256) * 256;
  if (!tiles && (xt == 1 || xt == 2) && M >= 256 && (wide_rows - M) * 4 <= wide_rows &&
      q4_wide_tiles(M, N, ncols, epi) >= kWideMinTiles)
    return q4_gemm_wide(codes, scales, N, K, x, xt, M, ldx, y, ldy, epi, ncols, st, qr);
  BLArgs a{codes, scales, x, y, M, N, K, ldx, ldy, ncols, 0, 0, 0,
           tiles, ntiles, goff, rowidx, cstride, sstride, nullptr, K / 128};
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
    ws = nullptr;  // the RoPE epilogue needs whole output tiles: no K split
  }
  const bool swiglu = epi >= 3 && epi <= 5;
  const int64_t logical_cols = swiglu ? 2 * (int64_t)ncols : N;
  // Tile shape (measured on MI355X over the configs' decode, prefill and
  // recompute shapes): 32 rows per wave (128-row tiles; grouped plan tiles are
  // 128 rows) above 256 rows or when 128 x 128 tiles still number >= 512,
  // else 16; 128-column tiles (half the activation re-reads of 64) when that
  // still gives >= 256 tiles.
  const int wr = (tiles || M > 256 ||
                  (M > 128 && ceil_div(M, 128) * ceil_div(logical_cols, 128) >= 512)) ? 32 : 16;
  const int tm = 4 * wr;
  const int64_t mtiles = tiles ? max_tiles : ceil_div(M, tm);
  const int tn = (ceil_div(logical_cols, 128) * mtiles >= 256) ? 128 : 64;
  const int ngroups = K / 128;
  const int64_t cnt_bytes = bl_counter_bytes();
  const int64_t ks_cap = (ws && !tiles && ws_bytes > cnt_bytes)
                             ? std::max<int64_t>(1, std::min<int64_t>(8, ngroups / 2)) : 1;
  a.ntiles = (int)ceil_div(logical_cols, tn);
  a.mtiles = (int)mtiles;
  a.mtiles8 = (int)(tiles ? mtiles : (mtiles >= 8 ? ceil_div(mtiles, 8) * 8 : mtiles));
  const int64_t blocks = (int64_t)a.mtiles8 * a.ntiles;
  if (blocks > 0x7fffffff) {
    set_error("sm_q4_matmul: problem too large");
    return SM_ERR_UNSUPPORTED;
  }
  if (tiles) a.mtiles = 0;  // grouped: tile order comes from the plan
  // split-K (measured): only for K >= 16 groups, as many splits as still fit
  // one wave of workgroups (512 at two per CU), >= 4 groups per split; the
  // reduction launch costs more than it saves on shorter K
  int ks = 1;
  if (ks_cap > 1 && ngroups >= 16 && blocks <= 256) {
    ks = (int)std::min<int64_t>(std::min<int64_t>(ks_cap, ngroups / 4), 512 / blocks);
    const int64_t part_cap = (ws_bytes - cnt_bytes) / 4;
    while (ks > 1 && (int64_t)ks * M * logical_cols > part_cap) --ks;
    if (ks > 1) {
      a.gper = (int)ceil_div(ngroups, ks);
      ks = (int)ceil_div(ngroups, a.gper);  // every split non-empty
    }
    if (ks > 1) a.part = reinterpret_cast<float*>(static_cast<char*>(ws) + cnt_bytes);
  }
  const dim3 grid((unsigned)blocks, (unsigned)ks);
  int s;
  if (wr == 16) s = (tn == 128) ? launch_bl_x<16, 128>(a, epi, xt, grid, st)
                                : launch_bl_x<16, 64>(a, epi, xt, grid, st);
  else s = (tn == 128) ? launch_bl_x<32, 128>(a, epi, xt, grid, st)
                       : launch_bl_x<32, 64>(a, epi, xt, grid, st);
  if (s != SM_OK || ks == 1) return s;
  return splitk_reduce(a.part, ks, M, N, ncols, y, ldy, epi, st);
}

int splitk_reduce(const float* part, int ks, int M, int N, int ncols, void* y, int ldy, int epi,
                  hipStream_t st) {
  const bool swiglu = epi >= 3 && epi <= 5;
  const int64_t width = swiglu ? ncols : N;
  const unsigned rb = (unsigned)ceil_div((int64_t)M * width, 256);
  switch (epi) {
#define SM_RED(E)                                                                       \
    case E:                                                                             \
      splitk_reduce_kernel<E><<<rb, 256, 0, st>>>(part, ks, M, N, ncols, y, ldy);        \
      break;
    SM_RED(0)
    SM_RED(1)
    SM_RED(2)
    SM_RED(3)
    SM_RED(4)
    SM_RED(5)
#undef SM_RED
    default: set_error("sm_q4_matmul: split-K reduction of epilogue %d", epi); return SM_ERR_INVALID;
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace sm
