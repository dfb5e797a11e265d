// Causal flash attention for prefill and log-prob recompute (16-bit MFMA;
// q and cache bf16 or f16).
//
// Semantics: Transformer full-sequence attention (sdpa with causal mask,
// summa-llm/src/model/attention.rs:216-298; CubeK flash forward
// cube_attention.rs:127-220): query row r of sequence s sits at absolute
// position pos0[s] + r and attends keys 0..=pos0[s]+r of the cache, scale
// 1/sqrt(hd), GQA head h -> KV head h / (H/KVH).
//
// Tiling: one workgroup per (128 query rows, head, sequence), 8 waves x 16
// query rows. Per 64-key tile the workgroup stages K [64][hd] and V transposed
// [hd][64] in LDS (padded rows); the next tile's global loads are issued into
// registers before the current tile's math, so their latency hides behind it.
// The tile math is transposed so that each lane owns one query:
//   S^T = K.Q^T  (v_mfma_f32_16x16x32_{bf16,f16}; A = K rows from LDS, B = the
//                 wave's Q fragments, kept in registers for the whole sweep):
//                 lane (j, g) receives 16 scores of query j;
//   softmax      running max / sum per lane in raw-score units, the scale folded
//                into one FMA before exp2; the only cross-lane steps are two
//                shuffles (lanes j, j+16, j+32, j+48) per reduction; the causal
//                mask runs on the diagonal tiles only;
//   P            written to the wave's LDS slice P[query][key] as an f16 pair
//                (hi + lo, ~21 significant bits), 4 consecutive keys per store;
//   O^T += V^T.P^T  two f16 MFMAs (hi, lo) per k-step, A = the transposed V
//                tile (f16 as stored, or bf16 -> f16 while staging, exact for
//                |v| < 65504 and above the f16 subnormal range), B = P^T;
//                lane (j, g) accumulates dims 4g..4g+3 of every 16-dim block of
//                query j, so rescaling by the softmax correction needs no
//                cross-lane traffic and the epilogue stores 8 bytes at a time.
// A wave skips the key tiles past its last row's position (fully masked for
// it). Without the causal mask (AttentionBackend::attention_inner with
// causal = false) every query attends keys 0..L-1. q and out are addressed
// through element strides (sequence, position, head), so the same kernel
// serves the model's [S, L, H, hd] rows and the reference's [B, H, S, hd]
// tensors. The f16 pair keeps P.V at fp32-like precision, so the prefill path
// matches the decode path's fp32 probabilities; a single bf16 or f16 P costs
// measurable log-prob accuracy.
#include <cmath>

#include "attn_common.hpp"
#include "common.hpp"

namespace sm {
namespace {

template <int HD, bool KF16, int OM>
__global__ __launch_bounds__(512) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ pos0,
    void* __restrict__ out, float* __restrict__ lse, int L, int H, int KVH, int cap,
    float scale, AttnStrides qs, AttnStrides os, int causal) {
  typedef typename Op8<KF16>::T op8;
  constexpr int NW = 8;                  // waves, 16 query rows each
  constexpr int NT = NW * kWave;         // threads
  constexpr int STEPS = HD / 32;
  // Padded LDS rows (elements). 16 elements of padding: the fragment reads
  // (16 rows x one 16-byte chunk column per wave instruction) measured 1.7-1.9x
  // faster on MI355X than with 8 (128-byte rows: 565 against 979 ns, 256-byte
  // rows: 573 against 1069 ns per 16 reads of 8 waves); in this kernel 1-2 %
  // (config[2] recompute 1139-1147 -> 1130 us, bits unchanged).
  constexpr int KP = HD + 16;  // K row
  constexpr int VP = 64 + 16;  // transposed-V row
  constexpr int PP = 64 + 16;  // P row
  constexpr int CH = HD / 8;             // 16-byte chunks per key row
  constexpr int KCH = 64 * CH;           // K chunks per tile
  constexpr int VU = 32 * CH;            // V units per tile: 2 keys x 8 dims
  constexpr int KPT = (KCH + NT - 1) / NT;
  constexpr int VPT = (VU + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) uint16_t ks[64 * KP];
  __shared__ __attribute__((aligned(16))) _Float16 vts[HD * VP];
  __shared__ __attribute__((aligned(16))) _Float16 ps[NW][2][16 * PP];  // P = hi + lo

  const int qt = blockIdx.x, h = blockIdx.y, s = blockIdx.z;
  const int kvh = h / (H / KVH);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int p0 = pos0 ? pos0[s] : 0;
  const int r0 = qt * (16 * NW) + wave * 16;  // first query row of this wave
  const size_t kv_base = ((size_t)s * KVH + kvh) * cap * HD;

  // Q fragments (A operand): lane (row j, group g)
  op8 qa[STEPS];
  {
    const int r = r0 + j;
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      if (r < L)
        qa[st] = *reinterpret_cast<const op8*>(q + qs.at(s, r, h) + st * 32 + g * 8);
      else
        qa[st] = op8{};
    }
  }
  // Transposed tile math: S^T = K.Q^T and O^T = V^T.P^T, so lane (j, g) owns
  // query r0 + j: its running max m and sum l (in raw-score units; the scale
  // is folded into the exp2 argument), and o[d][r] = O[query][dim d*16 + 4g + r].
  f4 o[HD / 16];
#pragma unroll
  for (int d = 0; d < HD / 16; ++d) o[d] = f4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float c2 = scale * 1.44269504088896340736f;  // scale * log2(e)
  const int qpos = p0 + r0 + j;                       // this lane's query position

  const int last_row = min(qt * (16 * NW) + 16 * NW - 1, L - 1);
  // keys [0, kend) needed by this workgroup (all L of them without the mask)
  const int kend = causal ? p0 + last_row + 1 : L;
  // keys this wave attends to: [0, p0 + its last row]; later tiles are fully
  // masked for it (they would leave m, l and o bit-for-bit unchanged) and skipped
  const int wave_kmax = (r0 < L) ? (causal ? p0 + min(r0 + 15, L - 1) : L - 1) : -1;

  // ---- K/V tile staging: the next tile's global loads are issued into
  //      registers before the current tile's math and written to LDS after
  //      it (K row-major; V transposed, 2 keys x 8 dims per unit so each LDS
  //      store is 4 bytes of consecutive keys)
  u32x4 kreg[KPT], vreg[VPT][2];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = i * NT + threadIdx.x;
      const int key = kt + c / CH;
      kreg[i] = u32x4{0u, 0u, 0u, 0u};
      if (c < KCH && key < kend && key < cap)
        kreg[i] = *reinterpret_cast<const u32x4*>(kc + kv_base + (size_t)key * HD + (c % CH) * 8);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int u = i * NT + threadIdx.x;
      const int key = kt + 2 * (u % 32);
      const size_t off = kv_base + (size_t)key * HD + (u / 32) * 8;
      vreg[i][0] = vreg[i][1] = u32x4{0u, 0u, 0u, 0u};
      if (u < VU && key < kend && key < cap) vreg[i][0] = *reinterpret_cast<const u32x4*>(vc + off);
      if (u < VU && key + 1 < kend && key + 1 < cap)
        vreg[i][1] = *reinterpret_cast<const u32x4*>(vc + off + HD);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int c = i * NT + threadIdx.x;
      if (c < KCH) *reinterpret_cast<u32x4*>(&ks[(c / CH) * KP + (c % CH) * 8]) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int u = i * NT + threadIdx.x;
      if (u >= VU) continue;
      float f0[8], f1[8];
      unpack8<KF16>(vreg[i][0], f0);
      unpack8<KF16>(vreg[i][1], f1);
      const int kp = u % 32, dc = u / 32;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *reinterpret_cast<h2*>(&vts[(dc * 8 + e) * VP + 2 * kp]) =
            h2{(_Float16)f0[e], (_Float16)f1[e]};
    }
  };

  load_tile(0);
  store_tile();
  __syncthreads();
  for (int kt = 0; kt < kend; kt += 64) {
    const bool more = kt + 64 < kend;
    if (more) load_tile(kt + 64);
    if (kt <= wave_kmax) {  // uniform per wave
    // ---- S^T = K Q^T for 4 key blocks: A = K rows (lane key j), B = Q^T
    //      (lane query j); lane (j, g) receives keys kb*16 + 4g + r of query j
    f4 sc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        const op8 kf = *reinterpret_cast<const op8*>(&ks[(kb * 16 + j) * KP + st * 32 + g * 8]);
        acc = Op8<KF16>::mfma(kf, qa[st], acc);
      }
      sc[kb] = acc;
    }
    // ---- causal mask (only tiles that reach past the wave's first query)
    if (kt + 63 > (causal ? p0 + r0 : L - 1)) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (kt + kb * 16 + 4 * g + r > (causal ? qpos : L - 1)) sc[kb][r] = -INFINITY;
    }
    // ---- online softmax of query j over the 64 keys (16 here, 48 in the
    //      lanes j + 16, j + 32, j + 48)
    float mx = sc[0][0];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[kb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float mnew = fmaxf(m, mx);  // finite: key 0 <= every query position
    const float alpha = __builtin_amdgcn_exp2f((m - mnew) * c2);
    const float mc = mnew * c2;
    float sum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sc[kb][r], c2, -mc));
        sc[kb][r] = p;
        sum += p;
      }
    sum += __shfl_xor(sum, 16, kWave);
    sum += __shfl_xor(sum, 32, kWave);
    l = l * alpha + sum;
    m = mnew;
    if (__ballot(alpha != 1.f)) {  // a factor of 1 would leave O unchanged
#pragma unroll
      for (int d = 0; d < HD / 16; ++d)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[d][r] *= alpha;
    }
    // ---- P as an f16 pair (hi + lo carries ~21 significant bits) to this
    //      wave's LDS slice P[query j][key]: 4 consecutive keys per store
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      h4 hi, lo;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        _Float16 a, b;
        split_f16(sc[kb][r], a, b);
        hi[r] = a;
        lo[r] = b;
      }
      *reinterpret_cast<h4*>(&ps[wave][0][j * PP + kb * 16 + 4 * g]) = hi;
      *reinterpret_cast<h4*>(&ps[wave][1][j * PP + kb * 16 + 4 * g]) = lo;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- O^T += V^T P^T: A = V^T rows (lane dim j), B = P^T (lane query j)
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const h8 pa = *reinterpret_cast<const h8*>(&ps[wave][0][j * PP + st * 32 + g * 8]);
      const h8 pl = *reinterpret_cast<const h8*>(&ps[wave][1][j * PP + st * 32 + g * 8]);
#pragma unroll
      for (int d = 0; d < HD / 16; ++d) {
        const h8 vb = *reinterpret_cast<const h8*>(&vts[(d * 16 + j) * VP + st * 32 + g * 8]);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vb, pa, o[d], 0, 0, 0);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vb, pl, o[d], 0, 0, 0);
      }
    }
    }  // kt <= wave_kmax
    __syncthreads();  // every wave done with this tile
    if (more) store_tile();
    __syncthreads();
  }
  if (r0 >= L) return;
  const int row = r0 + j;
  if (row >= L) return;
  // log-sum-exp of the scaled, masked scores, [S*H, L] (fused_attention.rs:166-172)
  if (lse && g == 0) lse[((size_t)s * H + h) * L + row] = m * scale + logf(l);
  const float inv = 1.f / l;
  // lane (j, g) holds dims d*16 + 4g .. +3 of its query: 8-byte stores
  const size_t orow = (size_t)s * L + row;  // f16-pair rows: [S * L, 2 * H * hd]
  const int width = H * HD;
  const size_t obase = os.at(s, row, h);
#pragma unroll
  for (int d = 0; d < HD / 16; ++d) {
    const int col = h * HD + d * 16 + 4 * g;
    if constexpr (OM == 2) {
      h4 hi, lo;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        _Float16 a, b;
        split_f16(o[d][r] * inv, a, b);
        hi[r] = a;
        lo[r] = b;
      }
      _Float16* base = static_cast<_Float16*>(out) + orow * 2 * width;
      *reinterpret_cast<h4*>(base + col) = hi;
      *reinterpret_cast<h4*>(base + width + col) = lo;
    } else if constexpr (OM == 1) {
      const h4 v = h4{(_Float16)(o[d][0] * inv), (_Float16)(o[d][1] * inv),
                      (_Float16)(o[d][2] * inv), (_Float16)(o[d][3] * inv)};
      *reinterpret_cast<h4*>(static_cast<_Float16*>(out) + obase + d * 16 + 4 * g) = v;
    } else {
      const uint2 v = uint2{(uint32_t)f32_to_bf16(o[d][0] * inv) |
                                ((uint32_t)f32_to_bf16(o[d][1] * inv) << 16),
                            (uint32_t)f32_to_bf16(o[d][2] * inv) |
                                ((uint32_t)f32_to_bf16(o[d][3] * inv) << 16)};
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + obase + d * 16 + 4 * g) = v;
    }
  }
}

}  // namespace

int attn_prefill_16(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                    const int32_t* pos0, void* out, float* lse, bool kf16, int om, int S, int L,
                    int H, int KVH, int cap, int hd, hipStream_t st, const AttnStrides* qs_in,
                    const AttnStrides* os_in, bool causal) {
  if (S > 65535 || H > 65535) {
    set_error("sm_attn_prefill: S and H must be <= 65535");
    return SM_ERR_UNSUPPORTED;
  }
  const dim3 grid((unsigned)ceil_div(L, 128), (unsigned)H, (unsigned)S);
  const float scale = 1.0f / sqrtf((float)hd);
  const AttnStrides rows = AttnStrides::rows(L, H, hd);  // [S, L, H, hd]
  const AttnStrides qs = qs_in ? *qs_in : rows, os = os_in ? *os_in : rows;
  const int cz = causal ? 1 : 0;
#define SM_PF3(HD, KF, OM)                                                                \
  attn_prefill_kernel<HD, KF, OM><<<grid, 512, 0, st>>>(q, kc, vc, pos0, out, lse, L, H, KVH, cap, \
                                                        scale, qs, os, cz)
#define SM_PF2(HD, KF)                          \
  do {                                          \
    if (om == 2) SM_PF3(HD, KF, 2);             \
    else if (om == 1) SM_PF3(HD, KF, 1);        \
    else SM_PF3(HD, KF, 0);                     \
  } while (0)
#define SM_PF(HD)                               \
  do {                                          \
    if (kf16) SM_PF2(HD, true);                 \
    else SM_PF2(HD, false);                     \
  } while (0)
  if (hd == 64) SM_PF(64);
  else SM_PF(128);
#undef SM_PF
#undef SM_PF2
#undef SM_PF3
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace sm
