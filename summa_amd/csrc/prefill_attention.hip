// Causal flash attention for prefill and log-prob recompute (16-bit MFMA;
// q and cache bf16 or f16).
//
// Semantics: Transformer full-sequence attention (sdpa with causal mask,
// summa-llm/src/model/attention.rs:216-298; CubeK flash forward
// cube_attention.rs:127-220): query row r of sequence s sits at absolute
// position pos0[s] + r and attends keys 0..=pos0[s]+r of the cache, scale
// 1/sqrt(hd), GQA head h -> KV head h / (H/KVH).
//
// Tiling: one workgroup per (64 query rows, head, sequence), 4 waves x 16 rows.
// Per 64-key tile the workgroup stages K [64][hd] and V transposed [hd][64] in
// LDS (padded rows), then each wave computes S = Q.K^T with
// v_mfma_f32_16x16x32_{bf16,f16} (Q fragments stay in registers for the whole
// sweep), applies the causal mask and the online softmax on the MFMA output
// registers (row stats reduced across the 16 lanes that share a row), writes P
// to its LDS slice as a pair of f16 values (hi + lo, ~21 significant bits)
// and accumulates O += P.V with two f16 MFMAs whose B operand reads the
// transposed V tile (f16 as stored, or bf16 -> f16 while staging, exact for
// |v| < 65504 and above the f16 subnormal range). The split keeps P.V at
// fp32-like precision, so the prefill path matches the decode path's fp32
// probabilities; a single bf16 or f16 P costs measurable log-prob accuracy.
// O stays in registers; the final 1/l scaling and store happen once.
#include <cmath>

#include "attn_common.hpp"
#include "common.hpp"

namespace sm {
namespace {

template <int HD, bool KF16, int OM>
__global__ __launch_bounds__(256) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ pos0,
    void* __restrict__ out, float* __restrict__ lse, int L, int H, int KVH, int cap,
    float scale) {
  typedef typename Op8<KF16>::T op8;
  constexpr int STEPS = HD / 32;
  constexpr int KP = HD + 8;   // padded K row (elements)
  constexpr int VP = 64 + 8;   // padded transposed-V row
  constexpr int PP = 64 + 8;   // padded P row
  __shared__ __attribute__((aligned(16))) uint16_t ks[64 * KP];
  __shared__ __attribute__((aligned(16))) _Float16 vts[HD * VP];
  __shared__ __attribute__((aligned(16))) _Float16 ps[4][2][16 * PP];  // P = hi + lo

  const int qt = blockIdx.x, h = blockIdx.y, s = blockIdx.z;
  const int kvh = h / (H / KVH);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int p0 = pos0[s];
  const int r0 = qt * 64 + wave * 16;  // first query row of this wave
  const size_t kv_base = ((size_t)s * KVH + kvh) * cap * HD;

  // Q fragments (A operand): lane (row j, group g)
  op8 qa[STEPS];
  {
    const int r = r0 + j;
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      if (r < L)
        qa[st] = *reinterpret_cast<const op8*>(q + (((size_t)s * L + r) * H + h) * HD + st * 32 + g * 8);
      else
        qa[st] = op8{};
    }
  }
  f4 o[HD / 16];
#pragma unroll
  for (int d = 0; d < HD / 16; ++d) o[d] = f4{0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) { m[r] = -INFINITY; l[r] = 0.f; }

  const int last_row = min(qt * 64 + 63, L - 1);
  const int kend = p0 + last_row + 1;  // keys [0, kend) needed by this workgroup
  for (int kt = 0; kt < kend; kt += 64) {
    __syncthreads();  // previous tile fully consumed
    // ---- stage K tile (row-major, padded) and V tile transposed
    constexpr int CH = HD / 8;  // 16-byte chunks per row
    for (int c = threadIdx.x; c < 64 * CH; c += 256) {
      const int kr = c / CH, cc = c % CH;
      const int key = kt + kr;
      u32x4 kv = u32x4{0u, 0u, 0u, 0u}, vv = u32x4{0u, 0u, 0u, 0u};
      if (key < kend && key < cap) {
        kv = *reinterpret_cast<const u32x4*>(kc + kv_base + (size_t)key * HD + cc * 8);
        vv = *reinterpret_cast<const u32x4*>(vc + kv_base + (size_t)key * HD + cc * 8);
      }
      *reinterpret_cast<u32x4*>(&ks[kr * KP + cc * 8]) = kv;
      float vf[8];
      unpack8<KF16>(vv, vf);
#pragma unroll
      for (int e = 0; e < 8; ++e) vts[(cc * 8 + e) * VP + kr] = (_Float16)vf[e];
    }
    __syncthreads();
    if (r0 >= L) continue;  // wave has no rows (uniform per wave)
    // ---- S = Q K^T for 4 key blocks
    f4 sc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        const op8 kf = *reinterpret_cast<const op8*>(&ks[(kb * 16 + j) * KP + st * 32 + g * 8]);
        acc = Op8<KF16>::mfma(qa[st], kf, acc);
      }
      sc[kb] = acc;
    }
    // ---- mask + online softmax; lane holds rows 4g+r, key kb*16+j
    float alpha[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = r0 + 4 * g + r;
      const int qpos = p0 + row;
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const int key = kt + kb * 16 + j;
        const float v = (row < L && key <= qpos) ? sc[kb][r] * scale : -INFINITY;
        sc[kb][r] = v;
        mx = fmaxf(mx, v);
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
      const float mnew = fmaxf(m[r], mx);
      alpha[r] = (m[r] == -INFINITY) ? 0.f : __expf(m[r] - mnew);
      float sum = 0.f;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const float p = (sc[kb][r] == -INFINITY) ? 0.f : __expf(sc[kb][r] - mnew);
        sc[kb][r] = p;
        sum += p;
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off, kWave);
      l[r] = l[r] * alpha[r] + sum;
      m[r] = mnew;
    }
#pragma unroll
    for (int d = 0; d < HD / 16; ++d)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[d][r] *= alpha[r];
    // ---- P as an f16 pair (hi + lo carries ~21 significant bits) to this
    //      wave's LDS slice: P[row 4g+r][key kb*16+j]
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const _Float16 hi = (_Float16)sc[kb][r];
        ps[wave][0][(4 * g + r) * PP + kb * 16 + j] = hi;
        ps[wave][1][(4 * g + r) * PP + kb * 16 + j] = (_Float16)(sc[kb][r] - (float)hi);
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- O += P V: A = P rows (lane row j), B = V^T rows (lane dim j)
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const h8 pa = *reinterpret_cast<const h8*>(&ps[wave][0][j * PP + st * 32 + g * 8]);
      const h8 pl = *reinterpret_cast<const h8*>(&ps[wave][1][j * PP + st * 32 + g * 8]);
#pragma unroll
      for (int d = 0; d < HD / 16; ++d) {
        const h8 vb = *reinterpret_cast<const h8*>(&vts[(d * 16 + j) * VP + st * 32 + g * 8]);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, o[d], 0, 0, 0);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vb, o[d], 0, 0, 0);
      }
    }
  }
  if (r0 >= L) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = r0 + 4 * g + r;
    if (row >= L) continue;
    // log-sum-exp of the scaled, masked scores, [S*H, L] (fused_attention.rs:166-172)
    if (lse && j == 0) lse[((size_t)s * H + h) * L + row] = m[r] + logf(l[r]);
    const float inv = 1.f / l[r];
#pragma unroll
    for (int d = 0; d < HD / 16; ++d)
      store_out<OM>(out, (size_t)s * L + row, H * HD, h * HD + d * 16 + j, o[d][r] * inv);
  }
}

}  // namespace

int attn_prefill_16(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                    const int32_t* pos0, void* out, float* lse, bool kf16, int om, int S, int L,
                    int H, int KVH, int cap, int hd, hipStream_t st) {
  if (S > 65535 || H > 65535) {
    set_error("sm_attn_prefill: S and H must be <= 65535");
    return SM_ERR_UNSUPPORTED;
  }
  const dim3 grid((unsigned)ceil_div(L, 64), (unsigned)H, (unsigned)S);
  const float scale = 1.0f / sqrtf((float)hd);
#define SM_PF3(HD, KF, OM)                                                                \
  attn_prefill_kernel<HD, KF, OM><<<grid, 256, 0, st>>>(q, kc, vc, pos0, out, lse, L, H, KVH, cap, \
                                                        scale)
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
