// Backward-pass and optimizer kernels for the GRPO policy update of fp32
// models (prepare_device_batch's autodiff and optimizer_step,
// summa-train/src/posttrain.rs:1288-1305, trainer.rs:1974-1975):
//   * a general f32 GEMM with transposes, C = alpha op(A) op(B) + beta C, for
//     the data and weight gradients of every linear and Muon's Newton-Schulz
//     iterations (matmul backward of Linear::forward, matmul.rs:57-66);
//   * RMSNorm backward (Norm::forward, norm.rs:36-50), deterministic dgamma;
//   * in-place RoPE on the q / k heads of a qkv block and its backward
//     (adjacent-pair rotation, attention.rs:142-177);
//   * causal GQA attention backward from the forward's log-sum-exp
//     (fused_attention.rs:219-405: dq, dk, dv with delta = rowsum(dO * O));
//   * embedding backward (scatter-add of row gradients);
//   * AdamW and Muon's momentum step (burn_optim AdamW; BatchedMuon,
//     summa-train/src/muon.rs:196-215).
// All f32 with f32 accumulation: the precision of the reference CPU path.
#include <algorithm>
#include <cmath>

#include "attn_common.hpp"
#include "common.hpp"

namespace sm {
namespace {

// ------------------------------------------------------------------ GEMM ---
// 64 x 64 output tile per 256-thread workgroup, 4 x 4 outputs per thread, K in
// steps of 16 through LDS; op(A) is [M, K] (A stored [M, K] or, transposed,
// [K, M]), op(B) is [K, N] (B stored [K, N] or [N, K]).
template <bool TA, bool TB>
__global__ __launch_bounds__(256) void gemm_ex_kernel(const float* __restrict__ A, int64_t lda,
                                                      const float* __restrict__ B, int64_t ldb,
                                                      float* __restrict__ C, int64_t ldc, int M,
                                                      int N, int K, float alpha, float beta) {
  __shared__ float as[16][64 + 4];
  __shared__ float bs[16][64 + 4];
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    for (int e = threadIdx.x; e < 64 * 16; e += 256) {
      // consecutive threads walk the contiguous dimension of each operand
      int r, kk;
      if (TA) { kk = e / 64; r = e % 64; } else { r = e / 16; kk = e % 16; }
      const int gm = m0 + r, gk = k0 + kk;
      as[kk][r] = (gm < M && gk < K) ? (TA ? A[(size_t)gk * lda + gm] : A[(size_t)gm * lda + gk])
                                     : 0.f;
      int c, kb;
      if (TB) { c = e / 16; kb = e % 16; } else { kb = e / 64; c = e % 64; }
      const int gn = n0 + c, gkb = k0 + kb;
      bs[kb][c] = (gn < N && gkb < K) ? (TB ? B[(size_t)gn * ldb + gkb] : B[(size_t)gkb * ldb + gn])
                                      : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = as[kk][ty * 4 + i];
        b[i] = bs[kk][tx * 4 + i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int gm = m0 + ty * 4 + i;
    if (gm >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gn = n0 + tx * 4 + j;
      if (gn >= N) continue;
      float* cp = C + (size_t)gm * ldc + gn;
      *cp = alpha * acc[i][j] + (beta != 0.f ? beta * *cp : 0.f);
    }
  }
}

// --------------------------------------------------------------- RMSNorm ---
// y = x r gamma with r = 1 / sqrt(mean(x^2) + eps):
// dx = r gamma dy - x r^3 / d * sum_c(gamma dy x); dgamma_c = sum_rows dy x r.
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ gamma,
                                                          const float* __restrict__ dy, int d,
                                                          float eps, int accumulate,
                                                          float* __restrict__ dx,
                                                          float* __restrict__ rinv) {
  __shared__ float part[2][4];
  const int64_t r = blockIdx.x;
  const float* xr = x + r * d;
  const float* gr = dy + r * d;
  float ss = 0.f, dot = 0.f;
  for (int c = threadIdx.x; c < d; c += 256) {
    ss = fmaf(xr[c], xr[c], ss);
    dot = fmaf(gamma[c] * gr[c], xr[c], dot);
  }
  ss = wave_sum(ss);
  dot = wave_sum(dot);
  if (threadIdx.x % kWave == 0) {
    part[0][threadIdx.x / kWave] = ss;
    part[1][threadIdx.x / kWave] = dot;
  }
  __syncthreads();
  const float tot = part[0][0] + part[0][1] + part[0][2] + part[0][3];
  const float sdot = part[1][0] + part[1][1] + part[1][2] + part[1][3];
  const float rs = 1.f / sqrtf(tot / (float)d + eps);
  const float k = rs * rs * rs / (float)d * sdot;
  for (int c = threadIdx.x; c < d; c += 256) {
    const float v = rs * gamma[c] * gr[c] - xr[c] * k;
    dx[r * d + c] = accumulate ? dx[r * d + c] + v : v;
  }
  if (threadIdx.x == 0) rinv[r] = rs;
}

// dgamma_c = sum over rows in order (deterministic), one thread per column
// dgamma[c] (=, or += with accumulate) = sum_r dy[r, c] x[r, c] rinv[r]: one
// workgroup per 64 columns; thread t sums columns 4 (t % 16) + j over rows
// t / 16, t / 16 + 16, ... (a wave reads four 256-byte row segments per
// step), and the 16 row-lane partials are added in order.
__global__ __launch_bounds__(256) void rmsnorm_dgamma_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ dy,
                                                             const float* __restrict__ rinv,
                                                             int64_t rows, int d, int accumulate,
                                                             float* __restrict__ dgamma) {
  __shared__ float part[16][64];
  const int cg = threadIdx.x % 16, rl = threadIdx.x / 16;
  const int c0 = blockIdx.x * 64 + 4 * cg;
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t r = rl; r < rows; r += 16) {
    const float ri = rinv[r];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (c0 + j < d) s[j] = fmaf(dy[r * d + c0 + j] * x[r * d + c0 + j], ri, s[j]);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) part[rl][4 * cg + j] = s[j];
  __syncthreads();
  const int c = blockIdx.x * 64 + (int)threadIdx.x;
  if (threadIdx.x >= 64 || c >= d) return;
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) tot += part[i][threadIdx.x];
  dgamma[c] = accumulate ? dgamma[c] + tot : tot;
}

// dgamma over row chunks: block (x, y) sums rows [y * rpc, (y + 1) * rpc) of
// columns 64x .. 64x + 63 (as rmsnorm_dgamma_kernel does over all rows) into
// parts[y][col]; dgamma_finish_kernel then adds the chunks in order. For the
// policy update's 8k-row norms, where 32 column blocks cannot fill the GPU.
__global__ __launch_bounds__(256) void rmsnorm_dgamma_parts_kernel(
    const float* __restrict__ x, const float* __restrict__ dy, const float* __restrict__ rinv,
    int64_t rows, int d, int64_t rpc, float* __restrict__ parts) {
  __shared__ float part[16][64];
  const int cg = threadIdx.x % 16, rl = threadIdx.x / 16;
  const int c0 = blockIdx.x * 64 + 4 * cg;
  const int64_t r0 = (int64_t)blockIdx.y * rpc, r1 = min(rows, r0 + rpc);
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  for (int64_t r = r0 + rl; r < r1; r += 16) {
    const float ri = rinv[r];
    if (c0 + 4 <= d && d % 4 == 0) {
      const float4 a = *reinterpret_cast<const float4*>(dy + r * d + c0);
      const float4 b = *reinterpret_cast<const float4*>(x + r * d + c0);
      s[0] = fmaf(a.x * b.x, ri, s[0]);
      s[1] = fmaf(a.y * b.y, ri, s[1]);
      s[2] = fmaf(a.z * b.z, ri, s[2]);
      s[3] = fmaf(a.w * b.w, ri, s[3]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (c0 + j < d) s[j] = fmaf(dy[r * d + c0 + j] * x[r * d + c0 + j], ri, s[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) part[rl][4 * cg + j] = s[j];
  __syncthreads();
  const int c = blockIdx.x * 64 + (int)threadIdx.x;
  if (threadIdx.x >= 64 || c >= d) return;
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) tot += part[i][threadIdx.x];
  parts[(int64_t)blockIdx.y * d + c] = tot;
}

__global__ void dgamma_finish_kernel(const float* __restrict__ parts, int chunks, int d,
                                     int accumulate, float* __restrict__ dgamma) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= d) return;
  float tot = 0.f;
  for (int i = 0; i < chunks; ++i) tot += parts[(int64_t)i * d + c];
  dgamma[c] = accumulate ? dgamma[c] + tot : tot;
}

// ------------------------------------------------------------------ RoPE ---
// qkv rows [rows, (H + 2 KVH) hd]: rotate the q and k heads in place (DIR = +1)
// or apply the transposed rotation to their gradients (DIR = -1).
template <int DIR>
__global__ void rope_qk_kernel(float* __restrict__ qkv, const float2* __restrict__ rope,
                               const int32_t* __restrict__ pos0, int L, int H, int KVH, int hd,
                               int64_t rows) {
  const int half = hd / 2, slots = H + KVH;  // q and k heads
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * slots * half) return;
  const int p = idx % half;
  const int slot = (idx / half) % slots;
  const int64_t row = idx / ((int64_t)half * slots);
  const int pos = pos0[row / L] + (int)(row % L);
  float* e = qkv + row * (int64_t)(H + 2 * KVH) * hd + (int64_t)slot * hd + 2 * p;
  const float2 cs = rope[(size_t)pos * half + p];
  const float a = e[0], b = e[1];
  if (DIR > 0) {
    e[0] = a * cs.x - b * cs.y;
    e[1] = b * cs.x + a * cs.y;
  } else {
    e[0] = a * cs.x + b * cs.y;
    e[1] = b * cs.x - a * cs.y;
  }
}

// ------------------------------------------------------------- attention ---
// Forward inputs: q, o and dO addressed by element strides (the model's
// [S*L, H, hd] rows or the reference's [B, H, S, hd] tensors), k / v
// [S, KVH, L, hd] (positions 0..L-1, causal or not), lse [S*H, L].
// delta[s,h,r] = <dO, O>; with p_t = exp(scale <q, k_t> - lse) and
// ds_t = p_t (<dO, v_t> - delta) scale: dq = sum_t ds_t k_t, and for a key t
// of KV head g, dk_t = sum over the group's heads and rows r of ds q_r,
// dv_t = the same sum of p dO_r (fused_attention.rs:219-405).
//
// FlashAttention-2 style on 32 x 32 tiles: the dK / dV kernel holds one
// 32-key block of K and V and walks the query blocks of every head of its
// group (rows >= the block's first key under the causal mask), recomputing
// the scores and dP = dO V^T per tile; the dQ kernel holds one 32-row block
// of Q and dO and walks the key blocks. Each output has one owner and a
// fixed order of additions (deterministic, no atomics). Staged rows padded to
// hd + 4 floats. Under the causal mask the heaviest blocks are dispatched
// first. Measured at one GRPO group's shape (8 x 1023 positions, 16 / 4
// heads, hd 128; 120 GFLOP per layer): 2.6-2.8 ms per layer with f32 FMAs on
// LDS tiles, 1.50 ms (80 TF/s, 0.51 of the f32 matrix-core peak) on the
// matrix cores.
constexpr int kAB = 32;  // query rows and keys per tile

// delta = <dO, O> per (s, h, r), row (s H + h) L + r; one wave per row
template <int HD>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const float* __restrict__ o,
                                                             const float* __restrict__ dout,
                                                             int S, int L, int H, AttnStrides qs,
                                                             float* __restrict__ delta) {
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= (int64_t)S * H * L) return;  // uniform per wave
  const int r = (int)(row % L), sh = (int)(row / L);
  const size_t at = qs.at(sh / H, r, sh % H);
  float acc = 0.f;
#pragma unroll
  for (int d = lane; d < HD; d += kWave) acc = fmaf(dout[at + d], o[at + d], acc);
  acc = wave_sum(acc);
  if (lane == 0) delta[row] = acc;
}

// T rows of HD floats (row i at src(i), or 0 past `valid`) -> LDS rows of stride RS
template <int HD, int RS, typename Src>
__device__ inline void stage_rows(float* __restrict__ dst, int valid, Src src) {
  constexpr int C4 = HD / 4;
  for (int e = threadIdx.x; e < kAB * C4; e += 256) {
    const int i = e / C4, c = e % C4;
    f4 x = f4{0.f, 0.f, 0.f, 0.f};
    if (i < valid) x = *reinterpret_cast<const f4*>(src(i) + 4 * c);
    *reinterpret_cast<f4*>(dst + i * RS + 4 * c) = x;
  }
}

// Both passes run on the f32 matrix cores (v_mfma_f32_16x16x4_f32: f32
// operands, f32 accumulation). MFMA lane (g, j) = (lane / 16, lane % 16)
// supplies A[j][k = g] and B[k = g][j] and receives D[4 g + r][j], r = 0..3.
// A 32 x 32 score tile is 2 x 2 blocks of 16, one per wave. The head-dim
// contraction takes in step (c, e) dim 16 c + 4 g + e from lane group g, so
// every lane reads its operands as 16-byte chunks; the row / key contractions
// take row 4 c + g in step c. dK / dV pass: the workgroup's 32 keys of K and
// V sit in registers as A operands for the whole kernel; per (head, query
// block) the waves form S^T = K Q^T and dP^T = V dO^T, write P^T and dS^T
// to LDS, and each wave adds its 16 keys x 64 dims of dV += P^T dO and
// dK += dS^T Q. dQ pass: Q and dO rows in registers; per key block S = Q K^T,
// dP = dO V^T, dS to LDS, dQ += dS K. One owner per output and a fixed order
// of additions (deterministic).
// LP: bf16 operands on v_mfma_f32_16x16x16bf16_1k (f32 accumulation), the
// 16-bit precision of the reference's CUDA-path attention backward
// (cube_attention.rs:53-95 forms P and dS in bf16). The head-dim contractions
// take each run of four f32 steps e = 0..3 as one MFMA (lane group g: k =
// 4 g .. 4 g + 3, the same operands rounded to bf16); the row / key
// contractions take rows (keys) 16 q + 4 g .. 16 q + 4 g + 3 from lane group g
// in step q, so the P / dS operand is one 16-byte LDS read.
template <int HD, bool LP>
__global__ __launch_bounds__(256, 2) void attn_bwd_dkv_mfma_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    int S, int L, int H, int KVH, float scale, float* __restrict__ dk, float* __restrict__ dv,
    AttnStrides qs, int causal) {
  constexpr int T = kAB, RS = HD + 4, PS = T + 4, NC = HD / 16, DBW = HD / 32;
  __shared__ __attribute__((aligned(16))) float Qs[T * RS], Gs[T * RS];
  __shared__ __attribute__((aligned(16))) float Ps[T * PS], Ds[T * PS];  // [key][row]
  __shared__ float ls_s[T], dl_s[T];
  const int sk = (int)blockIdx.x, s = sk / KVH, kvh = sk % KVH;  // (sequence, KV head)
  const int k0 = (int)blockIdx.y * T;                            // heaviest (first) keys first
  const int t = (int)threadIdx.x, wave = t / kWave, lane = t % kWave;
  const int g = lane / 16, j = lane % 16, group = H / KVH;
  const int kb = wave / 2, rb = wave % 2;   // score block: keys kb*16.., rows rb*16..
  const int db0 = (wave % 2) * DBW;         // dK / dV: keys kb*16.., dim blocks db0..
  f4 kf[NC], vf[NC];
  {
    const int key = min(k0 + kb * 16 + j, L - 1);  // past L: a valid row, masked below
    const float* kr = k + ((size_t)sk * L + key) * HD + 4 * g;
    const float* vr = v + ((size_t)sk * L + key) * HD + 4 * g;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      kf[c] = *reinterpret_cast<const f4*>(kr + 16 * c);
      vf[c] = *reinterpret_cast<const f4*>(vr + 16 * c);
    }
  }
  bf16x4_t kb16[LP ? NC : 1], vb16[LP ? NC : 1];  // LP: K and V fragments as bf16
  if constexpr (LP) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      kb16[c] = to_bf16x4(kf[c]);
      vb16[c] = to_bf16x4(vf[c]);
    }
  }
  f4 adk[DBW], adv[DBW];
#pragma unroll
  for (int b = 0; b < DBW; ++b) adk[b] = adv[b] = f4{0.f, 0.f, 0.f, 0.f};
  const int nqb = (L + T - 1) / T;
  for (int hh = 0; hh < group; ++hh) {
    const int h = kvh * group + hh;
    for (int qb = causal ? k0 / T : 0; qb < nqb; ++qb) {
      const int r0 = qb * T;
      __syncthreads();  // the previous tile's readers are done
      stage_rows<HD, RS>(Qs, L - r0, [&](int i) { return q + qs.at(s, r0 + i, h); });
      stage_rows<HD, RS>(Gs, L - r0, [&](int i) { return dout + qs.at(s, r0 + i, h); });
      if (t < T) {
        const bool in = r0 + t < L;
        const size_t li = ((size_t)s * H + h) * L + r0 + t;
        ls_s[t] = in ? lse[li] : 0.f;
        dl_s[t] = in ? delta[li] : 0.f;
      }
      __syncthreads();
      f4 st = f4{0.f, 0.f, 0.f, 0.f}, dpt = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const f4 qv = *reinterpret_cast<const f4*>(Qs + (rb * 16 + j) * RS + 16 * c + 4 * g);
        const f4 gv = *reinterpret_cast<const f4*>(Gs + (rb * 16 + j) * RS + 16 * c + 4 * g);
        if constexpr (LP) {
          st = mfma_bf16_16x16x16(kb16[c], to_bf16x4(qv), st);
          dpt = mfma_bf16_16x16x16(vb16[c], to_bf16x4(gv), dpt);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            st = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[c][e], qv[e], st, 0, 0, 0);
            dpt = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[c][e], gv[e], dpt, 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {  // key kb*16 + 4g + r, row rb*16 + j
        const int kl = kb * 16 + 4 * g + r, rl = rb * 16 + j;
        const int kc = k0 + kl, qr = r0 + rl;
        float p = 0.f;
        if (qr < L && kc < L && (!causal || kc <= qr)) p = expf(st[r] * scale - ls_s[rl]);
        Ps[kl * PS + rl] = p;
        Ds[kl * PS + rl] = p * (dpt[r] - dl_s[rl]) * scale;
      }
      __syncthreads();
      if constexpr (LP) {
#pragma unroll
        for (int qq = 0; qq < T / 16; ++qq) {  // rows 16 qq + 4 g .. + 3
          const int row = 16 * qq + 4 * g;
          const bf16x4_t pa = to_bf16x4(*reinterpret_cast<const f4*>(Ps + (kb * 16 + j) * PS + row));
          const bf16x4_t da = to_bf16x4(*reinterpret_cast<const f4*>(Ds + (kb * 16 + j) * PS + row));
#pragma unroll
          for (int b = 0; b < DBW; ++b) {
            const int dim = (db0 + b) * 16 + j;
            const float* gp = Gs + row * RS + dim;
            const float* qp = Qs + row * RS + dim;
            adv[b] = mfma_bf16_16x16x16(pa, to_bf16x4(f4{gp[0], gp[RS], gp[2 * RS], gp[3 * RS]}),
                                        adv[b]);
            adk[b] = mfma_bf16_16x16x16(da, to_bf16x4(f4{qp[0], qp[RS], qp[2 * RS], qp[3 * RS]}),
                                        adk[b]);
          }
        }
      } else {
#pragma unroll
        for (int c = 0; c < T / 4; ++c) {  // rows 4c + g
          const int row = 4 * c + g;
          const float pa = Ps[(kb * 16 + j) * PS + row];
          const float da = Ds[(kb * 16 + j) * PS + row];
#pragma unroll
          for (int b = 0; b < DBW; ++b) {
            const int dim = (db0 + b) * 16 + j;
            adv[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, Gs[row * RS + dim], adv[b], 0, 0, 0);
            adk[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(da, Qs[row * RS + dim], adk[b], 0, 0, 0);
          }
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < DBW; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = k0 + kb * 16 + 4 * g + r;
      if (key >= L) continue;
      const size_t o = ((size_t)sk * L + key) * HD + (db0 + b) * 16 + j;
      dk[o] = adk[b][r];
      dv[o] = adv[b][r];
    }
}

template <int HD, bool LP>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_mfma_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ dout, const float* __restrict__ lse, const float* __restrict__ delta,
    int S, int L, int H, int KVH, float scale, float* __restrict__ dq, AttnStrides qs,
    int causal) {
  constexpr int T = kAB, RS = HD + 4, PS = T + 4, NC = HD / 16, DBW = HD / 32;
  __shared__ __attribute__((aligned(16))) float Ks[T * RS], Vs[T * RS];
  __shared__ __attribute__((aligned(16))) float Ds[T * PS];  // [row][key]
  const int sh = (int)blockIdx.x, s = sh / H, h = sh % H;
  const int sk = s * KVH + h / (H / KVH);
  const int nqb = (L + T - 1) / T;
  const int qb = causal ? nqb - 1 - (int)blockIdx.y : (int)blockIdx.y;  // heaviest first
  const int r0 = qb * T, t = (int)threadIdx.x, wave = t / kWave, lane = t % kWave;
  const int g = lane / 16, j = lane % 16;
  const int rb = wave / 2, kb = wave % 2;  // score block: rows rb*16.., keys kb*16..
  const int db0 = (wave % 2) * DBW;        // dQ: rows rb*16.., dim blocks db0..
  f4 qf[NC], gf[NC];
  {
    const int row = min(r0 + rb * 16 + j, L - 1);  // past L: a valid row, not stored
    const float* qr = q + qs.at(s, row, h) + 4 * g;
    const float* gr = dout + qs.at(s, row, h) + 4 * g;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qf[c] = *reinterpret_cast<const f4*>(qr + 16 * c);
      gf[c] = *reinterpret_cast<const f4*>(gr + 16 * c);
    }
  }
  bf16x4_t qb16[LP ? NC : 1], gb16[LP ? NC : 1];  // LP: Q and dO fragments as bf16
  if constexpr (LP) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      qb16[c] = to_bf16x4(qf[c]);
      gb16[c] = to_bf16x4(gf[c]);
    }
  }
  float ls[4], dl[4];  // rows rb*16 + 4g + r of the score block
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = r0 + rb * 16 + 4 * g + r;
    const size_t li = ((size_t)s * H + h) * L + min(row, L - 1);
    ls[r] = lse[li];
    dl[r] = delta[li];
  }
  f4 adq[DBW];
#pragma unroll
  for (int b = 0; b < DBW; ++b) adq[b] = f4{0.f, 0.f, 0.f, 0.f};
  const float* kbase = k + (size_t)sk * L * HD;
  const float* vbase = v + (size_t)sk * L * HD;
  const int nkb = causal ? qb + 1 : nqb;  // key blocks holding keys <= the block's last row
  for (int kbk = 0; kbk < nkb; ++kbk) {
    const int k0 = kbk * T;
    __syncthreads();  // the previous tile's readers are done
    stage_rows<HD, RS>(Ks, L - k0, [&](int i) { return kbase + (size_t)(k0 + i) * HD; });
    stage_rows<HD, RS>(Vs, L - k0, [&](int i) { return vbase + (size_t)(k0 + i) * HD; });
    __syncthreads();
    f4 sc = f4{0.f, 0.f, 0.f, 0.f}, dp = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const f4 kv = *reinterpret_cast<const f4*>(Ks + (kb * 16 + j) * RS + 16 * c + 4 * g);
      const f4 vv = *reinterpret_cast<const f4*>(Vs + (kb * 16 + j) * RS + 16 * c + 4 * g);
      if constexpr (LP) {
        sc = mfma_bf16_16x16x16(qb16[c], to_bf16x4(kv), sc);
        dp = mfma_bf16_16x16x16(gb16[c], to_bf16x4(vv), dp);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sc = __builtin_amdgcn_mfma_f32_16x16x4f32(qf[c][e], kv[e], sc, 0, 0, 0);
          dp = __builtin_amdgcn_mfma_f32_16x16x4f32(gf[c][e], vv[e], dp, 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {  // row rb*16 + 4g + r, key kb*16 + j
      const int rl = rb * 16 + 4 * g + r, kl = kb * 16 + j;
      const int qr = r0 + rl, kc = k0 + kl;
      float p = 0.f;
      if (qr < L && kc < L && (!causal || kc <= qr)) p = expf(sc[r] * scale - ls[r]);
      Ds[rl * PS + kl] = p * (dp[r] - dl[r]) * scale;
    }
    __syncthreads();
    if constexpr (LP) {
#pragma unroll
      for (int qq = 0; qq < T / 16; ++qq) {  // keys 16 qq + 4 g .. + 3
        const int key = 16 * qq + 4 * g;
        const bf16x4_t a = to_bf16x4(*reinterpret_cast<const f4*>(Ds + (rb * 16 + j) * PS + key));
#pragma unroll
        for (int b = 0; b < DBW; ++b) {
          const float* kp = Ks + key * RS + (db0 + b) * 16 + j;
          adq[b] = mfma_bf16_16x16x16(a, to_bf16x4(f4{kp[0], kp[RS], kp[2 * RS], kp[3 * RS]}),
                                      adq[b]);
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < T / 4; ++c) {  // keys 4c + g
        const int key = 4 * c + g;
        const float a = Ds[(rb * 16 + j) * PS + key];
#pragma unroll
        for (int b = 0; b < DBW; ++b)
          adq[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, Ks[key * RS + (db0 + b) * 16 + j],
                                                        adq[b], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < DBW; ++b)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = r0 + rb * 16 + 4 * g + r;
      if (row >= L) continue;
      dq[qs.at(s, row, h) + (db0 + b) * 16 + j] = adq[b][r];
    }
}

// ------------------------------------------------------------- embedding ---
__global__ void embed_bwd_kernel(const int32_t* __restrict__ ids, const float* __restrict__ dx,
                                 int64_t rows, int d, int vocab, float* __restrict__ dtable) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * d) return;
  const int id = ids[i / d];
  if (id < 0 || id >= vocab) return;
  atomicAdd(&dtable[(int64_t)id * d + i % d], dx[i]);
}

// ------------------------------------------------------------ optimizers ---
// AdamW with decoupled weight decay: m, v moments, bias-corrected step.
__global__ void adamw_kernel(float* __restrict__ p, const float* __restrict__ g,
                             float* __restrict__ m, float* __restrict__ v, int64_t n, float lr,
                             float b1, float b2, float eps, float wd, float c1, float c2) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float gi = g[i];
  const float mi = b1 * m[i] + (1.f - b1) * gi;
  const float vi = b2 * v[i] + (1.f - b2) * gi * gi;
  m[i] = mi;
  v[i] = vi;
  const float upd = (mi / c1) / (sqrtf(vi / c2) + eps);
  p[i] = p[i] * (1.f - lr * wd) - lr * upd;
}

// Muon momentum (muon.rs:200-204): velocity = g + mu * velocity (g alone on
// the first step), update = mu * velocity + g.
__global__ void muon_momentum_kernel(const float* __restrict__ g, float* __restrict__ vel,
                                     float* __restrict__ upd, int64_t n, float mu, int first) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float vi = first ? g[i] : g[i] + vel[i] * mu;
  vel[i] = vi;
  upd[i] = vi * mu + g[i];
}

// y = a * x + b * y over n elements
__global__ void axpby_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n,
                             float a, float b) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  y[i] = a * x[i] + b * y[i];
}

// out[0] = max(sqrt(sum x^2), eps) in f64 partial order (one workgroup)
__global__ __launch_bounds__(1024) void frob_norm_kernel(const float* __restrict__ x, int64_t n,
                                                          float eps, float* __restrict__ out) {
  __shared__ double part[16];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += 1024) s += (double)x[i] * x[i];
  s = wave_sum_f64(s);
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < 16; ++w) t += part[w];
    out[0] = fmaxf((float)sqrt(t), eps);
  }
}

__global__ void scale_by_kernel(float* __restrict__ x, int64_t n, const float* __restrict__ div) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] = x[i] / div[0];
}

inline unsigned g256(int64_t n) { return (unsigned)ceil_div(n, 256); }

}  // namespace

int gemm_planes(int planes, bool ta, bool tb, int64_t M, int64_t N, int64_t K, float alpha,
                const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
                int64_t ldc, hipStream_t st, float* scratch = nullptr,
                int64_t scratch_floats = 0, int b_planes = 3);  // gemm_mfma.hip
int64_t gemm_planes_scratch_floats(bool ta, bool tb, int64_t M, int64_t N, int64_t K);

// sm_gemm_ex with the matrix-core launches on `planes` bf16 planes per operand
// (3: f32-grade; 2: 16-bit operands; 1: bf16 operands); the small problems
// stay on the f32 FMA kernel. scratch (optional, 16-byte aligned): room for
// the matrix-core launch's transposed operands (gemm_planes_scratch_floats).
// b_planes 2: B's values are exact in two bf16 planes (fake-quantized
// weights), so three-plane products skip the zero third plane of B.
int gemm_ex_planes(int planes, int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                   float alpha, const float* A, int64_t lda, const float* B, int64_t ldb,
                   float beta, float* C, int64_t ldc, void* stream, float* scratch,
                   int64_t scratch_floats, int b_planes) {
  SM_REQUIRE(A && B && C, "sm_gemm_ex: null buffer");
  SM_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M < (1 << 30) && N < (1 << 30) && K < (1 << 30),
             "sm_gemm_ex: bad shape");
  SM_REQUIRE(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N) && ldc >= N,
             "sm_gemm_ex: leading dimension too small");
  if (M == 0 || N == 0) return SM_OK;
  SM_REQUIRE(ceil_div(M, 64) <= 65535, "sm_gemm_ex: M above 65535 x 64 rows");
  hipStream_t st = as_stream(stream);
  // large problems on the matrix cores (bf16 plane products, gemm_mfma.hip);
  // small ones, where a launch has few 128 x 128 tiles, here
  if (K >= 32 && M * N >= (int64_t)128 * 128 * 16 && M * N * K >= ((int64_t)1 << 27))
    return gemm_planes(planes, trans_a != 0, trans_b != 0, M, N, K, alpha, A, lda, B, ldb, beta,
                       C, ldc, st, scratch, scratch_floats, b_planes);
  const dim3 grid((unsigned)ceil_div(N, 64), (unsigned)ceil_div(M, 64));
#define SM_GX(TA, TB)                                                                        \
  gemm_ex_kernel<TA, TB><<<grid, 256, 0, st>>>(A, lda, B, ldb, C, ldc, (int)M, (int)N, (int)K, \
                                               alpha, beta)
  if (trans_a && trans_b) SM_GX(true, true);
  else if (trans_a) SM_GX(true, false);
  else if (trans_b) SM_GX(false, true);
  else SM_GX(false, false);
#undef SM_GX
  SM_LAUNCH_CHECK();
  return SM_OK;
}
}  // namespace sm

using namespace sm;

extern "C" int sm_gemm_ex(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K, float alpha,
                          const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
                          float* C, int64_t ldc, void* stream) {
  return gemm_ex_planes(3, trans_a, trans_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, stream,
                        nullptr, 0, 3);
}

extern "C" int sm_rmsnorm_backward(const float* x, const float* gamma, const float* dy,
                                   int64_t rows, int64_t d, float eps, int accumulate, float* dx,
                                   float* dgamma, float* rinv_scratch, void* stream) {
  SM_REQUIRE(x && gamma && dy && dx && rinv_scratch, "sm_rmsnorm_backward: null buffer");
  SM_REQUIRE(rows >= 0 && d > 0, "sm_rmsnorm_backward: bad shape");
  if (rows == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  rmsnorm_bwd_kernel<<<(unsigned)rows, 256, 0, st>>>(x, gamma, dy, (int)d, eps, accumulate, dx,
                                                     rinv_scratch);
  if (dgamma)
    rmsnorm_dgamma_kernel<<<(unsigned)ceil_div(d, 64), 256, 0, st>>>(x, dy, rinv_scratch, rows,
                                                                     (int)d, accumulate, dgamma);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

namespace sm {
// Row chunks of rmsnorm_backward_parts: up to kDgammaChunks chunks of at least
// 128 rows; parts needs chunks x d floats.
constexpr int kDgammaChunks = 64;
int64_t rmsnorm_dgamma_chunks(int64_t rows) {
  return std::max<int64_t>(1, std::min<int64_t>(kDgammaChunks, rows / 128));
}
// sm_rmsnorm_backward with dgamma summed over row chunks (parts: at least
// rmsnorm_dgamma_chunks(rows) * d floats of scratch).
int rmsnorm_backward_parts(const float* x, const float* gamma, const float* dy, int64_t rows,
                           int64_t d, float eps, int accumulate, float* dx, float* dgamma,
                           float* rinv_scratch, float* parts, hipStream_t st) {
  SM_REQUIRE(x && gamma && dy && dx && rinv_scratch && dgamma && parts,
             "sm_rmsnorm_backward: null buffer");
  SM_REQUIRE(rows >= 0 && d > 0, "sm_rmsnorm_backward: bad shape");
  if (rows == 0) return SM_OK;
  rmsnorm_bwd_kernel<<<(unsigned)rows, 256, 0, st>>>(x, gamma, dy, (int)d, eps, accumulate, dx,
                                                     rinv_scratch);
  const int64_t chunks = rmsnorm_dgamma_chunks(rows), rpc = ceil_div(rows, chunks);
  rmsnorm_dgamma_parts_kernel<<<dim3((unsigned)ceil_div(d, 64), (unsigned)chunks), 256, 0, st>>>(
      x, dy, rinv_scratch, rows, (int)d, rpc, parts);
  dgamma_finish_kernel<<<(unsigned)ceil_div(d, 256), 256, 0, st>>>(parts, (int)chunks, (int)d,
                                                                   accumulate, dgamma);
  SM_LAUNCH_CHECK();
  return SM_OK;
}
}  // namespace sm

extern "C" int sm_rope_qk(float* qkv, const float* rope_table, const int32_t* pos0, int64_t S,
                          int64_t L, int64_t H, int64_t KVH, int64_t head_dim, int backward,
                          void* stream) {
  SM_REQUIRE(qkv && rope_table && pos0, "sm_rope_qk: null buffer");
  SM_REQUIRE(S >= 0 && L >= 0 && H > 0 && KVH > 0 && head_dim > 0 && head_dim % 2 == 0,
             "sm_rope_qk: bad shape");
  const int64_t rows = S * L, n = rows * (H + KVH) * (head_dim / 2);
  if (n == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  const float2* rt = reinterpret_cast<const float2*>(rope_table);
  if (backward)
    rope_qk_kernel<-1><<<g256(n), 256, 0, st>>>(qkv, rt, pos0, (int)L, (int)H, (int)KVH,
                                                (int)head_dim, rows);
  else
    rope_qk_kernel<1><<<g256(n), 256, 0, st>>>(qkv, rt, pos0, (int)L, (int)H, (int)KVH,
                                               (int)head_dim, rows);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

namespace sm {
namespace {
int attn_backward_f32(const float* q, const float* k, const float* v, const float* o,
                      const float* dout, const float* lse, int64_t S, int64_t L, int64_t H,
                      int64_t KVH, int64_t head_dim, float* dq, float* dk, float* dv,
                      float* delta_scratch, const AttnStrides& qs, bool causal, hipStream_t st,
                      bool bf16_ops = false) {
  auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  SM_REQUIRE(al16(q) && al16(k) && al16(v) && al16(dout) && qs.seq % 4 == 0 && qs.pos % 4 == 0 &&
                 qs.head % 4 == 0,
             "attention backward: q, k, v and grad_out need 16-byte aligned rows");
  SM_REQUIRE(ceil_div(L, kAB) <= 65535, "attention backward: sequence longer than %d",
             65535 * kAB);
  const float scale = 1.0f / sqrtf((float)head_dim);
  const int cz = causal ? 1 : 0;
  const unsigned rows_blocks = (unsigned)ceil_div(S * H * L, 4);
  const dim3 gkv((unsigned)(S * KVH), (unsigned)ceil_div(L, kAB));
  const dim3 gq((unsigned)(S * H), (unsigned)ceil_div(L, kAB));
#define SM_AB(HD, LP)                                                                          \
  do {                                                                                         \
    attn_bwd_delta_kernel<HD><<<rows_blocks, 256, 0, st>>>(o, dout, (int)S, (int)L, (int)H, qs, \
                                                           delta_scratch);                     \
    attn_bwd_dkv_mfma_kernel<HD, LP><<<gkv, 256, 0, st>>>(q, k, v, dout, lse, delta_scratch,  \
                                                          (int)S, (int)L, (int)H, (int)KVH,    \
                                                          scale, dk, dv, qs, cz);              \
    attn_bwd_dq_mfma_kernel<HD, LP><<<gq, 256, 0, st>>>(q, k, v, dout, lse, delta_scratch,    \
                                                        (int)S, (int)L, (int)H, (int)KVH,      \
                                                        scale, dq, qs, cz);                    \
  } while (0)
  if (head_dim == 64) {
    if (bf16_ops) SM_AB(64, true);
    else SM_AB(64, false);
  } else {
    if (bf16_ops) SM_AB(128, true);
    else SM_AB(128, false);
  }
#undef SM_AB
  SM_LAUNCH_CHECK();
  return SM_OK;
}
}  // namespace
}  // namespace sm

extern "C" int sm_attn_backward_f32(const float* q, const float* k, const float* v, const float* o,
                                    const float* dout, const float* lse, int64_t S, int64_t L,
                                    int64_t H, int64_t KVH, int64_t head_dim, float* dq,
                                    float* dk, float* dv, float* delta_scratch, void* stream) {
  SM_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv && delta_scratch,
             "sm_attn_backward_f32: null buffer");
  SM_REQUIRE(S >= 0 && L >= 0 && H > 0 && KVH > 0 && H % KVH == 0, "sm_attn_backward_f32: bad shape");
  SM_REQUIRE(head_dim == 64 || head_dim == 128, "sm_attn_backward_f32: head_dim must be 64 or 128");
  if (S == 0 || L == 0) return SM_OK;
  return attn_backward_f32(q, k, v, o, dout, lse, S, L, H, KVH, head_dim, dq, dk, dv,
                           delta_scratch, AttnStrides::rows(L, H, head_dim), true,
                           as_stream(stream));
}

extern "C" int sm_attn_backward_bf16ops(const float* q, const float* k, const float* v,
                                        const float* o, const float* dout, const float* lse,
                                        int64_t S, int64_t L, int64_t H, int64_t KVH,
                                        int64_t head_dim, float* dq, float* dk, float* dv,
                                        float* delta_scratch, void* stream) {
  SM_REQUIRE(q && k && v && o && dout && lse && dq && dk && dv && delta_scratch,
             "sm_attn_backward_bf16ops: null buffer");
  SM_REQUIRE(S >= 0 && L >= 0 && H > 0 && KVH > 0 && H % KVH == 0,
             "sm_attn_backward_bf16ops: bad shape");
  SM_REQUIRE(head_dim == 64 || head_dim == 128,
             "sm_attn_backward_bf16ops: head_dim must be 64 or 128");
  if (S == 0 || L == 0) return SM_OK;
  return attn_backward_f32(q, k, v, o, dout, lse, S, L, H, KVH, head_dim, dq, dk, dv,
                           delta_scratch, AttnStrides::rows(L, H, head_dim), true,
                           as_stream(stream), true);
}

extern "C" int sm_attention_backward(const float* q, const float* k, const float* v,
                                     const float* out, const float* grad_out, const float* lse,
                                     int64_t B, int64_t H, int64_t KVH, int64_t S,
                                     int64_t head_dim, int causal, float* dq, float* dk, float* dv,
                                     float* delta_scratch, void* stream) {
  SM_REQUIRE(q && k && v && out && grad_out && lse && dq && dk && dv && delta_scratch,
             "sm_attention_backward: null buffer");
  SM_REQUIRE(B >= 0 && S >= 0 && H > 0 && KVH > 0 && H % KVH == 0,
             "sm_attention_backward: bad shape (query heads must be a multiple of key/value heads)");
  SM_REQUIRE(head_dim == 64 || head_dim == 128, "sm_attention_backward: head_dim must be 64 or 128");
  SM_REQUIRE(causal == 0 || causal == 1, "sm_attention_backward: causal must be 0 or 1");
  if (B == 0 || S == 0) return SM_OK;
  return attn_backward_f32(q, k, v, out, grad_out, lse, B, S, H, KVH, head_dim, dq, dk, dv,
                           delta_scratch, AttnStrides::bhsd(S, H, head_dim), causal != 0,
                           as_stream(stream));
}

extern "C" int sm_embed_backward(const int32_t* ids, const float* dx, int64_t rows, int64_t d,
                                 int64_t vocab, float* dtable, void* stream) {
  SM_REQUIRE(ids && dx && dtable, "sm_embed_backward: null buffer");
  SM_REQUIRE(rows >= 0 && d > 0 && vocab > 0, "sm_embed_backward: bad shape");
  if (rows == 0) return SM_OK;
  embed_bwd_kernel<<<g256(rows * d), 256, 0, as_stream(stream)>>>(ids, dx, rows, (int)d,
                                                                  (int)vocab, dtable);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_adamw_step(float* param, const float* grad, float* m, float* v, int64_t n,
                             float lr, float beta1, float beta2, float eps, float weight_decay,
                             int64_t step, void* stream) {
  SM_REQUIRE(param && grad && m && v, "sm_adamw_step: null buffer");
  SM_REQUIRE(n >= 0 && step >= 1, "sm_adamw_step: step counts from 1");
  SM_REQUIRE(std::isfinite(lr) && beta1 >= 0.f && beta1 < 1.f && beta2 >= 0.f && beta2 < 1.f &&
                 eps > 0.f && weight_decay >= 0.f,
             "sm_adamw_step: invalid hyperparameters");
  if (n == 0) return SM_OK;
  const float c1 = 1.f - powf(beta1, (float)step), c2 = 1.f - powf(beta2, (float)step);
  adamw_kernel<<<g256(n), 256, 0, as_stream(stream)>>>(param, grad, m, v, n, lr, beta1, beta2,
                                                       eps, weight_decay, c1, c2);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_muon_momentum(const float* grad, float* velocity, float* update, int64_t n,
                                float momentum, int first_step, void* stream) {
  SM_REQUIRE(grad && velocity && update, "sm_muon_momentum: null buffer");
  if (n <= 0) return SM_OK;
  muon_momentum_kernel<<<g256(n), 256, 0, as_stream(stream)>>>(grad, velocity, update, n, momentum,
                                                               first_step);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_axpby(const float* x, float* y, int64_t n, float a, float b, void* stream) {
  SM_REQUIRE(x && y, "sm_axpby: null buffer");
  if (n <= 0) return SM_OK;
  axpby_kernel<<<g256(n), 256, 0, as_stream(stream)>>>(x, y, n, a, b);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_frobenius_normalize(float* x, int64_t n, float eps, float* norm_out,
                                      void* stream) {
  SM_REQUIRE(x && norm_out, "sm_frobenius_normalize: null buffer");
  if (n <= 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  frob_norm_kernel<<<1, 1024, 0, st>>>(x, n, eps, norm_out);
  scale_by_kernel<<<g256(n), 256, 0, st>>>(x, n, norm_out);
  SM_LAUNCH_CHECK();
  return SM_OK;
}
