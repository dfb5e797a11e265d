// Attention over a contiguous KV cache (kernel 2 and the prefill/recompute
// attention).
//
// Semantics: MultiHeadAttention::forward_cached / sdpa
// (summa-llm/src/model/attention.rs:216-265, 318-371): softmax(q.K^T / sqrt(hd)) . V
// over key positions 0..=pos of the query, GQA query head h reading KV head
// h / (H / KVH) (repeat_kv, fused_attention.rs:114-125 — here never
// materialised: each KV head is read once for its whole query-head group).
// Cache layout [S, KVH, cap, hd] as AttnCache (attention.rs:20-40, 115-134).
//
// 16-bit decode kernel (one query per sequence; q and cache bf16 or f16): one
// workgroup per (KV head, sequence); its four waves split the key range in
// tiles of 64. Scores Q.K^T come from v_mfma_f32_16x16x32_{bf16,f16} with the
// group's query heads
// as the 16-row A operand (padded) and K rows read straight from HBM as the B
// operand (natural [pos][hd] layout is already k-contiguous per lane). The
// online softmax runs on the MFMA output registers, probabilities go through a
// per-wave LDS slice, and P.V is a VALU FMA pass with hd/DPL lanes per V row,
// each lane owning DPL dims (DPL = 8: 16-byte loads; DPL = 4, 8-byte loads, for
// groups of 4 or more query heads, which halves the per-head accumulators:
// config[2]'s kernel 138 -> 133 VGPRs, 82 -> 80 us, and 16 heads per KV head
// no longer spill, 225 -> 52 us at S 64, KVH 2, len 512-1023). Tiles are 32 keys; all
// K and V loads of a tile are issued together before its math, so a tile costs
// one HBM round trip; 32-key tiles keep the kernel at 138 VGPRs, three waves
// per SIMD (measured on MI355X, config[2] decode S256 H16/4 len 768: 78-80 us
// against 81-83 us for 64-key tiles at two waves per SIMD, and the same again
// with 32-key tiles double-buffered in registers at two). Waves merge (max,
// sum, O) in LDS at the end in a fixed order.
//
// Prefill / recompute (many queries, causal) uses the flash-attention kernel
// in prefill_attention.hip; fp32 models (config[0]) use the simple VALU
// kernel below for both.
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "attn_common.hpp"
#include "common.hpp"

namespace sm {
namespace {

constexpr int kMaxQpk = 16;  // query heads per KV head handled by one WG
constexpr int kMaxPrefixSplits = 4;  // key splits of a shared prompt (attn_prefix_*)

// QM: query heads per KV head the kernel is built for (>= H / KVH); EX: exactly
// QM, so the per-head bounds are compile-time; DPL: V dims per lane in P.V.
// PRE: keys 0..k0-1 were done by attn_prefix_kernel (a prompt shared by a
// group of rollouts); this kernel takes keys k0..len-1 from the sequence's
// cache and folds the prefix's nsplit partials (max, sum, unnormalised O per
// query head) into its final merge.
template <int HD, int QM, bool KF16, int OM, bool EX, int DPL, bool PRE = false>
__global__ __launch_bounds__(256, PRE ? 4 : 1) void attn_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ lens,
    void* __restrict__ out, int H, int KVH, int cap, float scale, int k0 = 0,
    const float* __restrict__ pre_o = nullptr, const float* __restrict__ pre_ml = nullptr,
    int nsplit = 0) {
  typedef typename Op8<KF16>::T op8;
  static_assert(DPL == 4 || DPL == 8, "DPL is 4 or 8");
  constexpr int LPK = HD / DPL;    // lanes per V row in the P.V pass (DPL dims each)
  typedef typename std::conditional<DPL == 8, u32x4, u32x2>::type vrow;
  constexpr int PPI = 64 / LPK;    // keys per P.V iteration per wave
  constexpr int STEPS = HD / 32;   // MFMA k-steps over head_dim
  const int kvh = blockIdx.x, s = blockIdx.y;
  const int qpk = EX ? QM : H / KVH;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int len = min(lens[s], cap);
  const size_t kv_base = ((size_t)s * KVH + kvh) * cap * HD;

  constexpr int TK = 32;         // keys per tile
  constexpr int VR = TK / PPI;   // V rows of a tile held by each lane
  constexpr int KB = TK / 16;    // 16-key MFMA blocks per tile
  __shared__ float pbuf[4][QM][TK];
  __shared__ float mrg_m[4][QM], mrg_l[4][QM];
  __shared__ float mrg_o[4][QM][HD];
  // PRE: the prefix partials of this (sequence, KV head), [head][split][HD] O
  // and [head][split][2] (max, sum), staged in LDS for the final merge. Every
  // load is issued up front (16 bytes per thread per 1024 floats of O) next
  // to the query loads, and stored after them, so the start of the kernel
  // waits for one memory round trip instead of one per staging pass.
  __shared__ __attribute__((aligned(16))) float pre_os[PRE ? QM * kMaxPrefixSplits * HD : 1];
  __shared__ float pre_mls[PRE ? QM * kMaxPrefixSplits * 2 : 1];
  constexpr int PV = PRE ? (QM * kMaxPrefixSplits * HD + 1023) / 1024 : 1;  // f4 per thread
  f4 pv[PV];
  float pml = 0.f;
  const int n_o = qpk * nsplit * HD, n_ml = qpk * nsplit * 2;  // n_o % 4 == 0
  if constexpr (PRE) {
    const size_t first = ((size_t)s * H + kvh * qpk) * nsplit;  // this WG's first slot
    const f4* src = reinterpret_cast<const f4*>(pre_o + first * HD);
#pragma unroll
    for (int i = 0; i < PV; ++i) {
      const int e4 = (int)threadIdx.x + i * 256;
      if (4 * e4 < n_o) pv[i] = src[e4];
    }
    if ((int)threadIdx.x < n_ml) pml = pre_ml[first * 2 + threadIdx.x];
  }

  // A operand: query head (kvh*qpk + j) if j < qpk.
  op8 qa[STEPS];
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    if (j < qpk) {
      const uint16_t* qp = q + ((size_t)s * H + kvh * qpk + j) * HD + st * 32 + g * 8;
      qa[st] = *reinterpret_cast<const op8*>(qp);
    } else {
      qa[st] = op8{};
    }
  }
  if constexpr (PRE) {
#pragma unroll
    for (int i = 0; i < PV; ++i) {
      const int e4 = (int)threadIdx.x + i * 256;
      if (4 * e4 < n_o) reinterpret_cast<f4*>(pre_os)[e4] = pv[i];
    }
    if ((int)threadIdx.x < n_ml) pre_mls[threadIdx.x] = pml;
  }

  float m_i[QM], l_i[QM], o[QM][DPL];
#pragma unroll
  for (int i = 0; i < QM; ++i) {
    m_i[i] = -INFINITY;
    l_i[i] = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[i][e] = 0.f;
  }

  const int sub = lane / LPK;          // which key of the PPI group this lane handles
  const int dl = (lane % LPK) * DPL;   // first of the dims this lane owns

  // One tile's loads: K fragments for the score MFMAs and this lane's V rows.
  // Rows past the end are clamped to the last valid row and masked below.
  struct Tile {
    op8 kf[KB][STEPS];
    vrow vr[VR];
  };
  const int last = max(len - 1, 0);  // every load stays inside the sequence's cache rows
  auto load = [&](int t0, Tile& T) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int key = min(t0 + kb * 16 + j, last);
#pragma unroll
      for (int st = 0; st < STEPS; ++st)
        T.kf[kb][st] = *reinterpret_cast<const op8*>(kc + kv_base + (size_t)key * HD + st * 32 + g * 8);
    }
#pragma unroll
    for (int i = 0; i < VR; ++i) {
      const int key = min(t0 + sub + i * PPI, last);
      T.vr[i] = *reinterpret_cast<const vrow*>(vc + kv_base + (size_t)key * HD + dl);
    }
  };
  auto compute = [&](int t0, const Tile& T) {
    // ---- scores for TK keys: KB MFMA blocks of 16 keys
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int key = t0 + kb * 16 + j;
      f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < STEPS; ++st)
        acc = Op8<KF16>::mfma(qa[st], T.kf[kb][st], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * g + r;
        if (row < qpk) pbuf[wave][row][kb * 16 + j] = (key < len) ? acc[r] * scale : -INFINITY;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- online softmax per query head (lane = key within the tile)
#pragma unroll
    for (int i = 0; i < QM; ++i) {
      if (i >= qpk) break;
      const float v = lane < TK ? pbuf[wave][i][lane] : -INFINITY;
      const float mnew = fmaxf(m_i[i], wave_max(v));
      const float alpha = (m_i[i] == -INFINITY) ? 0.f : __expf(m_i[i] - mnew);
      const float p = (v == -INFINITY) ? 0.f : __expf(v - mnew);
      l_i[i] = l_i[i] * alpha + wave_sum(p);
      m_i[i] = mnew;
#pragma unroll
      for (int e = 0; e < DPL; ++e) o[i][e] *= alpha;
      if (lane < TK) pbuf[wave][i][lane] = p;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- P.V from the V rows already in registers (p = 0 past the end)
#pragma unroll
    for (int vi = 0; vi < VR; ++vi) {
      const int tt = sub + vi * PPI;
      float v[DPL];
      if constexpr (DPL == 8) unpack8<KF16>(T.vr[vi], v);
      else unpack4<KF16>(T.vr[vi], v);
#pragma unroll
      for (int i = 0; i < QM; ++i) {
        if (i >= qpk) break;
        const float p = pbuf[wave][i][tt];
#pragma unroll
        for (int e = 0; e < DPL; ++e) o[i][e] = fmaf(p, v[e], o[i][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  };

  // Wave w takes tiles w, w + 4, ... (of keys k0.. with a shared prefix)
  constexpr int STRIDE = 4 * TK;
  for (int t0 = (PRE ? k0 : 0) + wave * TK; t0 < len; t0 += STRIDE) {
    Tile ta;
    load(t0, ta);
    compute(t0, ta);
  }
  // combine the PPI key-subsets inside the wave
  if constexpr (PPI > 1) {
#pragma unroll
    for (int i = 0; i < QM; ++i)
#pragma unroll
      for (int off = LPK; off < 64; off <<= 1)
#pragma unroll
        for (int e = 0; e < DPL; ++e) o[i][e] += __shfl_xor(o[i][e], off, kWave);
  }
#pragma unroll
  for (int i = 0; i < QM; ++i) {
    if (i >= qpk) break;
    if (lane == 0) { mrg_m[wave][i] = m_i[i]; mrg_l[wave][i] = l_i[i]; }
    if (lane < LPK) {
#pragma unroll
      for (int e = 0; e < DPL; ++e) mrg_o[wave][i][dl + e] = o[i][e];
    }
  }
  __syncthreads();
  // merge the four waves: thread t handles (head, dim) pairs
  for (int e = threadIdx.x; e < qpk * HD; e += 256) {
    const int i = e / HD, d = e % HD;
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) m = fmaxf(m, mrg_m[w][i]);
    const int slot = i * nsplit;  // in the staged partials
    if constexpr (PRE)
      for (int p = 0; p < nsplit; ++p) m = fmaxf(m, pre_mls[(slot + p) * 2]);
    float l = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (mrg_m[w][i] == -INFINITY) continue;
      const float c = __expf(mrg_m[w][i] - m);
      l += mrg_l[w][i] * c;
      o += mrg_o[w][i][d] * c;
    }
    if constexpr (PRE)
      for (int p = 0; p < nsplit; ++p) {
        const float pm = pre_mls[(slot + p) * 2];
        if (pm == -INFINITY) continue;
        const float c = __expf(pm - m);
        l += pre_mls[(slot + p) * 2 + 1] * c;
        o += pre_os[(slot + p) * HD + d] * c;
      }
    store_out<OM>(out, (size_t)s, H * HD, (kvh * qpk + i) * HD + d, o / l);
  }
}

// Decode attention over a prompt shared by a group of G rollouts (prompt
// groups): the prompt's K / V ([groups, KVH, P, hd], written once per group by
// the prefill) is read once per (group, KV head) for all G x qpk query heads
// of the group's rollouts at this decode step, instead of once per rollout.
// One workgroup per (KV head, group, key split); its four waves take 32-key
// tiles in turn. Per 16-key block:
//   scores S^T = K . Q^T: v_mfma_f32_16x16x32_{f16,bf16}, A = 16 key rows (read
//   straight from HBM, 16 bytes per lane), B = 16 queries (registers, loaded
//   once); lane (g, j) gets keys 4g..4g+3 of the block for query j;
//   online softmax per query = per lane column (max / sum over the block by
//   two cross-row shuffles), so the rescale of O is lane-local;
//   O^T += V^T . P^T: v_mfma_f32_16x16x4_f32 with P in f32 (the decode kernel's
//   f32 probabilities), one MFMA per (key 4g + r, dim block db). A-row i of dim
//   block db is dim i * (hd / 16) + db, so lane (g, j) loads dims
//   j*hd/16 .. +hd/16 of its key row as one 16-byte (hd 128) or 8-byte load,
//   and ends holding dims 4g*hd/16 .. +4*hd/16 of query j.
// The four waves merge in LDS; each (query head, split) writes its partial
// (max, sum, unnormalised O) for attn_decode_kernel<..., PRE>, which adds the
// rollout's own keys P..len-1 and normalises. QB: 16-query blocks (G * qpk <=
// 16 * QB).
template <int HD, bool KF16, int QB>
__global__ __launch_bounds__(256) void attn_prefix_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ pk,
    const uint16_t* __restrict__ pv, float* __restrict__ part_o, float* __restrict__ part_ml,
    int H, int KVH, int G, int P, int per, float scale) {
  typedef typename Op8<KF16>::T op8;
  constexpr int STEPS = HD / 32;  // score MFMA k-steps over head_dim
  constexpr int DB = HD / 16;     // dim blocks of the P.V MFMA = V dims per lane
  typedef typename std::conditional<DB == 8, u32x4, u32x2>::type vrow;
  constexpr int TK = 32;          // keys per tile: two 16-key blocks
  const int kvh = blockIdx.x, grp = blockIdx.y, sp = blockIdx.z, splits = gridDim.z;
  const int qpk = H / KVH, nq = G * qpk;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int k_lo = sp * per, k_hi = min(P, k_lo + per);
  const size_t base = ((size_t)grp * KVH + kvh) * P * HD;
  __shared__ float mrg_m[4][QB * 16], mrg_l[4][QB * 16];
  __shared__ float mrg_o[4][QB * 16][HD + 1];

  // B operand of the scores: query column j of block qb is query qb*16 + j =
  // (rollout grp*G + qi / qpk, head kvh*qpk + qi % qpk); zero past nq.
  op8 qf[QB][STEPS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qi = qb * 16 + j;
#pragma unroll
    for (int st = 0; st < STEPS; ++st) qf[qb][st] = op8{};
    if (qi < nq) {
      const int s = grp * G + qi / qpk, h = kvh * qpk + qi % qpk;
      const uint16_t* qp = q + ((size_t)s * H + h) * HD + g * 8;
#pragma unroll
      for (int st = 0; st < STEPS; ++st) qf[qb][st] = *reinterpret_cast<const op8*>(qp + st * 32);
    }
  }
  float m_i[QB], l_i[QB];
  f4 o[QB][DB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = -INFINITY;
    l_i[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[qb][db] = f4{0.f, 0.f, 0.f, 0.f};
  }

  const int last = k_hi - 1;  // loads past the split's end re-read its last key (masked)
  for (int t0 = k_lo + wave * TK; t0 < k_hi; t0 += 4 * TK) {
    op8 kf[2][STEPS];
    vrow vr[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const uint16_t* kp = pk + base + (size_t)min(t0 + kb * 16 + j, last) * HD + g * 8;
#pragma unroll
      for (int st = 0; st < STEPS; ++st) kf[kb][st] = *reinterpret_cast<const op8*>(kp + st * 32);
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        vr[kb][r] = *reinterpret_cast<const vrow*>(
            pv + base + (size_t)min(t0 + kb * 16 + 4 * g + r, last) * HD + j * DB);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      f4 sc[2];
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sc[kb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < STEPS; ++st) sc[kb] = Op8<KF16>::mfma(kf[kb][st], qf[qb][st], sc[kb]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = (t0 + kb * 16 + 4 * g + r < k_hi) ? sc[kb][r] * scale : -INFINITY;
          sc[kb][r] = v;
          mx = fmaxf(mx, v);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float mnew = fmaxf(m_i[qb], mx);  // finite: key t0 is in range
      const float alpha = (m_i[qb] == -INFINITY) ? 0.f : __expf(m_i[qb] - mnew);
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = (sc[kb][r] == -INFINITY) ? 0.f : __expf(sc[kb][r] - mnew);
          sc[kb][r] = p;
          ps += p;
        }
      ps += __shfl_xor(ps, 16, kWave);
      ps += __shfl_xor(ps, 32, kWave);
      l_i[qb] = l_i[qb] * alpha + ps;
      m_i[qb] = mnew;
#pragma unroll
      for (int db = 0; db < DB; ++db) o[qb][db] *= alpha;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v[DB];
          if constexpr (DB == 8) unpack8<KF16>(vr[kb][r], v);
          else unpack4<KF16>(vr[kb][r], v);
#pragma unroll
          for (int db = 0; db < DB; ++db)
            o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[db], sc[kb][r], o[qb][db], 0, 0, 0);
        }
    }
  }
  // lane (g, j) holds dims (4g + r) * DB + db of query qb*16 + j
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r) mrg_o[wave][qb * 16 + j][(4 * g + r) * DB + db] = o[qb][db][r];
    if (g == 0) {
      mrg_m[wave][qb * 16 + j] = m_i[qb];
      mrg_l[wave][qb * 16 + j] = l_i[qb];
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < nq * HD; e += 256) {
    const int qi = e / HD, d = e % HD;
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) m = fmaxf(m, mrg_m[w][qi]);
    float l = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (mrg_m[w][qi] == -INFINITY) continue;
      const float c = __expf(mrg_m[w][qi] - m);
      l += mrg_l[w][qi] * c;
      acc += mrg_o[w][qi][d] * c;
    }
    const int s = grp * G + qi / qpk, h = kvh * qpk + qi % qpk;
    const size_t slot = ((size_t)s * H + h) * splits + sp;
    part_o[slot * HD + d] = acc;
    if (d == 0) {
      part_ml[slot * 2] = m;
      part_ml[slot * 2 + 1] = l;
    }
  }
}

// The f16-cache form of attn_prefix_kernel (the quantized models' cache):
// P.V on the f16 matrix cores instead of f32 ones. Per 16-key tile,
// O^T += V^T . P^T with v_mfma_f32_16x16x16_f16: B = P^T, lane (g, j) holding
// p of keys 4g..4g+3 for query j, which is exactly the score MFMA's output
// layout; A = V^T for dim block db, lane (g, j) holding dim j*hd/16 + db of
// keys 4g..4g+3, gathered from the same 16-byte V loads as before (a 4 x 8
// transpose of 16-bit values per lane and tile). P enters as an f16 hi + lo
// pair (about 22 significant bits, so the f32 probabilities of the decode
// kernel), scaled by 2^14 first so that probabilities far below the row's
// maximum stay normal f16 numbers; O is scaled back before the merge. Two
// MFMAs per (dim block, query block) replace the f32 form's four and run
// 4x faster each. The next tile's K / V loads are issued before the current
// tile's math (a 16-key tile, so both fit the registers).
template <int HD, int QB>
__global__ __launch_bounds__(256) void attn_prefix_f16_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ pk,
    const uint16_t* __restrict__ pv, float* __restrict__ part_o, float* __restrict__ part_ml,
    int H, int KVH, int G, int P, int per, float scale) {
  constexpr int STEPS = HD / 32;  // score MFMA k-steps over head_dim
  constexpr int DB = HD / 16;     // dim blocks of the P.V MFMA = V dims per lane
  typedef typename std::conditional<DB == 8, u32x4, u32x2>::type vrow;
  constexpr int TK = 16;          // keys per tile
  constexpr float kPS = 16384.f;  // P scale before the f16 split
  const int qpk = H / KVH, nq = G * qpk;
  // blockIdx.z = split * nqg + query group: each workgroup takes QB 16-query
  // blocks, so a group's query blocks run in several workgroups (fewer
  // registers, more of them resident); their K / V reads after the first hit
  // L2 (the workgroups of one split are KVH * groups apart in launch order, a
  // multiple of the 8 XCDs at the configs' shapes, so on one XCD).
  const int nqg = (nq + QB * 16 - 1) / (QB * 16);
  const int kvh = blockIdx.x, grp = blockIdx.y, sp = blockIdx.z / nqg;
  const int splits = gridDim.z / nqg, qbase = (blockIdx.z % nqg) * QB * 16;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16;
  const int k_lo = sp * per, k_hi = min(P, k_lo + per);
  const size_t base = ((size_t)grp * KVH + kvh) * P * HD;
  __shared__ float mrg_m[4][QB * 16], mrg_l[4][QB * 16];
  __shared__ float mrg_o[4][QB * 16][HD + 1];

  h8 qf[QB][STEPS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qi = qbase + qb * 16 + j;
#pragma unroll
    for (int st = 0; st < STEPS; ++st) qf[qb][st] = h8{};
    if (qi < nq) {
      const int s = grp * G + qi / qpk, h = kvh * qpk + qi % qpk;
      const uint16_t* qp = q + ((size_t)s * H + h) * HD + g * 8;
#pragma unroll
      for (int st = 0; st < STEPS; ++st) qf[qb][st] = *reinterpret_cast<const h8*>(qp + st * 32);
    }
  }
  float m_i[QB], l_i[QB];
  f4 o[QB][DB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_i[qb] = -INFINITY;
    l_i[qb] = 0.f;
#pragma unroll
    for (int db = 0; db < DB; ++db) o[qb][db] = f4{0.f, 0.f, 0.f, 0.f};
  }

  struct Tile {
    h8 kf[STEPS];
    vrow vr[4];
  };
  const int last = k_hi - 1;  // loads past the split's end re-read its last key (masked)
  auto load = [&](int t0, Tile& T) {
    const uint16_t* kp = pk + base + (size_t)min(t0 + j, last) * HD + g * 8;
#pragma unroll
    for (int st = 0; st < STEPS; ++st) T.kf[st] = *reinterpret_cast<const h8*>(kp + st * 32);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      T.vr[r] = *reinterpret_cast<const vrow*>(pv + base + (size_t)min(t0 + 4 * g + r, last) * HD +
                                               j * DB);
  };
  auto half_of = [](const vrow& v, int e) -> uint32_t {
    const uint32_t w = (e >> 1) == 0 ? v[0] : (e >> 1) == 1 ? v[1] : (e >> 1) == 2 ? v[2] : v[3];
    return (e & 1) ? (w >> 16) : (w & 0xffffu);
  };
  auto compute = [&](int t0, const Tile& T) {
    h4 a[DB];  // V^T: dim j*DB + db of keys t0 + 4g + r, r = 0..3
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      u32x2 w;
      w[0] = half_of(T.vr[0], db) | (half_of(T.vr[1], db) << 16);
      w[1] = half_of(T.vr[2], db) | (half_of(T.vr[3], db) << 16);
      a[db] = __builtin_bit_cast(h4, w);
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      f4 sc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < STEPS; ++st)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(T.kf[st], qf[qb][st], sc, 0, 0, 0);
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = (t0 + 4 * g + r < k_hi) ? sc[r] * scale : -INFINITY;
        sc[r] = v;
        mx = fmaxf(mx, v);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      const float mnew = fmaxf(m_i[qb], mx);  // finite: key t0 is in range
      const float alpha = (m_i[qb] == -INFINITY) ? 0.f : __expf(m_i[qb] - mnew);
      float ps = 0.f;
      h4 bh, bl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = (sc[r] == -INFINITY) ? 0.f : __expf(sc[r] - mnew);
        ps += p;
        _Float16 hi, lo;
        split_f16(p * kPS, hi, lo);
        bh[r] = hi;
        bl[r] = lo;
      }
      ps += __shfl_xor(ps, 16, kWave);
      ps += __shfl_xor(ps, 32, kWave);
      l_i[qb] = l_i[qb] * alpha + ps;
      m_i[qb] = mnew;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        o[qb][db] *= alpha;
        o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x16f16(a[db], bh, o[qb][db], 0, 0, 0);
        o[qb][db] = __builtin_amdgcn_mfma_f32_16x16x16f16(a[db], bl, o[qb][db], 0, 0, 0);
      }
    }
  };
  int t0 = k_lo + wave * TK;
  if (t0 < k_hi) {
    Tile cur;
    load(t0, cur);
    for (; t0 < k_hi; t0 += 4 * TK) {
      Tile nxt;
      load(t0 + 4 * TK, nxt);  // clamped into the split: in bounds past its end too
      compute(t0, cur);
      cur = nxt;
    }
  }
  // lane (g, j) holds dims (4g + r) * DB + db of query qb*16 + j (times kPS)
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        mrg_o[wave][qb * 16 + j][(4 * g + r) * DB + db] = o[qb][db][r] * (1.f / kPS);
    if (g == 0) {
      mrg_m[wave][qb * 16 + j] = m_i[qb];
      mrg_l[wave][qb * 16 + j] = l_i[qb];
    }
  }
  __syncthreads();
  const int nql = min(nq - qbase, QB * 16);  // this workgroup's queries
  for (int e = threadIdx.x; e < nql * HD; e += 256) {
    const int ql = e / HD, d = e % HD, qi = qbase + ql;
    float m = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) m = fmaxf(m, mrg_m[w][ql]);
    float l = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if (mrg_m[w][ql] == -INFINITY) continue;
      const float c = __expf(mrg_m[w][ql] - m);
      l += mrg_l[w][ql] * c;
      acc += mrg_o[w][ql][d] * c;
    }
    const int s = grp * G + qi / qpk, h = kvh * qpk + qi % qpk;
    const size_t slot = ((size_t)s * H + h) * splits + sp;
    part_o[slot * HD + d] = acc;
    if (d == 0) {
      part_ml[slot * 2] = m;
      part_ml[slot * 2 + 1] = l;
    }
  }
}

// fp32 attention (fp32 models: decode, prefill and recompute; any strides of
// q / out, causal or not): one wave per query (sequence s, query row r, head
// h), over keys in chunks of 64. Scores: lane l takes key t0 + l and reads
// its K row itself (float4 loads, all in flight together), q sits in
// registers; the chunk's max and sum are wave reductions (online softmax
// across chunks). P.V: the chunk's probabilities go through a per-wave LDS
// slice and lane l owns output dims l (and l + 64 for hd 128), reading each
// V row coalesced. q [S, L, H, hd] at qs (or [B, H, S, hd]); cache
// [S, KVH, cap, hd] f32; keys 0..pos (pos = pos0[s] + r + pos_off, or L - 1
// without the causal mask).
template <int HD>
__global__ __launch_bounds__(256) void attn_valu_f32_kernel(
    const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc,
    const int32_t* __restrict__ pos0, int pos_off, float* __restrict__ out,
    float* __restrict__ lse, int S, int L, int H,
    int KVH, int cap, float scale, AttnStrides qs, AttnStrides os, int causal) {
  constexpr int DL = HD / 64;  // output dims per lane
  __shared__ float pbuf[4][64];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t wid = (int64_t)blockIdx.x * 4 + wave;
  if (wid >= (int64_t)S * L * H) return;  // uniform per wave; no workgroup barrier below
  const int h = wid % H;
  const int r = (wid / H) % L;
  const int s = wid / ((int64_t)H * L);
  const int kvh = h / (H / KVH);
  const int pos = causal ? (pos0 ? pos0[s] : 0) + r + pos_off : L - 1;
  const float* qp = q + qs.at(s, r, h);
  const float* kb = kc + ((size_t)s * KVH + kvh) * cap * HD;
  const float* vb = vc + ((size_t)s * KVH + kvh) * cap * HD;
  float qv[HD];
#pragma unroll
  for (int d = 0; d < HD; d += 4) {
    const float4 t = *reinterpret_cast<const float4*>(qp + d);
    qv[d] = t.x; qv[d + 1] = t.y; qv[d + 2] = t.z; qv[d + 3] = t.w;
  }
  float m = -INFINITY, l = 0.f, o[DL];
#pragma unroll
  for (int e = 0; e < DL; ++e) o[e] = 0.f;
  for (int t0 = 0; t0 <= pos; t0 += 64) {
    const int t = t0 + lane;
    const bool ok = t <= pos;
    const float* kr = kb + (size_t)(ok ? t : t0) * HD;
    float sc = 0.f;
#pragma unroll
    for (int d = 0; d < HD; d += 4) {
      const float4 k4 = *reinterpret_cast<const float4*>(kr + d);
      sc = fmaf(qv[d], k4.x, sc);
      sc = fmaf(qv[d + 1], k4.y, sc);
      sc = fmaf(qv[d + 2], k4.z, sc);
      sc = fmaf(qv[d + 3], k4.w, sc);
    }
    sc = ok ? sc * scale : -INFINITY;
    const float mnew = fmaxf(m, wave_max(sc));
    const float alpha = (m == -INFINITY) ? 0.f : expf(m - mnew);
    const float p = ok ? expf(sc - mnew) : 0.f;
    l = l * alpha + wave_sum(p);
    m = mnew;
    pbuf[wave][lane] = p;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int nt = min(64, pos + 1 - t0);
    float acc[DL];
#pragma unroll
    for (int e = 0; e < DL; ++e) acc[e] = 0.f;
#pragma unroll 8
    for (int tt = 0; tt < nt; ++tt) {
      const float pt = pbuf[wave][tt];
      const float* vr = vb + (size_t)(t0 + tt) * HD + lane;
#pragma unroll
      for (int e = 0; e < DL; ++e) acc[e] = fmaf(pt, vr[e * 64], acc[e]);
    }
#pragma unroll
    for (int e = 0; e < DL; ++e) o[e] = fmaf(o[e], alpha, acc[e]);
    __builtin_amdgcn_wave_barrier();  // the next chunk rewrites pbuf
  }
  float* op = out + os.at(s, r, h);
#pragma unroll
  for (int e = 0; e < DL; ++e) op[lane + e * 64] = o[e] / l;
  if (lse && lane == 0) lse[((size_t)s * H + h) * L + r] = m + logf(l);
}

// fp32 attention over many queries (prefill, recompute, the policy's forward;
// L >= 32), FlashAttention-style on the f32 matrix cores
// (v_mfma_f32_16x16x4_f32; MFMA lane (g, j) = (lane / 16, lane % 16) supplies
// A[j][k = g], B[k = g][j] and receives D[4 g + r][j]): one workgroup per
// (sequence, head) and 64 query rows, the heaviest (last) blocks first, each
// wave owning 16 rows, K and V in 32-key tiles through LDS. Per tile a wave
// forms S^T = K Q^T (A = K rows from LDS, B = its rows of Q held in
// registers; the head-dim contraction takes dim 16 c + 4 g + e from lane
// group g in step (c, e)), so lane (g, j) holds keys 4 g + r of each 16-key
// block for row j: the row's max and sum reduce over the four lane groups
// (two shuffles), and O^T += V^T P^T takes P^T straight from those registers
// as the B operand (step r: key 4 g + r from lane group g), with V^T read from
// LDS as the A operand. Lane (g, j) ends holding dims 4 g + r of each 16-dim
// block of row j. Same semantics and arguments as attn_valu_f32_kernel.
// Measured at one GRPO group's shape (8 x 1023 positions, 16 / 4 heads, hd
// 128): 0.87-0.93 ms per layer with f32 FMAs on 32 x 32 LDS tiles, 0.38-0.40
// ms here.
// LP: bf16 operands (v_mfma_f32_16x16x16bf16_1k, f32 accumulation), the
// 16-bit precision of the reference's CUDA-path flash attention: each run of
// four f32 steps e = 0..3 (lane group g: k = 4 g + e) is one bf16 MFMA whose
// lane group g supplies k = 4 g .. 4 g + 3, the same operands rounded to
// bf16 (round to nearest even) and the same output layout.
template <int HD, bool LP>
__global__ __launch_bounds__(256, 2) void attn_f32_mfma_kernel(
    const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc,
    const int32_t* __restrict__ pos0, int pos_off, float* __restrict__ out,
    float* __restrict__ lse, int S, int L, int H, int KVH, int cap, float scale, AttnStrides qs,
    AttnStrides os, int causal) {
  constexpr int TR = 64, TK = 32, RS = HD + 4, NC = HD / 16, DB = HD / 16, C4 = HD / 4;
  __shared__ __attribute__((aligned(16))) float Ks[TK * RS], Vs[TK * RS];
  const int sh = (int)blockIdx.x, s = sh / H, h = sh % H, kvh = h / (H / KVH);
  const int nrb = (L + TR - 1) / TR;
  const int r0 = (nrb - 1 - (int)blockIdx.y) * TR, t = (int)threadIdx.x;
  const int wave = t / kWave, lane = t % kWave, g = lane / 16, j = lane % 16;
  const int base = causal ? (pos0 ? pos0[s] : 0) + pos_off : 0;
  const int rlast = min(r0 + TR, L) - 1;
  const int kend = causal ? base + rlast + 1 : L;  // keys [0, kend)
  const float* kb = kc + ((size_t)s * KVH + kvh) * cap * HD;
  const float* vb = vc + ((size_t)s * KVH + kvh) * cap * HD;
  const int row = r0 + wave * 16 + j;  // this lane's query row (B column)
  const bool rin = row < L;
  const int qpos = base + row;
  f4 qf[NC];
  {
    const float* qr = q + qs.at(s, min(row, L - 1), h) + 4 * g;  // past L: a valid row, not stored
#pragma unroll
    for (int c = 0; c < NC; ++c) qf[c] = *reinterpret_cast<const f4*>(qr + 16 * c);
  }
  bf16x4_t qb[NC];  // LP: the query fragments as bf16, formed once
  if constexpr (LP) {
#pragma unroll
    for (int c = 0; c < NC; ++c) qb[c] = to_bf16x4(qf[c]);
  }
  float m = -INFINITY, l = 0.f;
  f4 o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d) o[d] = f4{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < kend; k0 += TK) {
    __syncthreads();  // the previous tile's readers are done
    for (int e = t; e < TK * C4; e += 256) {
      const int i = e / C4, c = e % C4;
      f4 x = f4{0.f, 0.f, 0.f, 0.f}, y = x;
      if (k0 + i < kend) {
        x = *reinterpret_cast<const f4*>(kb + (size_t)(k0 + i) * HD + 4 * c);
        y = *reinterpret_cast<const f4*>(vb + (size_t)(k0 + i) * HD + 4 * c);
      }
      *reinterpret_cast<f4*>(Ks + i * RS + 4 * c) = x;
      *reinterpret_cast<f4*>(Vs + i * RS + 4 * c) = y;
    }
    __syncthreads();
    f4 st[2];  // [16-key block]: keys 16 b + 4 g + r of row j
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      st[b] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const f4 kv = *reinterpret_cast<const f4*>(Ks + (b * 16 + j) * RS + 16 * c + 4 * g);
        if constexpr (LP) {
          st[b] = mfma_bf16_16x16x16(to_bf16x4(kv), qb[c], st[b]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            st[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[e], qf[c][e], st[b], 0, 0, 0);
        }
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + b * 16 + 4 * g + r;
        const bool ok = rin && key < kend && (!causal || key <= qpos);
        st[b][r] = ok ? st[b][r] * scale : -INFINITY;
        mx = fmaxf(mx, st[b][r]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float mnew = fmaxf(m, mx);
    const float alpha = (m == -INFINITY) ? (mnew == -INFINITY ? 1.f : 0.f) : expf(m - mnew);
    float sum = 0.f;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = st[b][r] == -INFINITY ? 0.f : expf(st[b][r] - mnew);
        st[b][r] = p;
        sum += p;
      }
    sum += __shfl_xor(sum, 16, kWave);
    sum += __shfl_xor(sum, 32, kWave);
    l = l * alpha + sum;
    m = mnew;
    if constexpr (LP) {
      const bf16x4_t pb[2] = {to_bf16x4(st[0]), to_bf16x4(st[1])};
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        o[d] *= alpha;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const float* vp = Vs + (b * 16 + 4 * g) * RS + d * 16 + j;
          const f4 va = f4{vp[0], vp[RS], vp[2 * RS], vp[3 * RS]};
          o[d] = mfma_bf16_16x16x16(to_bf16x4(va), pb[b], o[d]);
        }
      }
    } else {
#pragma unroll
      for (int d = 0; d < DB; ++d) {
        o[d] *= alpha;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                Vs[(b * 16 + 4 * g + r) * RS + d * 16 + j], st[b][r], o[d], 0, 0, 0);
      }
    }
  }
  if (!rin) return;
  // lane (g, j): dims 16 d + 4 g + r of row j
  float* op = out + os.at(s, row, h) + 4 * g;
#pragma unroll
  for (int d = 0; d < DB; ++d) {
    f4 y;
#pragma unroll
    for (int r = 0; r < 4; ++r) y[r] = o[d][r] / l;
    *reinterpret_cast<f4*>(op + 16 * d) = y;
  }
  if (lse && g == 0) lse[((size_t)s * H + h) * L + row] = m + logf(l);
}

// bf16_ops: the matrix-core path (L >= 32, hd 64 or 128) with bf16 operands;
// shorter rows keep the f32 VALU kernel.
int attn_valu_f32(const float* q, const float* kc, const float* vc, const int32_t* pos0,
                  int pos_off, float* out, float* lse, int S, int L, int H, int KVH, int cap,
                  int hd, hipStream_t st, const AttnStrides* qs_in = nullptr,
                  const AttnStrides* os_in = nullptr, bool causal = true, bool bf16_ops = false) {
  const int64_t n = (int64_t)S * L * H;  // queries, one wave each
  if (n == 0) return SM_OK;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kc) |
       reinterpret_cast<uintptr_t>(vc) | reinterpret_cast<uintptr_t>(out)) % 16 != 0) {
    set_error("f32 attention: q, the caches and out must be 16-byte aligned");
    return SM_ERR_INVALID;
  }
  const unsigned blocks = (unsigned)ceil_div(n, 4);
  const float scale = 1.0f / sqrtf((float)hd);
  const AttnStrides rows = AttnStrides::rows(L, H, hd);
  const AttnStrides qs = qs_in ? *qs_in : rows, os = os_in ? *os_in : rows;
  const int cz = causal ? 1 : 0;
  if (L >= 32 && ceil_div(L, 64) <= 65535 && (hd == 64 || hd == 128)) {  // many queries
    const dim3 grid((unsigned)((int64_t)S * H), (unsigned)ceil_div(L, 64));
#define SM_AF(HD, LP)                                                                       \
  attn_f32_mfma_kernel<HD, LP><<<grid, 256, 0, st>>>(q, kc, vc, pos0, pos_off, out, lse, S, L, \
                                                     H, KVH, cap, scale, qs, os, cz)
    if (hd == 64) {
      if (bf16_ops) SM_AF(64, true);
      else SM_AF(64, false);
    } else {
      if (bf16_ops) SM_AF(128, true);
      else SM_AF(128, false);
    }
#undef SM_AF
    SM_LAUNCH_CHECK();
    return SM_OK;
  }
  if (hd == 64)
    attn_valu_f32_kernel<64><<<blocks, 256, 0, st>>>(q, kc, vc, pos0, pos_off, out, lse, S, L, H,
                                                     KVH, cap, scale, qs, os, cz);
  else if (hd == 128)
    attn_valu_f32_kernel<128><<<blocks, 256, 0, st>>>(q, kc, vc, pos0, pos_off, out, lse, S, L, H,
                                                      KVH, cap, scale, qs, os, cz);
  else {
    set_error("f32 attention: head_dim must be 64 or 128 (got %d)", hd);
    return SM_ERR_UNSUPPORTED;
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace

int attn_prefill_16(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                    const int32_t* pos0, void* out, float* lse, bool kf16, int om, int S, int L,
                    int H, int KVH, int cap, int hd, hipStream_t st,
                    const AttnStrides* qs = nullptr, const AttnStrides* os = nullptr,
                    bool causal = true);

inline int out_mode(int out_dtype) {
  return out_dtype == SM_BF16 ? 0 : out_dtype == SM_F16 ? 1 : out_dtype == SM_F16X2 ? 2 : -1;
}

}  // namespace sm

extern "C" int sm_attn_decode(const void* q, const void* kcache, const void* vcache,
                              const int32_t* lens, void* out, int dtype, int out_dtype, int64_t S,
                              int64_t H, int64_t KVH, int64_t cap, int64_t head_dim,
                              void* stream) {
  using namespace sm;
  SM_REQUIRE(q && kcache && vcache && lens && out, "sm_attn_decode: null buffer");
  SM_REQUIRE(S >= 0 && S <= 65535 && H > 0 && KVH > 0 && H % KVH == 0,
             "sm_attn_decode: need 0 <= S <= 65535 and H a multiple of KVH");
  SM_REQUIRE(cap > 0 && cap <= (1 << 24), "sm_attn_decode: bad cache capacity");
  SM_REQUIRE(head_dim == 64 || head_dim == 128, "sm_attn_decode: head_dim must be 64 or 128");
  if (S == 0) return SM_OK;
  const float scale = 1.0f / sqrtf((float)head_dim);
  hipStream_t st = as_stream(stream);
  if (dtype == SM_F32) {
    SM_REQUIRE(out_dtype == SM_F32, "sm_attn_decode: f32 attention writes f32");
    return attn_valu_f32((const float*)q, (const float*)kcache, (const float*)vcache, lens, -1,
                         (float*)out, nullptr, (int)S, 1, (int)H, (int)KVH, (int)cap, (int)head_dim, st);
  }
  SM_REQUIRE(dtype == SM_BF16 || dtype == SM_F16,
             "sm_attn_decode: dtype must be SM_BF16, SM_F16 or SM_F32");
  const int om = out_mode(out_dtype);
  SM_REQUIRE(om >= 0, "sm_attn_decode: 16-bit attention writes bf16, f16 or f16 pairs");
  const int qpk = (int)(H / KVH);
  SM_REQUIRE(qpk <= kMaxQpk, "sm_attn_decode: at most %d query heads per KV head", kMaxQpk);
  const dim3 grid((unsigned)KVH, (unsigned)S);
  const uint16_t *qq = (const uint16_t*)q, *kk = (const uint16_t*)kcache,
                 *vv = (const uint16_t*)vcache;
#define SM_DEC_K(HD, QM, KF, EX, DPL)                                                         \
  do {                                                                                         \
    if (om == 2)                                                                               \
      attn_decode_kernel<HD, QM, KF, 2, EX, DPL><<<grid, 256, 0, st>>>(                        \
          qq, kk, vv, lens, out, (int)H, (int)KVH, (int)cap, scale);                           \
    else if (om == 1)                                                                          \
      attn_decode_kernel<HD, QM, KF, 1, EX, DPL><<<grid, 256, 0, st>>>(                        \
          qq, kk, vv, lens, out, (int)H, (int)KVH, (int)cap, scale);                           \
    else                                                                                       \
      attn_decode_kernel<HD, QM, KF, 0, EX, DPL><<<grid, 256, 0, st>>>(                        \
          qq, kk, vv, lens, out, (int)H, (int)KVH, (int)cap, scale);                           \
  } while (0)
#define SM_DEC_X(HD, QM, EX)                                          \
  do {                                                                \
    if (dtype == SM_F16) SM_DEC_K(HD, QM, true, EX, (QM >= 4 ? 4 : 8)); \
    else SM_DEC_K(HD, QM, false, EX, (QM >= 4 ? 4 : 8));              \
  } while (0)
#define SM_DEC(HD, QM)                     \
  do {                                     \
    if (qpk == QM) SM_DEC_X(HD, QM, true); \
    else SM_DEC_X(HD, QM, false);          \
  } while (0)
  if (head_dim == 64) {
    if (qpk == 1) SM_DEC(64, 1); else if (qpk <= 4) SM_DEC(64, 4); else SM_DEC(64, 16);
  } else {
    if (qpk == 1) SM_DEC(128, 1); else if (qpk <= 4) SM_DEC(128, 4); else SM_DEC(128, 16);
  }
#undef SM_DEC
#undef SM_DEC_X
#undef SM_DEC_K
  SM_LAUNCH_CHECK();
  return SM_OK;
}

namespace sm {
namespace {

// Key splits of a shared prompt per (group, KV head): enough workgroups to
// cover the CUs (>= 256) while each split keeps >= 256 keys (two 32-key tiles
// per wave) and its partials stay small next to the keys it reads.
int prefix_splits(int64_t groups, int64_t KVH, int64_t P) {
  const int64_t pairs = groups * KVH;
  int64_t sp = std::max<int64_t>(1, std::min<int64_t>((256 + pairs - 1) / pairs, P / 256));
  sp = std::min<int64_t>(sp, kMaxPrefixSplits);
  const int64_t per = (P + sp - 1) / sp;
  const int64_t per32 = (per + 31) / 32 * 32;
  return (int)((P + per32 - 1) / per32);  // no empty split
}

}  // namespace
}  // namespace sm

extern "C" int64_t sm_attn_decode_prefix_workspace_bytes(int64_t S, int64_t G, int64_t P,
                                                         int64_t H, int64_t KVH,
                                                         int64_t head_dim) {
  if (S <= 0 || G <= 0 || S % G || P <= 0 || H <= 0 || KVH <= 0 || H % KVH || head_dim <= 0)
    return -1;
  const int64_t sp = sm::prefix_splits(S / G, KVH, P);
  return S * H * sp * (head_dim + 2) * 4;
}

extern "C" int sm_attn_decode_prefix(const void* q, const void* prefix_k, const void* prefix_v,
                                     const void* kcache, const void* vcache, const int32_t* lens,
                                     void* out, void* workspace, int64_t workspace_bytes,
                                     int dtype, int out_dtype, int64_t S, int64_t G, int64_t P,
                                     int64_t H, int64_t KVH, int64_t cap, int64_t head_dim,
                                     void* stream) {
  using namespace sm;
  SM_REQUIRE(q && prefix_k && prefix_v && kcache && vcache && lens && out && workspace,
             "sm_attn_decode_prefix: null buffer");
  SM_REQUIRE(S > 0 && S <= 65535 && G > 0 && S % G == 0,
             "sm_attn_decode_prefix: need 0 < S <= 65535 rollouts in whole groups of G");
  SM_REQUIRE(H > 0 && KVH > 0 && H % KVH == 0, "sm_attn_decode_prefix: H must be a multiple of KVH");
  const int64_t qpk = H / KVH;
  SM_REQUIRE(qpk <= kMaxQpk && G * qpk <= 32,
             "sm_attn_decode_prefix: at most %d query heads per KV head and 32 per group",
             kMaxQpk);
  SM_REQUIRE(P > 0 && P <= cap && cap <= (1 << 24), "sm_attn_decode_prefix: need 0 < P <= cap");
  SM_REQUIRE(head_dim == 64 || head_dim == 128,
             "sm_attn_decode_prefix: head_dim must be 64 or 128");
  SM_REQUIRE(dtype == SM_F16 || dtype == SM_BF16,
             "sm_attn_decode_prefix: dtype must be SM_F16 or SM_BF16");
  SM_REQUIRE(out_dtype == SM_F16X2, "sm_attn_decode_prefix: writes f16 pairs (SM_F16X2)");
  const int64_t need = sm_attn_decode_prefix_workspace_bytes(S, G, P, H, KVH, head_dim);
  SM_REQUIRE(workspace_bytes >= need, "sm_attn_decode_prefix: workspace of %lld bytes, %lld needed",
             (long long)workspace_bytes, (long long)need);
  SM_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
             "sm_attn_decode_prefix: workspace must be 16-byte aligned");
  const int splits = prefix_splits(S / G, KVH, P);
  const int per = (int)(((P + splits - 1) / splits + 31) / 32 * 32);
  const float scale = 1.0f / sqrtf((float)head_dim);
  hipStream_t st = as_stream(stream);
  float* part_o = (float*)workspace;
  float* part_ml = part_o + (size_t)S * H * splits * head_dim;
  const uint16_t *qq = (const uint16_t*)q, *pk = (const uint16_t*)prefix_k,
                 *pv = (const uint16_t*)prefix_v, *kk = (const uint16_t*)kcache,
                 *vv = (const uint16_t*)vcache;
  const dim3 ga((unsigned)KVH, (unsigned)(S / G), (unsigned)splits);
  const bool f16 = dtype == SM_F16;
  const bool two = G * qpk > 16;
#define SM_PRE_A(HD, KF, QB)                                                              \
  attn_prefix_kernel<HD, KF, QB><<<ga, 256, 0, st>>>(qq, pk, pv, part_o, part_ml, (int)H, \
                                                      (int)KVH, (int)G, (int)P, per, scale)
#define SM_PRE_AK(HD, KF) \
  do { if (two) SM_PRE_A(HD, KF, 2); else SM_PRE_A(HD, KF, 1); } while (0)
  const dim3 ga16((unsigned)KVH, (unsigned)(S / G), (unsigned)(splits * (two ? 2 : 1)));
#define SM_PRE_A16(HD)                                                                   \
  attn_prefix_f16_kernel<HD, 1><<<ga16, 256, 0, st>>>(qq, pk, pv, part_o, part_ml, (int)H, \
                                                       (int)KVH, (int)G, (int)P, per, scale)
  if (f16) {  // P.V on the f16 matrix cores, one 16-query block per workgroup
    if (head_dim == 64) SM_PRE_A16(64);
    else SM_PRE_A16(128);
  } else if (head_dim == 64) {
    SM_PRE_AK(64, false);
  } else {
    SM_PRE_AK(128, false);
  }
#undef SM_PRE_A16
#undef SM_PRE_AK
#undef SM_PRE_A
  const dim3 gb((unsigned)KVH, (unsigned)S);
#define SM_PRE_B(HD, QM, KF, EX)                                                              \
  attn_decode_kernel<HD, QM, KF, 2, EX, (QM >= 4 ? 4 : 8), true><<<gb, 256, 0, st>>>(        \
      qq, kk, vv, lens, out, (int)H, (int)KVH, (int)cap, scale, (int)P, part_o, part_ml, splits)
#define SM_PRE_BX(HD, QM, EX) \
  do { if (f16) SM_PRE_B(HD, QM, true, EX); else SM_PRE_B(HD, QM, false, EX); } while (0)
#define SM_PRE_BQ(HD, QM) \
  do { if (qpk == QM) SM_PRE_BX(HD, QM, true); else SM_PRE_BX(HD, QM, false); } while (0)
  if (head_dim == 64) {
    if (qpk == 1) SM_PRE_BQ(64, 1); else if (qpk <= 4) SM_PRE_BQ(64, 4); else SM_PRE_BQ(64, 16);
  } else {
    if (qpk == 1) SM_PRE_BQ(128, 1); else if (qpk <= 4) SM_PRE_BQ(128, 4); else SM_PRE_BQ(128, 16);
  }
#undef SM_PRE_BQ
#undef SM_PRE_BX
#undef SM_PRE_B
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_attn_prefill_lse(const void* q, const void* kcache, const void* vcache,
                                   const int32_t* pos0, void* out, float* lse, int dtype,
                                   int out_dtype, int64_t S, int64_t L, int64_t H, int64_t KVH,
                                   int64_t cap, int64_t head_dim, void* stream);

extern "C" int sm_attn_prefill(const void* q, const void* kcache, const void* vcache,
                               const int32_t* pos0, void* out, int dtype, int out_dtype,
                               int64_t S, int64_t L, int64_t H, int64_t KVH, int64_t cap,
                               int64_t head_dim, void* stream) {
  return sm_attn_prefill_lse(q, kcache, vcache, pos0, out, nullptr, dtype, out_dtype, S, L, H, KVH,
                             cap, head_dim, stream);
}

extern "C" int sm_attn_prefill_lse(const void* q, const void* kcache, const void* vcache,
                                   const int32_t* pos0, void* out, float* lse, int dtype,
                                   int out_dtype, int64_t S, int64_t L, int64_t H, int64_t KVH,
                                   int64_t cap, int64_t head_dim, void* stream) {
  using namespace sm;
  SM_REQUIRE(q && kcache && vcache && pos0 && out, "sm_attn_prefill: null buffer");
  SM_REQUIRE(S >= 0 && L >= 0 && H > 0 && KVH > 0 && H % KVH == 0,
             "sm_attn_prefill: bad shape");
  SM_REQUIRE(head_dim == 64 || head_dim == 128, "sm_attn_prefill: head_dim must be 64 or 128");
  SM_REQUIRE(cap > 0 && cap <= (1 << 24), "sm_attn_prefill: bad cache capacity");
  if (S == 0 || L == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  if (dtype == SM_F32) {
    SM_REQUIRE(out_dtype == SM_F32, "sm_attn_prefill: f32 attention writes f32");
    return attn_valu_f32((const float*)q, (const float*)kcache, (const float*)vcache, pos0, 0,
                         (float*)out, lse, (int)S, (int)L, (int)H, (int)KVH, (int)cap, (int)head_dim,
                         st);
  }
  SM_REQUIRE(dtype == SM_BF16 || dtype == SM_F16,
             "sm_attn_prefill: dtype must be SM_BF16, SM_F16 or SM_F32");
  const int om = out_mode(out_dtype);
  SM_REQUIRE(om >= 0, "sm_attn_prefill: 16-bit attention writes bf16, f16 or f16 pairs");
  SM_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(kcache) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(vcache) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(out) % 8 == 0,
             "sm_attn_prefill: q and the caches must be 16-byte aligned, out 8-byte aligned");
  return attn_prefill_16((const uint16_t*)q, (const uint16_t*)kcache, (const uint16_t*)vcache,
                         pos0, out, lse, dtype == SM_F16, om, (int)S, (int)L, (int)H, (int)KVH,
                         (int)cap, (int)head_dim, st);
}

extern "C" int sm_attn_prefill_lse_bf16ops(const float* q, const float* kcache,
                                           const float* vcache, const int32_t* pos0, float* out,
                                           float* lse, int64_t S, int64_t L, int64_t H,
                                           int64_t KVH, int64_t cap, int64_t head_dim,
                                           void* stream) {
  using namespace sm;
  SM_REQUIRE(q && kcache && vcache && pos0 && out, "sm_attn_prefill_lse_bf16ops: null buffer");
  SM_REQUIRE(S >= 0 && L >= 0 && H > 0 && KVH > 0 && H % KVH == 0,
             "sm_attn_prefill_lse_bf16ops: bad shape");
  SM_REQUIRE(head_dim == 64 || head_dim == 128,
             "sm_attn_prefill_lse_bf16ops: head_dim must be 64 or 128");
  SM_REQUIRE(cap > 0 && cap <= (1 << 24), "sm_attn_prefill_lse_bf16ops: bad cache capacity");
  if (S == 0 || L == 0) return SM_OK;
  return attn_valu_f32(q, kcache, vcache, pos0, 0, out, lse, (int)S, (int)L, (int)H, (int)KVH,
                       (int)cap, (int)head_dim, as_stream(stream), nullptr, nullptr, true, true);
}

extern "C" int sm_attention(const void* q, const void* k, const void* v, int dtype, int64_t B,
                            int64_t H, int64_t KVH, int64_t S, int64_t head_dim, int causal,
                            void* out, float* lse, void* stream) {
  using namespace sm;
  SM_REQUIRE(q && k && v && out, "sm_attention: null buffer");
  SM_REQUIRE(B >= 0 && B <= 65535 && S >= 0 && S <= (1 << 24) && H > 0 && H <= 65535 &&
                 KVH > 0 && H % KVH == 0,
             "sm_attention: bad shape (query heads must be a multiple of key/value heads)");
  SM_REQUIRE(head_dim == 64 || head_dim == 128, "sm_attention: head_dim must be 64 or 128");
  SM_REQUIRE(causal == 0 || causal == 1, "sm_attention: causal must be 0 or 1");
  if (B == 0 || S == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  const AttnStrides ts = AttnStrides::bhsd(S, H, head_dim);
  if (dtype == SM_F32)
    return attn_valu_f32((const float*)q, (const float*)k, (const float*)v, nullptr, 0,
                         (float*)out, lse, (int)B, (int)S, (int)H, (int)KVH, (int)S,
                         (int)head_dim, st, &ts, &ts, causal != 0);
  SM_REQUIRE(dtype == SM_BF16 || dtype == SM_F16,
             "sm_attention: dtype must be SM_F32, SM_BF16 or SM_F16");
  SM_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(out) % 8 == 0,
             "sm_attention: q, k and v must be 16-byte aligned, out 8-byte aligned");
  return attn_prefill_16((const uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v, nullptr, out,
                         lse, dtype == SM_F16, dtype == SM_F16 ? 1 : 0, (int)B, (int)S, (int)H,
                         (int)KVH, (int)S, (int)head_dim, st, &ts, &ts, causal != 0);
}
