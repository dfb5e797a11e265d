// Top-2 mixture-of-experts FFN on one GPU (config[4]).
//
// Semantics of SparseMoe::forward (summa-llm/src/model/ffn.rs:478-711):
//   router logits = fp32 x . W_r (:489-490)
//   top-2 indices, strict '>' scan so the first index wins ties
//     (top2_indices_kernel, moe_topk.rs:74-104)
//   route weights = softmax over the two selected logits (:514)
//   routes r = t*k + j sorted stably by expert, inverse permutation
//     (host_route_plan ffn.rs:888-929, stable_route_pack moe_route.rs:88-142)
//   per-expert SwiGLU MLP on each expert's contiguous rows (forward_grouped_swiglu)
//   out[t] = sum_j w[t,j] * routed[inverse[t*k+j]] (route_combine_forward,
//     moe_dispatch.rs:290-312), added to the residual stream.
//
// MI355X design: no host round trip anywhere. The route plan (one workgroup,
// deterministic stable counting sort) also emits two device tile lists
// (16-row and 128-row tiles per expert), which the grouped Q4 matmuls consume
// directly: the small-M kernel for decode (q4.hip) and the LDS kernel for
// prefill / recompute (q4_gemm_bl.hip). The token gather is folded into the
// first grouped matmul's A-operand addressing (row index = src_rows[p]), so
// routed inputs are never materialised.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "moe_plan.hpp"

namespace sm {

int64_t moe_max_tiles(int64_t routes, int64_t experts, int64_t rows) {
  return ceil_div(routes, rows) + experts;
}

PlanView plan_view(int32_t* plan, int64_t routes, int64_t experts) {
  PlanView v;
  int32_t* p = plan;
  v.counts = p; p += experts;
  v.offsets = p; p += experts + 1;
  v.order = p; p += routes;
  v.inverse = p; p += routes;
  v.src_rows = p; p += routes;
  v.ntiles16 = p; p += 1;
  v.tiles16 = p; p += 2 * moe_max_tiles(routes, experts, 16);
  v.ntiles128 = p; p += 1;
  v.tiles128 = p;
  return v;
}

namespace {

constexpr int kRouterThreads = 512;  // 8 waves: four experts each at E = 32
constexpr int kRouterLds = 64 * 1024;  // dynamic LDS budget (h rows + logits)

// One workgroup per TT tokens: their h rows go to LDS (f32), then each of the
// 8 waves takes experts e = wave, wave + 8, ...: its lanes stream W_r[e] once
// (coalesced, c = lane + 64 u; for d = 768 and 2048 all of the expert's loads
// in flight together, else eight) and accumulate the dot products of all TT
// tokens, reduced across the wave in a fixed order; the router weights are
// read once per TT tokens instead of once per token. (Four waves walking the
// experts with eight loads in flight waited one L2 round trip per 512 weights:
// 31 us per call at config[4].) One
// thread per token then does the strict top-2 scan and the softmax over the
// pair. Rows past the last token repeat the last token (their results are
// not stored), so the inner loops carry no per-token branches.
// TH: f32, f16, or f16 pair (PAIR: row t is hi[d] | lo[d]); VEC: d % 64 == 0.
// Top-2 of one token's E router logits, strict '>' so the first index wins
// ties (top2_indices_kernel, moe_topk.rs:74-104), and the softmax over the
// selected pair (ffn.rs:514).
__device__ inline void top2_of(const float* l, int E, int& i0, int& i1, float& w0, float& w1) {
  float v0 = -INFINITY, v1 = -INFINITY;
  i0 = 0;
  i1 = 0;
  for (int e = 0; e < E; ++e) {
    const float v = l[e];
    if (v > v0) { v1 = v0; i1 = i0; v0 = v; i0 = e; }
    else if (v > v1) { v1 = v; i1 = e; }
  }
  const float e1 = expf(v1 - v0);  // softmax over [v0, v1] (v0 >= v1)
  w0 = 1.f / (1.f + e1);
  w1 = e1 / (1.f + e1);
}

template <typename TH, bool PAIR, int TT, bool VEC, int CH = 0>
__global__ __launch_bounds__(kRouterThreads) void router_top2_kernel(
    const TH* __restrict__ h, const float* __restrict__ wr, int64_t tokens, int d, int E,
    float* __restrict__ logits_out, int32_t* __restrict__ top_idx, float* __restrict__ top_w) {
  extern __shared__ float smem[];
  float* hs = smem;            // [TT][d]
  float* lg = smem + TT * d;   // [TT][E]
  const int64_t t0 = (int64_t)blockIdx.x * TT;
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int64_t r = min<int64_t>(t0 + t, tokens - 1);
    const TH* row = h + r * (PAIR ? 2 * d : d);
    if constexpr (VEC && sizeof(TH) == 2) {
      for (int c8 = threadIdx.x; c8 < d / 8; c8 += kRouterThreads) {
        const h8 lo8 = *reinterpret_cast<const h8*>(row + 8 * c8);
        h8 hi8 = h8{0, 0, 0, 0, 0, 0, 0, 0};
        if constexpr (PAIR) hi8 = *reinterpret_cast<const h8*>(row + d + 8 * c8);
#pragma unroll
        for (int u = 0; u < 8; ++u) hs[t * d + 8 * c8 + u] = (float)lo8[u] + (float)hi8[u];
      }
    } else {
      for (int c = threadIdx.x; c < d; c += kRouterThreads) {
        float v = (float)row[c];
        if constexpr (PAIR) v += (float)row[d + c];
        hs[t * d + c] = v;
      }
    }
  }
  __syncthreads();
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  for (int e = wave; e < E; e += kRouterThreads / kWave) {
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = 0.f;
    const float* we = wr + (size_t)e * d;
    if constexpr (CH > 0) {
      // d = 64 * CH: every weight load of the expert in flight at once (one
      // L2 round trip per expert), then the same FMA order as below
      float w[CH];
#pragma unroll
      for (int ch = 0; ch < CH; ++ch) w[ch] = we[ch * kWave + lane];
#pragma unroll
      for (int ch = 0; ch < CH; ++ch)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[t] = fmaf(hs[t * d + ch * kWave + lane], w[ch], acc[t]);
    } else if constexpr (VEC) {
      const int chunks = d / kWave;
      int ch = 0;
      for (; ch + 8 <= chunks; ch += 8) {
        float w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = we[(ch + u) * kWave + lane];
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int t = 0; t < TT; ++t)
            acc[t] = fmaf(hs[t * d + (ch + u) * kWave + lane], w[u], acc[t]);
      }
      for (; ch < chunks; ++ch) {
        const float w = we[ch * kWave + lane];
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[t] = fmaf(hs[t * d + ch * kWave + lane], w, acc[t]);
      }
    } else {
      for (int c = lane; c < d; c += kWave) {
        const float w = we[c];
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[t] = fmaf(hs[t * d + c], w, acc[t]);
      }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      const float v = wave_sum(acc[t]);
      if (lane == 0) lg[t * E + e] = v;
    }
  }
  __syncthreads();
  if (threadIdx.x < TT && t0 + threadIdx.x < tokens) {
    const int t = threadIdx.x;
    const int64_t r = t0 + t;
    const float* l = lg + t * E;
    if (top_idx) {  // (logits only when top_idx is null)
      int i0, i1;
      float w0, w1;
      top2_of(l, E, i0, i1, w0, w1);
      top_idx[r * 2] = i0;
      top_idx[r * 2 + 1] = i1;
      top_w[r * 2] = w0;
      top_w[r * 2 + 1] = w1;
    }
    if (logits_out)
      for (int e = 0; e < E; ++e) logits_out[r * E + e] = l[e];
  }
}

template <typename TH, bool PAIR, int TT>
void launch_router(const void* h, const float* wr, int64_t tokens, int d, int E, float* lo,
                   int32_t* idx, float* w, hipStream_t st) {
  const size_t shmem = (size_t)TT * (d + E) * sizeof(float);
  const unsigned grid = (unsigned)ceil_div(tokens, TT);
  const bool vec = d % kWave == 0 && reinterpret_cast<uintptr_t>(h) % 16 == 0;
  // (d = 2048 rows hold at most four tokens in the LDS budget: TT <= 4 there)
  if (TT <= 4 && vec && d == 32 * kWave)
    router_top2_kernel<TH, PAIR, TT, true, (TT <= 4 ? 32 : 0)><<<grid, kRouterThreads, shmem, st>>>(
        static_cast<const TH*>(h), wr, tokens, d, E, lo, idx, w);
  else if (vec && d == 12 * kWave)
    router_top2_kernel<TH, PAIR, TT, true, 12><<<grid, kRouterThreads, shmem, st>>>(
        static_cast<const TH*>(h), wr, tokens, d, E, lo, idx, w);
  else if (vec)
    router_top2_kernel<TH, PAIR, TT, true><<<grid, kRouterThreads, shmem, st>>>(
        static_cast<const TH*>(h), wr, tokens, d, E, lo, idx, w);
  else
    router_top2_kernel<TH, PAIR, TT, false><<<grid, kRouterThreads, shmem, st>>>(
        static_cast<const TH*>(h), wr, tokens, d, E, lo, idx, w);
}

template <typename TH, bool PAIR>
void launch_router_tt(const void* h, const float* wr, int64_t tokens, int d, int E, float* lo,
                      int32_t* idx, float* w, hipStream_t st) {
  // tokens per workgroup: the largest of 8 / 4 / 2 / 1 whose rows fit the LDS budget
  const int64_t row = (int64_t)(d + E) * sizeof(float);
  if (8 * row <= kRouterLds) launch_router<TH, PAIR, 8>(h, wr, tokens, d, E, lo, idx, w, st);
  else if (4 * row <= kRouterLds) launch_router<TH, PAIR, 4>(h, wr, tokens, d, E, lo, idx, w, st);
  else if (2 * row <= kRouterLds) launch_router<TH, PAIR, 2>(h, wr, tokens, d, E, lo, idx, w, st);
  else launch_router<TH, PAIR, 1>(h, wr, tokens, d, E, lo, idx, w, st);
}

// Stable counting sort of the routes by expert in one workgroup. Thread i owns
// the contiguous route chunk [i*C, (i+1)*C); per-(thread, expert) counts live in
// LDS, an exclusive scan over threads per expert gives each thread's write
// base, and each thread then places its routes in order: the result equals the
// reference's host plan (experts ascending, route ids ascending within one).
constexpr int kPlanThreads = 128;
constexpr int kMaxExperts = 64;

__global__ __launch_bounds__(kPlanThreads) void route_plan_kernel(const int32_t* __restrict__ idx,
                                                                  int routes, int k, int E,
                                                                  PlanView pv, int max16,
                                                                  int max128,
                                                                  int32_t* __restrict__ error) {
  __shared__ int32_t cnt[kPlanThreads][kMaxExperts + 1];
  __shared__ int32_t offs[kMaxExperts + 1];
  const int t = threadIdx.x;
  const int C = (routes + kPlanThreads - 1) / kPlanThreads;
  const int r0 = min(t * C, routes), r1 = min(r0 + C, routes);
  for (int e = 0; e < E; ++e) cnt[t][e] = 0;
  int bad = 0;
  for (int r = r0; r < r1; ++r) {
    const int e = idx[r];
    if (e < 0 || e >= E) { bad = 1; continue; }
    cnt[t][e] += 1;
  }
  if (bad) atomicOr(error, 1);
  __syncthreads();
  // per expert: exclusive scan over threads (thread e does expert e)
  if (t < E) {
    int run = 0;
    for (int i = 0; i < kPlanThreads; ++i) {
      const int c = cnt[i][t];
      cnt[i][t] = run;
      run += c;
    }
    pv.counts[t] = run;
    offs[t] = run;  // total per expert, turned into offsets below
  }
  __syncthreads();
  if (t == 0) {
    int acc = 0;
    for (int e = 0; e < E; ++e) {
      const int c = offs[e];
      offs[e] = acc;
      pv.offsets[e] = acc;
      acc += c;
    }
    offs[E] = acc;
    pv.offsets[E] = acc;
    // tile lists: (expert, first row) for 16- and 128-row tiles
    int n16 = 0, n128 = 0;
    for (int e = 0; e < E; ++e) {
      const int c = offs[e + 1] - offs[e];
      for (int r = 0; r < c && n16 < max16; r += 16, ++n16) {
        pv.tiles16[2 * n16] = e;
        pv.tiles16[2 * n16 + 1] = r;
      }
      for (int r = 0; r < c && n128 < max128; r += 128, ++n128) {
        pv.tiles128[2 * n128] = e;
        pv.tiles128[2 * n128 + 1] = r;
      }
    }
    pv.ntiles16[0] = n16;
    pv.ntiles128[0] = n128;
  }
  __syncthreads();
  for (int r = r0; r < r1; ++r) {
    const int e = idx[r];
    if (e < 0 || e >= E) {
      pv.inverse[r] = -1;  // flagged route: combine skips it
      continue;
    }
    const int pos = offs[e] + cnt[t][e];
    cnt[t][e] += 1;
    pv.order[pos] = r;
    pv.inverse[r] = pos;
    pv.src_rows[pos] = r / k;
  }
}

// The same plan for at most kPlanSmall routes (decode batches): one thread per
// route and no serial scans. Per expert, a wave ballot gives the wave's count
// and each route's rank among the wave's routes of that expert (lanes, like
// waves, are in route order, so the sort stays stable); a 16-step pass per
// expert turns the wave counts into wave bases, and one wave scans the
// expert totals and tile counts with shuffles. Output identical to
// route_plan_kernel.
constexpr int kPlanSmall = 1024;
constexpr size_t kPlanLogitsLds = 64 * 1024;  // logits route_plan_small_kernel stages

// With logits (top-2 routing, k = 2): route r first takes the top-2 of its
// token's router logits [tokens, E] itself (top2_of, as router_top2_kernel),
// writing top_idx / top_w, so a decode step needs no router launch.
__global__ __launch_bounds__(kPlanSmall) void route_plan_small_kernel(
    const int32_t* __restrict__ idx, int routes, int k, int E, PlanView pv, int max16,
    int max128, int32_t* __restrict__ error, const float* __restrict__ logits = nullptr,
    int32_t* __restrict__ top_idx = nullptr, float* __restrict__ top_w = nullptr) {
  constexpr int NW = kPlanSmall / kWave;
  __shared__ int32_t wc[NW][kMaxExperts];  // wave counts, then wave bases
  __shared__ int32_t offs[kMaxExperts];
  const int r = threadIdx.x, wave = r / kWave, lane = r % kWave;
  int e = -1;
  if (logits) {  // the logits [routes / 2, E] staged in LDS (coalesced), then scanned there
    extern __shared__ float lgs[];
    for (int i = r; i < (routes / 2) * E; i += kPlanSmall) lgs[i] = logits[i];
    __syncthreads();
    if (r < routes) {
      int i0, i1;
      float w0, w1;
      top2_of(lgs + (r / 2) * E, E, i0, i1, w0, w1);
      e = (r & 1) ? i1 : i0;
      top_idx[r] = e;
      top_w[r] = (r & 1) ? w1 : w0;
    }
  } else if (r < routes) {
    e = idx[r];
    if (e < 0 || e >= E) {
      atomicOr(error, 1);
      pv.inverse[r] = -1;  // flagged route: combine skips it
      e = -1;
    }
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int rank = 0;
  for (int x = 0; x < E; ++x) {
    const uint64_t m = __ballot(e == x);
    if (e == x) rank = __popcll(m & below);
    if (lane == 0) wc[wave][x] = __popcll(m);
  }
  __syncthreads();
  if (wave == 0) {
    // lane x: expert x's wave bases and total; then the exclusive scans of
    // the totals and of the 16- / 128-row tile counts across the experts
    int tot = 0;
    if (lane < E) {
      for (int w = 0; w < NW; ++w) {
        const int c = wc[w][lane];
        wc[w][lane] = tot;
        tot += c;
      }
    }
    const int t16 = (tot + 15) / 16, t128 = (tot + 127) / 128;
    int s0 = tot, s16 = t16, s128 = t128;  // inclusive scans
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int a0 = __shfl_up(s0, o, kWave), a16 = __shfl_up(s16, o, kWave),
                a128 = __shfl_up(s128, o, kWave);
      if (lane >= o) { s0 += a0; s16 += a16; s128 += a128; }
    }
    if (lane < E) {
      const int off = s0 - tot;
      offs[lane] = off;
      pv.counts[lane] = tot;
      pv.offsets[lane] = off;
      if (lane == E - 1) pv.offsets[E] = s0;
      for (int i = 0, n = s16 - t16; i < t16; ++i, ++n)
        if (n < max16) { pv.tiles16[2 * n] = lane; pv.tiles16[2 * n + 1] = 16 * i; }
      for (int i = 0, n = s128 - t128; i < t128; ++i, ++n)
        if (n < max128) { pv.tiles128[2 * n] = lane; pv.tiles128[2 * n + 1] = 128 * i; }
      if (lane == E - 1) {
        pv.ntiles16[0] = min(s16, max16);
        pv.ntiles128[0] = min(s128, max128);
      }
    }
  }
  __syncthreads();
  if (e >= 0) {
    const int pos = offs[e] + wc[wave][e] + rank;
    pv.order[pos] = r;
    pv.inverse[r] = pos;
    pv.src_rows[pos] = r / k;
  }
}

// top_idx / top_w [tokens, 2] from router logits [tokens, E], one thread per
// token (the batches too large for route_plan_small_kernel's fused form).
__global__ void top2_from_logits_kernel(const float* __restrict__ logits, int64_t tokens, int E,
                                        int32_t* __restrict__ top_idx, float* __restrict__ top_w) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= tokens) return;
  int i0, i1;
  float w0, w1;
  top2_of(logits + t * E, E, i0, i1, w0, w1);
  top_idx[t * 2] = i0;
  top_idx[t * 2 + 1] = i1;
  top_w[t * 2] = w0;
  top_w[t * 2 + 1] = w1;
}

// x[t, c] += sum_j w[t, j] * routed[inverse[t*k + j], c]   (f32); routes the
// plan flagged (inverse < 0) contribute nothing
__global__ void combine_kernel(const float* __restrict__ routed, const float* __restrict__ w,
                               const int32_t* __restrict__ inverse, int64_t tokens, int k, int d,
                               float* __restrict__ x) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tokens * d) return;
  const int64_t t = i / d;
  const int c = i % d;
  const int64_t routes = tokens * k;
  float sum = 0.f;
  for (int j = 0; j < k; ++j) {
    const int64_t route = t * k + j;
    const int p = inverse[route];
    if (p >= 0 && p < routes) sum += routed[(int64_t)p * d + c] * w[route];
  }
  x[i] += sum;
}

// combine_kernel's sum for one token row (its routes in order, x += sum),
// then the next RMSNorm of the row as f16 pairs (row_rmsnorm_pair): one
// workgroup per token, wave i owning float4s i * 64 + lane of the row.
template <int V>
__global__ __launch_bounds__(64 * V) void combine_rmsnorm_kernel(
    const float* __restrict__ routed, const float* __restrict__ w,
    const int32_t* __restrict__ inverse, int64_t tokens, int k, float* __restrict__ x,
    const float* __restrict__ gamma, float eps, _Float16* __restrict__ h) {
  constexpr int D = 256 * V;
  __shared__ float4 sq[V][64];
  __shared__ float rms_s;
  const int64_t t = blockIdx.x;
  const int c4 = threadIdx.x;
  const int64_t routes = tokens * k;
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int j = 0; j < k; ++j) {
    const int64_t route = t * k + j;
    const int p = inverse[route];
    if (p >= 0 && p < routes) {
      const float4 r4 = reinterpret_cast<const float4*>(routed + (int64_t)p * D)[c4];
      const float wj = w[route];
      sum.x += r4.x * wj;
      sum.y += r4.y * wj;
      sum.z += r4.z * wj;
      sum.w += r4.w * wj;
    }
  }
  float4* xr = reinterpret_cast<float4*>(x + t * D) + c4;
  const float4 x4 = *xr;
  const float4 v = make_float4(x4.x + sum.x, x4.y + sum.y, x4.z + sum.z, x4.w + sum.w);
  *xr = v;
  row_rmsnorm_pair<V>(v, reinterpret_cast<const float4*>(gamma)[c4], eps, sq, rms_s,
                      h + t * 2 * D);
}

}  // namespace
}  // namespace sm

using namespace sm;

extern "C" int sm_rmsnorm(const float* x, const float* gamma, int64_t rows, int64_t d, float eps,
                          void* y, int out_dtype, void* stream);
extern "C" int sm_moe_combine(const float* routed, const float* top_w, const int32_t* plan,
                              int64_t tokens, int64_t top_k, int64_t experts, int64_t d, float* x,
                              void* stream);

extern "C" int sm_moe_combine_rmsnorm(const float* routed, const float* top_w,
                                      const int32_t* plan, int64_t tokens, int64_t top_k,
                                      int64_t experts, int64_t d, float* x, const float* gamma,
                                      float eps, void* h_out, void* stream) {
  SM_REQUIRE(routed && top_w && plan && x && gamma && h_out,
             "sm_moe_combine_rmsnorm: null buffer");
  SM_REQUIRE(tokens >= 0 && top_k >= 1 && d > 0, "sm_moe_combine_rmsnorm: bad shape");
  if (tokens == 0) return SM_OK;
  const int64_t v = d / 256;
  const bool fused = d % 256 == 0 && (v == 3 || v == 4 || v == 8 || v == 12 || v == 16) &&
                     tokens <= 0x7fffffff && reinterpret_cast<uintptr_t>(routed) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(gamma) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(h_out) % 8 == 0;
  if (!fused) {  // the two steps
    SM_TRY(sm_moe_combine(routed, top_w, plan, tokens, top_k, experts, d, x, stream));
    return sm_rmsnorm(x, gamma, tokens, d, eps, h_out, SM_F16X2, stream);
  }
  PlanView pv = plan_view(const_cast<int32_t*>(plan), tokens * top_k, experts);
  hipStream_t st = as_stream(stream);
  _Float16* h = static_cast<_Float16*>(h_out);
#define SM_CRN(V)                                                                        \
  case V:                                                                                \
    combine_rmsnorm_kernel<V><<<(unsigned)tokens, 64 * V, 0, st>>>(                      \
        routed, top_w, pv.inverse, tokens, (int)top_k, x, gamma, eps, h);                \
    break;
  switch (v) {
    SM_CRN(3)
    SM_CRN(4)
    SM_CRN(8)
    SM_CRN(12)
    SM_CRN(16)
    default: break;
  }
#undef SM_CRN
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int64_t sm_moe_plan_words(int64_t tokens, int64_t top_k, int64_t experts) {
  const int64_t routes = tokens * top_k;
  return experts + (experts + 1) + 3 * routes + 1 + 2 * moe_max_tiles(routes, experts, 16) + 1 +
         2 * moe_max_tiles(routes, experts, 128);
}

extern "C" int sm_moe_router_top2(const void* h, int h_dtype, const float* w_router,
                                  int64_t tokens, int64_t d, int64_t experts, float* logits_out,
                                  int32_t* top_idx, float* top_w, void* stream) {
  SM_REQUIRE(h && w_router && ((top_idx && top_w) || (logits_out && !top_idx && !top_w)),
             "sm_moe_router_top2: null buffer");
  SM_REQUIRE(experts >= 2, "top-2 routing needs at least two experts");
  SM_REQUIRE(tokens >= 0 && tokens <= 0x7fffffff && d > 0 && d <= 8192 && experts <= kMaxExperts,
             "sm_moe_router_top2: bad shape (d <= 8192, experts <= %d)", kMaxExperts);
  static_assert(kRouterLds >= (8192 + kMaxExperts) * 4, "one token must fit the router LDS");
  if (tokens == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  if (h_dtype == SM_F16X2)
    launch_router_tt<_Float16, true>(h, w_router, tokens, (int)d, (int)experts, logits_out,
                                     top_idx, top_w, st);
  else if (h_dtype == SM_F16)
    launch_router_tt<_Float16, false>(h, w_router, tokens, (int)d, (int)experts, logits_out,
                                      top_idx, top_w, st);
  else if (h_dtype == SM_F32)
    launch_router_tt<float, false>(h, w_router, tokens, (int)d, (int)experts, logits_out,
                                   top_idx, top_w, st);
  else SM_REQUIRE(false, "sm_moe_router_top2: h must be f32, f16 or f16 pairs");
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_moe_route_plan(const int32_t* top_idx, int64_t tokens, int64_t top_k,
                                 int64_t experts, int32_t* plan, int32_t* error, void* stream) {
  SM_REQUIRE((top_idx || tokens == 0) && plan && error, "sm_moe_route_plan: null buffer");
  SM_REQUIRE(experts >= 1 && experts <= kMaxExperts, "sm_moe_route_plan: experts must be <= %d",
             kMaxExperts);
  SM_REQUIRE(top_k >= 1 && tokens >= 0 && tokens * top_k <= 0x7fffffff,
             "sm_moe_route_plan: bad shape");
  const int64_t routes = tokens * top_k;
  PlanView pv = plan_view(plan, routes, experts);
  const int max16 = (int)moe_max_tiles(routes, experts, 16);
  const int max128 = (int)moe_max_tiles(routes, experts, 128);
  if (routes <= kPlanSmall)
    route_plan_small_kernel<<<1, kPlanSmall, 0, as_stream(stream)>>>(
        top_idx, (int)routes, (int)top_k, (int)experts, pv, max16, max128, error);
  else
    route_plan_kernel<<<1, kPlanThreads, 0, as_stream(stream)>>>(
        top_idx, (int)routes, (int)top_k, (int)experts, pv, max16, max128, error);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_moe_route_plan_logits(const float* logits, int64_t tokens, int64_t experts,
                                        int32_t* top_idx, float* top_w, int32_t* plan,
                                        int32_t* error, void* stream) {
  SM_REQUIRE((logits || tokens == 0) && top_idx && top_w && plan && error,
             "sm_moe_route_plan_logits: null buffer");
  SM_REQUIRE(experts >= 2 && experts <= kMaxExperts,
             "sm_moe_route_plan_logits: experts must be in 2..=%d", kMaxExperts);
  SM_REQUIRE(tokens >= 0 && tokens * 2 <= 0x7fffffff, "sm_moe_route_plan_logits: bad shape");
  const int64_t routes = tokens * 2;
  PlanView pv = plan_view(plan, routes, experts);
  const int max16 = (int)moe_max_tiles(routes, experts, 16);
  const int max128 = (int)moe_max_tiles(routes, experts, 128);
  hipStream_t st = as_stream(stream);
  const size_t lds = (size_t)tokens * experts * sizeof(float);  // the staged logits
  if (routes <= kPlanSmall && lds <= kPlanLogitsLds) {
    route_plan_small_kernel<<<1, kPlanSmall, lds, st>>>(nullptr, (int)routes, 2, (int)experts, pv,
                                                       max16, max128, error, logits, top_idx,
                                                       top_w);
  } else {
    top2_from_logits_kernel<<<(unsigned)ceil_div(tokens, 256), 256, 0, st>>>(
        logits, tokens, (int)experts, top_idx, top_w);
    route_plan_kernel<<<1, kPlanThreads, 0, st>>>(top_idx, (int)routes, 2, (int)experts, pv,
                                                  max16, max128, error);
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_moe_combine(const float* routed, const float* top_w, const int32_t* plan,
                              int64_t tokens, int64_t top_k, int64_t experts, int64_t d, float* x,
                              void* stream) {
  SM_REQUIRE(routed && top_w && plan && x, "sm_moe_combine: null buffer");
  SM_REQUIRE(tokens >= 0 && top_k >= 1 && d > 0, "sm_moe_combine: bad shape");
  if (tokens == 0) return SM_OK;
  PlanView pv = plan_view(const_cast<int32_t*>(plan), tokens * top_k, experts);
  combine_kernel<<<(unsigned)ceil_div(tokens * d, 256), 256, 0, as_stream(stream)>>>(
      routed, top_w, pv.inverse, tokens, (int)top_k, (int)d, x);
  SM_LAUNCH_CHECK();
  return SM_OK;
}
