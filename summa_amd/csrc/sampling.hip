// Next-token selection with the TextGenerator options (summa-llm/src/generate.rs:
// 127-250): sign-aware repetition penalty, exact top-k, EOS tracking, and an
// opt-in nucleus (top-p) filter, one logits row per workgroup, all on the device.
//
// Order of operations per row (select_next_token, generate.rs:127-153):
//   val[v] = penalised logit (apply_repetition_penalty, :155-182: a token seen
//            in the context is multiplied by p when negative, else divided by p,
//            once per distinct token — the caller's seen-bitmap is a set);
//   T <= 0 : argmax of val, lowest index on ties (:141-152);
//   T > 0  : candidates = the top_k largest val, ordered by value (IEEE total
//            order, f32::total_cmp) then index (select_nth_unstable_by, :218-225),
//            then optionally the smallest value-ordered prefix of them whose
//            softmax(val / T) mass reaches top_p; one Gumbel-max draw among the
//            candidates samples softmax(val / T) restricted to them — the
//            distribution of sample_from_values (:228-249).
// The selection thresholds come from a byte-wise radix select over the
// order-preserving key of val (four passes over the row, 256-bin LDS histogram
// scanned by one wave), counting elements for top-k and summing 2^-32 fixed-point
// probability masses for top-p, so the result does not depend on thread order.
// The Gumbel noise is the counter stream of sm_sample (seed, row, step * vocab + v),
// so with the options off the draw equals sm_sample's.
#include "common.hpp"
#include "sampling.hpp"

namespace sm {
namespace {

constexpr int kExThreads = 1024;
constexpr int kExWaves = kExThreads / kWave;

struct ExArgs {
  const float* logits;
  int64_t ld;
  int vocab;
  float inv_temp;  // 0: greedy
  float penalty;
  const uint32_t* seen_r;  // read side of the seen bitmap (null: no penalty)
  uint32_t* seen_w;        // chosen token recorded here (nullable)
  int64_t seen_ld;
  int top_k;    // 0: off
  float top_p;  // applied when < 1 and apply_top_p
  int apply_top_p;
  int eos;  // -1: none
  uint64_t seed;
  int64_t step;
  int32_t* done;
  int32_t* lengths;
  int32_t* ndone;
  int32_t* tok;
  int64_t tok_stride;
  float* lp;
  int64_t lp_stride;
  int32_t* next_ids;
};

// IEEE total order as an unsigned key (f32::total_cmp): -NaN < -inf < ... < -0 <
// +0 < ... < +inf < +NaN.
__device__ inline uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k ^ 0x80000000u) : ~k);
}

__device__ inline float penalised(const float* row, const uint32_t* seen, float pen, int v) {
  const float x = row[v];
  if (seen == nullptr || !((seen[v >> 5] >> (v & 31)) & 1u)) return x;
  return x < 0.f ? x * pen : __fdiv_rn(x, pen);
}

// softmax(val / T) mass relative to the row maximum, as 2^-32 fixed point.
__device__ inline unsigned long long mass_of(float val, float maxv, float inv_temp) {
  const float w = expf((val - maxv) * inv_temp);
  return w > 0.f ? (unsigned long long)(w * 4294967296.0f) : 0ull;  // NaN (inf - inf) -> 0
}

// Set kept by a radix-select cut: keys above T, and ties at T up to index `cut`.
struct Cut {
  uint32_t T = 0;
  int cut = 0;
  bool on = false;
};
__device__ inline bool kept(const Cut& c, uint32_t key, int v) {
  return !c.on || key > c.T || (key == c.T && v <= c.cut);
}

struct Smem {
  unsigned long long hist[256];
  int wtot[kExWaves];
  float bf[kExWaves];
  int bi[kExWaves];
  float bm[kExWaves], bs[kExWaves];
  int bin;
  unsigned long long above, binm, target;
  int cut;
  float maxv;
};

__device__ inline int block_excl_scan(int c, Smem& sh) {
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  int inc = c;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int t = __shfl_up(inc, o, kWave);
    if (lane >= o) inc += t;
  }
  if (lane == kWave - 1) sh.wtot[w] = inc;
  __syncthreads();
  int base = 0;
  for (int i = 0; i < w; ++i) base += sh.wtot[i];
  __syncthreads();
  return base + inc - c;
}

__device__ inline float block_max(float x, Smem& sh) {
  x = wave_max(x);
  if (threadIdx.x % kWave == 0) sh.bf[threadIdx.x / kWave] = x;
  __syncthreads();
  float m = sh.bf[0];
  for (int i = 1; i < kExWaves; ++i) m = fmaxf(m, sh.bf[i]);
  __syncthreads();
  return m;
}

// Threshold of the `target`-th unit of measure (counts, or masses for MASS)
// among the elements kept by `outer`, in descending (value, -index) order.
// For MASS the target is ceil(top_p * total mass), taken from the first pass.
template <bool MASS>
__device__ Cut radix_select(const ExArgs& a, const float* row, const Cut& outer,
                            unsigned long long target, float maxv, Smem& sh) {
  uint32_t prefix = 0, mask = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += kExThreads) sh.hist[i] = 0;
    __syncthreads();
    for (int v = threadIdx.x; v < a.vocab; v += kExThreads) {
      const float val = penalised(row, a.seen_r, a.penalty, v);
      const uint32_t key = order_key(val);
      if ((key & mask) != prefix || !kept(outer, key, v)) continue;
      const unsigned long long w = MASS ? mass_of(val, maxv, a.inv_temp) : 1ull;
      if (w) atomicAdd(&sh.hist[(key >> shift) & 255u], w);
    }
    if (threadIdx.x == 0) {  // degenerate rows (no finite mass) keep these
      sh.bin = 0;
      sh.above = sh.binm = sh.target = 0;
    }
    __syncthreads();
    if (threadIdx.x < kWave) {
      const int lane = threadIdx.x;
      unsigned long long h[4], s = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        h[i] = sh.hist[255 - 4 * lane - i];  // lane 0 holds the top bins
        s += h[i];
      }
      unsigned long long inc = s;
#pragma unroll
      for (int o = 1; o < kWave; o <<= 1) {
        const unsigned long long t = __shfl_up(inc, o, kWave);
        if (lane >= o) inc += t;
      }
      unsigned long long tgt = target;
      if (MASS && shift == 24) {
        const unsigned long long total = __shfl(inc, kWave - 1, kWave);
        double x = ceil((double)a.top_p * (double)total);
        tgt = x < 1.0 ? 1ull : (unsigned long long)x;
        if (tgt > total) tgt = total;
      }
      unsigned long long acc = inc - s;
      if (acc < tgt && tgt <= inc) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (acc + h[i] >= tgt) {
            sh.bin = 255 - 4 * lane - i;
            sh.above = acc;
            sh.binm = h[i];
            sh.target = tgt - acc;
            break;
          }
          acc += h[i];
        }
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sh.bin << shift;
    mask |= 255u << shift;
    target = sh.target;
    __syncthreads();
  }
  // ties at the threshold key: how many the target still needs, lowest index first
  const unsigned long long eqm = sh.binm;
  unsigned long long need = target, eq = eqm;
  if (MASS) {
    const unsigned long long q = mass_of(key_value(prefix), maxv, a.inv_temp);
    need = q ? (target + q - 1) / q : 0;
    eq = q ? eqm / q : 0;
  }
  Cut c;
  c.T = prefix;
  c.on = true;
  c.cut = 0x7fffffff;
  if (need > 0 && need < eq) {
    if (threadIdx.x == 0) sh.cut = -1;  // set by the one thread that holds the need-th tie
    const int chunk = (a.vocab + kExThreads - 1) / kExThreads;
    const int b0 = min(a.vocab, (int)threadIdx.x * chunk), b1 = min(a.vocab, b0 + chunk);
    int cnt = 0;
    for (int v = b0; v < b1; ++v) {
      const uint32_t key = order_key(penalised(row, a.seen_r, a.penalty, v));
      cnt += (key == prefix && kept(outer, key, v)) ? 1 : 0;
    }
    const int e = block_excl_scan(cnt, sh);
    if ((unsigned long long)e < need && need <= (unsigned long long)(e + cnt)) {
      int left = (int)(need - (unsigned long long)e);
      for (int v = b0; v < b1; ++v) {
        const uint32_t key = order_key(penalised(row, a.seen_r, a.penalty, v));
        if (key == prefix && kept(outer, key, v) && --left == 0) {
          sh.cut = v;
          break;
        }
      }
    }
    __syncthreads();
    c.cut = sh.cut;
    __syncthreads();
  }
  return c;
}

__global__ __launch_bounds__(kExThreads) void sample_ex_kernel(ExArgs a) {
  __shared__ Smem sh;
  const int64_t r = blockIdx.x;
  if (a.done && a.done[r]) {  // finished rollout: EOS padding, zero log-prob
    if (threadIdx.x == 0) {
      a.tok[r * a.tok_stride] = a.eos;
      if (a.lp) a.lp[r * a.lp_stride] = 0.f;
      if (a.next_ids) a.next_ids[r] = a.eos;
    }
    return;
  }
  const float* row = a.logits + r * a.ld;
  const uint32_t* seen = a.seen_r ? a.seen_r + r * a.seen_ld : nullptr;
  ExArgs ar = a;
  ar.seen_r = seen;
  Cut ck, cp;
  if (a.inv_temp > 0.f && a.top_k > 0 && a.top_k < a.vocab)
    ck = radix_select<false>(ar, row, Cut{}, (unsigned long long)a.top_k, 0.f, sh);
  if (a.inv_temp > 0.f && a.apply_top_p && a.top_p < 1.f) {
    float mx = -INFINITY;
    for (int v = threadIdx.x; v < a.vocab; v += kExThreads)
      mx = fmaxf(mx, penalised(row, seen, a.penalty, v));
    mx = block_max(mx, sh);
    cp = radix_select<true>(ar, row, ck, 0ull, mx, sh);
  }
  // Gumbel-max (or argmax) over the candidates, and log_softmax of the raw row
  float m = -INFINITY, s = 0.f, best = -INFINITY;
  int bidx = 0x7fffffff;
  const uint64_t row_key = mix64(a.seed + 0x9e3779b97f4a7c15ull * ((uint64_t)r + 1));
  const uint64_t cbase = (uint64_t)a.step * (uint64_t)a.vocab;
  for (int v = threadIdx.x; v < a.vocab; v += kExThreads) {
    const float x = row[v];
    if (x > m) {
      s = s * __expf(m - x) + 1.f;
      m = x;
    } else if (x != -INFINITY) {
      s += __expf(x - m);
    }
    const float val = penalised(row, seen, a.penalty, v);
    const uint32_t key = order_key(val);
    if (!kept(ck, key, v) || !kept(cp, key, v)) continue;
    float g = val;
    if (a.inv_temp > 0.f) {
      const float u = u01(mix64(row_key ^ ((cbase + (uint64_t)v) * 0xd1b54a32d192ed03ull)));
      g = val * a.inv_temp - logf(-logf(u));
    }
    if (g > best) {  // v increases per thread: first max kept
      best = g;
      bidx = v;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ob = __shfl_xor(best, o, kWave);
    const int oi = __shfl_xor(bidx, o, kWave);
    if (ob > best || (ob == best && oi < bidx)) {
      best = ob;
      bidx = oi;
    }
    const float om = __shfl_xor(m, o, kWave), os = __shfl_xor(s, o, kWave);
    lse_merge(m, s, om, os);
  }
  const int w = threadIdx.x / kWave;
  if (threadIdx.x % kWave == 0) {
    sh.bf[w] = best;
    sh.bi[w] = bidx;
    sh.bm[w] = m;
    sh.bs[w] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kExWaves; ++k) {
      if (sh.bf[k] > best || (sh.bf[k] == best && sh.bi[k] < bidx)) {
        best = sh.bf[k];
        bidx = sh.bi[k];
      }
      lse_merge(m, s, sh.bm[k], sh.bs[k]);
    }
    if (bidx >= a.vocab) bidx = 0;  // no finite candidate: deterministic fallback
    a.tok[r * a.tok_stride] = bidx;
    if (a.next_ids) a.next_ids[r] = bidx;
    if (a.lp) a.lp[r * a.lp_stride] = row[bidx] - (m + __logf(s));
    if (a.seen_w) a.seen_w[r * a.seen_ld + (bidx >> 5)] |= 1u << (bidx & 31);
    if (a.eos >= 0 && bidx == a.eos) {
      if (a.done) a.done[r] = 1;
      if (a.lengths) a.lengths[r] = (int32_t)(a.step + 1);
      if (a.ndone) atomicAdd(a.ndone, 1);
    }
  }
}

__global__ void seen_clear_kernel(uint32_t* seen, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) seen[i] = 0u;
}

__global__ void seen_mark_kernel(const int32_t* ids, int64_t rows, int64_t n, int64_t ids_ld,
                                 int vocab, uint32_t* seen, int64_t seen_ld) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * n) return;
  const int64_t r = i / n;
  const int t = ids[r * ids_ld + i % n];
  if (t < 0 || t >= vocab) return;  // ids outside the vocabulary mark nothing
  atomicOr(&seen[r * seen_ld + (t >> 5)], 1u << (t & 31));
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

int validate_sampling(const sm_sampling* c, int64_t vocab) {
  SM_REQUIRE(c != nullptr, "sampling options are null");
  SM_REQUIRE(!std::isnan(c->temperature), "temperature must not be NaN");
  SM_REQUIRE(c->top_k != 0, "top_k must be >= 1 (got 0)");
  SM_REQUIRE(std::isfinite(c->repetition_penalty) && c->repetition_penalty >= 1.f,
             "repetition_penalty must be finite and >= 1 (got %g)", (double)c->repetition_penalty);
  SM_REQUIRE(std::isfinite(c->top_p) && c->top_p > 0.f && c->top_p <= 1.f,
             "rollout top_p must be finite and in (0, 1]");
  SM_REQUIRE(c->apply_top_p == 0 || c->apply_top_p == 1, "apply_top_p must be 0 or 1");
  SM_REQUIRE(c->eos_token >= -1 && c->eos_token < vocab,
             "eos_token %d is outside the model vocabulary of %lld entries", c->eos_token,
             (long long)vocab);
  return SM_OK;
}

int sample_ex_launch(const float* logits, int64_t rows, int64_t ld, int64_t vocab,
                     const sm_sampling* c, uint64_t seed, int64_t step, uint32_t* seen,
                     int64_t seen_ld, int32_t* done, int32_t* lengths, int32_t* ndone,
                     int32_t* tokens, int64_t tok_stride, float* logprobs, int64_t lp_stride,
                     int32_t* next_ids, hipStream_t st) {
  ExArgs a{};
  a.logits = logits;
  a.ld = ld;
  a.vocab = (int)vocab;
  a.inv_temp = c->temperature > 0.f ? 1.f / c->temperature : 0.f;
  a.penalty = c->repetition_penalty;
  const bool pen = c->repetition_penalty != 1.f;
  a.seen_r = pen ? seen : nullptr;
  a.seen_w = seen;
  a.seen_ld = seen_ld;
  a.top_k = c->top_k > 0 ? c->top_k : 0;
  a.top_p = c->top_p;
  a.apply_top_p = c->apply_top_p;
  a.eos = c->eos_token;
  a.seed = seed;
  a.step = step;
  a.done = done;
  a.lengths = lengths;
  a.ndone = ndone;
  a.tok = tokens;
  a.tok_stride = tok_stride;
  a.lp = logprobs;
  a.lp_stride = lp_stride;
  a.next_ids = next_ids;
  sample_ex_kernel<<<(unsigned)rows, kExThreads, 0, st>>>(a);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

int seen_tokens(const int32_t* ids, int64_t rows, int64_t n, int64_t ids_ld, int64_t vocab,
                uint32_t* seen, int64_t seen_ld, bool clear, hipStream_t st) {
  if (clear && rows > 0)
    seen_clear_kernel<<<(unsigned)ceil_div(rows * seen_ld, 256), 256, 0, st>>>(seen,
                                                                                rows * seen_ld);
  if (rows > 0 && n > 0)
    seen_mark_kernel<<<(unsigned)ceil_div(rows * n, 256), 256, 0, st>>>(ids, rows, n, ids_ld,
                                                                       (int)vocab, seen, seen_ld);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

int fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t st) {
  if (n <= 0) return SM_OK;
  fill_i32_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, st>>>(p, n, v);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace sm

using namespace sm;

extern "C" int sm_sample_ex(const float* logits, int64_t rows, int64_t ld, int64_t vocab,
                            const sm_sampling* sampling, uint64_t seed, int64_t step,
                            uint32_t* seen, int64_t seen_ld, int32_t* done, int32_t* lengths,
                            int32_t* tokens, int64_t tok_stride, float* logprobs,
                            int64_t lp_stride, int32_t* next_ids, void* stream) {
  SM_REQUIRE(logits && tokens, "sm_sample_ex: null buffer");
  SM_REQUIRE(rows >= 0 && vocab > 0 && vocab <= ld && vocab < (1 << 30), "sm_sample_ex: bad shape");
  SM_TRY(validate_sampling(sampling, vocab));
  SM_REQUIRE(sampling->repetition_penalty == 1.f || seen != nullptr,
             "sm_sample_ex: repetition_penalty needs the seen-token bitmap");
  SM_REQUIRE(seen == nullptr || seen_ld >= ceil_div(vocab, 32),
             "sm_sample_ex: seen_ld must be >= ceil(vocab / 32)");
  SM_REQUIRE(done == nullptr || sampling->eos_token >= 0,
             "sm_sample_ex: done flags need an eos_token");
  if (rows == 0) return SM_OK;
  return sample_ex_launch(logits, rows, ld, vocab, sampling, seed, step, seen, seen_ld, done,
                          lengths, nullptr, tokens, tok_stride, logprobs, lp_stride, next_ids,
                          as_stream(stream));
}

extern "C" int sm_seen_tokens(const int32_t* ids, int64_t rows, int64_t n, int64_t ids_ld,
                              int64_t vocab, uint32_t* seen, int64_t seen_ld, int clear,
                              void* stream) {
  SM_REQUIRE(seen && (ids || n == 0), "sm_seen_tokens: null buffer");
  SM_REQUIRE(rows >= 0 && n >= 0 && ids_ld >= n && vocab > 0 && seen_ld >= ceil_div(vocab, 32),
             "sm_seen_tokens: bad shape");
  return seen_tokens(ids, rows, n, ids_ld, vocab, seen, seen_ld, clear != 0, as_stream(stream));
}
