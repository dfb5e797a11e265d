/*
 * CPU oracle, model level — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates the reference decoder forward, generation loop and GRPO log-prob
 * recompute for the configs' architecture:
 *   embed                 summa-llm/src/model/transformer.rs:511-518
 *   pre-norm block        summa-llm/src/model/block.rs:80-157
 *   RMSNorm (fp32 stats)  summa-llm/src/model/norm.rs:36-50
 *   qkv / RoPE / cache    summa-llm/src/model/attention.rs:92, 142-177, 318-371
 *   attention             attention.rs:216-265 (softmax(qK^T/sqrt(hd))V, GQA repeat_kv)
 *   SwiGLU FFN            summa-llm/src/model/ffn.rs:854-886
 *   final norm + head     transformer.rs:802-909
 *   generation            summa-llm/src/generate.rs:53-250
 *   log-prob recompute    summa-train/src/tensor_sleep.rs:2531-2689
 * in fp32, as the reference's CPU path computes, with one storage rounding
 * for quantized models: q, k and v are rounded to f16 (the device's 16-bit KV
 * cache and query; kv_f32 keeps them f32, the policy's training forward); the
 * embedding table is bf16 (rounded by the caller). The
 * device keeps matmul inputs at fp32-grade precision (f16 hi + lo pairs), so
 * no activation rounding is modelled here. Matmul dot products accumulate
 * sequentially in fp32 (the order PackedTensor::matrix_vector uses,
 * quantization.rs:642-651) or, with acc64, in f64, the exactly-accumulated
 * value the quantized parity checks compare against.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

typedef struct or_model {
  int32_t layers, d, H, KVH, hd, F, V, quantized;
  int32_t acc64; /* 1: accumulate matmul dot products in f64 (exact sum of the
                    same products); 0: sequential f32 as matrix_vector does */
  float eps, theta;
  const float* embed;      /* [V, d] */
  const float* attn_norm;  /* [layers, d] */
  const float* ffn_norm;   /* [layers, d] */
  const float* final_norm; /* [d] */
  const float *qkv, *o, *in, *down, *lm_head;           /* dense [N, K] per layer */
  const uint8_t *qkv_c, *o_c, *in_c, *down_c, *lm_c;    /* Q4 codes per layer */
  const uint16_t *qkv_s, *o_s, *in_s, *down_s, *lm_s;   /* Q4 scales per layer */
  /* top-2 MoE FFN (experts > 0): router [layers][E][d] f32, expert weights
   * [layers][E][2Fe, d] and [layers][E][d, Fe], dense or Q4 like the rest */
  int32_t experts, expert_ffn;
  const float* router;
  const float *exp_in, *exp_down;
  const uint8_t *exp_in_c, *exp_down_c;
  const uint16_t *exp_in_s, *exp_down_s;
  /* optional diagnostics: when set, moe_ffn stores for layer l and row t the
   * router margin (2nd-largest minus 3rd-largest logit) at [l * M + t] */
  float* router_gap;
  /* optional route hints [layers][M][2] (expert ids of another computation of
   * the same forward): a token whose margin is below hint_margin is an
   * ambiguous top-2 decision and takes the hinted pair; elsewhere a hinted
   * pair that differs from the oracle's own is counted in *hint_conflicts */
  const int32_t* route_hint;
  float hint_margin;
  int32_t* hint_conflicts;
  /* 1: keep q, k and v in f32 for a quantized model (the trainable policy's
   * forward, whose attention runs in f32 over f32 K / V); 0: round them to
   * f16 as the device's inference path stores them */
  int32_t kv_f32;
} or_model;

/* f16 rounding of q, k and v (the 16-bit KV cache) of quantized models. */
static float rkv(const or_model* m, float v) {
  return (m->quantized && !m->kv_f32) ? or_round_f16(v) : v;
}

static float q4_at(const uint8_t* codes, const uint16_t* scales, int64_t i) {
  const uint8_t byte = codes[i / 2];
  int q = (i & 1) ? (byte >> 4) : (byte & 0xf);
  if (q >= 8) q -= 16;
  return or_bf16_to_f32(scales[i / 128]) * (float)q;
}

/* Decode row n ([K] values) of a Q4 tensor whose rows start at n * K. */
static void q4_row(const uint8_t* c, const uint16_t* s, int64_t n, int64_t K, float* out) {
  for (int64_t k = 0; k < K; ++k) out[k] = q4_at(c, s, n * K + k);
}

/* f64 dot product of f32 vectors: the products are exact in f64, and eight
 * interleaved partial sums (k mod 8) are added at the end. The result differs
 * from a sequential f64 sum only far below f32 resolution; it stands for the
 * exactly accumulated value. */
static double dot64(const float* a, const float* b, int64_t K) {
  double p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t k = 0;
  for (; k + 8 <= K; k += 8)
    for (int j = 0; j < 8; ++j) p[j] += (double)a[k + j] * (double)b[k + j];
  for (; k < K; ++k) p[0] += (double)a[k] * (double)b[k];
  return ((p[0] + p[4]) + (p[1] + p[5])) + ((p[2] + p[6]) + (p[3] + p[7]));
}

/* dot64 of four rows w0..w3 (stride K) with one x, each computed exactly as
 * dot64 computes it; the four are interleaved only for instruction-level
 * parallelism. */
static void dot64x4(const float* w, const float* x, int64_t K, double* out) {
  double p[4][8] = {{0}};
  int64_t k = 0;
  for (; k + 8 <= K; k += 8)
    for (int r = 0; r < 4; ++r)
      for (int j = 0; j < 8; ++j) p[r][j] += (double)w[r * K + k + j] * (double)x[k + j];
  for (; k < K; ++k)
    for (int r = 0; r < 4; ++r) p[r][0] += (double)w[r * K + k] * (double)x[k];
  for (int r = 0; r < 4; ++r)
    out[r] = ((p[r][0] + p[r][4]) + (p[r][1] + p[r][5])) + ((p[r][2] + p[r][6]) + (p[r][3] + p[r][7]));
}

/* y[r, n] (+)= sum_k x[r, k] * W[n, k]; W dense f32 (w) or Q4 codes/scales
 * (c, s); sequential f32 accumulation, or f64 with acc64. Weight rows are
 * decoded once, in blocks of 16, and each input row is applied to a whole
 * block while it sits in cache; every output is still its own dot product. */
#define OR_NB 16
static void linear_w(const or_model* m, int64_t N, int64_t K, const float* w, const uint8_t* c,
                     const uint16_t* s, const float* x, int64_t M, float* y, int add) {
  const int64_t nblk = (N + OR_NB - 1) / OR_NB;
#pragma omp parallel
  {
    float* buf = w ? NULL : malloc(sizeof(float) * K * OR_NB);
#pragma omp for schedule(dynamic, 1)
    for (int64_t b = 0; b < nblk; ++b) {
      const int64_t n0 = b * OR_NB, nn = N - n0 < OR_NB ? N - n0 : OR_NB;
      const float* wb = w ? w + n0 * K : buf;
      if (!w)
        for (int64_t j = 0; j < nn; ++j) q4_row(c, s, n0 + j, K, buf + j * K);
      for (int64_t r = 0; r < M; ++r) {
        const float* xr = x + r * K;
        int64_t j = 0;
        if (m->acc64)
          for (; j + 4 <= nn; j += 4) {
            double o[4];
            dot64x4(wb + j * K, xr, K, o);
            for (int q = 0; q < 4; ++q) {
              if (add) y[r * N + n0 + j + q] += (float)o[q];
              else y[r * N + n0 + j + q] = (float)o[q];
            }
          }
        for (; j < nn; ++j) {
          const float* wr = wb + j * K;
          float acc = 0.f;
          if (m->acc64) acc = (float)dot64(wr, xr, K);
          else for (int64_t k = 0; k < K; ++k) acc += wr[k] * xr[k];
          if (add) y[r * N + n0 + j] += acc; else y[r * N + n0 + j] = acc;
        }
      }
    }
    free(buf);
  }
}

/* kind: 0 qkv, 1 o, 2 in, 3 down, 4 lm_head */
static void linear(const or_model* m, int kind, int layer, const float* x, int64_t M, float* y,
                   int add) {
  int64_t N, K;
  const int64_t qdim = (int64_t)m->H * m->hd, kvdim = (int64_t)m->KVH * m->hd;
  switch (kind) {
    case 0: N = qdim + 2 * kvdim; K = m->d; break;
    case 1: N = m->d; K = qdim; break;
    case 2: N = 2 * (int64_t)m->F; K = m->d; break;
    case 3: N = m->d; K = m->F; break;
    default: N = m->V; K = m->d; break;
  }
  const int64_t off = (kind == 4) ? 0 : (int64_t)layer * N * K;
  if (m->quantized) {
    const uint8_t* cs[] = {m->qkv_c, m->o_c, m->in_c, m->down_c, m->lm_c};
    const uint16_t* ss[] = {m->qkv_s, m->o_s, m->in_s, m->down_s, m->lm_s};
    linear_w(m, N, K, NULL, cs[kind] + off / 2, ss[kind] + off / 128, x, M, y, add);
  } else {
    const float* ws[] = {m->qkv, m->o, m->in, m->down, m->lm_head};
    linear_w(m, N, K, ws[kind] + off, NULL, NULL, x, M, y, add);
  }
}

/* x += SparseMoe(h) (ffn.rs:478-711) for M tokens: fp32 router, strict top-2,
 * softmax over the pair, per-route SwiGLU expert MLP, weighted sum. The routes
 * are grouped by expert so that each expert's weights are decoded once; every
 * route's values are computed exactly as for a token on its own. */
static void moe_ffn(const or_model* m, int layer, const float* h, int64_t M, float* x) {
  const int E = m->experts, Fe = m->expert_ffn, d = m->d;
  const float* wr = m->router + (size_t)layer * E * d;
  const int64_t nin = 2 * (int64_t)Fe * d, ndown = (int64_t)d * Fe;
  int32_t* sel = malloc(sizeof(int32_t) * M * 2);
  float* rw = malloc(sizeof(float) * M * 2);
#pragma omp parallel
  {
    float* lg = malloc(sizeof(float) * E);
#pragma omp for schedule(static)
    for (int64_t t = 0; t < M; ++t) {
      const float* ht = h + t * d;
      for (int e = 0; e < E; ++e) {
        float acc = 0.f;
        double acc64 = 0.0;
        if (m->acc64) { for (int c = 0; c < d; ++c) acc64 += (double)ht[c] * wr[(size_t)e * d + c]; acc = (float)acc64; }
        else for (int c = 0; c < d; ++c) acc += ht[c] * wr[(size_t)e * d + c];
        lg[e] = acc;
      }
      float v0 = -INFINITY, v1 = -INFINITY, v2 = -INFINITY;
      int i0 = 0, i1 = 0;
      for (int e = 0; e < E; ++e) {
        if (lg[e] > v0) { v2 = v1; v1 = v0; i1 = i0; v0 = lg[e]; i0 = e; }
        else if (lg[e] > v1) { v2 = v1; v1 = lg[e]; i1 = e; }
        else if (lg[e] > v2) v2 = lg[e];
      }
      if (m->router_gap) m->router_gap[(int64_t)layer * M + t] = v1 - v2;
      if (m->route_hint) {
        const int32_t* hp = m->route_hint + ((int64_t)layer * M + t) * 2;
        const int a = hp[0], b = hp[1];
        const int same = (a == i0 && b == i1) || (a == i1 && b == i0);
        if (!same && v1 - v2 < m->hint_margin && a >= 0 && a < E && b >= 0 && b < E && a != b) {
          /* the first of the pair by logit (equal logits: the lower index) */
          const int first = (lg[a] > lg[b] || (lg[a] == lg[b] && a < b)) ? a : b;
          i0 = first;
          i1 = first == a ? b : a;
          v0 = lg[i0];
          v1 = lg[i1];
        } else if (!same && m->hint_conflicts) {
#pragma omp atomic
          *m->hint_conflicts += 1;
        }
      }
      const float e1 = expf(v1 - v0);
      sel[2 * t] = i0;
      sel[2 * t + 1] = i1;
      rw[2 * t] = 1.f / (1.f + e1);
      rw[2 * t + 1] = e1 / (1.f + e1);
    }
    free(lg);
  }
  float* yr = malloc(sizeof(float) * M * 2 * d);   /* expert output per route t*2+j */
  int64_t* rt = malloc(sizeof(int64_t) * M * 2);   /* routes of one expert */
  float* hx = malloc(sizeof(float) * M * 2 * d);
  float* gv = malloc(sizeof(float) * M * 2 * 2 * Fe);
  float* u = malloc(sizeof(float) * M * 2 * Fe);
  float* yv = malloc(sizeof(float) * M * 2 * d);
  for (int e = 0; e < E; ++e) {
    int64_t cnt = 0;
    for (int64_t r = 0; r < 2 * M; ++r)
      if (sel[r] == e) rt[cnt++] = r;
    if (cnt == 0) continue;
    for (int64_t i = 0; i < cnt; ++i) memcpy(hx + i * d, h + (rt[i] / 2) * d, sizeof(float) * d);
    const int64_t base_in = ((int64_t)layer * E + e) * nin, base_down = ((int64_t)layer * E + e) * ndown;
    if (m->quantized)
      linear_w(m, 2 * Fe, d, NULL, m->exp_in_c + base_in / 2, m->exp_in_s + base_in / 128, hx, cnt, gv, 0);
    else
      linear_w(m, 2 * Fe, d, m->exp_in + base_in, NULL, NULL, hx, cnt, gv, 0);
    for (int64_t i = 0; i < cnt; ++i)
      for (int c = 0; c < Fe; ++c) {
        const float g = gv[i * 2 * Fe + c], v = gv[i * 2 * Fe + Fe + c];
        u[i * Fe + c] = g / (1.0f + expf(-g)) * v;
      }
    if (m->quantized)
      linear_w(m, d, Fe, NULL, m->exp_down_c + base_down / 2, m->exp_down_s + base_down / 128, u, cnt, yv, 0);
    else
      linear_w(m, d, Fe, m->exp_down + base_down, NULL, NULL, u, cnt, yv, 0);
    for (int64_t i = 0; i < cnt; ++i) memcpy(yr + rt[i] * d, yv + i * d, sizeof(float) * d);
  }
  for (int64_t t = 0; t < M; ++t)
    for (int c = 0; c < d; ++c) {
      float sum = 0.f;
      sum += yr[(2 * t) * d + c] * rw[2 * t];
      sum += yr[(2 * t + 1) * d + c] * rw[2 * t + 1];
      x[t * d + c] += sum;
    }
  free(sel); free(rw); free(yr); free(rt); free(hx); free(gv); free(u); free(yv);
}

static void rmsnorm(const or_model* m, const float* x, const float* g, int64_t M, float* y) {
  const int d = m->d;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < M; ++r) {
    float ss = 0.f;
    for (int c = 0; c < d; ++c) ss += x[r * d + c] * x[r * d + c];
    const float rms = sqrtf(ss / (float)d + m->eps);
    for (int c = 0; c < d; ++c) y[r * d + c] = x[r * d + c] / rms * g[c];
  }
}

/* RoPE cos/sin of (pos, pair): theta^(-2p/hd) and the angle in double, then f32. */
static void rope_cs(const or_model* m, int pos, int p, float* cs, float* sn) {
  const double freq = pow((double)m->theta, -2.0 * p / (double)m->hd);
  const double ang = (double)pos * freq;
  *cs = (float)cos(ang);
  *sn = (float)sin(ang);
}

/* Forward S sequences x L new tokens at positions pos0..pos0+L-1 through all
 * layers, appending K/V to caches [layers][S][KVH][cap][hd]; x [S*L, d] out. */
void or_model_forward(const or_model* m, const int32_t* ids, int S, int L, int pos0, float* kc,
                      float* vc, int cap, float* x) {
  const int d = m->d, H = m->H, KVH = m->KVH, hd = m->hd, F = m->F;
  const int64_t rows = (int64_t)S * L;
  const int64_t qdim = (int64_t)H * hd, kvdim = (int64_t)KVH * hd, qn = qdim + 2 * kvdim;
  float* h = malloc(sizeof(float) * rows * (d > qdim ? d : qdim));
  float* qkv = malloc(sizeof(float) * rows * qn);
  float* q = malloc(sizeof(float) * rows * qdim);
  float* att = malloc(sizeof(float) * rows * qdim);
  float* gv = malloc(sizeof(float) * rows * 2 * F);
  float* u = malloc(sizeof(float) * rows * F);
  const float scale = 1.0f / sqrtf((float)hd);
  /* cos / sin of (position pos0 + i, pair p), the same values rope_cs gives */
  float* rcos = malloc(sizeof(float) * (size_t)L * (hd / 2));
  float* rsin = malloc(sizeof(float) * (size_t)L * (hd / 2));
  for (int i = 0; i < L; ++i)
    for (int p = 0; p < hd / 2; ++p)
      rope_cs(m, pos0 + i, p, &rcos[(size_t)i * (hd / 2) + p], &rsin[(size_t)i * (hd / 2) + p]);
  for (int64_t r = 0; r < rows; ++r)
    for (int c = 0; c < d; ++c) x[r * d + c] = m->embed[(int64_t)ids[r] * d + c];
  for (int l = 0; l < m->layers; ++l) {
    float* kl = kc + (size_t)l * S * KVH * cap * hd;
    float* vl = vc + (size_t)l * S * KVH * cap * hd;
    rmsnorm(m, x, m->attn_norm + (size_t)l * d, rows, h);
    linear(m, 0, l, h, rows, qkv, 0);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
      const int s = (int)(r / L), pos = pos0 + (int)(r % L);
      const float* src = qkv + r * qn;
      for (int slot = 0; slot < H + 2 * KVH; ++slot)
        for (int p = 0; p < hd / 2; ++p) {
          const float a = src[slot * hd + 2 * p], b = src[slot * hd + 2 * p + 1];
          float ra = a, rbv = b;
          if (slot < H + KVH) {
            const float cs = rcos[(size_t)(pos - pos0) * (hd / 2) + p];
            const float sn = rsin[(size_t)(pos - pos0) * (hd / 2) + p];
            ra = a * cs - b * sn;
            rbv = b * cs + a * sn;
          }
          if (slot < H) {
            q[r * qdim + slot * hd + 2 * p] = rkv(m, ra);
            q[r * qdim + slot * hd + 2 * p + 1] = rkv(m, rbv);
          } else {
            const int kv = slot < H + KVH ? slot - H : slot - H - KVH;
            float* dst = (slot < H + KVH ? kl : vl) + (((size_t)s * KVH + kv) * cap + pos) * hd;
            dst[2 * p] = rkv(m, ra);
            dst[2 * p + 1] = rkv(m, rbv);
          }
        }
    }
    /* causal attention, each query over keys 0..pos (two-pass softmax in f32) */
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t r = 0; r < rows; ++r)
      for (int hh = 0; hh < H; ++hh) {
        const int s = (int)(r / L), pos = pos0 + (int)(r % L);
        const int kv = hh / (H / KVH);
        const float* qp = q + r * qdim + hh * hd;
        const float* kb = kl + ((size_t)s * KVH + kv) * cap * hd;
        const float* vb = vl + ((size_t)s * KVH + kv) * cap * hd;
        float* sc = malloc(sizeof(float) * (pos + 1));
        float mx = -INFINITY;
        for (int t = 0; t <= pos; ++t) {
          float acc = 0.f;
          for (int e = 0; e < hd; ++e) acc += qp[e] * kb[(size_t)t * hd + e];
          sc[t] = acc * scale;
          if (sc[t] > mx) mx = sc[t];
        }
        float sum = 0.f;
        for (int t = 0; t <= pos; ++t) {
          sc[t] = expf(sc[t] - mx);
          sum += sc[t];
        }
        for (int e = 0; e < hd; ++e) {
          float acc = 0.f;
          for (int t = 0; t <= pos; ++t) acc += sc[t] * vb[(size_t)t * hd + e];
          att[r * qdim + hh * hd + e] = acc / sum;
        }
        free(sc);
      }
    linear(m, 1, l, att, rows, x, 1);
    rmsnorm(m, x, m->ffn_norm + (size_t)l * d, rows, h);
    if (m->experts > 0) {
      moe_ffn(m, l, h, rows, x);
      continue;
    }
    linear(m, 2, l, h, rows, gv, 0);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
      for (int c = 0; c < F; ++c) {
        const float g = gv[r * 2 * F + c], v = gv[r * 2 * F + F + c];
        u[r * F + c] = g / (1.0f + expf(-g)) * v;
      }
    linear(m, 3, l, u, rows, x, 1);
  }
  free(h); free(qkv); free(q); free(att); free(gv); free(u); free(rcos); free(rsin);
}

void or_model_logits(const or_model* m, const float* x, int64_t M, float* logits) {
  float* h = malloc(sizeof(float) * M * m->d);
  rmsnorm(m, x, m->final_norm, M, h);
  linear(m, 4, 0, h, M, logits, 0);
  free(h);
}

/* Counter RNG identical to the device sampler's (SplitMix64 finaliser). */
static uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
static uint64_t rng_key(uint64_t seed, uint64_t stream, uint64_t counter) {
  return mix64(mix64(seed + 0x9e3779b97f4a7c15ull * (stream + 1)) ^ (counter * 0xd1b54a32d192ed03ull));
}
static float u01(uint64_t bits) { return ((float)(bits >> 40) + 0.5f) * (1.0f / 16777216.0f); }

/* select_next_token (generate.rs:127-202): greedy first-max argmax, or a
 * Gumbel-max draw from softmax(l/T); lp = log_softmax(l)[token] in f64. */
void or_sample(const float* logits, int64_t rows, int64_t V, float temperature, uint64_t seed,
               int64_t step, int32_t* tok, int64_t tok_stride, double* lp, int64_t lp_stride) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* l = logits + r * V;
    float best = -INFINITY;
    int bi = 0;
    double mx = -INFINITY;
    for (int64_t v = 0; v < V; ++v) {
      float key = l[v];
      if (temperature > 0.f) {
        const float u = u01(rng_key(seed, (uint64_t)r, (uint64_t)step * (uint64_t)V + (uint64_t)v));
        key = l[v] * (1.0f / temperature) - logf(-logf(u));
      }
      if (key > best) { best = key; bi = (int)v; }
      if (l[v] > mx) mx = l[v];
    }
    double s = 0.0;
    for (int64_t v = 0; v < V; ++v) s += exp((double)l[v] - mx);
    tok[r * tok_stride] = bi;
    if (lp) lp[r * lp_stride] = (double)l[bi] - (mx + log(s));
  }
}

/* generate (generate.rs:68-124, no EOS) for S rollouts at once. */
void or_generate(const or_model* m, const int32_t* prompts, int S, int P, int N, float temperature,
                 uint64_t seed, int32_t* tokens, double* lp) {
  const int cap = P + N - 1, d = m->d;
  const size_t cache = (size_t)m->layers * S * m->KVH * cap * m->hd;
  float* kc = calloc(cache, sizeof(float));
  float* vc = calloc(cache, sizeof(float));
  float* x = malloc(sizeof(float) * (size_t)S * P * d);
  float* last = malloc(sizeof(float) * (size_t)S * d);
  float* logits = malloc(sizeof(float) * (size_t)S * m->V);
  int32_t* ids = malloc(sizeof(int32_t) * S);
  or_model_forward(m, prompts, S, P, 0, kc, vc, cap, x);
  for (int s = 0; s < S; ++s) memcpy(last + (size_t)s * d, x + ((size_t)s * P + P - 1) * d, sizeof(float) * d);
  or_model_logits(m, last, S, logits);
  or_sample(logits, S, m->V, temperature, seed, 0, tokens, N, lp, N);
  for (int t = 1; t < N; ++t) {
    for (int s = 0; s < S; ++s) ids[s] = tokens[(size_t)s * N + t - 1];
    or_model_forward(m, ids, S, 1, P + t - 1, kc, vc, cap, last);
    or_model_logits(m, last, S, logits);
    or_sample(logits, S, m->V, temperature, seed, t, tokens + t, N, lp ? lp + t : NULL, N);
  }
  free(kc); free(vc); free(x); free(last); free(logits); free(ids);
}

/* apply_repetition_penalty (generate.rs:155-182): every distinct token of
 * prior[0..n) has its value divided by p (>= 0) or multiplied by p (< 0),
 * once. Returns -1 (and changes nothing further) for a token outside [0, V). */
int or_apply_penalty(float* values, int64_t V, const int32_t* prior, int64_t n, float penalty) {
  if (penalty == 1.0f) return 0;
  unsigned char* seen = calloc((size_t)V, 1);
  int rc = 0;
  for (int64_t i = 0; i < n; ++i) {
    const int32_t t = prior[i];
    if (t < 0 || t >= V) { rc = -1; break; }
    if (seen[t]) continue;
    seen[t] = 1;
    values[t] = values[t] < 0.0f ? values[t] * penalty : values[t] / penalty;
  }
  free(seen);
  return rc;
}

/* f32::total_cmp as an unsigned key. */
static uint32_t total_key(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

static const float* g_sort_vals;
/* value descending (total order), then index ascending (generate.rs:218-225) */
static int by_value_desc(const void* a, const void* b) {
  const int32_t i = *(const int32_t*)a, j = *(const int32_t*)b;
  const uint32_t ki = total_key(g_sort_vals[i]), kj = total_key(g_sort_vals[j]);
  if (ki != kj) return ki > kj ? -1 : 1;
  return i < j ? -1 : (i > j);
}

/* select_next_token with the full option set (generate.rs:127-250), one row:
 * penalty over prior[0..n), greedy max (lowest index on ties) or a Gumbel-max
 * draw (the device counter stream) among the top_k (top_k <= 0: all) largest,
 * optionally narrowed to the smallest value-ordered prefix whose 2^-32
 * fixed-point softmax(val / T) mass reaches ceil(top_p * total) (apply_top_p;
 * the reference validates top_p but has no nucleus sampler: parity unpinned,
 * checked against the definition in the tests). lp = log_softmax(raw)[token]. */
int or_sample_ex_row(const float* logits, int64_t V, float temperature, int top_k, float penalty,
                     float top_p, int apply_top_p, uint64_t seed, int64_t row, int64_t step,
                     const int32_t* prior, int64_t n, int32_t* tok, double* lp) {
  float* val = malloc(sizeof(float) * V);
  memcpy(val, logits, sizeof(float) * V);
  if (or_apply_penalty(val, V, prior, n, penalty) != 0) { free(val); return -1; }
  int best_i = 0;
  if (temperature <= 0.0f) {
    uint32_t bk = 0;
    int have = 0;
    for (int64_t v = 0; v < V; ++v) {
      const uint32_t k = total_key(val[v]);
      if (!have || k > bk) { bk = k; best_i = (int)v; have = 1; }
    }
  } else {
    int32_t* idx = malloc(sizeof(int32_t) * V);
    for (int64_t v = 0; v < V; ++v) idx[v] = (int32_t)v;
    g_sort_vals = val;
    qsort(idx, (size_t)V, sizeof(int32_t), by_value_desc);
    int64_t nc = (top_k > 0 && top_k < V) ? top_k : V;
    const float inv_t = 1.0f / temperature;
    if (apply_top_p && top_p < 1.0f) {
      const float mx = val[idx[0]];
      uint64_t* q = malloc(sizeof(uint64_t) * nc);
      uint64_t total = 0;
      for (int64_t i = 0; i < nc; ++i) {
        const float w = expf((val[idx[i]] - mx) * inv_t);
        q[i] = w > 0.0f ? (uint64_t)(w * 4294967296.0f) : 0;
        total += q[i];
      }
      double x = ceil((double)top_p * (double)total);
      uint64_t tgt = x < 1.0 ? 1 : (uint64_t)x;
      if (tgt > total) tgt = total;
      uint64_t cum = 0;
      int64_t keep = 0;
      while (keep < nc && cum < tgt) cum += q[keep++];
      if (keep == 0) keep = 1;
      nc = keep;
      free(q);
    }
    unsigned char* cand = calloc((size_t)V, 1);
    for (int64_t i = 0; i < nc; ++i) cand[idx[i]] = 1;
    float best = -INFINITY;
    best_i = -1;
    for (int64_t v = 0; v < V; ++v) {
      if (!cand[v]) continue;
      const float u = u01(rng_key(seed, (uint64_t)row, (uint64_t)step * (uint64_t)V + (uint64_t)v));
      const float key = val[v] * inv_t - logf(-logf(u));
      if (key > best) { best = key; best_i = (int)v; }
    }
    if (best_i < 0) best_i = 0;
    free(cand);
    free(idx);
  }
  double mx = -INFINITY, s = 0.0;
  for (int64_t v = 0; v < V; ++v) if (logits[v] > mx) mx = logits[v];
  for (int64_t v = 0; v < V; ++v) s += exp((double)logits[v] - mx);
  *tok = best_i;
  if (lp) *lp = (double)logits[best_i] - (mx + log(s));
  free(val);
  return 0;
}

/* TextGenerator::generate (generate.rs:68-124) for S rollouts with the full
 * options: the penalty sees prompt + generated tokens; a rollout stops at
 * eos (>= 0): its later tokens are eos with lp 0, lengths = tokens generated
 * including the EOS (N when none). */
void or_generate_ex(const or_model* m, const int32_t* prompts, int S, int P, int N,
                    float temperature, int top_k, float penalty, float top_p, int apply_top_p,
                    int eos, uint64_t seed, int32_t* tokens, double* lp, int32_t* lengths) {
  const int cap = P + N - 1, d = m->d;
  const size_t cache = (size_t)m->layers * S * m->KVH * cap * m->hd;
  float* kc = calloc(cache, sizeof(float));
  float* vc = calloc(cache, sizeof(float));
  float* x = malloc(sizeof(float) * (size_t)S * P * d);
  float* last = malloc(sizeof(float) * (size_t)S * d);
  float* logits = malloc(sizeof(float) * (size_t)S * m->V);
  int32_t* ids = malloc(sizeof(int32_t) * S);
  int32_t* hist = malloc(sizeof(int32_t) * (size_t)S * (P + N));
  int* done = calloc((size_t)S, sizeof(int));
  for (int s = 0; s < S; ++s) {
    memcpy(hist + (size_t)s * (P + N), prompts + (size_t)s * P, sizeof(int32_t) * P);
    lengths[s] = N;
  }
  or_model_forward(m, prompts, S, P, 0, kc, vc, cap, x);
  for (int s = 0; s < S; ++s) memcpy(last + (size_t)s * d, x + ((size_t)s * P + P - 1) * d, sizeof(float) * d);
  for (int t = 0; t < N; ++t) {
    if (t > 0) {
      for (int s = 0; s < S; ++s) ids[s] = tokens[(size_t)s * N + t - 1];
      or_model_forward(m, ids, S, 1, P + t - 1, kc, vc, cap, last);
    }
    or_model_logits(m, last, S, logits);
    for (int s = 0; s < S; ++s) {
      int32_t* out = tokens + (size_t)s * N + t;
      double* lo = lp ? lp + (size_t)s * N + t : NULL;
      if (done[s]) { *out = eos; if (lo) *lo = 0.0; continue; }
      or_sample_ex_row(logits + (size_t)s * m->V, m->V, temperature, top_k, penalty, top_p,
                       apply_top_p, seed, s, t, hist + (size_t)s * (P + N), P + t, out, lo);
      hist[(size_t)s * (P + N) + P + t] = *out;
      if (eos >= 0 && *out == eos) { done[s] = 1; lengths[s] = t + 1; }
    }
  }
  free(kc); free(vc); free(x); free(last); free(logits); free(ids); free(hist); free(done);
}

/* Log-probs of tokens[:, n] given prompt ‖ tokens[:, :n] (tensor_sleep.rs:2531-2615). */
void or_logprobs(const or_model* m, const int32_t* prompts, const int32_t* tokens, int S, int P,
                 int N, double* lp) {
  const int L = P + N - 1, d = m->d;
  const size_t cache = (size_t)m->layers * S * m->KVH * L * m->hd;
  float* kc = calloc(cache, sizeof(float));
  float* vc = calloc(cache, sizeof(float));
  int32_t* ids = calloc((size_t)S * L, sizeof(int32_t));
  float* x = malloc(sizeof(float) * (size_t)S * L * d);
  float* rows = malloc(sizeof(float) * (size_t)S * N * d);
  float* logits = malloc(sizeof(float) * (size_t)S * N * m->V);
  for (int s = 0; s < S; ++s)
    for (int t = 0; t < L; ++t)
      ids[(size_t)s * L + t] = t < P ? prompts[(size_t)s * P + t] : tokens[(size_t)s * N + t - P];
  or_model_forward(m, ids, S, L, 0, kc, vc, L, x);
  for (int s = 0; s < S; ++s)
    for (int n = 0; n < N; ++n)
      memcpy(rows + ((size_t)s * N + n) * d, x + ((size_t)s * L + P - 1 + n) * d, sizeof(float) * d);
  or_model_logits(m, rows, (int64_t)S * N, logits);
  or_ce_rows(logits, 0, tokens, (int64_t)S * N, m->V, m->V, lp, NULL, NULL, 1.0, NULL);
  free(kc); free(vc); free(ids); free(x); free(rows); free(logits);
}
