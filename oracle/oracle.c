/*
 * CPU oracle — TEST INFRASTRUCTURE ONLY (see oracle.h). Restates the
 * reference's CPU path; never linked into the product library.
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <string.h>

/* OpenMP thread count of the oracle's parallel loops (n <= 0: every core). */
void or_set_threads(int n) { omp_set_num_threads(n > 0 ? n : omp_get_num_procs()); }
int or_max_threads(void) { return omp_get_max_threads(); }

float or_bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t or_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

void or_bf16_bits(const float* x, int64_t n, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = or_f32_to_bf16(x[i]);
}

float or_round_f16(float f) {
  if (!isfinite(f)) return f;
  const float a = fabsf(f);
  if (a >= 65520.0f) return copysignf(INFINITY, f); /* halfway above 65504 rounds to inf */
  float q;
  if (a < 6.103515625e-05f) {
    q = 5.9604644775390625e-08f; /* subnormal quantum 2^-24 */
  } else {
    int e;
    frexpf(a, &e);          /* a in [2^(e-1), 2^e) */
    q = ldexpf(1.0f, e - 11); /* 10 fraction bits */
  }
  return copysignf(nearbyintf(a / q) * q, f); /* ties to even (default rounding mode) */
}

static double load_logit(const void* p, int dtype, int64_t i) {
  if (dtype == 1) return (double)or_bf16_to_f32(((const uint16_t*)p)[i]);
  return (double)((const float*)p)[i];
}

/* linear_cross_entropy/reference.rs:21-40 masks padded columns to -inf, so
 * they contribute exp(-inf) = 0; here they are simply skipped. The loss of
 * reference.rs:60-92 is mean(-log_softmax[target]); the gradient of
 * reference.rs:128-137 / gpu.rs:143-152 is (softmax - onehot) * scale. */
void or_ce_rows(const void* logits, int dtype, const int32_t* targets, int64_t rows,
                int64_t stored, int64_t logical, double* lp, double* lse, float* grad,
                double grad_scale, const double* row_scale) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t base = r * stored;
    double m = -INFINITY;
    for (int64_t c = 0; c < logical; ++c) {
      double x = load_logit(logits, dtype, base + c);
      if (x > m) m = x;
    }
    double s = 0.0;
    for (int64_t c = 0; c < logical; ++c) s += exp(load_logit(logits, dtype, base + c) - m);
    const double l = m + log(s);
    const int32_t t = targets[r];
    if (lse) lse[r] = l;
    if (lp) lp[r] = (t >= 0 && t < logical) ? load_logit(logits, dtype, base + t) - l : NAN;
    if (grad) {
      const double sc = grad_scale * (row_scale ? row_scale[r] : 1.0);
      for (int64_t c = 0; c < stored; ++c) {
        double g = 0.0;
        if (c < logical) {
          g = exp(load_logit(logits, dtype, base + c) - l) * sc;
          if (c == t) g -= sc;
        }
        grad[base + c] = (float)g;
      }
    }
  }
}

/* Bits match include/summa_amd.h SM_GRPO_*. */
enum {
  OR_BAD_REWARD = 1 << 0,
  OR_BAD_CURRENT = 1 << 1,
  OR_BAD_BEHAVIOR = 1 << 2,
  OR_MASK_NOT_BINARY = 1 << 3,
  OR_MASK_EMPTY_ROW = 1 << 4,
  OR_RATIO_NONFINITE = 1 << 5,
  OR_RATIO_UNSAFE = 1 << 6,
  OR_REWARD_OVERFLOW = 1 << 7,
  OR_LOSS_OVERFLOW = 1 << 8,
  OR_BAD_REFERENCE = 1 << 9,
  OR_REF_RATIO_NONFINITE = 1 << 10,
  OR_REF_RATIO_UNSAFE = 1 << 11
};

/* posttrain.rs:720-868, statement by statement, per group; mask semantics of
 * posttrain.rs:957-961 (masked sum over tokens / active count per rollout). */
int or_grpo_loss(const double* rewards, const double* lp_cur, const double* lp_beh,
                 const double* lp_ref, const double* mask, int64_t groups, int64_t G,
                 int64_t T, double clip, double adv_eps, double beta, double* stats,
                 double* adv, double* dlp) {
  int first_error = 0;
  for (int64_t g = 0; g < groups; ++g) {
    int err = 0;
    const double* r = rewards + g * G;
    double sum = 0.0;
    for (int64_t i = 0; i < G; ++i) {
      if (!isfinite(r[i])) err |= OR_BAD_REWARD;
      sum += r[i];
    }
    const double mean = sum / (double)G;
    double var = 0.0;
    for (int64_t i = 0; i < G; ++i) var += (r[i] - mean) * (r[i] - mean);
    var /= (double)G;
    if (!isfinite(mean) || !isfinite(var)) err |= OR_REWARD_OVERFLOW;
    const double sd = sqrt(var);
    const double den = sd > adv_eps ? sd : adv_eps;
    const double group_scale = 1.0 / (double)G;
    const double lower = 1.0 - clip, upper = 1.0 + clip;
    double objective = 0.0, total_kl = 0.0, clipped = 0.0, tokens = 0.0;
    for (int64_t i = 0; i < G; ++i) {
      const double a = (r[i] - mean) / den;
      if (adv) adv[g * G + i] = a;
      const int64_t off = (g * G + i) * T;
      double len = 0.0;
      for (int64_t t = 0; t < T; ++t) {
        const double mk = mask ? mask[off + t] : 1.0;
        if (!(mk == 0.0 || mk == 1.0)) err |= OR_MASK_NOT_BINARY;
        len += mk;
      }
      if (len <= 0.0) err |= OR_MASK_EMPTY_ROW;
      const double token_scale = len > 0.0 ? group_scale / len : 0.0;
      for (int64_t t = 0; t < T; ++t) {
        const double mk = mask ? mask[off + t] : 1.0;
        const double cur = lp_cur[off + t], beh = lp_beh[off + t];
        if (!isfinite(cur)) err |= OR_BAD_CURRENT;
        if (!isfinite(beh)) err |= OR_BAD_BEHAVIOR;
        const double log_ratio = cur - beh;
        if (!isfinite(log_ratio)) err |= OR_RATIO_NONFINITE;
        if (!(log_ratio <= 80.0)) err |= OR_RATIO_UNSAFE;
        const double ratio = exp(log_ratio > 80.0 ? 80.0 : log_ratio);
        const double clipped_ratio = ratio < lower ? lower : (ratio > upper ? upper : ratio);
        const double unclipped_surrogate = ratio * a;
        const double clipped_surrogate = clipped_ratio * a;
        const double surrogate =
            unclipped_surrogate < clipped_surrogate ? unclipped_surrogate : clipped_surrogate;
        const int is_clipped = surrogate == clipped_surrogate && ratio != clipped_ratio;
        double kl = 0.0, d_kl = 0.0;
        if (lp_ref) {
          const double ref = lp_ref[off + t];
          if (!isfinite(ref)) err |= OR_BAD_REFERENCE;
          const double lrp = ref - cur;
          if (!isfinite(lrp)) err |= OR_REF_RATIO_NONFINITE;
          if (!(lrp <= 80.0)) err |= OR_REF_RATIO_UNSAFE;
          const double rop = exp(lrp > 80.0 ? 80.0 : lrp);
          kl = rop - lrp - 1.0;
          d_kl = 1.0 - rop;
        }
        const double ts = token_scale * mk;
        objective += ts * (surrogate - beta * kl);
        total_kl += ts * kl;
        if (mk != 0.0) {
          clipped += is_clipped ? 1.0 : 0.0;
          tokens += 1.0;
        }
        const int active = (a >= 0.0 && ratio <= upper) || (a < 0.0 && ratio >= lower);
        const double d_surrogate = active ? ratio * a : 0.0;
        if (dlp) dlp[off + t] = ts * (-d_surrogate + beta * d_kl);
      }
    }
    if (!isfinite(objective) || !isfinite(total_kl)) err |= OR_LOSS_OVERFLOW;
    if (stats) {
      stats[g * 5 + 0] = -objective;
      stats[g * 5 + 1] = mean;
      stats[g * 5 + 2] = sd;
      stats[g * 5 + 3] = total_kl;
      stats[g * 5 + 4] = tokens > 0.0 ? clipped / tokens : 0.0;
    }
    if (err && !first_error) first_error = err;
  }
  return first_error;
}

/* ------------------------------------------------------------ Q4G128 --- */

/* Rust f32::round: half away from zero. */
static float round_half_away(float v) { return v >= 0.f ? floorf(v + 0.5f) : -floorf(-v + 0.5f); }

void or_q4_quantize(const float* w, int64_t n, uint8_t* codes, uint16_t* scales) {
  const int64_t groups = (n + 127) / 128;
  memset(codes, 0, (size_t)(groups * 64));
  /* groups own disjoint 64-byte code ranges */
#pragma omp parallel for schedule(static)
  for (int64_t g = 0; g < groups; ++g) {
    const int64_t lo = g * 128, hi = lo + 128 < n ? lo + 128 : n;
    float amax = 0.f;
    for (int64_t i = lo; i < hi; ++i) {
      float a = fabsf(w[i]);
      if (a > amax) amax = a;
    }
    const uint16_t sb = or_f32_to_bf16(amax / 7.0f);
    scales[g] = sb;
    const float s = or_bf16_to_f32(sb);
    for (int64_t i = lo; i < hi; ++i) {
      int q = 0;
      if (s > 0.f) {
        float v = round_half_away(w[i] / s);
        q = v < -8.f ? -8 : (v > 7.f ? 7 : (int)v);
      }
      const uint8_t nib = (uint8_t)(q & 0xf);
      codes[i / 2] |= (uint8_t)((i & 1) ? (nib << 4) : nib);
    }
  }
}

static float q4_value(const uint8_t* codes, const uint16_t* scales, int64_t i) {
  const uint8_t byte = codes[i / 2];
  int q = (i & 1) ? (byte >> 4) : (byte & 0xf);
  if (q >= 8) q -= 16;
  return or_bf16_to_f32(scales[i / 128]) * (float)q;
}

void or_q4_decode(const uint8_t* codes, const uint16_t* scales, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = q4_value(codes, scales, i);
}

void or_q4_matvec(const uint8_t* codes, const uint16_t* scales, int64_t rows, int64_t cols,
                  const float* x, float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float sum = 0.f;
    for (int64_t c = 0; c < cols; ++c) sum += q4_value(codes, scales, r * cols + c) * x[c];
    y[r] = sum;
  }
}
