/*
 * HQUANT codec restatement — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * quantize_tensor (summa-train/src/quantization.rs:691-773), optimal_ternary
 * (:934-978), PackedTensor::decode (:445-497), the container layout of
 * to_bytes (:502-528) and fnv1a64 (:2274-2281). Pinned in tests/test_oracle.py
 * by the reference's codec tests (:2495-2618: storage rates, identical ternary
 * decodes, the 137-element partial group, decode . x == matrix_vector), FNV-1a
 * published test vectors, and brute force over every nonzero count for the
 * ternary error minimiser.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* f32 -> IEEE binary16 bits, round to nearest even (half::f16::from_f32). */
uint16_t or_f32_to_f16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  if (isnan(f)) return sign | 0x7e00u;
  const float r = or_round_f16(fabsf(f));
  if (isinf(r)) return sign | 0x7c00u;
  if (r == 0.0f) return sign;
  int e;
  const float m = frexpf(r, &e); /* r = m * 2^e, m in [0.5, 1) */
  if (e < -13) {                 /* subnormal: r = k * 2^-24 */
    return sign | (uint16_t)lrintf(ldexpf(r, 24));
  }
  const uint16_t exp = (uint16_t)(e + 14);
  const uint16_t frac = (uint16_t)lrintf((m * 2.0f - 1.0f) * 1024.0f);
  return sign | (uint16_t)(exp << 10) | frac;
}

float or_f16_bits_to_f32(uint16_t b) {
  const int e = (b >> 10) & 31, m = b & 1023;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m + 1024), e - 25);
  return (b & 0x8000) ? -v : v;
}

uint64_t or_fnv1a64(const uint8_t* p, int64_t n) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (int64_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

int64_t or_hq_bytes_per_group(int format) {
  return format == 1 ? 16 : format == 2 ? 32 : format == 3 ? 26 : 64;
}

typedef struct {
  int64_t i;
  double m;
} ranked_t;

static int by_magnitude(const void* a, const void* b) {
  const ranked_t* x = a;
  const ranked_t* y = b;
  if (x->m != y->m) return x->m > y->m ? -1 : 1; /* descending magnitude */
  return x->i < y->i ? -1 : (x->i > y->i);       /* then index */
}

/* optimal_ternary (:934-978): the k largest magnitudes are nonzero, with k and
 * scale = mean of those k magnitudes minimising the squared error. */
static float optimal_ternary(const float* g, int64_t n, uint8_t* trits) {
  ranked_t* r = malloc(sizeof(ranked_t) * (size_t)n);
  for (int64_t i = 0; i < n; ++i) {
    r[i].i = i;
    r[i].m = fabs((double)g[i]);
  }
  qsort(r, (size_t)n, sizeof(ranked_t), by_magnitude);
  double total = 0.0;
  for (int64_t i = 0; i < n; ++i) total += r[i].m * r[i].m;
  double prefix = 0.0, best_err = total, best_scale = 0.0;
  int64_t best_k = 0;
  for (int64_t i = 0; i < n; ++i) {
    prefix += r[i].m;
    const double err = total - prefix * prefix / (double)(i + 1);
    if (err < best_err) {
      best_err = err;
      best_k = i + 1;
      best_scale = prefix / (double)(i + 1);
    }
  }
  unsigned char* sel = calloc((size_t)n, 1);
  for (int64_t i = 0; i < best_k; ++i) sel[r[i].i] = 1;
  for (int64_t i = 0; i < n; ++i)
    trits[i] = (!sel[i] || best_scale == 0.0) ? 1 : (g[i] < 0.0f ? 0 : 2);
  free(sel);
  free(r);
  return (float)best_scale;
}

/* quantize_tensor (:691-773) for formats 1-3; codes zero-initialised by the
 * caller ([groups * bytes_per_group]). Returns 0, or -1 for a scale outside
 * the finite FP16 range. */
int or_hq_quantize(const float* v, int64_t n, int format, uint16_t* scales, uint8_t* codes) {
  const int64_t groups = (n + 127) / 128, bpg = or_hq_bytes_per_group(format);
  uint8_t trits[128];
  for (int64_t gi = 0; gi < groups; ++gi) {
    const float* g = v + gi * 128;
    const int64_t len = (gi + 1) * 128 <= n ? 128 : n - gi * 128;
    float scale;
    if (format == 1) {
      double s = 0.0;
      for (int64_t i = 0; i < len; ++i) s += fabs((double)g[i]);
      scale = (float)(s / (double)len);
    } else {
      scale = optimal_ternary(g, len, trits);
    }
    const uint16_t sb = or_f32_to_f16_bits(scale);
    const float sf = or_f16_bits_to_f32(sb);
    if (!isfinite(sf) || sf < 0.0f) return -1;
    scales[gi] = sb;
    uint8_t* c = codes + gi * bpg;
    if (format == 1) {
      for (int64_t i = 0; i < len; ++i)
        if (g[i] >= 0.0f) c[i / 8] |= (uint8_t)(1u << (i % 8));
    } else if (format == 2) {
      for (int64_t i = 0; i < len; ++i) c[i / 4] |= (uint8_t)(trits[i] << ((i % 4) * 2));
    } else {
      for (int64_t b = 0; b * 5 < len; ++b) {
        unsigned packed = 0, mult = 1;
        for (int64_t k = b * 5; k < len && k < b * 5 + 5; ++k) {
          packed += trits[k] * mult;
          mult *= 3;
        }
        c[b] = (uint8_t)packed;
      }
    }
  }
  return 0;
}

/* PackedTensor::decode (:445-497) for formats 1-3; format 4 is the Q4G128
 * codec of oracle.c (bf16 scale x two's-complement nibble). */
void or_hq_decode(int format, int64_t n, const uint16_t* scales, const uint8_t* codes,
                  float* out) {
  const int64_t bpg = or_hq_bytes_per_group(format);
  for (int64_t i = 0; i < n; ++i) {
    const int64_t gi = i / 128, l = i % 128;
    const uint8_t* c = codes + gi * bpg;
    if (format == 4) {
      const int nib = (l & 1) ? (c[l / 2] >> 4) : (c[l / 2] & 15);
      out[i] = or_bf16_to_f32(scales[gi]) * (float)((nib ^ 8) - 8);
      continue;
    }
    const float s = or_f16_bits_to_f32(scales[gi]);
    int code;
    if (format == 1) code = ((c[l / 8] >> (l % 8)) & 1) ? 2 : 0;
    else if (format == 2) code = (c[l / 4] >> ((l % 4) * 2)) & 3;
    else {
      int d = 1;
      for (int k = 0; k < l % 5; ++k) d *= 3;
      code = (c[l / 5] / d) % 3;
    }
    out[i] = code == 0 ? -s : code == 1 ? 0.0f : s;
  }
}
