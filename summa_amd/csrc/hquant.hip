// HQUANT packed tensors: the single-tensor container (PackedTensor::to_bytes /
// from_bytes, summa-train/src/quantization.rs:502-597, validate_packed
// :980-1071, fnv1a64 :2274-2281) as host code, and the device decode of its
// formats (PackedTensor::decode / value_at, :445-497, :656-689) feeding the
// model loader (QuantizedModelBackend::load_quantized_matrix, :1183-1189).
//
// Formats: 1 binary g128 (one sign bit, FP16 group scale), 2 ternary g128
// (2-bit slots 0/1/2 = -s/0/+s), 3 ternary entropy g128 (five base-3 trits per
// byte, 26 bytes per group), and 4 = this build's Q4G128 (two's-complement
// nibbles, low nibble first, bf16 group scale), which has no counterpart in
// the reference codec.
#include <cmath>
#include <cstring>

#include "common.hpp"

namespace sm {
namespace {

constexpr uint8_t kMagic[8] = {'H', 'Q', 'U', 'A', 'N', 'T', '1', 0};
constexpr uint16_t kCodecVersion = 1;
constexpr int kMaxRank = 32;
constexpr int kGroup = 128;

uint64_t fnv1a64(const uint8_t* p, int64_t n) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (int64_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

int64_t bytes_per_group(int format) {
  switch (format) {
    case SM_HQ_BINARY: return kGroup / 8;
    case SM_HQ_TERNARY: return kGroup / 4;
    case SM_HQ_TERNARY_ENTROPY: return (kGroup + 4) / 5;
    case SM_HQ_Q4G128: return kGroup / 2;
    default: return -1;
  }
}

float f16_bits_to_f32(uint16_t b) {
  const uint32_t s = (uint32_t)(b >> 15) << 31, e = (b >> 10) & 31, m = b & 1023;
  uint32_t u;
  if (e == 0) {
    if (m == 0) {
      u = s;
    } else {  // subnormal: renormalise
      int ee = -1;
      uint32_t mm = m;
      while (!(mm & 1024)) {
        mm <<= 1;
        --ee;
      }
      u = s | (uint32_t)(127 - 15 + 1 + ee) << 23 | (mm & 1023) << 13;
    }
  } else if (e == 31) {
    u = s | 0x7f800000u | m << 13;
  } else {
    u = s | (e + 112) << 23 | m << 13;
  }
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

float bf16_bits_to_f32(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Slot `slot` of a group's code bytes (the padding check of
// validate_zero_padding, :1036-1056).
int code_at(int format, const uint8_t* g, int64_t slot) {
  switch (format) {
    case SM_HQ_BINARY: return (g[slot / 8] >> (slot % 8)) & 1;
    case SM_HQ_TERNARY: return (g[slot / 4] >> ((slot % 4) * 2)) & 3;
    case SM_HQ_TERNARY_ENTROPY: {
      int d = 1;
      for (int i = 0; i < slot % 5; ++i) d *= 3;
      return (g[slot / 5] / d) % 3;
    }
    default: return (g[slot / 2] >> ((slot % 2) * 4)) & 15;
  }
}

int validate(const sm_hquant* t) {
  SM_REQUIRE(t->group_size == kGroup, "packed tensor is not g128");
  SM_REQUIRE(t->rank >= 1 && t->rank <= kMaxRank, "packed tensor rank must be in 1..=%d",
             kMaxRank);
  int64_t elements = 1;
  for (int i = 0; i < t->rank; ++i) {
    SM_REQUIRE(t->shape[i] >= 0 && (t->shape[i] == 0 || elements <= INT64_MAX / t->shape[i]),
               "tensor element count overflows usize");
    elements *= t->shape[i];
  }
  SM_REQUIRE(elements > 0, "packed tensor is empty");
  SM_REQUIRE(elements == t->elements, "packed tensor element count mismatch");
  const int64_t bpg = bytes_per_group(t->format);
  SM_REQUIRE(bpg > 0, "unknown ultra-quant format tag %d", t->format);
  const int64_t groups = ceil_div(elements, kGroup);
  SM_REQUIRE(t->nscales == groups, "packed tensor scale count mismatch");
  SM_REQUIRE(t->ncodes == groups * bpg, "packed tensor code size mismatch");
  for (int64_t i = 0; i < groups; ++i) {
    const uint16_t b = t->scales[i];
    const float s = t->format == SM_HQ_Q4G128 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
    SM_REQUIRE(std::isfinite(s) && s >= 0.f && !(b & 0x8000),
               "packed tensor contains an invalid or non-canonical scale");
    if (t->format == SM_HQ_Q4G128)  // q * scale must stay exact in f16
      SM_REQUIRE(s == 0.f || (s >= 6.103515625e-05f && s * 8.f <= 65504.f),
                 "Q4G128 scale %g is outside the f16 normal range", (double)s);
  }
  if (t->format == SM_HQ_TERNARY) {
    for (int64_t i = 0; i < t->ncodes; ++i)
      for (int slot = 0; slot < 4; ++slot)
        SM_REQUIRE(((t->codes[i] >> (slot * 2)) & 3) != 3,
                   "packed tensor contains reserved ternary code 3");
  } else if (t->format == SM_HQ_TERNARY_ENTROPY) {
    for (int64_t i = 0; i < t->ncodes; ++i)
      SM_REQUIRE(t->codes[i] < 243, "packed tensor contains an invalid base-3 byte");
  }
  // canonical padding: unused slots of the final group are code 0, and the
  // two spare trits of every full base-3 group are 0
  const int64_t valid_last = elements - (groups - 1) * kGroup;
  const int slots_per_byte = t->format == SM_HQ_BINARY ? 8 : t->format == SM_HQ_TERNARY ? 4
                           : t->format == SM_HQ_TERNARY_ENTROPY ? 5 : 2;
  const uint8_t* last = t->codes + (groups - 1) * bpg;
  for (int64_t slot = valid_last; slot < bpg * slots_per_byte; ++slot)
    SM_REQUIRE(code_at(t->format, last, slot) == 0,
               "packed tensor contains non-canonical final-group padding");
  if (t->format == SM_HQ_TERNARY_ENTROPY)
    for (int64_t g = 0; g + 1 < groups; ++g)
      SM_REQUIRE(t->codes[g * bpg + bpg - 1] < 27,
                 "packed tensor contains non-canonical base-3 group padding");
  return SM_OK;
}

template <typename T>
bool rd(const uint8_t* p, int64_t n, int64_t& at, T& v) {
  if (at + (int64_t)sizeof(T) > n) return false;
  std::memcpy(&v, p + at, sizeof(T));  // little-endian host
  at += sizeof(T);
  return true;
}

// ---- device decode: one element per thread
__device__ inline float f16bits(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

template <int FMT>
__global__ void hq_decode_kernel(const uint16_t* __restrict__ scales,
                                 const uint8_t* __restrict__ codes, int64_t n, int64_t rows,
                                 int64_t cols, int transpose, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int64_t g = i / kGroup, l = i % kGroup;
  float v;
  if constexpr (FMT == SM_HQ_Q4G128) {
    const uint8_t byte = codes[g * 64 + l / 2];
    const int q = ((int)((l & 1) ? (byte >> 4) : (byte & 15)) ^ 8) - 8;
    v = bf16_to_f32(scales[g]) * (float)q;
  } else {
    const float s = f16bits(scales[g]);
    int code;
    if constexpr (FMT == SM_HQ_BINARY) {
      code = ((codes[g * 16 + l / 8] >> (l % 8)) & 1) ? 2 : 0;
    } else if constexpr (FMT == SM_HQ_TERNARY) {
      code = (codes[g * 32 + l / 4] >> ((l % 4) * 2)) & 3;
    } else {
      const int byte = codes[g * 26 + l / 5];
      const int pw[5] = {1, 3, 9, 27, 81};
      code = (byte / pw[l % 5]) % 3;
    }
    v = code == 0 ? -s : code == 1 ? 0.f : s;
  }
  // [rows, cols] row-major, or written transposed as [cols, rows]
  out[transpose ? (i % cols) * rows + i / cols : i] = v;
}

}  // namespace

int hquant_decode_device(const sm_hquant* t, float* out, int transpose, hipStream_t st) {
  SM_REQUIRE(!transpose || t->rank == 2, "a transposed decode needs a rank-2 tensor");
  const int64_t n = t->elements;
  const int64_t rows = transpose ? t->shape[0] : 1, cols = transpose ? t->shape[1] : n;
  const unsigned blocks = (unsigned)ceil_div(n, 256);
  switch (t->format) {
#define SM_HQ(F)                                                                            \
    case F: hq_decode_kernel<F><<<blocks, 256, 0, st>>>(t->scales, t->codes, n, rows, cols, \
                                                         transpose, out); break;
    SM_HQ(SM_HQ_BINARY)
    SM_HQ(SM_HQ_TERNARY)
    SM_HQ(SM_HQ_TERNARY_ENTROPY)
    SM_HQ(SM_HQ_Q4G128)
#undef SM_HQ
    default: SM_REQUIRE(false, "unknown ultra-quant format tag %d", t->format);
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace sm

using namespace sm;

extern "C" uint64_t sm_fnv1a64(const uint8_t* bytes, int64_t n) {
  return bytes && n > 0 ? fnv1a64(bytes, n) : 0xcbf29ce484222325ull;
}

extern "C" int sm_hquant_parse(const uint8_t* b, int64_t n, sm_hquant* out) {
  SM_REQUIRE(out && (b || n == 0), "sm_hquant_parse: null argument");
  SM_REQUIRE(n >= 8 + 2 + 1 + 2 + 1 + 8, "quantized tensor is truncated");
  const int64_t pn = n - 8;
  uint64_t expected;
  std::memcpy(&expected, b + pn, 8);
  SM_REQUIRE(fnv1a64(b, pn) == expected, "quantized tensor checksum mismatch");
  SM_REQUIRE(std::memcmp(b, kMagic, 8) == 0, "invalid quantized tensor magic");
  int64_t at = 8;
  uint16_t version, gs;
  uint8_t tag, rank;
  SM_REQUIRE(rd(b, pn, at, version), "quantized tensor is truncated");
  SM_REQUIRE(version == kCodecVersion, "unsupported quantized tensor version %u",
             (unsigned)version);
  SM_REQUIRE(rd(b, pn, at, tag), "quantized tensor is truncated");
  SM_REQUIRE(tag >= 1 && tag <= 4, "unknown ultra-quant format tag %u", (unsigned)tag);
  SM_REQUIRE(rd(b, pn, at, gs) && rd(b, pn, at, rank), "quantized tensor is truncated");
  SM_REQUIRE(rank >= 1 && rank <= kMaxRank, "packed tensor rank must be in 1..=%d", kMaxRank);
  sm_hquant t{};
  t.format = tag;
  t.group_size = gs;
  t.rank = rank;
  int64_t elements = 1;
  for (int i = 0; i < rank; ++i) {
    uint64_t d;
    SM_REQUIRE(rd(b, pn, at, d), "quantized tensor is truncated");
    SM_REQUIRE(d <= (uint64_t)INT64_MAX && (d == 0 || elements <= INT64_MAX / (int64_t)d),
               "tensor element count overflows usize");
    t.shape[i] = (int64_t)d;
    elements *= (int64_t)d;
  }
  SM_REQUIRE(elements > 0, "packed tensor is empty");
  t.elements = elements;
  uint64_t ns, nc;
  SM_REQUIRE(rd(b, pn, at, ns) && rd(b, pn, at, nc), "quantized tensor is truncated");
  const uint64_t remaining = (uint64_t)(pn - at);
  SM_REQUIRE(ns <= remaining / 2 && nc <= remaining && ns * 2 + nc == remaining,
             "quantized tensor declared payload size mismatch");
  t.nscales = (int64_t)ns;
  t.ncodes = (int64_t)nc;
  t.scales = reinterpret_cast<const uint16_t*>(b + at);  // 2-byte aligned when b is
  t.codes = b + at + 2 * ns;
  SM_REQUIRE(((uintptr_t)t.scales & 1) == 0, "sm_hquant_parse: buffer must be 2-byte aligned");
  SM_TRY(validate(&t));
  *out = t;
  return SM_OK;
}

extern "C" int64_t sm_hquant_bytes(const sm_hquant* t) {
  if (!t || t->rank < 1 || t->rank > kMaxRank) return -1;
  return 8 + 2 + 1 + 2 + 1 + 8 * (int64_t)t->rank + 8 + 8 + 2 * t->nscales + t->ncodes + 8;
}

extern "C" int sm_hquant_write(const sm_hquant* t, uint8_t* out, int64_t cap, int64_t* written) {
  SM_REQUIRE(t && out && t->scales && t->codes, "sm_hquant_write: null argument");
  SM_TRY(validate(t));
  const int64_t need = sm_hquant_bytes(t);
  SM_REQUIRE(cap >= need, "sm_hquant_write: buffer holds %lld bytes, %lld needed",
             (long long)cap, (long long)need);
  int64_t at = 0;
  auto put = [&](const void* p, size_t k) {
    std::memcpy(out + at, p, k);
    at += (int64_t)k;
  };
  put(kMagic, 8);
  put(&kCodecVersion, 2);
  const uint8_t tag = (uint8_t)t->format, rank = (uint8_t)t->rank;
  const uint16_t gs = (uint16_t)t->group_size;
  put(&tag, 1);
  put(&gs, 2);
  put(&rank, 1);
  for (int i = 0; i < t->rank; ++i) {
    const uint64_t d = (uint64_t)t->shape[i];
    put(&d, 8);
  }
  const uint64_t ns = (uint64_t)t->nscales, nc = (uint64_t)t->ncodes;
  put(&ns, 8);
  put(&nc, 8);
  put(t->scales, 2 * (size_t)ns);
  put(t->codes, (size_t)nc);
  const uint64_t h = fnv1a64(out, at);
  put(&h, 8);
  if (written) *written = at;
  return SM_OK;
}

extern "C" int sm_hquant_decode(const sm_hquant* t, float* out, int transpose, void* stream) {
  SM_REQUIRE(t && out && t->scales && t->codes, "sm_hquant_decode: null argument");
  SM_REQUIRE(t->elements > 0 && t->nscales == ceil_div(t->elements, 128) &&
                 t->ncodes == t->nscales * bytes_per_group(t->format),
             "sm_hquant_decode: inconsistent tensor description");
  return hquant_decode_device(t, out, transpose, as_stream(stream));
}
