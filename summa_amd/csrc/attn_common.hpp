// Shared pieces of the 16-bit attention kernels (decode and prefill): the
// score-MFMA operand type per cache dtype (bf16 or f16), the 8-value cache
// unpack, and the output store per output mode.
#pragma once

#include "common.hpp"

namespace sm {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// Four f32 values rounded to bf16 (nearest even), as the 16-bit lanes the
// k = 16 bf16 MFMA takes (lane group g supplies k = 4 g .. 4 g + 3).
typedef short bf16x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16v4_t __attribute__((ext_vector_type(4)));
__device__ inline bf16x4_t to_bf16x4(f4 v) {
  return __builtin_bit_cast(bf16x4_t, __builtin_convertvector(v, bf16v4_t));
}
__device__ inline f4 mfma_bf16_16x16x16(bf16x4_t a, bf16x4_t b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// 8 x 16-bit operand for the score MFMA: raw bits of q / K, typed per cache dtype.
template <bool KF16> struct Op8;
template <> struct Op8<false> {
  typedef bf8 T;
  static __device__ inline f4 mfma(T a, T b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Op8<true> {
  typedef h8 T;
  static __device__ inline f4 mfma(T a, T b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// 8 cache values (one 16-byte load) -> f32.
template <bool KF16>
__device__ inline void unpack8(u32x4 v, float (&f)[8]) {
  if constexpr (KF16) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const h2 p = as_h2(w[i]);
      f[2 * i] = (float)p[0];
      f[2 * i + 1] = (float)p[1];
    }
  } else {
    f[0] = bf16lo(v.x); f[1] = bf16hi(v.x); f[2] = bf16lo(v.y); f[3] = bf16hi(v.y);
    f[4] = bf16lo(v.z); f[5] = bf16hi(v.z); f[6] = bf16lo(v.w); f[7] = bf16hi(v.w);
  }
}

// 4 cache values (one 8-byte load) -> f32.
template <bool KF16>
__device__ inline void unpack4(u32x2 v, float (&f)[4]) {
  if constexpr (KF16) {
    const h2 a = as_h2(v.x), b = as_h2(v.y);
    f[0] = (float)a[0]; f[1] = (float)a[1]; f[2] = (float)b[0]; f[3] = (float)b[1];
  } else {
    f[0] = bf16lo(v.x); f[1] = bf16hi(v.x); f[2] = bf16lo(v.y); f[3] = bf16hi(v.y);
  }
}

// Element strides of a q / output tensor over (sequence, position, head); the
// head_dim values of one (sequence, position, head) are contiguous.
struct AttnStrides {
  int64_t seq, pos, head;
  __host__ __device__ inline size_t at(int s, int r, int h) const {
    return (size_t)((int64_t)s * seq + (int64_t)r * pos + (int64_t)h * head);
  }
  // the model's rows [S, L, H, hd]
  static inline AttnStrides rows(int64_t L, int64_t H, int64_t hd) {
    return AttnStrides{L * H * hd, H * hd, hd};
  }
  // the reference's tensors [B, H, S, hd] (AttentionBackend, fused_attention.rs:37-55)
  static inline AttnStrides bhsd(int64_t S, int64_t H, int64_t hd) {
    return AttnStrides{H * S * hd, hd, S * hd};
  }
};

// Output modes: 0 bf16, 1 f16, 2 f16 pair (a row of `width` values is
// hi[width] | lo[width], the SM_F16X2 layout).
template <int OM>
__device__ inline void store_out(void* out, size_t row, int width, int col, float v) {
  if constexpr (OM == 2) {
    _Float16* o = static_cast<_Float16*>(out) + row * 2 * width;
    split_f16(v, o[col], o[width + col]);
  } else if constexpr (OM == 1) {
    static_cast<_Float16*>(out)[row * width + col] = (_Float16)v;
  } else {
    static_cast<uint16_t*>(out)[row * width + col] = f32_to_bf16(v);
  }
}

}  // namespace sm
