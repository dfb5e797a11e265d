// Internal interface between q4.hip (entry points, small-M kernel) and
// q4_gemm_bl.hip (batch kernel).
#pragma once

#include <cstddef>
#include <cstdint>

#include <hip/hip_runtime.h>

namespace sm {

// Arguments of the qkv + RoPE + cache-append epilogue (sm_q4_qkv_rope).
struct QkvRope {
  const float* rope;     // [max_pos][hd/2][2] f32 (cos, sin)
  const int32_t* pos0;   // [S] first position of each sequence
  int L, cap, H, KVH, hd;
  void *q_out, *kc, *vc; // f16
};

// Batch-M Q4 matmul (q4_gemm_bl.hip). epi: 0..5 as sm_q4_matmul, 6 = qkv +
// RoPE + cache append (qr non-null). Grouped (MoE) mode when tiles != nullptr.
int q4_gemm_bl(const uint8_t* codes, const uint16_t* scales, int N, int K, const void* x, int xt,
               int M, int ldx, void* y, int ldy, int epi, int ncols, hipStream_t st,
               const int32_t* tiles, const int32_t* ntiles, int64_t max_tiles,
               const int32_t* goff, const int32_t* rowidx, size_t cstride, size_t sstride,
               void* ws, int64_t ws_bytes, const QkvRope* qr);
int64_t bl_counter_bytes();

// Sums split-K partials part[ks][M][cols] (cols = N, or 2*ncols gate | value
// for SwiGLU) in split order and applies epilogue epi (0..5) into y.
int splitk_reduce(const float* part, int ks, int M, int N, int ncols, void* y, int ldy, int epi,
                  hipStream_t st);

// Dense large-M Q4 matmul with 256 x 256 tiles (q4_gemm_wide.hip): f16 (xt 1)
// or f16-pair (xt 2) activations, epilogues 0..6; the same results as
// q4_gemm_bl. q4_wide_tiles: its workgroup count for a shape.
int q4_gemm_wide(const uint8_t* codes, const uint16_t* scales, int N, int K, const void* x,
                 int xt, int M, int ldx, void* y, int ldy, int epi, int ncols, hipStream_t st,
                 const QkvRope* qr);
int64_t q4_wide_tiles(int M, int N, int ncols, int epi);

}  // namespace sm
