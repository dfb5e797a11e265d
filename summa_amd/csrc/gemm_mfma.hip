// f32 GEMM on the bf16 matrix cores, for the policy update's large matmuls
// (the forward with activations kept, every data and weight gradient, Muon's
// Newton-Schulz): C = alpha op(A) op(B) + beta C with op = identity or
// transpose, f32 in and out, any shape and leading dimensions. The reference
// trains through Burn's matmul (summa-llm/src/model/matmul.rs:132-143; bf16
// operands on its CUDA path, f32 on its CPU path).
//
// Each f32 operand value is split into P bf16 planes, round to nearest even
// at each step (bf16 has f32's exponent range, so no scaling is needed):
// - P = 3 (the default): x = x0 + x1 + x2 exactly (24 significant bits, f32's
//   own precision), and a product x y is the sum of the six plane products of
//   weight >= 2^-16 relative (x2 y0, x1 y1, x0 y2, x1 y0, x0 y1, x0 y0,
//   smallest first). The dropped terms (x1 y2, x2 y1, x2 y2) are below 2^-23
//   relative, so the result is an f32 GEMM's up to the order of its f32
//   additions.
// - P = 2: x = x0 + x1 + r with |r| <= 2^-17 |x|, products x1 y0, x0 y1,
//   x0 y0: each product within about 2^-15 relative (16-bit operands).
// - P = 1: x0 y0, the product of the bf16-rounded operands (each within 2^-9
//   relative): the reference's CUDA-path matmul, bf16 operands with f32
//   accumulation.
// Products are accumulated in f32 by v_mfma_f32_32x32x16_bf16.
//
// Workgroup = 128 x 128 output tile, 4 waves of 64 x 64 (2 x 2 blocks of
// 32 x 32); K in steps of 32. Each thread loads 16 values of each operand
// tile per step, splits them once into the planes and stores them to LDS as
// [plane][row][k] bf16, rows padded to 40 elements so that the 16-byte writes
// and fragment reads of consecutive rows spread over the banks; the next
// step's loads are in flight while the current step's MFMAs run. A thread
// holds 16 consecutive k of one row: four 16-byte loads when k is the
// operand's contiguous dimension, else 16 scalar loads, each instruction 64
// consecutive rows. (16-byte loads along the rows of a transposed operand, a
// thread holding 4 rows x 4 k, measured 1.1-1.6x slower at the policy
// update's shapes: their 8-byte LDS stores conflict.) One LDS buffer (20 KB
// per plane), two workgroups per CU. Per 16-k slice a
// wave reads its 2 + 2 fragments of each plane and issues the MFMAs product
// by product across its four blocks, so four independent accumulations
// separate two dependent ones.
#include <algorithm>

#include "common.hpp"

namespace sm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef f32x4 f4;

constexpr int kBM = 128, kBK = 32, kRS = kBK + 8;  // tile rows, k per step, LDS row stride
constexpr int kPlane = kBM * kRS;                   // bf16 per plane of one operand tile

// (a, b) -> P bf16 planes as packed words (a in the low half); for P = 3,
// v = p0 + p1 + p2 exactly (finite v)
template <int P>
__device__ inline void split_pair(float a, float b, uint32_t (&w)[P]) {
  w[0] = pack_bf16x2(a, b);
  if constexpr (P > 1) {
    const float ra = a - bf16lo(w[0]), rb = b - bf16hi(w[0]);
    w[1] = pack_bf16x2(ra, rb);
    if constexpr (P > 2) w[2] = pack_bf16x2(ra - bf16lo(w[1]), rb - bf16hi(w[1]));
  }
}

// 8 consecutive k of one row -> the P planes at LDS offset o (16 bytes each)
template <int P>
__device__ inline void store8(const float* v, __bf16* lds, int o) {
  u32x4 w[P];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t x[P];
    split_pair<P>(v[2 * i], v[2 * i + 1], x);
#pragma unroll
    for (int p = 0; p < P; ++p) w[p][i] = x[p];
  }
#pragma unroll
  for (int p = 0; p < P; ++p) *reinterpret_cast<u32x4*>(lds + p * kPlane + o) = w[p];
}

// One operand tile (128 rows x 32 k) of X, element (r, k) at X[r * ld + k]
// when KC (k contiguous), else at X[k * ld + r]; 16 values per thread.
// Thread t: 16 consecutive k of one row, v[i] = (row, k + i): KC: row t / 2,
// k 16 (t % 2) (four 16-byte loads when `vec`); otherwise row t % 128,
// k 16 (t / 128) (one scalar load per k, each instruction 64 consecutive
// rows). Out-of-range elements are 0.
template <bool KC>
struct TileLoader {
  const float* X;
  int64_t ld;
  int r0, R, K;
  bool vec;  // 16-byte aligned rows along k (uniform; KC only)
  int ra, ka;
  __device__ inline void init(int t) {
    ra = KC ? t / 2 : t % kBM;
    ka = KC ? 16 * (t % 2) : 16 * (t / kBM);
  }
  __device__ inline void load(int k0, float (&v)[16]) const {
    const int gr = r0 + ra, gk = k0 + ka;
    if constexpr (KC) {
      const float* p = X + (int64_t)min(gr, R - 1) * ld;
      if (vec && gr < R && gk + 16 <= K) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x4 q = *reinterpret_cast<const f32x4*>(p + gk + 4 * i);
          v[4 * i] = q[0]; v[4 * i + 1] = q[1]; v[4 * i + 2] = q[2]; v[4 * i + 3] = q[3];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i)
          v[i] = (gr < R && gk + i < K) ? p[min(gk + i, K - 1)] : 0.f;
      }
    } else {
      const int c = min(gr, R - 1);
#pragma unroll
      for (int i = 0; i < 16; ++i)
        v[i] = (gr < R && gk + i < K) ? X[(int64_t)min(gk + i, K - 1) * ld + c] : 0.f;
    }
  }
  // this thread's values as P planes into the LDS tile [plane][row][k]
  template <int P>
  __device__ inline void store(const float (&v)[16], __bf16* lds) const {
    store8<P>(v, lds, ra * kRS + ka);
    store8<P>(v + 8, lds, ra * kRS + ka + 8);
  }
};

// plane pairs (pa, pb) of each product, smallest weight first. PB = 2 with
// P = 3: B's values are exact in two planes (b2 = 0; a fake-quantized weight,
// a bf16 scale times a 4-bit code, has at most 11 significant bits, so its
// residual after the first plane has at most 3 and fits the second), so the
// a0 b2 product, exactly zero, is not formed; the other five keep their order
// and the result its bits.
template <int P, int PB = P> struct Products;
template <> struct Products<3, 3> {
  static constexpr int n = 6;
  static constexpr int a[6] = {2, 1, 0, 1, 0, 0}, b[6] = {0, 1, 2, 0, 1, 0};
};
template <> struct Products<3, 2> {
  static constexpr int n = 5;
  static constexpr int a[5] = {2, 1, 1, 0, 0}, b[5] = {0, 1, 0, 1, 0};
};
template <> struct Products<2, 2> {
  static constexpr int n = 3;
  static constexpr int a[3] = {1, 0, 0}, b[3] = {0, 1, 0};
};
template <> struct Products<1, 1> {
  static constexpr int n = 1;
  static constexpr int a[1] = {0}, b[1] = {0};
};

template <bool TA, bool TB, int P, int PB = P>
__global__ __launch_bounds__(256, 2) void gemm_planes_kernel(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ B, int64_t ldb,
    float* __restrict__ C, int64_t ldc, int M, int N, int K, float alpha, float beta, int vec_a,
    int vec_b) {
  __shared__ __attribute__((aligned(16))) __bf16 As[P * kPlane];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[PB * kPlane];
  const int t = threadIdx.x, wave = t / kWave, lane = t % kWave;
  const int wm = wave / 2, wn = wave % 2;
  const int m0 = (int)blockIdx.y * kBM, n0 = (int)blockIdx.x * kBM;
  // op(A) row m = A row m (TA false: k contiguous) or A column m (TA true);
  // op(B) column n = B column n (TB false: B[k][n], n contiguous) or B row n
  TileLoader<!TA> la{A, lda, m0, M, K, vec_a != 0};
  TileLoader<TB> lb{B, ldb, n0, N, K, vec_b != 0};
  la.init(t);
  lb.init(t);
  float va[16], vb[16];
  la.load(0, va);
  lb.load(0, vb);
  la.template store<P>(va, As);
  lb.template store<PB>(vb, Bs);
  __syncthreads();

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  // fragment of lane l: row / column l % 32 of the block, k 8 (l / 32) .. +7
  const int fo = (lane % 32) * kRS + 8 * (lane / 32);
  for (int k0 = 0; k0 < K; k0 += kBK) {
    const bool more = k0 + kBK < K;  // uniform
    if (more) {
      la.load(k0 + kBK, va);
      lb.load(k0 + kBK, vb);
    }
#pragma unroll
    for (int ks = 0; ks < kBK; ks += 16) {
      bf16x8 a[P][2], b[PB][2];
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          a[p][i] = *reinterpret_cast<const bf16x8*>(As + p * kPlane + (wm * 64 + i * 32) * kRS +
                                                     fo + ks);
#pragma unroll
      for (int p = 0; p < PB; ++p)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          b[p][i] = *reinterpret_cast<const bf16x8*>(Bs + p * kPlane + (wn * 64 + i * 32) * kRS +
                                                     fo + ks);
#pragma unroll
      for (int q = 0; q < Products<P, PB>::n; ++q)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                a[Products<P, PB>::a[q]][i], b[Products<P, PB>::b[q]][j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      __syncthreads();  // every wave is done with this step's tiles
      la.template store<P>(va, As);
      lb.template store<PB>(vb, Bs);
      __syncthreads();
    }
  }
  // acc[i][j][e]: row 8 (e / 4) + 4 (lane / 32) + e % 4, column lane % 32 of block (i, j)
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + lane % 32;
      if (col >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
        if (row >= M) continue;
        float* o = C + (int64_t)row * ldc + col;
        *o = beta == 0.f ? alpha * acc[i][j][e] : fmaf(alpha, acc[i][j][e], beta * *o);
      }
    }
}

// ---- pre-split operands: each operand split once into its bf16 planes,
// padded and zero-filled, [P][Rp][Kp] (Rp a multiple of 128 rows, Kp of 32
// k), so that the GEMM's K loop only copies 16-byte chunks into LDS. The
// planes are those the tile loader forms (split_pair on the same values, 0
// past the matrix), in the same LDS layout, so the products and their order,
// and the result, are the same bit for bit.

// op(X) row r, k contiguous: element (r, k) at X[r * ld + k]. Thread: 8
// consecutive k of one row (two 16-byte loads when aligned), one 16-byte
// store per plane.
template <int P>
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ X, int64_t ld,
                                                         int R, int K, __bf16* __restrict__ out,
                                                         int Rp, int Kp, int vec) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int kc = Kp / 8;
  if (c >= (int64_t)Rp * kc) return;
  const int r = (int)(c / kc), k = (int)(c % kc) * 8;
  float v[8];
  if (vec && r < R && k + 8 <= K) {
    const f4 a = *reinterpret_cast<const f4*>(X + (int64_t)r * ld + k);
    const f4 b = *reinterpret_cast<const f4*>(X + (int64_t)r * ld + k + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a[e];
      v[4 + e] = b[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (r < R && k + e < K) ? X[(int64_t)r * ld + k + e] : 0.f;
  }
  u32x4 w[P];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t x[P];
    split_pair<P>(v[2 * i], v[2 * i + 1], x);
#pragma unroll
    for (int p = 0; p < P; ++p) w[p][i] = x[p];
  }
#pragma unroll
  for (int p = 0; p < P; ++p)
    *reinterpret_cast<u32x4*>(out + (int64_t)p * Rp * Kp + (int64_t)r * Kp + k) = w[p];
}

// op(X) row r = column r of X: element (r, k) at X[k * ld + r]. 64 k x 64 r
// tiles through LDS (reads 64 consecutive r per wave instruction), then
// thread: 8 consecutive k of one r, one 16-byte store per plane.
template <int P>
__global__ __launch_bounds__(256) void split_cols_kernel(const float* __restrict__ X, int64_t ld,
                                                         int R, int K, __bf16* __restrict__ out,
                                                         int Rp, int Kp) {
  __shared__ float t[64][65];  // [k][r]
  const int k0 = (int)blockIdx.x * 64, r0 = (int)blockIdx.y * 64;
  const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
  for (int i = ty; i < 64; i += 4) {
    const int k = k0 + i, r = r0 + tx;
    t[i][tx] = (k < K && r < R) ? X[(int64_t)k * ld + r] : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = (int)threadIdx.x + 256 * h, rl = c / 8, kl = (c % 8) * 8;
    if (k0 + kl >= Kp) continue;
    u32x4 w[P];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t x[P];
      split_pair<P>(t[kl + 2 * i][rl], t[kl + 2 * i + 1][rl], x);
#pragma unroll
      for (int p = 0; p < P; ++p) w[p][i] = x[p];
    }
#pragma unroll
    for (int p = 0; p < P; ++p)
      *reinterpret_cast<u32x4*>(out + (int64_t)p * Rp * Kp + (int64_t)(r0 + rl) * Kp + k0 + kl) =
          w[p];
  }
}

// C = alpha op(A) op(B) + beta C from pre-split planes: A [P][Mp][Kp], B
// [PB][Np][Kp] (B's rows are op(B)'s columns; Kp a multiple of BK).
// gemm_planes_kernel's tiles, waves and MFMA order, with BK k per step (rows
// of BK + 8 in LDS); per step a thread copies BK / 16 16-byte chunks (8 k of
// one row) of each plane of each operand, requested one step ahead.
template <int P, int PB, int BK = kBK>
__global__ __launch_bounds__(256, 2) void gemm_split_kernel(
    const __bf16* __restrict__ A, const __bf16* __restrict__ B, int Kp, int64_t pa, int64_t pb,
    float* __restrict__ C, int64_t ldc, int M, int N, float alpha, float beta) {
  constexpr int RS = BK + 8, PL = kBM * RS, CH = BK / 16;  // LDS row, plane, chunks per thread
  __shared__ __attribute__((aligned(16))) __bf16 As[P * PL];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[PB * PL];
  const int t = threadIdx.x, wave = t / kWave, lane = t % kWave;
  const int wm = wave / 2, wn = wave % 2;
  const int m0 = (int)blockIdx.y * kBM, n0 = (int)blockIdx.x * kBM;
  // chunk h of this thread: row (t + 256 h) / (BK / 8), k 8 ((t + 256 h) % (BK / 8))
  int64_t ga[CH], gb[CH];
  int lo[CH];
#pragma unroll
  for (int h = 0; h < CH; ++h) {
    const int c = t + 256 * h, row = c / (BK / 8), k8 = (c % (BK / 8)) * 8;
    ga[h] = (int64_t)(m0 + row) * Kp + k8;
    gb[h] = (int64_t)(n0 + row) * Kp + k8;
    lo[h] = row * RS + k8;
  }
  u32x4 ra[P][CH], rb[PB][CH];
  auto gload = [&](int k0) {
#pragma unroll
    for (int h = 0; h < CH; ++h) {
#pragma unroll
      for (int p = 0; p < P; ++p) ra[p][h] = *reinterpret_cast<const u32x4*>(A + p * pa + ga[h] + k0);
#pragma unroll
      for (int p = 0; p < PB; ++p) rb[p][h] = *reinterpret_cast<const u32x4*>(B + p * pb + gb[h] + k0);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int h = 0; h < CH; ++h) {
#pragma unroll
      for (int p = 0; p < P; ++p) *reinterpret_cast<u32x4*>(As + p * PL + lo[h]) = ra[p][h];
#pragma unroll
      for (int p = 0; p < PB; ++p) *reinterpret_cast<u32x4*>(Bs + p * PL + lo[h]) = rb[p][h];
    }
  };
  gload(0);
  lstore();
  __syncthreads();
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  const int fo = (lane % 32) * RS + 8 * (lane / 32);
  for (int k0 = 0; k0 < Kp; k0 += BK) {
    const bool more = k0 + BK < Kp;  // uniform
    if (more) gload(k0 + BK);
#pragma unroll
    for (int ks = 0; ks < BK; ks += 16) {
      bf16x8 a[P][2], b[PB][2];
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          a[p][i] = *reinterpret_cast<const bf16x8*>(As + p * PL + (wm * 64 + i * 32) * RS +
                                                     fo + ks);
#pragma unroll
      for (int p = 0; p < PB; ++p)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          b[p][i] = *reinterpret_cast<const bf16x8*>(Bs + p * PL + (wn * 64 + i * 32) * RS +
                                                     fo + ks);
#pragma unroll
      for (int q = 0; q < Products<P, PB>::n; ++q)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                a[Products<P, PB>::a[q]][i], b[Products<P, PB>::b[q]][j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      __syncthreads();  // every wave is done with this step's tiles
      lstore();
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + wn * 64 + j * 32 + lane % 32;
      if (col >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
        if (row >= M) continue;
        float* o = C + (int64_t)row * ldc + col;
        *o = beta == 0.f ? alpha * acc[i][j][e] : fmaf(alpha, acc[i][j][e], beta * *o);
      }
    }
}

// op(X) (rows r, k along kc or across) -> planes [P][Rp][Kp] at out
template <int P>
void split_operand(const float* X, int64_t ld, bool kc, int64_t R, int64_t K, __bf16* out,
                   int64_t Rp, int64_t Kp, hipStream_t st) {
  if (kc) {
    const int vec = (ld % 4 == 0 && reinterpret_cast<uintptr_t>(X) % 16 == 0) ? 1 : 0;
    split_rows_kernel<P><<<(unsigned)ceil_div(Rp * (Kp / 8), 256), 256, 0, st>>>(
        X, ld, (int)R, (int)K, out, (int)Rp, (int)Kp, vec);
  } else {
    const dim3 grid((unsigned)ceil_div(Kp, 64), (unsigned)(Rp / 64));
    split_cols_kernel<P><<<grid, 256, 0, st>>>(X, ld, (int)R, (int)K, out, (int)Rp, (int)Kp);
  }
}

// out[c * ldo + r] = in[r * ld + c] for an R x C f32 matrix: 64 x 64 tiles
// through LDS (65-float rows, so the column reads of the write phase spread
// over the banks); each wave instruction reads and writes 64 consecutive
// floats.
__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict__ in,
                                                            int64_t ld, int R, int C,
                                                            float* __restrict__ out, int64_t ldo) {
  __shared__ float t[64][65];
  const int r0 = (int)blockIdx.y * 64, c0 = (int)blockIdx.x * 64;
  const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
  for (int i = ty; i < 64; i += 4) {
    const int r = r0 + i, c = c0 + tx;
    if (r < R && c < C) t[i][tx] = in[(int64_t)r * ld + c];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int c = c0 + i, r = r0 + tx;
    if (c < C && r < R) out[(int64_t)c * ldo + r] = t[tx][i];
  }
}

// The same with 16-byte accesses (R, C, ld, ldo multiples of 4, 16-byte
// aligned rows): thread (row group, f4 column) reads four consecutive floats
// of an input row and, after the barrier, gathers four consecutive input rows
// of one column from LDS into one 16-byte store of an output row.
__global__ __launch_bounds__(256) void transpose_f32x4_kernel(const float* __restrict__ in,
                                                              int64_t ld, int R, int C,
                                                              float* __restrict__ out,
                                                              int64_t ldo) {
  __shared__ float t[64][65];
  const int r0 = (int)blockIdx.y * 64, c0 = (int)blockIdx.x * 64;
  const int q = threadIdx.x % 16, rg = threadIdx.x / 16;  // f4 column, row (group)
  f4 v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + rg + 16 * i, c = c0 + 4 * q;
    v[i] = (r < R && c < C) ? *reinterpret_cast<const f4*>(in + (int64_t)r * ld + c)
                            : f4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) t[rg + 16 * i][4 * q + e] = v[i][e];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int cl = rg + 16 * i, c = c0 + cl, r = r0 + 4 * q;  // output row c, columns r..r+3
    if (c < C && r < R) {
      const f4 w = f4{t[4 * q][cl], t[4 * q + 1][cl], t[4 * q + 2][cl], t[4 * q + 3][cl]};
      *reinterpret_cast<f4*>(out + (int64_t)c * ldo + r) = w;
    }
  }
}

void transpose_f32(const float* in, int64_t ld, int64_t R, int64_t C, float* out, int64_t ldo,
                   hipStream_t st) {
  const dim3 grid((unsigned)ceil_div(C, 64), (unsigned)ceil_div(R, 64));
  const bool v4 = R % 4 == 0 && C % 4 == 0 && ld % 4 == 0 && ldo % 4 == 0 &&
                  reinterpret_cast<uintptr_t>(in) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(out) % 16 == 0;
  if (v4) transpose_f32x4_kernel<<<grid, 256, 0, st>>>(in, ld, (int)R, (int)C, out, ldo);
  else transpose_f32_kernel<<<grid, 256, 0, st>>>(in, ld, (int)R, (int)C, out, ldo);
}

template <int P, int PB = P>
void launch_planes(bool ta, bool tb, dim3 grid, hipStream_t st, const float* A, int64_t lda,
                   const float* B, int64_t ldb, float* C, int64_t ldc, int M, int N, int K,
                   float alpha, float beta, int vec_a, int vec_b) {
#define SM_GB(TA, TB)                                                                      \
  gemm_planes_kernel<TA, TB, P, PB><<<grid, 256, 0, st>>>(A, lda, B, ldb, C, ldc, M, N, K,\
                                                       alpha, beta, vec_a, vec_b)
  if (ta && tb) SM_GB(true, true);
  else if (ta) SM_GB(true, false);
  else if (tb) SM_GB(false, true);
  else SM_GB(false, false);
#undef SM_GB
}

}  // namespace

// scratch for the transposed-operand path (floats)
int64_t transpose_scratch_floats(bool ta, bool tb, int64_t M, int64_t N, int64_t K) {
  const int64_t kp = (K + 3) / 4 * 4;
  return (ta ? M * kp : 0) + (tb ? 0 : N * kp);
}

// k per step of the one-plane pre-split GEMM. Measured against 32 (two
// barriers per 8 MFMAs a wave): 7-18 % faster on the policy update's shapes
// (LM head forward 2.00 -> 1.67 ms); 128 (two waves per SIMD) mixed, the
// FFN-in forward and LM head slower.
constexpr int kSplitBK = 64;

// scratch for the pre-split path with P planes of A and PB of B (floats)
int64_t split_scratch_floats(int P, int PB, int64_t M, int64_t N, int64_t K) {
  const int64_t Mp = ceil_div(M, kBM) * kBM, Np = ceil_div(N, kBM) * kBM;
  const int64_t Kp = ceil_div(K, kSplitBK) * kSplitBK;
  return (P * Mp * Kp + PB * Np * Kp + 1) / 2;
}

// the most any call needs (the pre-split path runs at one plane)
int64_t gemm_planes_scratch_floats(bool ta, bool tb, int64_t M, int64_t N, int64_t K) {
  return std::max(split_scratch_floats(1, 1, M, N, K), transpose_scratch_floats(ta, tb, M, N, K));
}

int gemm_planes(int planes, bool ta, bool tb, int64_t M, int64_t N, int64_t K, float alpha,
                const float* A, int64_t lda, const float* B, int64_t ldb, float beta, float* C,
                int64_t ldc, hipStream_t st, float* scratch, int64_t scratch_floats,
                int b_planes) {
  const int P = planes, PB = (planes == 3 && b_planes == 2) ? 2 : planes;
  const bool al16 = scratch && reinterpret_cast<uintptr_t>(scratch) % 16 == 0;
  // One plane, with room for both operands' bf16 copies: each is converted
  // once (transposed on the way where its k is not contiguous) and
  // gemm_split_kernel only copies chunks into LDS in its K loop: the same
  // values and MFMA order, so the same bits. Measured on the policy update's
  // config[2] shapes: 1.4-1.9x faster at one plane with 32-k steps (FFN-in
  // forward 780 -> 517 us, LM head forward 3.90 -> 2.04 ms; 430 us and 1.65 ms
  // with 64-k steps); at two and three planes
  // the same form was 0-35 % slower (its staged chunks of every plane leave
  // two waves per SIMD where the in-loop split keeps three), so they keep the
  // in-loop split.
  if (P == 1 && al16 && split_scratch_floats(P, PB, M, N, K) <= scratch_floats) {
    const int64_t Mp = ceil_div(M, kBM) * kBM, Np = ceil_div(N, kBM) * kBM;
    const int64_t Kp = ceil_div(K, kSplitBK) * kSplitBK;
    __bf16* sa = reinterpret_cast<__bf16*>(scratch);
    __bf16* sb = sa + Mp * Kp;  // 16-byte aligned: Mp Kp is a multiple of 8192
    split_operand<1>(A, lda, !ta, M, K, sa, Mp, Kp, st);
    split_operand<1>(B, ldb, tb, N, K, sb, Np, Kp, st);
    const dim3 g2((unsigned)(Np / kBM), (unsigned)(Mp / kBM));
    gemm_split_kernel<1, 1, kSplitBK><<<g2, 256, 0, st>>>(sa, sb, (int)Kp, Mp * Kp, Np * Kp, C,
                                                          ldc, (int)M, (int)N, alpha, beta);
    SM_LAUNCH_CHECK();
    return SM_OK;
  }
  // Else, with a smaller scratch, an operand whose k is not its contiguous
  // dimension (op(A) of a transposed A, op(B) of an untransposed B) is first
  // transposed into it, rows padded to a multiple of 4 floats, so that the
  // GEMM runs with 16-byte loads along k on both operands. The tiles reach
  // LDS with the same values in the same k order, so the result is the same
  // bit for bit. Measured on one GRPO group's shapes (config[2], three
  // planes, event-timed, transposes included): FFN-in weight gradient 2.78 ->
  // 2.30 ms, its data gradient 2.28 -> 1.99 ms; LM head 7.40 -> 6.21 and 6.45
  // -> 5.93 ms.
  const int64_t need = transpose_scratch_floats(ta, tb, M, N, K);
  if (scratch && need > 0 && need <= scratch_floats &&
      reinterpret_cast<uintptr_t>(scratch) % 16 == 0) {
    const int64_t kp = (K + 3) / 4 * 4;
    float* s = scratch;
    if (ta) {  // A is [K][M]: A' = A^T, [M][kp]
      transpose_f32(A, lda, K, M, s, kp, st);
      A = s;
      lda = kp;
      ta = false;
      s += M * kp;
    }
    if (!tb) {  // B is [K][N]: B' = B^T, [N][kp]
      transpose_f32(B, ldb, K, N, s, kp, st);
      B = s;
      ldb = kp;
      tb = true;
    }
    SM_LAUNCH_CHECK();
  }
  // 16-byte loads along k need aligned rows (op(A) rows of an untransposed
  // A, op(B) columns of a transposed B)
  auto aligned = [](const float* p, int64_t ld) {
    return ld % 4 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0 ? 1 : 0;
  };
  const int vec_a = !ta && aligned(A, lda), vec_b = tb && aligned(B, ldb);
  const dim3 grid((unsigned)ceil_div(N, kBM), (unsigned)ceil_div(M, kBM));
  if (planes == 1)
    launch_planes<1>(ta, tb, grid, st, A, lda, B, ldb, C, ldc, (int)M, (int)N, (int)K, alpha,
                     beta, vec_a, vec_b);
  else if (planes == 2)
    launch_planes<2>(ta, tb, grid, st, A, lda, B, ldb, C, ldc, (int)M, (int)N, (int)K, alpha,
                     beta, vec_a, vec_b);
  else if (b_planes == 2)  // B exact in two planes: five products (Products<3, 2>)
    launch_planes<3, 2>(ta, tb, grid, st, A, lda, B, ldb, C, ldc, (int)M, (int)N, (int)K, alpha,
                        beta, vec_a, vec_b);
  else
    launch_planes<3>(ta, tb, grid, st, A, lda, B, ldb, C, ldc, (int)M, (int)N, (int)K, alpha,
                     beta, vec_a, vec_b);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace sm

namespace {
int check_gemm(const char* fn, int64_t M, int64_t N, int64_t K, const float* A, int64_t lda,
               const float* B, int64_t ldb, const float* C, int64_t ldc, int trans_a,
               int trans_b) {
  using namespace sm;
  SM_REQUIRE(A && B && C, "%s: null buffer", fn);
  SM_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M < (1 << 30) && N < (1 << 30) && K < (1 << 30),
             "%s: bad shape", fn);
  SM_REQUIRE(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N) && ldc >= N,
             "%s: leading dimension too small", fn);
  if (M == 0 || N == 0) return SM_OK;
  SM_REQUIRE(K > 0, "%s: K must be positive", fn);
  SM_REQUIRE(ceil_div(M, 128) <= 65535, "%s: M above 65535 x 128 rows", fn);
  return SM_OK;
}
}  // namespace

extern "C" int sm_gemm_mfma(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                            float alpha, const float* A, int64_t lda, const float* B, int64_t ldb,
                            float beta, float* C, int64_t ldc, void* stream) {
  using namespace sm;
  SM_TRY(check_gemm("sm_gemm_mfma", M, N, K, A, lda, B, ldb, C, ldc, trans_a, trans_b));
  if (M == 0 || N == 0) return SM_OK;
  return gemm_planes(3, trans_a != 0, trans_b != 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc,
                     as_stream(stream), nullptr, 0, 3);
}

extern "C" int sm_gemm_planes(int planes, int trans_a, int trans_b, int64_t M, int64_t N,
                              int64_t K, float alpha, const float* A, int64_t lda, const float* B,
                              int64_t ldb, float beta, float* C, int64_t ldc, void* stream) {
  using namespace sm;
  SM_REQUIRE(planes >= 1 && planes <= 3, "sm_gemm_planes: planes must be 1, 2 or 3 (got %d)",
             planes);
  SM_TRY(check_gemm("sm_gemm_planes", M, N, K, A, lda, B, ldb, C, ldc, trans_a, trans_b));
  if (M == 0 || N == 0) return SM_OK;
  return gemm_planes(planes, trans_a != 0, trans_b != 0, M, N, K, alpha, A, lda, B, ldb, beta, C,
                     ldc, as_stream(stream), nullptr, 0, 3);
}

extern "C" int64_t sm_gemm_planes_scratch_bytes(int trans_a, int trans_b, int64_t M, int64_t N,
                                                int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return 4 * sm::gemm_planes_scratch_floats(trans_a != 0, trans_b != 0, M, N, K);
}

extern "C" int sm_gemm_planes_ws(int planes, int b_planes, int trans_a, int trans_b, int64_t M,
                                 int64_t N, int64_t K, float alpha, const float* A, int64_t lda,
                                 const float* B, int64_t ldb, float beta, float* C, int64_t ldc,
                                 void* scratch, int64_t scratch_bytes, void* stream) {
  using namespace sm;
  SM_REQUIRE(planes >= 1 && planes <= 3, "sm_gemm_planes: planes must be 1, 2 or 3 (got %d)",
             planes);
  SM_REQUIRE(b_planes == 0 || b_planes == 2 || b_planes == 3,
             "sm_gemm_planes_ws: b_planes must be 0, 2 or 3 (got %d)", b_planes);
  SM_TRY(check_gemm("sm_gemm_planes", M, N, K, A, lda, B, ldb, C, ldc, trans_a, trans_b));
  SM_REQUIRE(scratch_bytes >= 0 && (scratch || scratch_bytes == 0) &&
                 reinterpret_cast<uintptr_t>(scratch) % 16 == 0,
             "sm_gemm_planes_ws: bad scratch");
  if (M == 0 || N == 0) return SM_OK;
  return gemm_planes(planes, trans_a != 0, trans_b != 0, M, N, K, alpha, A, lda, B, ldb, beta, C,
                     ldc, as_stream(stream), static_cast<float*>(scratch), scratch_bytes / 4,
                     b_planes == 2 ? 2 : 3);
}
