// f32 GEMM on the bf16 matrix cores, for the policy update's large matmuls
// (the forward with activations kept, every data and weight gradient, Muon's
// Newton-Schulz): C = alpha op(A) op(B) + beta C with op = identity or
// transpose, f32 in and out, any shape and leading dimensions. The reference
// trains through Burn's matmul (summa-llm/src/model/matmul.rs:132-143; bf16
// operands on its CUDA path, f32 on its CPU path); this keeps f32 results.
//
// Each f32 operand value is split exactly into three bf16 planes,
// x = x0 + x1 + x2 (round to nearest even at each step: 24 significant bits,
// f32's own precision; bf16 has f32's exponent range, so no scaling is
// needed), and a product x y is the sum of the six plane products of weight
// >= 2^-16 relative (x2 y0, x1 y1, x0 y2, x1 y0, x0 y1, x0 y0, smallest
// first), accumulated in f32 by v_mfma_f32_32x32x16_bf16. The dropped terms
// (x1 y2, x2 y1, x2 y2) are below 2^-23 relative, so the result is an f32
// GEMM's up to the order of its f32 additions.
//
// Workgroup = 128 x 128 output tile, 4 waves of 64 x 64 (2 x 2 blocks of
// 32 x 32); K in steps of 32. Each thread holds 16 consecutive k of one row
// of each operand tile (16-byte loads when k is the contiguous dimension,
// else scalar loads that are coalesced along the rows), splits them once into
// the three planes and stores them to LDS as [plane][row][k] bf16, rows
// padded to 40 elements so that the 16-byte writes and fragment reads of
// consecutive rows spread over the banks; the next step's loads are in
// flight while the current step's MFMAs run. One LDS buffer (60 KB), two
// workgroups per CU. Per 16-k slice a wave reads its 2 + 2 fragments of each
// plane and issues the 24 MFMAs product by product across its four blocks,
// so four independent accumulations separate two dependent ones.
#include "common.hpp"

namespace sm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 128, kBK = 32, kRS = kBK + 8;  // tile rows, k per step, LDS row stride
constexpr int kPlane = kBM * kRS;                   // bf16 per plane of one operand tile

// (a, b) -> bf16 planes with v = p0 + p1 + p2 exactly (finite v), as packed
// words (a in the low half).
__device__ inline void split3x2(float a, float b, uint32_t& p0, uint32_t& p1, uint32_t& p2) {
  p0 = pack_bf16x2(a, b);
  const float ra = a - bf16lo(p0), rb = b - bf16hi(p0);
  p1 = pack_bf16x2(ra, rb);
  p2 = pack_bf16x2(ra - bf16lo(p1), rb - bf16hi(p1));
}

// 8 consecutive k of one row -> the three planes at LDS offset o (16 bytes each)
__device__ inline void store8(const float* v, __bf16* lds, int o) {
  u32x4 w0, w1, w2;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t x0, x1, x2;
    split3x2(v[2 * i], v[2 * i + 1], x0, x1, x2);
    w0[i] = x0; w1[i] = x1; w2[i] = x2;
  }
  *reinterpret_cast<u32x4*>(lds + o) = w0;
  *reinterpret_cast<u32x4*>(lds + kPlane + o) = w1;
  *reinterpret_cast<u32x4*>(lds + 2 * kPlane + o) = w2;
}

// One operand tile (128 rows x 32 k) of X, element (r, k) at X[r * ld + k]
// when KC (k contiguous), else at X[k * ld + r]; 16 values per thread.
// Thread t: 16 consecutive k of one row, v[i] = (row, k + i): KC: row t / 2,
// k 16 (t % 2) (four 16-byte loads); otherwise row t % 128, k 16 (t / 128)
// (one scalar load per k, each instruction 64 consecutive rows). Out-of-range
// elements are 0.
template <bool KC>
struct TileLoader {
  const float* X;
  int64_t ld;
  int r0, R, K;
  bool vec;  // aligned vectors along the contiguous dimension (uniform)
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
  // this thread's values as three planes into the LDS tile [plane][row][k]
  __device__ inline void store(const float (&v)[16], __bf16* lds) const {
    store8(v, lds, ra * kRS + ka);
    store8(v + 8, lds, ra * kRS + ka + 8);
  }
};

template <bool TA, bool TB>
__global__ __launch_bounds__(256, 2) void gemm_bf16x3_kernel(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ B, int64_t ldb,
    float* __restrict__ C, int64_t ldc, int M, int N, int K, float alpha, float beta, int vec_a,
    int vec_b) {
  __shared__ __attribute__((aligned(16))) __bf16 As[3 * kPlane];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[3 * kPlane];
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
  la.store(va, As);
  lb.store(vb, Bs);
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
      bf16x8 a[3][2], b[3][2];
#pragma unroll
      for (int p = 0; p < 3; ++p)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          a[p][i] = *reinterpret_cast<const bf16x8*>(As + p * kPlane + (wm * 64 + i * 32) * kRS +
                                                     fo + ks);
          b[p][i] = *reinterpret_cast<const bf16x8*>(Bs + p * kPlane + (wn * 64 + i * 32) * kRS +
                                                     fo + ks);
        }
      // plane pairs (pa, pb), smallest weight first
      constexpr int PA[6] = {2, 1, 0, 1, 0, 0}, PB[6] = {0, 1, 2, 0, 1, 0};
#pragma unroll
      for (int q = 0; q < 6; ++q)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[PA[q]][i], b[PB[q]][j],
                                                                 acc[i][j], 0, 0, 0);
    }
    if (more) {
      __syncthreads();  // every wave is done with this step's tiles
      la.store(va, As);
      lb.store(vb, Bs);
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

}  // namespace

int gemm_bf16x3(bool ta, bool tb, int64_t M, int64_t N, int64_t K, float alpha, const float* A,
                int64_t lda, const float* B, int64_t ldb, float beta, float* C, int64_t ldc,
                hipStream_t st) {
  // 16-byte loads along k need aligned rows (op(A) rows of an untransposed
  // A, op(B) columns of a transposed B)
  auto aligned = [](const float* p, int64_t ld) {
    return ld % 4 == 0 && reinterpret_cast<uintptr_t>(p) % 16 == 0 ? 1 : 0;
  };
  const int vec_a = !ta && aligned(A, lda), vec_b = tb && aligned(B, ldb);
  const dim3 grid((unsigned)ceil_div(N, kBM), (unsigned)ceil_div(M, kBM));
#define SM_GB(TA, TB)                                                                          \
  gemm_bf16x3_kernel<TA, TB><<<grid, 256, 0, st>>>(A, lda, B, ldb, C, ldc, (int)M, (int)N,     \
                                                   (int)K, alpha, beta, vec_a, vec_b)
  if (ta && tb) SM_GB(true, true);
  else if (ta) SM_GB(true, false);
  else if (tb) SM_GB(false, true);
  else SM_GB(false, false);
#undef SM_GB
  SM_LAUNCH_CHECK();
  return SM_OK;
}

}  // namespace sm

extern "C" int sm_gemm_mfma(int trans_a, int trans_b, int64_t M, int64_t N, int64_t K,
                            float alpha, const float* A, int64_t lda, const float* B, int64_t ldb,
                            float beta, float* C, int64_t ldc, void* stream) {
  using namespace sm;
  SM_REQUIRE(A && B && C, "sm_gemm_mfma: null buffer");
  SM_REQUIRE(M >= 0 && N >= 0 && K >= 0 && M < (1 << 30) && N < (1 << 30) && K < (1 << 30),
             "sm_gemm_mfma: bad shape");
  SM_REQUIRE(lda >= (trans_a ? M : K) && ldb >= (trans_b ? K : N) && ldc >= N,
             "sm_gemm_mfma: leading dimension too small");
  if (M == 0 || N == 0) return SM_OK;
  SM_REQUIRE(K > 0, "sm_gemm_mfma: K must be positive");
  SM_REQUIRE(ceil_div(M, 128) <= 65535, "sm_gemm_mfma: M above 65535 x 128 rows");
  return gemm_bf16x3(trans_a != 0, trans_b != 0, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc,
                     as_stream(stream));
}
