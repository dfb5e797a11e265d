// Dense fp32 matmul y = x . W^T for fp32 models (config[0]: the reference CPU
// path's precision, summa-llm/src/model/matmul.rs:57-66 with F32 weights),
// plus the SwiGLU combine of a [gate | value] projection (ffn.rs:854-886).
//
// Tiled 64x64 output per 256-thread workgroup, 4x4 outputs per thread, K in
// steps of 32 through two LDS buffers: the next step's tiles are loaded into
// registers before the current step's math and stored to the other buffer
// after it, so each step's global loads overlap a step of FMAs (one barrier
// per step). Used for the tiny fp32 model, where a launch has only a handful
// of workgroups and a load round trip per K step would set the pace; the
// quantized path uses q4.hip.
#include "common.hpp"

namespace sm {
namespace {

template <bool ADD>
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ w,
                                                       const float* __restrict__ x,
                                                       float* __restrict__ y, int M, int N,
                                                       int K, int ldx, int ldy) {
  constexpr int KT = 32;
  __shared__ float xs[2][KT][64 + 4];
  __shared__ float ws[2][KT][64 + 4];
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
  // loader: element e = i * 256 + t of a 64 x 32 tile is row e / 32, k e % 32
  float rx[8], rw[8];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = i * 256 + threadIdx.x, r = e / KT, kk = e % KT;
      const int gm = m0 + r, gn = n0 + r, gk = k0 + kk;
      rx[i] = (gm < M && gk < K) ? x[(size_t)gm * ldx + gk] : 0.f;
      rw[i] = (gn < N && gk < K) ? w[(size_t)gn * K + gk] : 0.f;
    }
  };
  auto lstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int e = i * 256 + threadIdx.x, r = e / KT, kk = e % KT;
      xs[buf][kk][r] = rx[i];
      ws[buf][kk][r] = rw[i];
    }
  };
  float acc[4][4] = {};
  gload(0);
  lstore(0);
  __syncthreads();
  for (int k0 = 0, buf = 0; k0 < K; k0 += KT, buf ^= 1) {
    const bool more = k0 + KT < K;  // uniform
    if (more) gload(k0 + KT);
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) { a[i] = xs[buf][kk][ty * 4 + i]; b[i] = ws[buf][kk][tx * 4 + i]; }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[i][jj] = fmaf(a[i], b[jj], acc[i][jj]);
    }
    if (more) lstore(buf ^ 1);  // the other buffer was last read before the previous barrier
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int gm = m0 + ty * 4 + i;
    if (gm >= M) continue;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int gn = n0 + tx * 4 + jj;
      if (gn >= N) continue;
      float* o = y + (size_t)gm * ldy + gn;
      if (ADD) *o += acc[i][jj]; else *o = acc[i][jj];
    }
  }
}

__global__ void swiglu_f32_kernel(const float* __restrict__ gv, int64_t rows, int F,
                                  float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * F) return;
  const int64_t r = i / F;
  const int c = i % F;
  const float g = gv[r * 2 * F + c], v = gv[r * 2 * F + F + c];
  out[i] = g / (1.f + expf(-g)) * v;
}

}  // namespace
}  // namespace sm

using namespace sm;

extern "C" int sm_gemm_f32(const float* w, int64_t N, int64_t K, const float* x, int64_t M,
                           int64_t ldx, float* y, int64_t ldy, int epilogue, void* stream) {
  SM_REQUIRE(w && x && y, "sm_gemm_f32: null buffer");
  SM_REQUIRE(N > 0 && K > 0 && M >= 0 && ldx >= K && ldy >= N, "sm_gemm_f32: bad shape");
  SM_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff, "sm_gemm_f32: shape too large");
  SM_REQUIRE(epilogue == SM_EPI_STORE_F32 || epilogue == SM_EPI_ADD_F32,
             "sm_gemm_f32: epilogue must be SM_EPI_STORE_F32 or SM_EPI_ADD_F32");
  if (M == 0) return SM_OK;
  const dim3 grid((unsigned)ceil_div(N, 64), (unsigned)ceil_div(M, 64));
  if (epilogue == SM_EPI_ADD_F32)
    gemm_f32_kernel<true><<<grid, 256, 0, as_stream(stream)>>>(w, x, y, (int)M, (int)N, (int)K,
                                                               (int)ldx, (int)ldy);
  else
    gemm_f32_kernel<false><<<grid, 256, 0, as_stream(stream)>>>(w, x, y, (int)M, (int)N, (int)K,
                                                                (int)ldx, (int)ldy);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_swiglu_f32(const float* gate_value, int64_t rows, int64_t F, float* out,
                             void* stream) {
  SM_REQUIRE(gate_value && out, "sm_swiglu_f32: null buffer");
  SM_REQUIRE(rows >= 0 && F > 0, "sm_swiglu_f32: bad shape");
  const int64_t n = rows * F;
  if (n == 0) return SM_OK;
  swiglu_f32_kernel<<<(unsigned)ceil_div(n, 256), 256, 0, as_stream(stream)>>>(gate_value, rows,
                                                                              (int)F, out);
  SM_LAUNCH_CHECK();
  return SM_OK;
}
