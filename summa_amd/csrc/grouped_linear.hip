// Float-weight grouped expert projections and the MoE row permutation at the
// reference's dispatch seam:
//   * GroupedLinearBackend::grouped_linear_inner / _backward
//     (summa-llm/src/model/grouped_linear.rs:23-60, 65-86): input [routes,
//     d_in] with its rows grouped by expert (counts[e] consecutive rows of
//     expert e, in expert order), weight [E, d_in, d_out] row-major, output
//     [routes, d_out] = each expert's rows times its matrix; the backward
//     gives grad_input = grad W_e^T per expert and grad_weight[e] =
//     input_e^T grad_e (zero for an expert without rows);
//   * grouped_swiglu_mlp_inner / _backward (grouped_linear.rs:40-60, 89-111,
//     779-826): projected = grouped_linear(input, in_weight) as [gate |
//     value] (fused_swiglu.rs:30-42), hidden = silu(gate) * value, output =
//     grouped_linear(hidden, down_weight); the backward chains the two
//     grouped backwards through the SwiGLU backward;
//   * RowPermutationBackend::row_permute_inner (row_permute.rs:33-41): out[i]
//     = input[order[i]] (float_select over rows; the backward is the same
//     selection by the inverse permutation).
// The counts are host values, as grouped_linear_inner takes them (Vec<usize>;
// the CUDA path reads device counts back to the host before its grouped GEMM,
// grouped_linear.rs:787). Each expert with rows is one f32-grade GEMM
// (sm_gemm_ex: the three-plane bf16 matrix-core kernel from 2^27
// multiply-adds, the f32 FMA kernel below), in expert order on the stream.
#include "common.hpp"

extern "C" {
int sm_gemm_ex(int, int, int64_t, int64_t, int64_t, float, const float*, int64_t, const float*,
               int64_t, float, float*, int64_t, void*);
int sm_swiglu(const void*, int, int64_t, int64_t, void*, void*);
int sm_swiglu_backward(const void*, const void*, int, int64_t, int64_t, void*, void*);
}

namespace sm {
namespace {

// out row i = in row order[i] (16-byte chunks when rows allow, else 4-byte
// words or 2-byte elements); an order entry outside [0, rows) gives a zero row.
template <typename T>
__global__ __launch_bounds__(256) void row_permute_kernel(const T* __restrict__ in,
                                                          const int32_t* __restrict__ order,
                                                          int64_t rows, int64_t units,
                                                          T* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * units) return;
  const int64_t r = i / units, u = i % units;
  const int32_t src = order[r];
  T v{};
  if (src >= 0 && src < rows) v = in[(int64_t)src * units + u];
  out[i] = v;
}

__global__ void zero_f32_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

int check_counts(const int64_t* counts, int64_t experts, int64_t routes, const char* who) {
  SM_REQUIRE(counts, "%s: null counts", who);
  int64_t sum = 0;
  for (int64_t e = 0; e < experts; ++e) {
    SM_REQUIRE(counts[e] >= 0, "%s: negative count for expert %lld", who, (long long)e);
    sum += counts[e];
  }
  SM_REQUIRE(sum == routes, "%s: route counts must cover the input (%lld != %lld)", who,
             (long long)sum, (long long)routes);
  return SM_OK;
}

// y = x W_e per expert (x rows grouped by expert, W [E, d_in, d_out])
int grouped_forward(const float* x, const float* w, const int64_t* counts, int64_t experts,
                    int64_t d_in, int64_t d_out, float* y, void* stream) {
  int64_t off = 0;
  for (int64_t e = 0; e < experts; ++e) {
    const int64_t c = counts[e];
    if (c > 0)
      SM_TRY(sm_gemm_ex(0, 0, c, d_out, d_in, 1.f, x + off * d_in, d_in,
                        w + e * d_in * d_out, d_out, 0.f, y + off * d_out, d_out, stream));
    off += c;
  }
  return SM_OK;
}

// grad_x = grad W_e^T; grad_w[e] = x_e^T grad_e (zero without rows)
int grouped_backward(const float* x, const float* w, const float* grad, const int64_t* counts,
                     int64_t experts, int64_t d_in, int64_t d_out, float* grad_x, float* grad_w,
                     void* stream) {
  hipStream_t st = as_stream(stream);
  int64_t off = 0;
  for (int64_t e = 0; e < experts; ++e) {
    const int64_t c = counts[e];
    float* gw = grad_w ? grad_w + e * d_in * d_out : nullptr;
    if (c > 0) {
      if (grad_x)
        SM_TRY(sm_gemm_ex(0, 1, c, d_in, d_out, 1.f, grad + off * d_out, d_out,
                          w + e * d_in * d_out, d_out, 0.f, grad_x + off * d_in, d_in, stream));
      if (gw)
        SM_TRY(sm_gemm_ex(1, 0, d_in, d_out, c, 1.f, x + off * d_in, d_in, grad + off * d_out,
                          d_out, 0.f, gw, d_out, stream));
    } else if (gw) {
      zero_f32_kernel<<<(unsigned)ceil_div(d_in * d_out, 256), 256, 0, st>>>(gw, d_in * d_out);
      SM_LAUNCH_CHECK();
    }
    off += c;
  }
  return SM_OK;
}

}  // namespace
}  // namespace sm

using namespace sm;

extern "C" int sm_row_permute(const void* input, int dtype, int64_t rows, int64_t cols,
                              const int32_t* order, void* out, void* stream) {
  SM_REQUIRE(input && order && out, "sm_row_permute: null buffer");
  SM_REQUIRE(rows >= 0 && cols > 0, "sm_row_permute: bad shape");
  SM_REQUIRE(dtype == SM_F32 || dtype == SM_BF16 || dtype == SM_F16,
             "sm_row_permute: dtype must be SM_F32, SM_BF16 or SM_F16");
  SM_REQUIRE(input != out, "sm_row_permute: out must not alias input");
  if (rows == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  const int64_t bytes = cols * (dtype == SM_F32 ? 4 : 2);
  const bool a16 = bytes % 16 == 0 && reinterpret_cast<uintptr_t>(input) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0;
  const bool a4 = bytes % 4 == 0 && reinterpret_cast<uintptr_t>(input) % 4 == 0 &&
                  reinterpret_cast<uintptr_t>(out) % 4 == 0;
  if (a16) {
    const int64_t units = bytes / 16;
    row_permute_kernel<u32x4><<<(unsigned)ceil_div(rows * units, 256), 256, 0, st>>>(
        static_cast<const u32x4*>(input), order, rows, units, static_cast<u32x4*>(out));
  } else if (a4) {
    const int64_t units = bytes / 4;
    row_permute_kernel<uint32_t><<<(unsigned)ceil_div(rows * units, 256), 256, 0, st>>>(
        static_cast<const uint32_t*>(input), order, rows, units, static_cast<uint32_t*>(out));
  } else {
    const int64_t units = bytes / 2;
    row_permute_kernel<uint16_t><<<(unsigned)ceil_div(rows * units, 256), 256, 0, st>>>(
        static_cast<const uint16_t*>(input), order, rows, units, static_cast<uint16_t*>(out));
  }
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_grouped_linear(const float* input, const float* weight, const int64_t* counts,
                                 int64_t experts, int64_t routes, int64_t d_in, int64_t d_out,
                                 float* out, void* stream) {
  SM_REQUIRE(input && weight && out, "sm_grouped_linear: null buffer");
  SM_REQUIRE(experts > 0 && routes >= 0 && d_in > 0 && d_out > 0, "sm_grouped_linear: bad shape");
  SM_TRY(check_counts(counts, experts, routes, "sm_grouped_linear"));
  return grouped_forward(input, weight, counts, experts, d_in, d_out, out, stream);
}

extern "C" int sm_grouped_linear_backward(const float* input, const float* weight,
                                          const float* grad, const int64_t* counts,
                                          int64_t experts, int64_t routes, int64_t d_in,
                                          int64_t d_out, float* grad_input, float* grad_weight,
                                          void* stream) {
  SM_REQUIRE(input && weight && grad && (grad_input || grad_weight),
             "sm_grouped_linear_backward: null buffer");
  SM_REQUIRE(experts > 0 && routes >= 0 && d_in > 0 && d_out > 0,
             "sm_grouped_linear_backward: bad shape");
  SM_TRY(check_counts(counts, experts, routes, "sm_grouped_linear_backward"));
  return grouped_backward(input, weight, grad, counts, experts, d_in, d_out, grad_input,
                          grad_weight, stream);
}

extern "C" int sm_grouped_swiglu_mlp(const float* input, const float* in_weight,
                                     const float* down_weight, const int64_t* counts,
                                     int64_t experts, int64_t routes, int64_t d,
                                     int64_t intermediate, int64_t d_out, float* out,
                                     float* projected, float* hidden, void* stream) {
  SM_REQUIRE(input && in_weight && down_weight && out && projected && hidden,
             "sm_grouped_swiglu_mlp: null buffer");
  SM_REQUIRE(experts > 0 && routes >= 0 && d > 0 && intermediate > 0 && d_out > 0,
             "sm_grouped_swiglu_mlp: bad shape");
  SM_TRY(check_counts(counts, experts, routes, "sm_grouped_swiglu_mlp"));
  if (routes == 0) return SM_OK;
  SM_TRY(grouped_forward(input, in_weight, counts, experts, d, 2 * intermediate, projected,
                         stream));
  SM_TRY(sm_swiglu(projected, SM_F32, routes, intermediate, hidden, stream));
  return grouped_forward(hidden, down_weight, counts, experts, intermediate, d_out, out, stream);
}

extern "C" int sm_grouped_swiglu_mlp_backward(const float* input, const float* in_weight,
                                              const float* down_weight, const int64_t* counts,
                                              int64_t experts, int64_t routes, int64_t d,
                                              int64_t intermediate, int64_t d_out,
                                              const float* projected, const float* hidden,
                                              const float* grad, float* grad_input,
                                              float* grad_in_weight, float* grad_down_weight,
                                              float* scratch, void* stream) {
  SM_REQUIRE(input && in_weight && down_weight && projected && hidden && grad && grad_input &&
                 grad_in_weight && grad_down_weight && scratch,
             "sm_grouped_swiglu_mlp_backward: null buffer");
  SM_REQUIRE(experts > 0 && routes >= 0 && d > 0 && intermediate > 0 && d_out > 0,
             "sm_grouped_swiglu_mlp_backward: bad shape");
  SM_TRY(check_counts(counts, experts, routes, "sm_grouped_swiglu_mlp_backward"));
  // scratch: grad_hidden [routes, I] then grad_projected [routes, 2I]
  float* grad_hidden = scratch;
  float* grad_projected = scratch + routes * intermediate;
  SM_TRY(grouped_backward(hidden, down_weight, grad, counts, experts, intermediate, d_out,
                          grad_hidden, grad_down_weight, stream));
  if (routes > 0)
    SM_TRY(sm_swiglu_backward(projected, grad_hidden, SM_F32, routes, intermediate,
                              grad_projected, stream));
  return grouped_backward(input, in_weight, grad_projected, counts, experts, d,
                          2 * intermediate, grad_input, grad_in_weight, stream);
}
