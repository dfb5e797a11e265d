// MoE training kernels: the token gather and its backward, the weighted
// combine's backward to the routed rows and to the routing weights, and the
// fused SwiGLU forward / backward over [gate | value] rows (route_gather_*,
// route_combine_*, summa-llm/src/model/moe_dispatch.rs:244-384;
// swiglu_forward / swiglu_backward, fused_swiglu.rs:106-150). Elementwise
// kernels are HBM-bound (one thread per output element, f32 arithmetic); the
// weight gradient is one workgroup per route reducing a d-long dot product.
// Tensors are f32 or bf16 (the reference's F: Float), routing weights f32;
// route order / inverse come from the sm_moe_route_plan buffer.
#include <cmath>

#include "common.hpp"
#include "moe_plan.hpp"

namespace sm {
namespace {

template <typename T>
__device__ inline float ld(const T* p, int64_t i);
template <>
__device__ inline float ld<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ inline float ld<uint16_t>(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
template <typename T>
__device__ inline void st(T* p, int64_t i, float v);
template <>
__device__ inline void st<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ inline void st<uint16_t>(uint16_t* p, int64_t i, float v) { p[i] = f32_to_bf16(v); }

// routed[p] = x[order[p] / k] (route_gather_forward)
template <typename T>
__global__ void gather_kernel(const T* __restrict__ x, const int32_t* __restrict__ order,
                              int64_t routes, int k, int d, T* __restrict__ routed) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= routes * d) return;
  const int64_t p = i / d;
  const int c = (int)(i % d);
  const int64_t t = order[p] / k;
  routed[i] = x[t * d + c];
}

// grad_x[t] = sum_j grad_routed[inverse[t*k + j]] in route order
// (route_gather_backward); routes left out of the plan (inverse < 0) add 0
template <typename T>
__global__ void gather_backward_kernel(const T* __restrict__ grad, const int32_t* __restrict__ inverse,
                                       int64_t tokens, int k, int d, T* __restrict__ grad_x) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tokens * d) return;
  const int64_t t = i / d;
  const int c = (int)(i % d);
  float sum = 0.f;
  for (int j = 0; j < k; ++j) {
    const int p = inverse[t * k + j];
    if (p >= 0) sum += ld(grad, (int64_t)p * d + c);
  }
  st(grad_x, i, sum);
}

// grad_routed[inverse[r]] = grad_x[r / k] * w[r] (route_combine_routed_backward)
template <typename T>
__global__ void combine_routed_backward_kernel(const float* __restrict__ w,
                                               const int32_t* __restrict__ inverse,
                                               const T* __restrict__ grad_x, int64_t routes, int k,
                                               int d, T* __restrict__ grad_routed) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= routes * d) return;
  const int64_t r = i / d;
  const int c = (int)(i % d);
  const int p = inverse[r];
  if (p < 0) return;
  st(grad_routed, (int64_t)p * d + c, ld(grad_x, (r / k) * d + c) * w[r]);
}

// grad_w[r] = <grad_x[r / k], routed[inverse[r]]> (route_combine_weight_backward):
// one workgroup per route, lane-strided partial sums, then a fixed tree.
constexpr int kWT = 256;
template <typename T>
__global__ __launch_bounds__(kWT) void combine_weight_backward_kernel(
    const T* __restrict__ routed, const int32_t* __restrict__ inverse, const T* __restrict__ grad_x,
    int k, int d, float* __restrict__ grad_w) {
  __shared__ float red[kWT / kWave];
  const int64_t r = blockIdx.x;
  const int p = inverse[r];
  float part = 0.f;
  if (p >= 0) {
    const int64_t t = r / k;
    for (int c = threadIdx.x; c < d; c += kWT)
      part += ld(grad_x, t * d + c) * ld(routed, (int64_t)p * d + c);
  }
  part = wave_sum(part);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = part;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.f;
    for (int w = 0; w < kWT / kWave; ++w) s += red[w];
    grad_w[r] = s;
  }
}

// out[r, c] = silu(g) * v over [gate | value] rows (swiglu_forward)
template <typename T>
__global__ void swiglu_kernel(const T* __restrict__ gv, int64_t rows, int F, T* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * F) return;
  const int64_t r = i / F;
  const int c = (int)(i % F);
  const float g = ld(gv, r * 2 * F + c), v = ld(gv, r * 2 * F + F + c);
  const float sg = 1.f / (1.f + expf(-g));
  st(out, i, g * sg * v);
}

// d gate = dy * v * sigma(g) (1 + g (1 - sigma(g))), d value = dy * silu(g)
// (swiglu_backward)
template <typename T>
__global__ void swiglu_backward_kernel(const T* __restrict__ gv, const T* __restrict__ grad,
                                       int64_t rows, int F, T* __restrict__ grad_gv) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * F) return;
  const int64_t r = i / F;
  const int c = (int)(i % F);
  const int64_t gi = r * 2 * F + c, vi = gi + F;
  const float g = ld(gv, gi), v = ld(gv, vi), dy = ld(grad, i);
  const float sg = 1.f / (1.f + expf(-g));
  st(grad_gv, gi, dy * v * (sg * (1.f + g * (1.f - sg))));
  st(grad_gv, vi, dy * (g * sg));
}

inline unsigned grid_for(int64_t n) { return (unsigned)ceil_div(n, 256); }

int check_dtype(int dtype, const char* who) {
  SM_REQUIRE(dtype == SM_F32 || dtype == SM_BF16, "%s: dtype must be SM_F32 or SM_BF16", who);
  return SM_OK;
}

}  // namespace
}  // namespace sm

using namespace sm;

extern "C" int sm_moe_gather(const void* x, int dtype, const int32_t* plan, int64_t tokens,
                             int64_t top_k, int64_t experts, int64_t d, void* routed,
                             void* stream) {
  SM_REQUIRE(x && plan && routed, "sm_moe_gather: null buffer");
  SM_REQUIRE(tokens >= 0 && top_k >= 1 && experts >= 1 && d > 0, "sm_moe_gather: bad shape");
  SM_TRY(check_dtype(dtype, "sm_moe_gather"));
  const int64_t routes = tokens * top_k;
  if (routes == 0) return SM_OK;
  PlanView pv = plan_view(const_cast<int32_t*>(plan), routes, experts);
  hipStream_t st = as_stream(stream);
  if (dtype == SM_F32)
    gather_kernel<float><<<grid_for(routes * d), 256, 0, st>>>(
        (const float*)x, pv.order, routes, (int)top_k, (int)d, (float*)routed);
  else
    gather_kernel<uint16_t><<<grid_for(routes * d), 256, 0, st>>>(
        (const uint16_t*)x, pv.order, routes, (int)top_k, (int)d, (uint16_t*)routed);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_moe_gather_backward(const void* grad_routed, int dtype, const int32_t* plan,
                                      int64_t tokens, int64_t top_k, int64_t experts, int64_t d,
                                      void* grad_x, void* stream) {
  SM_REQUIRE(grad_routed && plan && grad_x, "sm_moe_gather_backward: null buffer");
  SM_REQUIRE(tokens >= 0 && top_k >= 1 && experts >= 1 && d > 0,
             "sm_moe_gather_backward: bad shape");
  SM_TRY(check_dtype(dtype, "sm_moe_gather_backward"));
  if (tokens == 0) return SM_OK;
  PlanView pv = plan_view(const_cast<int32_t*>(plan), tokens * top_k, experts);
  hipStream_t st = as_stream(stream);
  if (dtype == SM_F32)
    gather_backward_kernel<float><<<grid_for(tokens * d), 256, 0, st>>>(
        (const float*)grad_routed, pv.inverse, tokens, (int)top_k, (int)d, (float*)grad_x);
  else
    gather_backward_kernel<uint16_t><<<grid_for(tokens * d), 256, 0, st>>>(
        (const uint16_t*)grad_routed, pv.inverse, tokens, (int)top_k, (int)d, (uint16_t*)grad_x);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_moe_combine_backward(const void* grad_x, const void* routed, int dtype,
                                       const float* top_w, const int32_t* plan, int64_t tokens,
                                       int64_t top_k, int64_t experts, int64_t d,
                                       void* grad_routed, float* grad_w, void* stream) {
  SM_REQUIRE(grad_x && top_w && plan, "sm_moe_combine_backward: null buffer");
  SM_REQUIRE(!grad_w || routed, "sm_moe_combine_backward: weight gradient needs routed rows");
  SM_REQUIRE(tokens >= 0 && top_k >= 1 && experts >= 1 && d > 0,
             "sm_moe_combine_backward: bad shape");
  SM_TRY(check_dtype(dtype, "sm_moe_combine_backward"));
  const int64_t routes = tokens * top_k;
  if (routes == 0) return SM_OK;
  PlanView pv = plan_view(const_cast<int32_t*>(plan), routes, experts);
  hipStream_t st = as_stream(stream);
  if (grad_routed) {
    if (dtype == SM_F32)
      combine_routed_backward_kernel<float><<<grid_for(routes * d), 256, 0, st>>>(
          top_w, pv.inverse, (const float*)grad_x, routes, (int)top_k, (int)d,
          (float*)grad_routed);
    else
      combine_routed_backward_kernel<uint16_t><<<grid_for(routes * d), 256, 0, st>>>(
          top_w, pv.inverse, (const uint16_t*)grad_x, routes, (int)top_k, (int)d,
          (uint16_t*)grad_routed);
    SM_LAUNCH_CHECK();
  }
  if (grad_w) {
    SM_REQUIRE(routes <= 0x7fffffff, "sm_moe_combine_backward: too many routes");
    if (dtype == SM_F32)
      combine_weight_backward_kernel<float><<<(unsigned)routes, kWT, 0, st>>>(
          (const float*)routed, pv.inverse, (const float*)grad_x, (int)top_k, (int)d, grad_w);
    else
      combine_weight_backward_kernel<uint16_t><<<(unsigned)routes, kWT, 0, st>>>(
          (const uint16_t*)routed, pv.inverse, (const uint16_t*)grad_x, (int)top_k, (int)d,
          grad_w);
    SM_LAUNCH_CHECK();
  }
  return SM_OK;
}

extern "C" int sm_swiglu(const void* gate_value, int dtype, int64_t rows, int64_t F, void* out,
                         void* stream) {
  SM_REQUIRE(gate_value && out, "sm_swiglu: null buffer");
  SM_REQUIRE(rows >= 0 && F > 0, "sm_swiglu: bad shape");
  SM_TRY(check_dtype(dtype, "sm_swiglu"));
  if (rows == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  if (dtype == SM_F32)
    swiglu_kernel<float><<<grid_for(rows * F), 256, 0, st>>>((const float*)gate_value, rows,
                                                             (int)F, (float*)out);
  else
    swiglu_kernel<uint16_t><<<grid_for(rows * F), 256, 0, st>>>((const uint16_t*)gate_value,
                                                                rows, (int)F, (uint16_t*)out);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_swiglu_backward(const void* gate_value, const void* grad, int dtype,
                                  int64_t rows, int64_t F, void* grad_gate_value, void* stream) {
  SM_REQUIRE(gate_value && grad && grad_gate_value, "sm_swiglu_backward: null buffer");
  SM_REQUIRE(rows >= 0 && F > 0, "sm_swiglu_backward: bad shape");
  SM_TRY(check_dtype(dtype, "sm_swiglu_backward"));
  if (rows == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  if (dtype == SM_F32)
    swiglu_backward_kernel<float><<<grid_for(rows * F), 256, 0, st>>>(
        (const float*)gate_value, (const float*)grad, rows, (int)F, (float*)grad_gate_value);
  else
    swiglu_backward_kernel<uint16_t><<<grid_for(rows * F), 256, 0, st>>>(
        (const uint16_t*)gate_value, (const uint16_t*)grad, rows, (int)F,
        (uint16_t*)grad_gate_value);
  SM_LAUNCH_CHECK();
  return SM_OK;
}
