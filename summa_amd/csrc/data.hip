// Seeded synthetic inputs generated on the device (bench and test data).
// Every value is a pure function of (seed, flat index) through the counter
// RNG in common.hpp, so any launch shape produces the same tensor. Parity
// tests copy the generated tensor to the host for the CPU oracle.
#include <cmath>

#include "common.hpp"

namespace sm {
namespace {

// Box-Muller on two 24-bit uniforms drawn from the key (seed, index).
__device__ inline float normal_at(uint64_t seed, int64_t i) {
  const uint64_t a = rng_key(seed, 0, (uint64_t)i);
  const float u1 = u01(a);
  const float u2 = u01(a << 24);
  return sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

__global__ void fill_normal_kernel(void* out, int dtype, int64_t n, float mean, float std,
                                   uint64_t seed) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = mean + std * normal_at(seed, i);
    if (dtype == SM_BF16) static_cast<uint16_t*>(out)[i] = f32_to_bf16(v);
    else if (dtype == SM_F16) static_cast<_Float16*>(out)[i] = (_Float16)v;
    else static_cast<float*>(out)[i] = v;
  }
}

__global__ void ce_spike_kernel(void* logits, int dtype, int32_t* targets, int64_t rows,
                                int64_t vocab, float spike, uint64_t seed) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int32_t t = (int32_t)(rng_key(seed, 1, (uint64_t)r) % (uint64_t)vocab);
  targets[r] = t;
  const int64_t i = r * vocab + t;
  if (dtype == SM_BF16) {
    uint16_t* p = static_cast<uint16_t*>(logits);
    p[i] = f32_to_bf16(bf16_to_f32(p[i]) + spike);
  } else {
    static_cast<float*>(logits)[i] += spike;
  }
}

int fill_grid(int64_t n) {
  int64_t blocks = ceil_div(n, 256);
  return (int)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace
}  // namespace sm

extern "C" int sm_fill_normal(void* out, int dtype, int64_t n, float mean, float std,
                              uint64_t seed, void* stream) {
  using namespace sm;
  SM_REQUIRE(out || n == 0, "sm_fill_normal: null output");
  SM_REQUIRE(dtype == SM_F32 || dtype == SM_BF16 || dtype == SM_F16, "sm_fill_normal: bad dtype");
  SM_REQUIRE(n >= 0, "sm_fill_normal: negative size");
  if (n == 0) return SM_OK;
  fill_normal_kernel<<<fill_grid(n), 256, 0, as_stream(stream)>>>(out, dtype, n, mean, std, seed);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" int sm_fill_ce_stress(void* logits, int dtype, int32_t* targets, int64_t rows,
                                 int64_t vocab, float std, float spike, uint64_t seed,
                                 void* stream) {
  using namespace sm;
  SM_REQUIRE(logits && targets, "sm_fill_ce_stress: null buffers");
  SM_REQUIRE(dtype == SM_F32 || dtype == SM_BF16, "sm_fill_ce_stress: bad dtype");
  SM_REQUIRE(rows >= 0 && vocab > 0, "sm_fill_ce_stress: bad shape");
  SM_TRY(sm_fill_normal(logits, dtype, rows * vocab, 0.f, std, seed, stream));
  if (rows == 0) return SM_OK;
  ce_spike_kernel<<<(unsigned)ceil_div(rows, 256), 256, 0, as_stream(stream)>>>(
      logits, dtype, targets, rows, vocab, spike, seed);
  SM_LAUNCH_CHECK();
  return SM_OK;
}
