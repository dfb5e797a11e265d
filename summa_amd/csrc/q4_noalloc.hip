// sm_q4_matmul_noalloc: the Q4G128 matmul with its split-K partials in a
// library-owned static device array, for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc). It has no counterpart in the reference.
//
// `scratch` below is the array. In host code its name is only a host-side
// stand-in: the device address comes from hipGetSymbolAddress, taken once per
// device on the first call made with that device current, and only that
// address is ever handed to kernels. Every call on one GPU shares that GPU's
// array; the split-K partials are fully rewritten by each call before they
// are read, so nothing needs clearing, but calls that overlap on one GPU (two
// streams at once) race.
#include <mutex>

#include "common.hpp"

extern "C" int64_t sm_q4_matmul_workspace_bytes(int64_t, int64_t, int64_t, int);
extern "C" int sm_q4_matmul_ws(const uint8_t*, const uint16_t*, int64_t, int64_t, const void*,
                               int, int64_t, int64_t, void*, int64_t, int, void*, int64_t, void*);

namespace sm {
namespace {

static __device__ __align__(256) float scratch[SM_Q4_NOALLOC_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device id

// The current device's address of `scratch` (looked up once per device).
int scratch_address(void** out) {
  int dev = 0;
  SM_HIP(hipGetDevice(&dev));
  SM_REQUIRE(dev >= 0 && dev < kMaxDevices, "sm_q4_matmul_noalloc: device id %d >= %d", dev,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    SM_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    SM_REQUIRE(p != nullptr, "sm_q4_matmul_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SM_OK;
}

}  // namespace
}  // namespace sm

extern "C" int64_t sm_q4_noalloc_scratch_bytes(void) { return SM_Q4_NOALLOC_SCRATCH_BYTES; }

extern "C" int sm_q4_matmul_noalloc(const uint8_t* codes, const uint16_t* scales, int64_t N,
                                    int64_t K, const void* x, int x_dtype, int64_t M, int64_t ldx,
                                    void* y, int64_t ldy, int epilogue, void* stream) {
  using namespace sm;
  const int64_t need = sm_q4_matmul_workspace_bytes(M, N, K, epilogue);
  SM_REQUIRE(need <= SM_Q4_NOALLOC_SCRATCH_BYTES,
             "sm_q4_matmul_noalloc: M=%lld x N=%lld needs %lld bytes of split-K scratch; the "
             "static scratch holds %lld (use sm_q4_matmul_ws with a workspace)",
             (long long)M, (long long)N, (long long)need,
             (long long)SM_Q4_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  SM_TRY(scratch_address(&ws));
  return sm_q4_matmul_ws(codes, scales, N, K, x, x_dtype, M, ldx, y, ldy, epilogue,
                         need > 0 ? ws : nullptr, need, stream);
}
