// Many independent M = 1 Q4G128 GEMVs in one launch (sm_q4_gemv_multi): one
// decode-step Linear::forward (summa-llm/src/model/matmul.rs:57-66) per job,
// for callers that hold several matrices whose inputs are ready at once
// (independent projections, a whole-model weight sweep). A single launch
// removes the per-launch gap and the ramp-down tail of each small GEMV: the
// blocks of all jobs share one grid, so the weight stream never pauses.
//
// Workgroup = one 16-row block of one job (block_job[b] names the job, its
// first block is job.first_block), the four waves splitting the K groups
// (wave w: groups w, w + 4, ...) and merged in LDS in wave order; each wave
// copies only its own activation groups into LDS, weight groups are
// double-buffered in registers. The arithmetic per group (codes x
// activations over 4 k-steps of v_mfma_f32_16x16x32_f16, then one FMA with
// the group scale) and the merge order are q4.hip's M = 1 kernel's (its
// K-split form), so each job's result equals sm_q4_matmul at M = 1 bit for
// bit wherever that kernel splits K (K >= 512).
#include <algorithm>

#include "common.hpp"

namespace sm {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

template <int NA>
__global__ __launch_bounds__(256) void q4_gemv_multi_kernel(const sm_q4_gemv_job* __restrict__ jobs,
                                                            const int32_t* __restrict__ block_job,
                                                            int njobs, int max_k) {
  extern __shared__ _Float16 xs[];  // NA * K activations of the block's job (hi, then lo)
  __shared__ float red[4][16];
  const int b = blockIdx.x;
  const int ji = block_job[b];
  if (ji < 0 || ji >= njobs) return;  // uniform per workgroup
  const sm_q4_gemv_job jb = jobs[ji];
  const int K = (int)jb.K, ng = K / 128;
  const int nrb = (int)((jb.N + 15) / 16), rb = b - jb.first_block;
  if (K > max_k || rb < 0 || rb >= nrb) return;  // (a table that does not match the plan)
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int j = lane % 16, g = lane / 16, part = wave;
  const uint8_t* cb = jb.codes + q4t_code_offset((int64_t)rb * 16 + j, 0, ng) + g * 16;
  const uint16_t* sb = jb.scales + q4t_scale_index((int64_t)rb * 16 + j, 0, ng);
  auto load = [&](int kc, u32x4& w, uint16_t& sc) {
    kc = min(kc, ng - 1);
    w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(cb + (size_t)kc * 1024));
    sc = sb[kc * 16];
  };
  u32x4 w0, w1;
  uint16_t s0, s1;
  load(part, w0, s0);
  // this wave's K groups (part + 4i) of the activation row into their places
  // in LDS; only this wave reads them, so no workgroup barrier
  const _Float16* x = static_cast<const _Float16*>(jb.x);
  const int mine = (ng - part + 3) / 4;
  for (int c = lane; c < NA * mine * 16; c += kWave) {
    const int h = c / (mine * 16), i = (c / 16) % mine, ch = c % 16;
    const int off = h * K + (part + 4 * i) * 128 + ch * 8;
    *reinterpret_cast<h8*>(xs + off) = *reinterpret_cast<const h8*>(x + off);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float acc = 0.f;
  auto group = [&](int kg, const u32x4& w, uint16_t sc) {
    f4 t = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const h8 bq = q4_unpack(w[q]);
      const h8 ah = *reinterpret_cast<const h8*>(xs + kg * 128 + g * 32 + q * 8);
      t = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq, t, 0, 0, 0);
      if constexpr (NA == 2) {
        const h8 al = *reinterpret_cast<const h8*>(xs + K + kg * 128 + g * 32 + q * 8);
        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq, t, 0, 0, 0);
      }
    }
    acc = fmaf(t[0], bf16_to_f32(sc), acc);
  };
  for (int kb = part; kb < ng; kb += 8) {
    load(kb + 4, w1, s1);
    group(kb, w0, s0);
    if (kb + 4 >= ng) break;
    load(kb + 8, w0, s0);
    group(kb + 4, w1, s1);
  }
  if (g == 0) red[part][j] = acc;
  __syncthreads();
  if (part != 0 || g != 0) return;
  acc = red[0][j];
#pragma unroll
  for (int p = 1; p < 4; ++p) acc += red[p][j];
  const int64_t col = (int64_t)rb * 16 + j;
  if (col >= jb.N) return;
  if (jb.epilogue == SM_EPI_STORE_F32) static_cast<float*>(jb.y)[col] = acc;
  else if (jb.epilogue == SM_EPI_STORE_BF16) static_cast<uint16_t*>(jb.y)[col] = f32_to_bf16(acc);
  else static_cast<float*>(jb.y)[col] += acc;
}

}  // namespace
}  // namespace sm

extern "C" int64_t sm_q4_gemv_multi_plan(sm_q4_gemv_job* jobs, int64_t njobs, int32_t* block_job) {
  using namespace sm;
  clear_error();
  if (!jobs || njobs <= 0 || njobs > 0x7fffffff) {
    set_error("sm_q4_gemv_multi_plan: need a host array of >= 1 jobs");
    return -1;
  }
  int64_t total = 0;
  for (int64_t i = 0; i < njobs; ++i) {
    sm_q4_gemv_job& jb = jobs[i];
    if (!jb.codes || !jb.scales || !jb.x || !jb.y || jb.N <= 0 || jb.N > 0x7fffffff ||
        jb.K <= 0 || jb.K % 128 != 0 || jb.K > 0x7fffffff ||
        reinterpret_cast<uintptr_t>(jb.x) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(jb.codes) % 16 != 0 ||
        (jb.epilogue != SM_EPI_STORE_F32 && jb.epilogue != SM_EPI_STORE_BF16 &&
         jb.epilogue != SM_EPI_ADD_F32)) {
      set_error("sm_q4_gemv_multi_plan: job %lld: non-null 16-byte aligned codes / x, N > 0, "
                "K a positive multiple of 128, epilogue store f32 / bf16 or add f32",
                (long long)i);
      return -1;
    }
    const int64_t nrb = (jb.N + 15) / 16;
    if (total + nrb > 0x7fffffff) {
      set_error("sm_q4_gemv_multi_plan: too many row blocks");
      return -1;
    }
    jb.first_block = (int32_t)total;
    if (block_job)
      for (int64_t r = 0; r < nrb; ++r) block_job[total + r] = (int32_t)i;
    total += nrb;
  }
  return total;
}

extern "C" int sm_q4_gemv_multi(const sm_q4_gemv_job* jobs, int64_t njobs, const int32_t* block_job,
                                int64_t nblocks, int64_t max_k, int x_dtype, void* stream) {
  using namespace sm;
  SM_REQUIRE(jobs && block_job, "sm_q4_gemv_multi: null job table");
  SM_REQUIRE(njobs > 0 && njobs <= 0x7fffffff && nblocks >= 0 && nblocks <= 0x7fffffff,
             "sm_q4_gemv_multi: bad job / block count");
  SM_REQUIRE(x_dtype == SM_F16 || x_dtype == SM_F16X2,
             "sm_q4_gemv_multi: x must be f16 or f16 pairs");
  const int na = x_dtype == SM_F16X2 ? 2 : 1;
  SM_REQUIRE(max_k > 0 && max_k % 128 == 0 && (int64_t)na * max_k * 2 <= 65536,
             "sm_q4_gemv_multi: max_k must be a positive multiple of 128 with the activation row "
             "within 64 KB of LDS");
  if (nblocks == 0) return SM_OK;
  hipStream_t st = as_stream(stream);
  const size_t lds = (size_t)na * max_k * 2;
  if (na == 2)
    q4_gemv_multi_kernel<2><<<(unsigned)nblocks, 256, lds, st>>>(jobs, block_job, (int)njobs,
                                                                 (int)max_k);
  else
    q4_gemv_multi_kernel<1><<<(unsigned)nblocks, 256, lds, st>>>(jobs, block_job, (int)njobs,
                                                                 (int)max_k);
  SM_LAUNCH_CHECK();
  return SM_OK;
}
