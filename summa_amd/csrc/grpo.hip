// GRPO clipped policy-gradient + k3-KL loss (kernel 4), batched over groups.
//
// Follows the scalar oracle grpo_loss (summa-train/src/posttrain.rs:720-868)
// and the masked tensor core grpo_loss_tensor (posttrain.rs:874-1028):
//   A_i   = (r_i - mean) / max(sqrt(pop. variance), eps_adv)
//   rho   = exp(lp - lp_beh)                       (log-ratio must be <= 80)
//   surr  = min(rho*A, clamp(rho, 1-eps, 1+eps)*A)
//   kl    = exp(lp_ref - lp) - (lp_ref - lp) - 1   (k3 estimator)
//   loss  = -mean_i [ sum_t mask*(surr - beta*kl) / L_i ]
//   dL/dlp = (1/G)(1/L_i) (-[active]*rho*A + beta*(1 - exp(lp_ref - lp)))
// with active <=> (A >= 0 and rho <= 1+eps) or (A < 0 and rho >= 1-eps)
// (posttrain.rs:839-845) and clipped <=> surr == clipped surr and rho != clip(rho)
// (posttrain.rs:816-818).
//
// One workgroup per prompt group, one wave per rollout; all reductions are in
// f64 and in a fixed order, so results are deterministic. The work is tiny
// (config[2]: 131072 tokens), so the kernel is latency-bound by design.
#include <cmath>

#include "common.hpp"

namespace sm {
namespace {

constexpr int kThreads = 512;
constexpr int kMaxGroup = 1024;

__device__ inline bool finite(double v) { return isfinite(v); }

__global__ __launch_bounds__(kThreads) void grpo_kernel(
    const float* __restrict__ rewards, const float* __restrict__ lp_cur,
    const float* __restrict__ lp_beh, const float* __restrict__ lp_ref,
    const float* __restrict__ mask, int G, int64_t T, double clip, double adv_eps, double beta,
    float* __restrict__ stats, float* __restrict__ adv_out, float* __restrict__ dlp,
    int32_t* __restrict__ flags_out) {
  __shared__ double s_adv[kMaxGroup];
  __shared__ double s_obj[kMaxGroup];
  __shared__ double s_kl[kMaxGroup];
  __shared__ double s_clip[kMaxGroup];
  __shared__ double s_cnt[kMaxGroup];
  __shared__ double s_mean, s_std;
  __shared__ int s_flags;

  const int64_t g = blockIdx.x;
  const float* r = rewards + g * G;
  const int64_t base = g * (int64_t)G * T;
  if (threadIdx.x == 0) {
    int f = 0;
    // Sequential sums in rollout order, as grpo_loss does.
    double sum = 0.0;
    for (int i = 0; i < G; ++i) {
      if (!finite(r[i])) f |= SM_GRPO_BAD_REWARD;
      sum += (double)r[i];
    }
    const double mean = sum / G;
    double var = 0.0;
    for (int i = 0; i < G; ++i) {
      const double c = (double)r[i] - mean;
      var += c * c;
    }
    var /= G;
    if (!finite(mean) || !finite(var)) f |= SM_GRPO_REWARD_OVERFLOW;
    const double sd = sqrt(var);
    const double den = fmax(sd, adv_eps);
    for (int i = 0; i < G; ++i) s_adv[i] = ((double)r[i] - mean) / den;
    s_mean = mean;
    s_std = sd;
    s_flags = f;
  }
  __syncthreads();

  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int nwaves = kThreads / kWave;
  const double lower = 1.0 - clip, upper = 1.0 + clip;
  int f = 0;
  for (int i = wave; i < G; i += nwaves) {
    const int64_t off = base + (int64_t)i * T;
    // Active-token count of this rollout.
    double cnt = 0.0;
    for (int64_t t = lane; t < T; t += kWave) {
      const float mk = mask ? mask[off + t] : 1.f;
      if (!(mk == 0.f || mk == 1.f)) f |= SM_GRPO_MASK_NOT_BINARY;
      cnt += (double)mk;
    }
    cnt = wave_sum_f64(cnt);
    if (cnt <= 0.0) f |= SM_GRPO_MASK_EMPTY_ROW;
    const double a = s_adv[i];
    const double tscale = (cnt > 0.0) ? 1.0 / ((double)G * cnt) : 0.0;
    double obj = 0.0, kls = 0.0, clipped = 0.0;
    for (int64_t t = lane; t < T; t += kWave) {
      const double cur = lp_cur[off + t];
      const double beh = lp_beh[off + t];
      const double mk = mask ? (double)mask[off + t] : 1.0;
      if (!finite(cur)) f |= SM_GRPO_BAD_CURRENT;
      if (!finite(beh)) f |= SM_GRPO_BAD_BEHAVIOR;
      const double lr = cur - beh;
      if (!finite(lr)) f |= SM_GRPO_RATIO_NONFINITE;
      if (!(lr <= 80.0)) f |= SM_GRPO_RATIO_UNSAFE;
      const double rho = exp(fmin(lr, 80.0));
      const double crho = fmin(fmax(rho, lower), upper);
      const double unc = rho * a, cs = crho * a;
      const double surr = fmin(unc, cs);
      const bool is_clipped = (surr == cs) && (rho != crho);
      double kl = 0.0, dkl = 0.0;
      if (lp_ref) {
        const double ref = lp_ref[off + t];
        if (!finite(ref)) f |= SM_GRPO_BAD_REFERENCE;
        const double lrr = ref - cur;
        if (!finite(lrr)) f |= SM_GRPO_REF_RATIO_NONFINITE;
        if (!(lrr <= 80.0)) f |= SM_GRPO_REF_RATIO_UNSAFE;
        const double e = exp(fmin(lrr, 80.0));
        kl = e - lrr - 1.0;
        dkl = 1.0 - e;
      }
      const bool active = (a >= 0.0 && rho <= upper) || (a < 0.0 && rho >= lower);
      const double dsurr = active ? rho * a : 0.0;
      const double ts = tscale * mk;
      obj += ts * (surr - beta * kl);
      kls += ts * kl;
      clipped += (is_clipped && mk != 0.0) ? 1.0 : 0.0;
      if (dlp) dlp[off + t] = (float)(ts * (-dsurr + beta * dkl));
    }
    obj = wave_sum_f64(obj);
    kls = wave_sum_f64(kls);
    clipped = wave_sum_f64(clipped);
    if (lane == 0) {
      s_obj[i] = obj;
      s_kl[i] = kls;
      s_clip[i] = clipped;
      s_cnt[i] = cnt;
    }
  }
  if (f) atomicOr(&s_flags, f);
  __syncthreads();
  if (threadIdx.x == 0) {
    double obj = 0.0, kls = 0.0, clipped = 0.0, tokens = 0.0;
    for (int i = 0; i < G; ++i) {
      obj += s_obj[i];
      kls += s_kl[i];
      clipped += s_clip[i];
      tokens += s_cnt[i];
    }
    int fl = s_flags;
    if (!finite(obj) || !finite(kls)) fl |= SM_GRPO_LOSS_OVERFLOW;
    if (stats) {
      stats[g * 5 + 0] = (float)(-obj);
      stats[g * 5 + 1] = (float)s_mean;
      stats[g * 5 + 2] = (float)s_std;
      stats[g * 5 + 3] = (float)kls;
      stats[g * 5 + 4] = (float)(tokens > 0.0 ? clipped / tokens : 0.0);
    }
    if (flags_out) flags_out[g] = fl;
  }
  if (adv_out) {
    for (int i = threadIdx.x; i < G; i += kThreads) adv_out[g * G + i] = (float)s_adv[i];
  }
}

}  // namespace
}  // namespace sm

extern "C" int sm_grpo_loss(const float* rewards, const float* lp_cur, const float* lp_beh,
                            const float* lp_ref, const float* mask, int64_t groups,
                            int64_t group_size, int64_t tokens, double clip_epsilon,
                            double advantage_epsilon, double kl_coefficient, float* group_stats,
                            float* advantages, float* dlp, int32_t* flags, void* stream) {
  using namespace sm;
  SM_REQUIRE(rewards && lp_cur && lp_beh, "sm_grpo_loss: rewards, lp_cur and lp_beh are required");
  SM_REQUIRE(group_size >= 2, "GRPO tensor group must contain at least two rollouts");
  SM_REQUIRE(group_size <= kMaxGroup, "sm_grpo_loss: group_size %lld exceeds %d",
             (long long)group_size, kMaxGroup);
  SM_REQUIRE(tokens > 0, "GRPO tensor rollouts have no token columns");
  SM_REQUIRE(groups >= 0 && groups <= 0x7fffffff, "sm_grpo_loss: groups out of range");
  SM_REQUIRE(std::isfinite(clip_epsilon) && clip_epsilon > 0.0 && clip_epsilon < 1.0,
             "GRPO clip_epsilon must be finite and in (0, 1)");
  SM_REQUIRE(std::isfinite(advantage_epsilon) && advantage_epsilon > 0.0,
             "GRPO advantage_epsilon must be finite and positive");
  SM_REQUIRE(std::isfinite(kl_coefficient) && kl_coefficient >= 0.0,
             "GRPO kl_coefficient must be finite and non-negative");
  SM_REQUIRE(lp_ref || kl_coefficient == 0.0,
             "GRPO tensor objective needs reference log-probs for positive KL coefficient");
  if (groups == 0) return SM_OK;
  grpo_kernel<<<dim3((unsigned)groups), kThreads, 0, as_stream(stream)>>>(
      rewards, lp_cur, lp_beh, lp_ref, mask, (int)group_size, tokens, clip_epsilon,
      advantage_epsilon, kl_coefficient, group_stats, advantages, dlp, flags);
  SM_LAUNCH_CHECK();
  return SM_OK;
}

extern "C" const char* sm_grpo_flags_message(int32_t flags) {
  // Order and wording of grpo_loss_tensor's validation list (posttrain.rs:976-1006).
  static const struct { int32_t bit; const char* msg; } kMessages[] = {
      {SM_GRPO_BAD_REWARD, "GRPO rewards contain a non-finite value"},
      {SM_GRPO_BAD_CURRENT, "GRPO current log probabilities contain a non-finite value"},
      {SM_GRPO_BAD_BEHAVIOR, "GRPO behavior log probabilities contain a non-finite value"},
      {SM_GRPO_MASK_NOT_BINARY, "GRPO active_mask must contain only binary zero/one values"},
      {SM_GRPO_MASK_EMPTY_ROW,
       "GRPO active_mask must contain at least one active token in every rollout"},
      {SM_GRPO_RATIO_NONFINITE, "GRPO importance log-ratio is non-finite"},
      {SM_GRPO_RATIO_UNSAFE, "GRPO importance log-ratio exceeds the safe exponential domain"},
      {SM_GRPO_REWARD_OVERFLOW, "GRPO reward normalization overflowed"},
      {SM_GRPO_LOSS_OVERFLOW, "GRPO tensor objective overflowed"},
      {SM_GRPO_BAD_REFERENCE, "GRPO reference log probabilities contain a non-finite value"},
      {SM_GRPO_REF_RATIO_NONFINITE, "GRPO reference log-ratio is non-finite"},
      {SM_GRPO_REF_RATIO_UNSAFE, "GRPO reference log-ratio exceeds the safe exponential domain"},
  };
  for (const auto& m : kMessages)
    if (flags & m.bit) return m.msg;
  return nullptr;
}
