// Host-side helpers of sampling.hip shared with the rollout driver (model.hip).
#pragma once

#include "common.hpp"

namespace sm {

// Argument checks of SamplingConfig / RolloutSampling (generate.rs:68-84,
// posttrain.rs:372-386); sets the error message and returns its status.
int validate_sampling(const sm_sampling* c, int64_t vocab);

// One sample_ex launch over `rows` logits rows. seen: [rows, seen_ld] bitmap,
// read for the penalty and updated with the chosen token; done/lengths/ndone:
// EOS bookkeeping (nullable).
int sample_ex_launch(const float* logits, int64_t rows, int64_t ld, int64_t vocab,
                     const sm_sampling* c, uint64_t seed, int64_t step, uint32_t* seen,
                     int64_t seen_ld, int32_t* done, int32_t* lengths, int32_t* ndone,
                     int32_t* tokens, int64_t tok_stride, float* logprobs, int64_t lp_stride,
                     int32_t* next_ids, hipStream_t st);

// seen[r] (|)= {ids[r, 0..n)}; clear zeroes the rows first.
int seen_tokens(const int32_t* ids, int64_t rows, int64_t n, int64_t ids_ld, int64_t vocab,
                uint32_t* seen, int64_t seen_ld, bool clear, hipStream_t st);

int fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t st);

}  // namespace sm
