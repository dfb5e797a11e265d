// Device MoE route plan layout shared by moe.hip (producer) and the grouped
// Q4 matmuls (consumers). All words are int32; sizes are sm_moe_plan_words().
#pragma once

#include <cstdint>

namespace sm {

struct PlanView {
  int32_t *counts;     // [E] routes per expert
  int32_t *offsets;    // [E+1] first sorted position of each expert
  int32_t *order;      // [R] sorted position -> route id (t*k + j)
  int32_t *inverse;    // [R] route id -> sorted position
  int32_t *src_rows;   // [R] sorted position -> token (route id / k)
  int32_t *ntiles16;   // [1] number of 16-row (expert, first row) tiles
  int32_t *tiles16;    // [max16][2]
  int32_t *ntiles128;  // [1] number of 128-row tiles
  int32_t *tiles128;   // [max128][2]
};

int64_t moe_max_tiles(int64_t routes, int64_t experts, int64_t rows);
PlanView plan_view(int32_t* plan, int64_t routes, int64_t experts);

}  // namespace sm
