// Internal view of the dispatch-plan workspace shared by the plan kernels and
// the grouped GEMMs.
#pragma once

#include "common.h"

namespace mx {

// Row-tile heights of the grouped GEMMs; the plan emits one (expert, first
// row) work item per tile for each height.
constexpr int kPlanTileM = 128;
constexpr int kPlanTileM2 = 256;
// Expert (group) count limit of the plan: MAGI-2 flattens heads x experts
// onto one group axis (12 x 256 = 3072 groups).
constexpr int kPlanMaxExperts = 8192;

// True when the scatter pass keeps its per-word popcount prefixes in LDS next
// to the masks (2 * E * EB bits within 64 KiB).
__host__ __device__ inline bool plan_prefix_in_lds(int num_experts, int slots_per_block) {
  return static_cast<int64_t>(num_experts) * slots_per_block <= 262144;
}

struct PlanLayout {
  int64_t rows = 0;
  int experts = 0;
  int slots_per_block = 0;
  int blocks = 0;
  int64_t max_tiles = 0;   // 128-row tiles
  int64_t max_tiles2 = 0;  // 256-row tiles
  size_t off_block_counts = 0, off_block_base = 0, off_seg = 0, off_tiles = 0, off_tiles2 = 0;
  size_t off_tiles2m = 0, off_tilesr = 0;
  size_t off_row_token = 0, off_row_slot = 0, off_block_err = 0;
  size_t bytes = 0;
};

struct PlanView {
  int32_t *err;            // invalid expert ids / inconsistent counts seen
  int32_t *num_tiles;      // 128-row tiles emitted
  int32_t *num_tiles2;     // 256-row tiles emitted
  int32_t *block_counts;   // [blocks, E]
  int32_t *block_base;     // [blocks, E]
  int64_t *seg;            // [2, E]: segment start, segment end (sorted rows)
  int2 *tiles;             // [max_tiles]: (expert, first row), 128-row tiles
  int2 *tiles2;            // [max_tiles2]: 256-row tiles
  // Split covering: 256-row tiles over each expert's rows except a final
  // remainder of at most 128 rows, which gets one 128-row tile of its own.
  int32_t *num_tiles2m;    // 256-row tiles of the split covering
  int32_t *num_tilesr;     // 128-row remainder tiles (at most one per expert)
  int2 *tiles2m;           // [max_tiles2]
  int2 *tilesr;            // [experts]
  int32_t *row_token;      // [R]: sorted row -> token
  int32_t *row_slot;       // [R]: sorted row -> flat route slot t*k+j
  int32_t *block_err;      // [blocks]: invalid expert ids per count block
};

int slots_per_plan_block(int num_experts, int64_t rows);
PlanLayout plan_layout(int64_t num_rows, int num_experts);
PlanView plan_view(void *ws, const PlanLayout &L);
int validate_plan_args(const char *name, int64_t num_tokens, int top_k, int num_experts);

int build_plan(const int64_t *top_idx, const void *top_scores, int score_dtype,
               int64_t num_tokens, int top_k, int num_experts, int64_t *counts, int64_t *starts,
               int32_t *offsets, int64_t *sort_positions, int64_t *sorted_token_indices,
               void *sorted_scores, int64_t *inverse_order, void *workspace, hipStream_t s);
int plan_from_counts(const int64_t *counts, int64_t num_rows, int num_experts, void *workspace,
                     hipStream_t s);

}  // namespace mx
