// Small kernels of the layer backward: LoRA factor transposes and the
// per-expert LoRA weight gradients.
#pragma once

#include "common.h"

namespace mx {

// One [E, rows, cols] -> [E, cols, rows] bf16 transpose (total = E*rows*cols).
struct FactorTranspose {
  const uint16_t *src;
  uint16_t *dst;
  int64_t rows, cols, total;
};
struct FactorTransposes {
  FactorTranspose job[6];
  int n;
};
// All jobs in one launch.
int transpose_factors_multi(const FactorTransposes &jobs, hipStream_t s);

// Per-expert outer-product sums over the expert's sorted rows, for one or
// two V blocks that share M:
//   G_b[e, c, j] = sum_{r in [seg_start[e], seg_end[e])} M[map(r), c] * V_b[r, j]
// for c < cols, j < rank[b] (fp32 accumulation, fp32 output at
// out[b] + e*stride_e[b] + c*stride_c[b] + j*stride_j[b]). M and V_b are bf16 with
// leading dimensions ldm / ldv; map (null: identity) sends a sorted row to its
// M row. Each V block holds 32 columns (those past its rank only feed
// unwritten outputs); rank <= 32, cols a multiple of 8.
struct WeightGradJob {
  const uint16_t *m;
  int64_t ldm;
  const int32_t *map;
  const uint16_t *v[2];
  int64_t ldv;
  int rank[2];
  int nv;
  int64_t cols;
  float *out[2];
  int64_t stride_e[2], stride_c[2], stride_j[2];
};
constexpr int kMaxGradJobs = 8;
struct WeightGradJobs {
  WeightGradJob job[kMaxGradJobs];
  int n;
};
// All jobs in one launch.
int lora_weight_grads(const WeightGradJobs &jobs, const int64_t *seg_start,
                      const int64_t *seg_end, int experts, hipStream_t s);

// Gated-activation backward in place over expert-sorted rows: row r of `dgu`
// (stride 2f) holds dh in its first f columns on entry and [dG | dU] on exit,
// for h = bf16(silu(g)) * u (MX_ACT_SILU) or h = swiglu7(g, u) (MX_ACT_SWIGLU7),
// g, u: [rows, f].
int swiglu_backward(uint16_t *dgu, const uint16_t *g, const uint16_t *u, int64_t rows,
                    int64_t f, int act, hipStream_t s);

}  // namespace mx
