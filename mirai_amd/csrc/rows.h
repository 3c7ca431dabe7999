// Row-wise helper kernels shared by the layer entry points (rows.hip).
#pragma once

#include "common.h"

namespace mx {

// fp32 [rows, cols] -> bf16 planes [rows, 3*cols] in MX_SPLIT_* order.
int split_f32(const float *x, int64_t rows, int64_t cols, int pattern, uint16_t *out,
              hipStream_t s);

// out[r, c] = sum over q < planes of in[r, q*cols + c] for fp32 in
// [rows, planes*cols], added from the last plane to the first and written as
// out_dtype (the fp32 layer's combine of its output planes).
int sum_planes(const float *in, int64_t rows, int64_t cols, int planes, void *out, int out_dtype,
               hipStream_t s);

// mx_combine with an optional addend [T, cols] of out's dtype:
// out = out_dtype(out_dtype(sum) + addend). With bf16_terms each term is
// bf16(y * bf16(score)) and the running sum is rounded to bf16 after every
// add (expert order), the bf16 index_add of the reference's MAGI-2 backend.
int combine_ex(const void *y, const int64_t *top_idx, const void *top_scores, int score_dtype,
               int64_t num_tokens, int top_k, int num_experts, int64_t cols, void *out,
               int out_dtype, const void *addend, void *stream, bool bf16_terms = false);

}  // namespace mx
