// Row-wise helper kernels shared by the layer entry points (rows.hip).
#pragma once

#include "common.h"

namespace mx {

// fp32 [rows, cols] -> bf16 planes [rows, 3*cols] in MX_SPLIT_* order.
int split_f32(const float *x, int64_t rows, int64_t cols, int pattern, uint16_t *out,
              hipStream_t s);

// out[r, c] = in[r, c] + in[r, cols + c] for fp32 in [rows, 2*cols], written
// as out_dtype (the fp32 layer's combine of its two output planes).
int sum_halves(const float *in, int64_t rows, int64_t cols, void *out, int out_dtype,
               hipStream_t s);

}  // namespace mx
