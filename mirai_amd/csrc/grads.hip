// LoRA factor transposes and per-expert LoRA weight gradients of the layer
// backward. The weight gradients follow the autograd of the reference's LoRA
// composition (ActiveExpertLoRA.forward,
// mirai/core/models/compressed_weights/execution/active_expert_lora.py:316-346,
// linear(linear(x, A_e), B_e) * scale):
//   dB_e = sum_rows dOut^T (s * x A_e^T)      dA_e = sum_rows dz^T x,
// with dz = s * dOut B_e, each a sum over the expert's sorted rows.
#include "grads.h"

namespace mx {
namespace {

__global__ __launch_bounds__(256) void transpose_factors_kernel(const uint16_t *src, int64_t rows,
                                                                int64_t cols, int64_t total,
                                                                uint16_t *dst) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= total) return;
  const int64_t per = rows * cols;
  const int64_t e = i / per, rem = i - e * per;
  const int64_t r = rem / cols, c = rem - r * cols;
  dst[e * per + c * rows + r] = src[i];
}

// One workgroup per (expert, 512-column slice); each thread owns two adjacent
// columns and RANK fp32 accumulators per column. The expert's V rows are
// staged in LDS 64 at a time and read back as broadcasts.
template <int RANK>
__global__ __launch_bounds__(256) void lora_weight_grad_kernel(
    const uint16_t *m, int64_t ldm, const int32_t *map, const uint16_t *v, int64_t ldv,
    int64_t cols, const int64_t *seg_start, const int64_t *seg_end, float *out, int64_t se,
    int64_t sc, int64_t sj) {
  constexpr int kRows = 64;
  __shared__ float sv[kRows][RANK];
  const int e = blockIdx.y;
  const int64_t c0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 2;
  const bool active = c0 < cols;
  const int64_t start = seg_start[e], end = seg_end[e];
  float acc0[RANK], acc1[RANK];
#pragma unroll
  for (int j = 0; j < RANK; ++j) acc0[j] = acc1[j] = 0.0f;
  for (int64_t r0 = start; r0 < end; r0 += kRows) {
    const int n = static_cast<int>(min(static_cast<int64_t>(kRows), end - r0));
    __syncthreads();
    for (int idx = threadIdx.x; idx < kRows * RANK; idx += 256) {
      const int rr = idx / RANK, j = idx - rr * RANK;
      sv[rr][j] = rr < n ? bf16_bits_to_f32(v[(r0 + rr) * ldv + j]) : 0.0f;
    }
    __syncthreads();
    if (!active) continue;
#pragma unroll 4
    for (int rr = 0; rr < n; ++rr) {
      const int64_t row = r0 + rr;
      const int64_t src = map ? static_cast<int64_t>(map[row]) : row;
      const uint32_t w = *reinterpret_cast<const uint32_t *>(m + src * ldm + c0);
      const float x0 = bf16_bits_to_f32(w & 0xffffu), x1 = bf16_bits_to_f32(w >> 16);
#pragma unroll
      for (int j = 0; j < RANK; ++j) {
        acc0[j] = fmaf(x0, sv[rr][j], acc0[j]);
        acc1[j] = fmaf(x1, sv[rr][j], acc1[j]);
      }
    }
  }
  if (!active) return;
  float *o = out + e * se;
#pragma unroll
  for (int j = 0; j < RANK; ++j) {
    o[c0 * sc + j * sj] = acc0[j];
    o[(c0 + 1) * sc + j * sj] = acc1[j];
  }
}

}  // namespace

int transpose_factors(const uint16_t *src, int64_t experts, int64_t rows, int64_t cols,
                      uint16_t *dst, hipStream_t s) {
  const int64_t total = experts * rows * cols;
  if (total <= 0) return MX_OK;
  hipLaunchKernelGGL(transpose_factors_kernel, dim3(static_cast<unsigned>(ceil_div(total, 256))),
                     dim3(256), 0, s, src, rows, cols, total, dst);
  return check_launch("LoRA factor transpose");
}

int lora_weight_grad(const uint16_t *m, int64_t ldm, const int32_t *map, const uint16_t *v,
                     int64_t ldv, int rank, int64_t cols, const int64_t *seg_start,
                     const int64_t *seg_end, int experts, float *out, int64_t stride_e,
                     int64_t stride_c, int64_t stride_j, hipStream_t s) {
  if (cols % 2 != 0) {
    set_error("LoRA weight gradient: cols must be even");
    return MX_ERR_INVALID;
  }
  const dim3 grid(static_cast<unsigned>(ceil_div(cols, 512)), static_cast<unsigned>(experts));
#define MX_LWG(R)                                                                              \
  hipLaunchKernelGGL(lora_weight_grad_kernel<R>, grid, dim3(256), 0, s, m, ldm, map, v, ldv,   \
                     cols, seg_start, seg_end, out, stride_e, stride_c, stride_j)
  switch (rank) {
    case 8: MX_LWG(8); break;
    case 16: MX_LWG(16); break;
    case 24: MX_LWG(24); break;
    case 32: MX_LWG(32); break;
    default:
      set_error("LoRA weight gradient: rank %d not in {8,16,24,32}", rank);
      return MX_ERR_INVALID;
  }
#undef MX_LWG
  return check_launch("LoRA weight gradient");
}

}  // namespace mx
