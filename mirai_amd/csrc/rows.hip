// Row movement between token order and expert-sorted order: gather (permute),
// scatter-add (permute backward), the gate-weighted combine and its backward.
#include "common.h"
#include "rows.h"

namespace mx {
namespace {

constexpr int kMaxK = 16;

// One thread per 16-byte chunk of a destination row.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint4 *src, int64_t src_rows,
                                                          const int64_t *index, int64_t rows,
                                                          int64_t chunks_per_row, uint4 *out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * chunks_per_row) return;
  const int64_t r = i / chunks_per_row, c = i - r * chunks_per_row;
  const int64_t s = index[r];
  uint4 v = make_uint4(0, 0, 0, 0);
  if (s >= 0 && s < src_rows) v = src[s * chunks_per_row + c];
  out[i] = v;
}

__global__ __launch_bounds__(256) void fill_f32_kernel(float *p, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.0f;
}

__global__ __launch_bounds__(256) void scatter_add_rows_kernel(const void *rows_in, int dtype,
                                                               const float *row_scale,
                                                               const int64_t *index, int64_t rows,
                                                               int64_t cols, int64_t out_rows,
                                                               float *out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * cols) return;
  const int64_t r = i / cols, c = i - r * cols;
  const int64_t t = index[r];
  if (t < 0 || t >= out_rows) return;
  float v = load_score(rows_in, i, dtype);
  if (row_scale) v = __fmul_rn(v, row_scale[r]);
  atomicAdd(out + t * cols + c, v);
}

// Order of the k slots of one token by ascending expert id (slot order for
// equal ids); invalid ids are marked -1 and skipped by the callers.
__device__ __forceinline__ int sorted_slots(const int64_t *idx_row, int k, int E, int *slot) {
  int ex[kMaxK];
  int n = 0;
  for (int j = 0; j < k; ++j) {
    const int64_t e = idx_row[j];
    if (e < 0 || e >= E) continue;
    int p = n++;
    while (p > 0 && ex[p - 1] > static_cast<int>(e)) {
      ex[p] = ex[p - 1];
      slot[p] = slot[p - 1];
      --p;
    }
    ex[p] = static_cast<int>(e);
    slot[p] = j;
  }
  return n;
}

// 16-byte load that bypasses cache retention: each y row is read exactly once.
__device__ __forceinline__ uint4 nt_load16(const uint16_t *p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Stores 8 combined columns at element offset `off`. With an addend (same
// dtype and layout as out) the value is out_dtype(out_dtype(sum) + addend):
// the routed sum is rounded to the output dtype first and then added, as the
// reference's `out + shared_output` on the block output
// (transformer_lingbot_video.py:2374-2377).
__device__ __forceinline__ void store_combined(void *out, int out_dtype, const void *addend,
                                               int64_t off, const float (&acc)[8]) {
  if (out_dtype == MX_DTYPE_BF16) {
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = acc[i];
    if (addend) {
      const uint4 a = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(addend) + off);
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[2 * q] = round_bf16(v[2 * q]) + bf16_bits_to_f32(aw[q] & 0xffffu);
        v[2 * q + 1] = round_bf16(v[2 * q + 1]) + bf16_bits_to_f32(aw[q] >> 16);
      }
    }
    const u32x4 o = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                     pack_bf16x2(v[6], v[7])};
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(out) + off));
  } else {
    float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + off);
    float4 lo = make_float4(acc[0], acc[1], acc[2], acc[3]);
    float4 hi = make_float4(acc[4], acc[5], acc[6], acc[7]);
    if (addend) {
      const float4 *a = reinterpret_cast<const float4 *>(static_cast<const float *>(addend) + off);
      const float4 a0 = a[0], a1 = a[1];
      lo = make_float4(lo.x + a0.x, lo.y + a0.y, lo.z + a0.z, lo.w + a0.w);
      hi = make_float4(hi.x + a1.x, hi.y + a1.y, hi.z + a1.z, hi.w + a1.w);
    }
    o[0] = lo;
    o[1] = hi;
  }
}

// One wave per token (four tokens per workgroup) for a compile-time top-k:
// the slot order (ascending expert id, slot order for ties, invalid ids last)
// is formed with static indices, and the KC slot rows of each 512-column span
// are all loaded before the fp32 accumulation, which runs in that order.
// BF16T: each term is formed and added in bf16 -- acc = bf16(acc +
// bf16(y * bf16(score))) in the same order -- the bf16 index_add of the
// reference's MAGI-2 backend (grouped_moe.py:750-754) run in expert order.
__device__ __forceinline__ float bf16_term_add(float acc, float y, float s_bf16) {
  return round_bf16(acc + round_bf16(y * s_bf16));
}

template <int KC, bool BF16T>
__global__ __launch_bounds__(256) void combine_wave_kernel(const uint16_t *y, const int64_t *top_idx,
                                                          const void *top_scores, int score_dtype,
                                                          int E, int64_t cols, int64_t num_tokens,
                                                          void *out, int out_dtype,
                                                          const void *addend) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= num_tokens) return;
  const int lane = threadIdx.x & 63;
  int key[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    const int64_t e = top_idx[t * KC + j];
    key[j] = (e < 0 || e >= E) ? 0x7fffffff : static_cast<int>(e);
  }
  const uint16_t *row[KC];
  float sc[KC];
  bool ok[KC];
#pragma unroll
  for (int q = 0; q < KC; ++q) {
    row[q] = y;
    sc[q] = 0.0f;
    ok[q] = false;
  }
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    int rank = 0;
#pragma unroll
    for (int i = 0; i < KC; ++i) rank += (key[i] < key[j] || (key[i] == key[j] && i < j)) ? 1 : 0;
    const bool valid = key[j] != 0x7fffffff;
    float s = valid ? (top_scores ? load_score(top_scores, t * KC + j, score_dtype) : 1.0f) : 0.0f;
    if (BF16T) s = round_bf16(s);
#pragma unroll
    for (int q = 0; q < KC; ++q) {
      if (rank == q) {
        row[q] = y + (t * KC + j) * cols;
        sc[q] = s;
        ok[q] = valid;
      }
    }
  }
  // Sums the KC rows of one 8-column span into acc, in rank order.
  auto span_sum = [&](const uint4 (&v)[KC], float (&acc)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int q = 0; q < KC; ++q) {
      if (!ok[q]) continue;
      const uint32_t w[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (BF16T) {
          acc[2 * i] = bf16_term_add(acc[2 * i], bf16_bits_to_f32(w[i] & 0xffffu), sc[q]);
          acc[2 * i + 1] = bf16_term_add(acc[2 * i + 1], bf16_bits_to_f32(w[i] >> 16), sc[q]);
          continue;
        }
        // Product then sum, each rounded once, as in index_add_(y.float() * score).
        acc[2 * i] = __fadd_rn(acc[2 * i], __fmul_rn(bf16_bits_to_f32(w[i] & 0xffffu), sc[q]));
        acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], __fmul_rn(bf16_bits_to_f32(w[i] >> 16), sc[q]));
      }
    }
  };
  // kSpans 512-column spans per round: all kSpans * KC row loads (at most 16
  // per lane, so the registers leave room for several waves per SIMD) are in
  // flight before the first sum.
  constexpr int kSpans = KC > 4 ? 2 : 4;
  int64_t c0 = static_cast<int64_t>(lane) * 8;
  for (; c0 + (kSpans - 1) * 512 < cols; c0 += kSpans * 512) {
    uint4 v[kSpans][KC];
#pragma unroll
    for (int u = 0; u < kSpans; ++u)
#pragma unroll
      for (int q = 0; q < KC; ++q)
        v[u][q] = ok[q] ? nt_load16(row[q] + c0 + 512 * u) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < kSpans; ++u) {
      float acc[8];
      span_sum(v[u], acc);
      store_combined(out, out_dtype, addend, t * cols + c0 + 512 * u, acc);
    }
  }
  for (; c0 < cols; c0 += 512) {
    uint4 v[KC];
#pragma unroll
    for (int q = 0; q < KC; ++q)
      v[q] = ok[q] ? *reinterpret_cast<const uint4 *>(row[q] + c0) : make_uint4(0, 0, 0, 0);
    float acc[8];
    span_sum(v, acc);
    store_combined(out, out_dtype, addend, t * cols + c0, acc);
  }
}

// One workgroup per token; each thread owns 8 consecutive columns per step.
template <bool BF16T>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t *y, const int64_t *top_idx,
                                                      const void *top_scores, int score_dtype,
                                                      int k, int E, int64_t cols, void *out,
                                                      int out_dtype, const void *addend) {
  const int64_t t = blockIdx.x;
  int slot[kMaxK];
  const int n = sorted_slots(top_idx + t * k, k, E, slot);
  float sc[kMaxK];
  for (int j = 0; j < n; ++j) {
    sc[j] = top_scores ? load_score(top_scores, t * k + slot[j], score_dtype) : 1.0f;
    if (BF16T) sc[j] = round_bf16(sc[j]);
  }
  for (int64_t c0 = static_cast<int64_t>(threadIdx.x) * 8; c0 < cols; c0 += 256 * 8) {
    float acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = 0.0f;
    for (int j = 0; j < n; ++j) {
      const uint4 v = *reinterpret_cast<const uint4 *>(y + (t * k + slot[j]) * cols + c0);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (BF16T) {
          acc[2 * q] = bf16_term_add(acc[2 * q], bf16_bits_to_f32(w[q] & 0xffffu), sc[j]);
          acc[2 * q + 1] = bf16_term_add(acc[2 * q + 1], bf16_bits_to_f32(w[q] >> 16), sc[j]);
          continue;
        }
        // Product then sum, each rounded once, as in index_add_(y.float() * score).
        acc[2 * q] = __fadd_rn(acc[2 * q], __fmul_rn(bf16_bits_to_f32(w[q] & 0xffffu), sc[j]));
        acc[2 * q + 1] = __fadd_rn(acc[2 * q + 1], __fmul_rn(bf16_bits_to_f32(w[q] >> 16), sc[j]));
      }
    }
    store_combined(out, out_dtype, addend, t * cols + c0, acc);
  }
}

// One wave per token (four per workgroup) for a compile-time top-k: grad_y
// rows for every valid slot, 16 bytes per lane, and the score gradients
// (wave reduction of grad_out . y, fp32).
template <int KC>
__global__ __launch_bounds__(256) void combine_backward_wave_kernel(
    const void *grad_out, int grad_dtype, const uint16_t *y, const int64_t *top_idx,
    const void *top_scores, int score_dtype, int E, int64_t cols, int64_t num_tokens,
    uint16_t *grad_y, float *grad_scores) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= num_tokens) return;
  const int lane = threadIdx.x & 63;
  bool ok[KC];
  float sc[KC], part[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    const int64_t e = top_idx[t * KC + j];
    ok[j] = e >= 0 && e < E;
    sc[j] = ok[j] ? load_score(top_scores, t * KC + j, score_dtype) : 0.0f;
    part[j] = 0.0f;
  }
  for (int64_t c0 = static_cast<int64_t>(lane) * 8; c0 < cols; c0 += 512) {
    float g[8];
    if (grad_dtype == MX_DTYPE_BF16) {
      const uint4 v = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(grad_out) + t * cols + c0);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
        g[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
      }
    } else {
      const float4 *gp = reinterpret_cast<const float4 *>(static_cast<const float *>(grad_out) + t * cols + c0);
      const float4 a = gp[0], b = gp[1];
      g[0] = a.x; g[1] = a.y; g[2] = a.z; g[3] = a.w;
      g[4] = b.x; g[5] = b.y; g[6] = b.z; g[7] = b.w;
    }
    uint4 yv[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j)
      yv[j] = ok[j] ? *reinterpret_cast<const uint4 *>(y + (t * KC + j) * cols + c0) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      if (!ok[j]) continue;
      const uint32_t w[4] = {yv[j].x, yv[j].y, yv[j].z, yv[j].w};
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        part[j] += g[2 * i] * bf16_bits_to_f32(w[i] & 0xffffu) + g[2 * i + 1] * bf16_bits_to_f32(w[i] >> 16);
        o[i] = pack_bf16x2(g[2 * i] * sc[j], g[2 * i + 1] * sc[j]);
      }
      *reinterpret_cast<uint4 *>(grad_y + (t * KC + j) * cols + c0) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    float v = part[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) grad_scores[t * KC + j] = ok[j] ? v : 0.0f;
  }
}

// One workgroup per token: grad_y rows for every valid slot and the score
// gradients (block reduction of grad_out . y).
__global__ __launch_bounds__(256) void combine_backward_kernel(
    const void *grad_out, int grad_dtype, const uint16_t *y, const int64_t *top_idx,
    const void *top_scores, int score_dtype, int k, int E, int64_t cols, uint16_t *grad_y,
    float *grad_scores) {
  __shared__ float red[kMaxK][4];
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float part[kMaxK];
  for (int j = 0; j < k; ++j) part[j] = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float g = load_score(grad_out, t * cols + c, grad_dtype);
    for (int j = 0; j < k; ++j) {
      const int64_t e = top_idx[t * k + j];
      if (e < 0 || e >= E) continue;
      const int64_t r = t * k + j;
      const float s = load_score(top_scores, r, score_dtype);
      grad_y[r * cols + c] = f32_to_bf16_bits(g * s);
      part[j] += g * bf16_bits_to_f32(y[r * cols + c]);
    }
  }
  for (int j = 0; j < k; ++j) {
    float v = part[j];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) red[j][wid] = v;
  }
  __syncthreads();
  if (threadIdx.x < k) {
    const int j = threadIdx.x;
    const int64_t e = top_idx[t * k + j];
    const float v = red[j][0] + red[j][1] + red[j][2] + red[j][3];
    grad_scores[t * k + j] = (e < 0 || e >= E) ? 0.0f : v;
  }
}

// fp32 -> bf16 planes: one thread per 8 values of a row; hi = bf16(x),
// lo = bf16(x - hi) (x - hi is exact in fp32).
__global__ __launch_bounds__(256) void split_f32_kernel(const float4 *x, int64_t rows,
                                                        int64_t chunks, int pattern, uint4 *out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * chunks) return;
  const int64_t r = i / chunks, c = i - r * chunks;
  const float4 a = x[2 * i], b = x[2 * i + 1];
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t hi[4], lo[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    hi[q] = pack_bf16x2(v[2 * q], v[2 * q + 1]);
    lo[q] = pack_bf16x2(v[2 * q] - bf16_bits_to_f32(hi[q] & 0xffffu),
                        v[2 * q + 1] - bf16_bits_to_f32(hi[q] >> 16));
  }
  const uint4 H = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  const uint4 L = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  uint4 *o = out + r * 3 * chunks + c;
  o[0] = H;
  o[chunks] = pattern == MX_SPLIT_ACT ? H : L;
  o[2 * chunks] = pattern == MX_SPLIT_ACT ? L : H;
}

// out[r, c] = sum over planes q of in[r, q cols + c], added from the last
// plane to the first (the low-order planes first).
template <int OUT_DTYPE>
__global__ __launch_bounds__(256) void sum_planes_kernel(const float4 *in, int64_t rows,
                                                         int64_t chunks, int planes, void *out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * chunks) return;
  const int64_t r = i / chunks, c = i - r * chunks;
  const float4 *row = in + r * planes * chunks + c;
  float4 v = row[(planes - 1) * chunks];
  for (int q = planes - 2; q >= 0; --q) {
    const float4 a = row[q * chunks];
    v = make_float4(v.x + a.x, v.y + a.y, v.z + a.z, v.w + a.w);
  }
  if (OUT_DTYPE == MX_DTYPE_F32) {
    static_cast<float4 *>(out)[i] = v;
  } else {
    static_cast<uint2 *>(out)[i] = make_uint2(pack_bf16x2(v.x, v.y), pack_bf16x2(v.z, v.w));
  }
}

}  // namespace

int sum_planes(const float *in, int64_t rows, int64_t cols, int planes, void *out, int out_dtype,
               hipStream_t s) {
  if (rows <= 0) return MX_OK;
  const int64_t chunks = cols / 4;
  const dim3 grid(static_cast<unsigned>(ceil_div(rows * chunks, 256)));
  if (out_dtype == MX_DTYPE_F32)
    hipLaunchKernelGGL(sum_planes_kernel<MX_DTYPE_F32>, grid, dim3(256), 0, s,
                       reinterpret_cast<const float4 *>(in), rows, chunks, planes, out);
  else
    hipLaunchKernelGGL(sum_planes_kernel<MX_DTYPE_BF16>, grid, dim3(256), 0, s,
                       reinterpret_cast<const float4 *>(in), rows, chunks, planes, out);
  return check_launch("fp32 layer plane sum");
}

int split_f32(const float *x, int64_t rows, int64_t cols, int pattern, uint16_t *out,
              hipStream_t s) {
  if (!x || !out || rows < 0 || cols <= 0 || cols % 8 != 0 ||
      (pattern != MX_SPLIT_ACT && pattern != MX_SPLIT_WEIGHT)) {
    set_error("mx_split_f32: need non-null buffers, cols a multiple of 8 and a known pattern");
    return MX_ERR_INVALID;
  }
  if (rows == 0) return MX_OK;
  const int64_t chunks = cols / 8;
  hipLaunchKernelGGL(split_f32_kernel, dim3(static_cast<unsigned>(ceil_div(rows * chunks, 256))),
                     dim3(256), 0, s, reinterpret_cast<const float4 *>(x), rows, chunks, pattern,
                     reinterpret_cast<uint4 *>(out));
  return check_launch("mx_split_f32");
}

}  // namespace mx

using namespace mx;

extern "C" int mx_split_f32(const float *x, int64_t rows, int64_t cols, int pattern, void *out,
                            void *stream) {
  clear_error();
  return split_f32(x, rows, cols, pattern, static_cast<uint16_t *>(out), as_stream(stream));
}

extern "C" int mx_gather_rows(const void *tokens, int64_t src_rows, const int64_t *index,
                              int64_t rows, int64_t cols, int dtype, void *out, void *stream) {
  clear_error();
  const int64_t esize = dtype == MX_DTYPE_BF16 ? 2 : 4;
  if (rows < 0 || cols <= 0 || (cols * esize) % 16 != 0 ||
      (rows > 0 && (!tokens || !index || !out))) {
    set_error("mx_gather_rows: need non-null buffers and rows of a multiple of 16 bytes");
    return MX_ERR_INVALID;
  }
  if (rows == 0) return MX_OK;
  const int64_t chunks = cols * esize / 16;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(ceil_div(rows * chunks, 256)), dim3(256), 0,
                     as_stream(stream), static_cast<const uint4 *>(tokens), src_rows, index, rows,
                     chunks, static_cast<uint4 *>(out));
  return check_launch("mx_gather_rows");
}

extern "C" int mx_scatter_add_rows(const void *rows_in, const float *row_scale,
                                   const int64_t *index, int64_t rows, int64_t cols, int dtype,
                                   int64_t out_rows, float *out, void *stream) {
  clear_error();
  float *grad_tokens = out;
  const void *grad = rows_in;
  if ((!grad_tokens && out_rows > 0) || out_rows < 0 || rows < 0 || cols <= 0 ||
      (rows > 0 && (!grad || !index))) {
    set_error("mx_scatter_add_rows: invalid arguments");
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  if (out_rows * cols > 0)
    hipLaunchKernelGGL(fill_f32_kernel, dim3(ceil_div(out_rows * cols, 256)), dim3(256), 0, s,
                       grad_tokens, out_rows * cols);
  if (rows > 0)
    hipLaunchKernelGGL(scatter_add_rows_kernel, dim3(ceil_div(rows * cols, 256)), dim3(256), 0, s,
                       grad, dtype, row_scale, index, rows, cols, out_rows, grad_tokens);
  return check_launch("mx_scatter_add_rows");
}

namespace mx {

int combine_ex(const void *y, const int64_t *top_idx, const void *top_scores, int score_dtype,
               int64_t num_tokens, int top_k, int num_experts, int64_t cols, void *out,
               int out_dtype, const void *addend, void *stream, bool bf16_terms) {
  if (num_tokens < 0 || top_k <= 0 || top_k > kMaxK || cols <= 0 || cols % 8 != 0 ||
      num_experts <= 0) {
    set_error("mx_combine: need top_k in [1,16], cols a positive multiple of 8");
    return MX_ERR_INVALID;
  }
  if (num_tokens == 0) return MX_OK;
  if (!y || !top_idx || !out) {
    set_error("mx_combine: y, top_idx and out must be non-null");
    return MX_ERR_INVALID;
  }
  const dim3 wave_grid(static_cast<unsigned>(ceil_div(num_tokens, 4)));
  const uint16_t *yb = static_cast<const uint16_t *>(y);
#define MX_COMBINE_K(KC)                                                                     \
  case KC:                                                                                   \
    if (bf16_terms)                                                                          \
      hipLaunchKernelGGL((combine_wave_kernel<KC, true>), wave_grid, dim3(256), 0,             \
                         as_stream(stream), yb, top_idx, top_scores, score_dtype, num_experts,  \
                         cols, num_tokens, out, out_dtype, addend);                            \
    else                                                                                     \
      hipLaunchKernelGGL((combine_wave_kernel<KC, false>), wave_grid, dim3(256), 0,            \
                         as_stream(stream), yb, top_idx, top_scores, score_dtype, num_experts,  \
                         cols, num_tokens, out, out_dtype, addend);                            \
    break;
  switch (top_k) {
    MX_COMBINE_K(1)
    MX_COMBINE_K(2)
    MX_COMBINE_K(3)
    MX_COMBINE_K(4)
    MX_COMBINE_K(6)
    MX_COMBINE_K(8)
    default:
      if (bf16_terms)
        hipLaunchKernelGGL(combine_kernel<true>, dim3(num_tokens), dim3(256), 0,
                           as_stream(stream), yb, top_idx, top_scores, score_dtype, top_k,
                           num_experts, cols, out, out_dtype, addend);
      else
        hipLaunchKernelGGL(combine_kernel<false>, dim3(num_tokens), dim3(256), 0,
                           as_stream(stream), yb, top_idx, top_scores, score_dtype, top_k,
                           num_experts, cols, out, out_dtype, addend);
  }
#undef MX_COMBINE_K
  return check_launch("mx_combine");
}

}  // namespace mx

extern "C" int mx_combine(const void *y, const int64_t *top_idx, const void *top_scores,
                          int score_dtype, int64_t num_tokens, int top_k, int num_experts,
                          int64_t cols, void *out, int out_dtype, void *stream) {
  clear_error();
  return combine_ex(y, top_idx, top_scores, score_dtype, num_tokens, top_k, num_experts, cols, out,
                    out_dtype, nullptr, stream);
}

extern "C" int mx_combine_backward(const void *grad_out, int grad_dtype, const void *y,
                                   const int64_t *top_idx, const void *top_scores,
                                   int score_dtype, int64_t num_tokens, int top_k,
                                   int num_experts, int64_t cols, void *grad_y,
                                   float *grad_scores, void *stream) {
  clear_error();
  if (num_tokens < 0 || top_k <= 0 || top_k > kMaxK || cols <= 0 || num_experts <= 0) {
    set_error("mx_combine_backward: need top_k in [1,16] and cols > 0");
    return MX_ERR_INVALID;
  }
  if (num_tokens == 0) return MX_OK;
  if (!grad_out || !y || !top_idx || !top_scores || !grad_y || !grad_scores) {
    set_error("mx_combine_backward: buffers must be non-null");
    return MX_ERR_INVALID;
  }
  const uint16_t *yb = static_cast<const uint16_t *>(y);
  uint16_t *gy = static_cast<uint16_t *>(grad_y);
  if (cols % 8 == 0) {
    const dim3 wave_grid(static_cast<unsigned>(ceil_div(num_tokens, 4)));
#define MX_COMBINE_BWD_K(KC)                                                                  \
  case KC:                                                                                    \
    hipLaunchKernelGGL(combine_backward_wave_kernel<KC>, wave_grid, dim3(256), 0,             \
                       as_stream(stream), grad_out, grad_dtype, yb, top_idx, top_scores,        \
                       score_dtype, num_experts, cols, num_tokens, gy, grad_scores);           \
    return check_launch("mx_combine_backward");
    switch (top_k) {
      MX_COMBINE_BWD_K(1)
      MX_COMBINE_BWD_K(2)
      MX_COMBINE_BWD_K(4)
      MX_COMBINE_BWD_K(8)
      default:
        break;
    }
#undef MX_COMBINE_BWD_K
  }
  hipLaunchKernelGGL(combine_backward_kernel, dim3(num_tokens), dim3(256), 0, as_stream(stream),
                     grad_out, grad_dtype, yb, top_idx, top_scores, score_dtype, top_k,
                     num_experts, cols, gy, grad_scores);
  return check_launch("mx_combine_backward");
}
