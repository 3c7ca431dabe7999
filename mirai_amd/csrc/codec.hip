// Frozen-weight codecs: NF4 (blocksize 64, bf16 absmax) and INT8 (per output
// row, bf16 scale). Quantisation runs once at weight load; dequantisation here
// is the standalone (bit-exact) form of the decode the grouped GEMMs perform
// in registers.
#include "common.h"

namespace mx {
namespace {

constexpr int kNF4Block = 64;

__device__ __forceinline__ float load_weight_as_bf16(const void *w, int64_t i, int dtype) {
  // Frozen weights are stored from their bf16 value, as the reference casts
  // them to bf16 before quantize_4bit (quant.py:328).
  if (dtype == MX_DTYPE_BF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(w)[i]);
  float f = reinterpret_cast<const float *>(w)[i];
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

// One wavefront per 64-element block: lane = element. Writes 32 code bytes
// (lanes with even index pack their odd neighbour as the high nibble) and one
// absmax.
__global__ __launch_bounds__(256) void nf4_quantize_kernel(const void *w, int w_dtype,
                                                           int64_t num_blocks, uint8_t *codes,
                                                           uint16_t *absmax) {
  const int lane = threadIdx.x & 63;
  const int64_t block = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  if (block >= num_blocks) return;
  const float v = load_weight_as_bf16(w, block * kNF4Block + lane, w_dtype);
  float amax = fabsf(v);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  // amax is the magnitude of one of the bf16 inputs, hence exactly a bf16 value.
  const float scaled = amax > 0.0f ? div_rn(v, amax) : 0.0f;
  int best = 0;
  float best_d = fabsf(scaled - kNF4Levels[0]);
#pragma unroll
  for (int j = 1; j < 16; ++j) {
    const float d = fabsf(scaled - kNF4Levels[j]);
    if (d < best_d) {  // strict: the first index wins ties
      best_d = d;
      best = j;
    }
  }
  const int hi = __shfl_down(best, 1, 64);
  if ((lane & 1) == 0) codes[block * (kNF4Block / 2) + (lane >> 1)] = static_cast<uint8_t>(best | (hi << 4));
  if (lane == 0) absmax[block] = f32_to_bf16_bits(amax);
}

// Each thread decodes one code byte (two elements).
__global__ __launch_bounds__(256) void nf4_dequantize_kernel(const uint8_t *codes,
                                                             const uint16_t *absmax,
                                                             int64_t num_bytes, void *out,
                                                             int out_dtype) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= num_bytes) return;
  const uint32_t byte = codes[i];
  const float a = bf16_bits_to_f32(absmax[i / (kNF4Block / 2)]);
  const float lo = kNF4Levels[byte & 15] * a;
  const float hi = kNF4Levels[byte >> 4] * a;
  if (out_dtype == MX_DTYPE_BF16) {
    reinterpret_cast<uint32_t *>(out)[i] = pack_bf16x2(lo, hi);
  } else {
    // fp32 output carries the bf16-rounded value (the codec's dequantized
    // weight is defined in bf16).
    float *o = reinterpret_cast<float *>(out);
    o[2 * i] = bf16_bits_to_f32(f32_to_bf16_bits(lo));
    o[2 * i + 1] = bf16_bits_to_f32(f32_to_bf16_bits(hi));
  }
}

// One workgroup per output row.
__global__ __launch_bounds__(256) void int8_quantize_kernel(const void *w, int w_dtype,
                                                            int64_t cols, int8_t *q,
                                                            uint16_t *scale) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const void *wrow = w;
  const int64_t base = row * cols;
  float amax = 0.0f;
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x)
    amax = fmaxf(amax, fabsf(load_weight_as_bf16(wrow, base + c, w_dtype)));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // scale = max(absmax / 127, 1e-30) in fp32, stored as bf16 (quant.py:227).
  // 0x0DA24260 is the fp32 value nearest to 1e-30.
  float s32 = fmaxf(div_rn(amax, 127.0f), __uint_as_float(0x0DA24260u));
  const uint16_t s_bits = f32_to_bf16_bits(s32);
  const float s = bf16_bits_to_f32(s_bits);
  for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
    const float v = load_weight_as_bf16(wrow, base + c, w_dtype);
    float r = rintf(div_rn(v, s));  // round half to even
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    q[base + c] = static_cast<int8_t>(r);
  }
  if (threadIdx.x == 0) scale[row] = s_bits;
}

__global__ __launch_bounds__(256) void int8_dequantize_kernel(const int8_t *q,
                                                              const uint16_t *scale,
                                                              int64_t cols, int64_t total,
                                                              void *out, int out_dtype) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const float s = bf16_bits_to_f32(scale[i / cols]);
  const float v = static_cast<float>(q[i]) * s;  // exact: 7-bit integer times 8-bit mantissa
  store_value(out, i, bf16_bits_to_f32(f32_to_bf16_bits(v)), out_dtype);
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_nf4_quantize(const void *w, int w_dtype, int64_t rows, int64_t cols,
                               uint8_t *codes, void *absmax, void *stream) {
  clear_error();
  if (!w || !codes || !absmax || rows < 0 || cols <= 0 || cols % 64 != 0) {
    set_error("mx_nf4_quantize: need non-null buffers and cols a positive multiple of 64 (got %lld)",
              static_cast<long long>(cols));
    return MX_ERR_INVALID;
  }
  if (w_dtype != MX_DTYPE_BF16 && w_dtype != MX_DTYPE_F32) {
    set_error("mx_nf4_quantize: weight dtype must be bf16 or fp32");
    return MX_ERR_INVALID;
  }
  const int64_t blocks = rows * (cols / 64);
  if (blocks == 0) return MX_OK;
  const int64_t threads = blocks * 64;
  hipLaunchKernelGGL(nf4_quantize_kernel, dim3(ceil_div(threads, 256)), dim3(256), 0,
                     as_stream(stream), w, w_dtype, blocks, codes,
                     reinterpret_cast<uint16_t *>(absmax));
  return check_launch("mx_nf4_quantize");
}

extern "C" int mx_nf4_dequantize(const uint8_t *codes, const void *absmax, int64_t rows,
                                 int64_t cols, void *out, int out_dtype, void *stream) {
  clear_error();
  if (!codes || !absmax || !out || rows < 0 || cols <= 0 || cols % 64 != 0) {
    set_error("mx_nf4_dequantize: need non-null buffers and cols a positive multiple of 64");
    return MX_ERR_INVALID;
  }
  const int64_t bytes = rows * cols / 2;
  if (bytes == 0) return MX_OK;
  hipLaunchKernelGGL(nf4_dequantize_kernel, dim3(ceil_div(bytes, 256)), dim3(256), 0,
                     as_stream(stream), codes, reinterpret_cast<const uint16_t *>(absmax), bytes,
                     out, out_dtype);
  return check_launch("mx_nf4_dequantize");
}

extern "C" int mx_int8_quantize(const void *w, int w_dtype, int64_t rows, int64_t cols,
                                int8_t *q, void *scale, void *stream) {
  clear_error();
  if (!w || !q || !scale || rows < 0 || cols <= 0) {
    set_error("mx_int8_quantize: need non-null buffers and cols > 0");
    return MX_ERR_INVALID;
  }
  if (w_dtype != MX_DTYPE_BF16 && w_dtype != MX_DTYPE_F32) {
    set_error("mx_int8_quantize: weight dtype must be bf16 or fp32");
    return MX_ERR_INVALID;
  }
  if (rows == 0) return MX_OK;
  if (rows > 0x7fffffff) {
    set_error("mx_int8_quantize: too many rows");
    return MX_ERR_INVALID;
  }
  hipLaunchKernelGGL(int8_quantize_kernel, dim3(rows), dim3(256), 0, as_stream(stream), w,
                     w_dtype, cols, q, reinterpret_cast<uint16_t *>(scale));
  return check_launch("mx_int8_quantize");
}

extern "C" int mx_int8_dequantize(const int8_t *q, const void *scale, int64_t rows, int64_t cols,
                                  void *out, int out_dtype, void *stream) {
  clear_error();
  if (!q || !scale || !out || rows < 0 || cols <= 0) {
    set_error("mx_int8_dequantize: need non-null buffers and cols > 0");
    return MX_ERR_INVALID;
  }
  const int64_t total = rows * cols;
  if (total == 0) return MX_OK;
  hipLaunchKernelGGL(int8_dequantize_kernel, dim3(ceil_div(total, 256)), dim3(256), 0,
                     as_stream(stream), q, reinterpret_cast<const uint16_t *>(scale), cols, total,
                     out, out_dtype);
  return check_launch("mx_int8_dequantize");
}
