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
// and one absmax. Packing: in each group of 8 elements, byte i holds element
// i in its low nibble and element i + 4 in its high nibble (lanes whose bit 2
// is clear pack their neighbour 4 lanes up as the high nibble).
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
  const int hi = __shfl_down(best, 4, 64);
  if ((lane & 4) == 0)
    codes[block * (kNF4Block / 2) + (lane >> 3) * 4 + (lane & 3)] = static_cast<uint8_t>(best | (hi << 4));
  if (lane == 0) absmax[block] = f32_to_bf16_bits(amax);
}

// Each thread decodes one packed dword: the 8 elements of one group (byte i
// holds element i in its low nibble and element i + 4 in its high nibble).
// The block absmax is bf16 (the build's quantiser) or fp32 (MX_FMT_NF4_F32).
template <bool F32_ABSMAX>
__global__ __launch_bounds__(256) void nf4_dequantize_kernel(const uint32_t *codes,
                                                             const void *absmax,
                                                             int64_t num_words, void *out,
                                                             int out_dtype) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= num_words) return;
  const uint32_t word = codes[i];
  const int64_t blk = i / (kNF4Block / 8);
  const float a = F32_ABSMAX ? static_cast<const float *>(absmax)[blk]
                             : bf16_bits_to_f32(static_cast<const uint16_t *>(absmax)[blk]);
  float v[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t byte = (word >> (8 * b)) & 0xffu;
    v[b] = kNF4Levels[byte & 15] * a;
    v[b + 4] = kNF4Levels[byte >> 4] * a;
  }
  if (out_dtype == MX_DTYPE_BF16) {
    reinterpret_cast<u32x4 *>(out)[i] =
        u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
              pack_bf16x2(v[6], v[7])};
  } else {
    // fp32 output carries the bf16-rounded value (the codec's dequantized
    // weight is defined in bf16).
    float *o = reinterpret_cast<float *>(out) + 8 * i;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = bf16_bits_to_f32(f32_to_bf16_bits(v[j]));
  }
}

// bitsandbytes double-quantised NF4 (quantize_4bit with compress_statistics,
// blocksize 64, nested blocksize 256; bitsandbytes 0.49.2 as called by
// mirai/core/models/compressed_weights/quantization/quant.py:315-358) ->
// MX_FMT_NF4_F32. One thread per group of 8 elements: bitsandbytes byte j of
// a row holds element 2j in its high nibble and 2j + 1 in its low nibble; the
// group is rewritten as byte i = element i | element i + 4 << 4. The thread
// that owns the first group of a 64-block also decodes the block's absmax,
// nested_code[absmax_q] * nested_absmax[block / 256] + offset in fp32 (the
// dequantize_blockwise + offset step of quant.py:413-424).
__global__ __launch_bounds__(256) void nf4_from_bnb_kernel(
    const uint32_t *packed, const uint8_t *absmax_q, const float *nested_absmax,
    const float *offsets, const float *nested_code, int64_t groups_per_expert,
    int64_t nested_per_expert, int64_t total_groups, uint32_t *codes, float *absmax) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= total_groups) return;
  const uint32_t w = packed[g];
  uint32_t out = 0;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t byte = (w >> (8 * m)) & 0xffu;
    const uint32_t e_even = byte >> 4, e_odd = byte & 15u;  // elements 2m, 2m + 1
    // element k of the group goes to byte k % 4, low nibble for k < 4.
    const int k0 = 2 * m, k1 = 2 * m + 1;
    out |= e_even << (8 * (k0 & 3) + 4 * (k0 >> 2));
    out |= e_odd << (8 * (k1 & 3) + 4 * (k1 >> 2));
  }
  codes[g] = out;
  if (absmax != nullptr && (g & 7) == 0) {  // first group of a 64-element block
#pragma clang fp contract(off)
    const int64_t e = g / groups_per_expert;
    const int64_t b = (g - e * groups_per_expert) >> 3;  // block within the expert
    const int64_t blk = g >> 3;
    // Two roundings (product, then sum), never one fused multiply-add.
    const float scaled = nested_code[absmax_q[blk]] * nested_absmax[e * nested_per_expert + (b >> 8)];
    absmax[blk] = scaled + offsets[e];
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

// absmax[e][b] = fp32(fp32(code[q[e][b]] * nested[e][b / 256]) + offsets[e]).
__global__ __launch_bounds__(256) void nf4_dq_absmax_kernel(const uint8_t *q, const float *nested,
                                                            const float *offsets, const float *code,
                                                            int64_t blocks_per_expert,
                                                            int64_t nested_per_expert, int64_t total,
                                                            float *absmax) {
#pragma clang fp contract(off)
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t e = i / blocks_per_expert, b = i - e * blocks_per_expert;
  // Two roundings (product, then sum), never one fused multiply-add.
  const float scaled = code[q[i]] * nested[e * nested_per_expert + (b >> 8)];
  absmax[i] = scaled + offsets[e];
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

extern "C" int mx_nf4_dequantize_ex(const uint8_t *codes, const void *absmax, int absmax_dtype,
                                    int64_t rows, int64_t cols, void *out, int out_dtype,
                                    void *stream) {
  clear_error();
  if (!codes || !absmax || !out || rows < 0 || cols <= 0 || cols % 64 != 0) {
    set_error("mx_nf4_dequantize: need non-null buffers and cols a positive multiple of 64");
    return MX_ERR_INVALID;
  }
  if (absmax_dtype != MX_DTYPE_BF16 && absmax_dtype != MX_DTYPE_F32) {
    set_error("mx_nf4_dequantize: absmax must be bf16 or fp32");
    return MX_ERR_INVALID;
  }
  if (reinterpret_cast<uintptr_t>(codes) % 4 != 0 ||
      (out_dtype == MX_DTYPE_BF16 && reinterpret_cast<uintptr_t>(out) % 16 != 0)) {
    set_error("mx_nf4_dequantize: codes must be 4-byte aligned and a bf16 output 16-byte aligned");
    return MX_ERR_INVALID;
  }
  const int64_t words = rows * cols / 8;
  if (words == 0) return MX_OK;
  const dim3 grid(static_cast<unsigned>(ceil_div(words, 256)));
  if (absmax_dtype == MX_DTYPE_F32)
    hipLaunchKernelGGL(nf4_dequantize_kernel<true>, grid, dim3(256), 0, as_stream(stream),
                       reinterpret_cast<const uint32_t *>(codes), absmax, words, out, out_dtype);
  else
    hipLaunchKernelGGL(nf4_dequantize_kernel<false>, grid, dim3(256), 0, as_stream(stream),
                       reinterpret_cast<const uint32_t *>(codes), absmax, words, out, out_dtype);
  return check_launch("mx_nf4_dequantize");
}

extern "C" int mx_nf4_dequantize(const uint8_t *codes, const void *absmax, int64_t rows,
                                 int64_t cols, void *out, int out_dtype, void *stream) {
  return mx_nf4_dequantize_ex(codes, absmax, MX_DTYPE_BF16, rows, cols, out, out_dtype, stream);
}

extern "C" int mx_nf4_from_bnb(const uint8_t *packed, const uint8_t *absmax_q,
                               const float *nested_absmax, const float *offsets,
                               const float *nested_code, int64_t experts, int64_t rows,
                               int64_t cols, uint8_t *codes, float *absmax, void *stream) {
  clear_error();
  if (!packed || !codes || (absmax && (!absmax_q || !nested_absmax || !offsets || !nested_code))) {
    set_error("mx_nf4_from_bnb: buffers must be non-null (absmax may be null: codes only)");
    return MX_ERR_INVALID;
  }
  if (experts < 0 || rows < 0 || cols <= 0 || cols % 64 != 0) {
    set_error("mx_nf4_from_bnb: need experts, rows >= 0 and cols a positive multiple of 64");
    return MX_ERR_INVALID;
  }
  if (reinterpret_cast<uintptr_t>(packed) % 4 != 0 || reinterpret_cast<uintptr_t>(codes) % 4 != 0) {
    set_error("mx_nf4_from_bnb: packed and codes must be 4-byte aligned");
    return MX_ERR_INVALID;
  }
  const int64_t groups_per_expert = rows * cols / 8;
  const int64_t total = experts * groups_per_expert;
  if (total == 0) return MX_OK;
  const int64_t nested_per_expert = ceil_div(rows * cols / 64, 256);
  hipLaunchKernelGGL(nf4_from_bnb_kernel, dim3(static_cast<unsigned>(ceil_div(total, 256))),
                     dim3(256), 0, as_stream(stream), reinterpret_cast<const uint32_t *>(packed),
                     absmax_q, nested_absmax, offsets, nested_code, groups_per_expert,
                     nested_per_expert, total, reinterpret_cast<uint32_t *>(codes), absmax);
  return check_launch("mx_nf4_from_bnb");
}

extern "C" int mx_nf4_dq_absmax(const mx_nf4_dq *dq, int64_t experts, int64_t blocks_per_expert,
                                float *absmax, void *stream) {
  clear_error();
  if (!dq || !absmax || !dq->absmax_q || !dq->nested_absmax || !dq->offsets || !dq->code) {
    set_error("mx_nf4_dq_absmax: buffers must be non-null");
    return MX_ERR_INVALID;
  }
  if (experts < 0 || blocks_per_expert < 0 ||
      dq->nested_per_expert < ceil_div(blocks_per_expert, 256)) {
    set_error("mx_nf4_dq_absmax: need experts, blocks >= 0 and ceil(blocks / 256) nested scales "
              "per expert");
    return MX_ERR_INVALID;
  }
  const int64_t total = experts * blocks_per_expert;
  if (total == 0) return MX_OK;
  hipLaunchKernelGGL(nf4_dq_absmax_kernel, dim3(static_cast<unsigned>(ceil_div(total, 256))),
                     dim3(256), 0, as_stream(stream), dq->absmax_q, dq->nested_absmax, dq->offsets,
                     dq->code, blocks_per_expert, dq->nested_per_expert, total, absmax);
  return check_launch("mx_nf4_dq_absmax");
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
