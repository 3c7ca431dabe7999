// Shared device and host helpers for libmirai_moe (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/mirai_moe.h"

typedef __bf16 bf16_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

namespace mx {

// ---------------------------------------------------------------- host side
// Thread-local error text returned by mx_last_error().
void set_error(const char *fmt, ...);
void clear_error();
// Returns MX_ERR_HIP (and records the message) when the last launch failed.
int check_launch(const char *what);

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }
inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// --------------------------------------------------------------- device side
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits) {
  return __uint_as_float(bits << 16);
}

// Round-to-nearest-even fp32 -> bf16 (hardware v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}


// Two fp32 values -> packed bf16 pair (lo in bits 0-15), round to nearest even,
// as one v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

// f rounded to bf16 (nearest even), as an fp32 value: one v_cvt_pk_bf16_f32
// with 0 in the low half, whose result bits are then the fp32 value itself.
__device__ __forceinline__ float round_bf16(float f) { return __uint_as_float(pack_bf16x2(0.0f, f)); }

// IEEE correctly rounded fp32 division: the quotient is formed in fp64 and
// rounded once to fp32. fp64 carries 53 >= 2*24+2 bits, so the double rounding
// is innocuous and the result equals the correctly rounded fp32 quotient,
// independent of the compiler's fp32 division lowering.
__device__ __forceinline__ float div_rn(float a, float b) {
  return static_cast<float>(static_cast<double>(a) / static_cast<double>(b));
}

__device__ __forceinline__ float load_score(const void *p, int64_t i, int dtype) {
  if (dtype == MX_DTYPE_BF16)
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(p)[i]);
  return reinterpret_cast<const float *>(p)[i];
}

__device__ __forceinline__ void store_value(void *p, int64_t i, float v, int dtype) {
  if (dtype == MX_DTYPE_BF16)
    reinterpret_cast<uint16_t *>(p)[i] = f32_to_bf16_bits(v);
  else
    reinterpret_cast<float *>(p)[i] = v;
}

// The 16 NF4 code values (QLoRA normal-float quantiles), as fp32.
// Same decimal values as mirai/core/models/quantization.py:100-117; each is an
// exactly representable fp32 number, so the literal is exact.
__constant__ static const float kNF4Levels[16] = {
    -1.0f,
    -0.6961928009986877f,
    -0.5250730514526367f,
    -0.39491748809814453f,
    -0.28444138169288635f,
    -0.18477343022823334f,
    -0.09105003625154495f,
    0.0f,
    0.07958029955625534f,
    0.16093020141124725f,
    0.24611230194568634f,
    0.33791524171829224f,
    0.44070982933044434f,
    0.5626170039176941f,
    0.7229568362236023f,
    1.0f,
};

}  // namespace mx
