/*
 * Plain-C restatement of the NF4 / INT8 frozen-weight codecs -- TEST
 * INFRASTRUCTURE ONLY (the checker for the HIP codec kernels; never linked
 * into the product library).
 *
 * Same rules as oracle/codec.py, which restates
 *   mirai/core/models/quantization.py:100-117 (NF4 codebook), :158-175
 *   (nearest level by argmin with first-index ties; packed per group of 8
 *   elements, byte i = element i | element i+4 << 4),
 *   mirai/core/models/compressed_weights/quantization/quant.py:189-260 (INT8
 *   per-row symmetric rule, scale floor 1e-30), :413-431 (fp32 product then
 *   cast on dequantisation),
 * in the BASELINE storage format (bf16 absmax / bf16 scale). Inputs and
 * outputs are bf16 bit patterns (uint16). Build: oracle/Makefile.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static const float kLevels[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if (isnan(f)) return 0x7FC0;
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

void oracle_nf4_levels(float *out) { memcpy(out, kLevels, sizeof(kLevels)); }

void oracle_nf4_quantize(const uint16_t *w, int64_t rows, int64_t cols, uint8_t *codes,
                         uint16_t *absmax) {
  const int64_t blocks = cols / 64;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t b = 0; b < blocks; ++b) {
      const uint16_t *src = w + r * cols + b * 64;
      float amax = 0.0f;
      for (int j = 0; j < 64; ++j) {
        const float a = fabsf(bf16_to_f32(src[j]));
        if (a > amax) amax = a;
      }
      absmax[r * blocks + b] = f32_to_bf16(amax);
      uint8_t q[64];
      for (int j = 0; j < 64; ++j) {
        const float s = amax > 0.0f ? bf16_to_f32(src[j]) / amax : 0.0f;
        int best = 0;
        float best_d = fabsf(s - kLevels[0]);
        for (int l = 1; l < 16; ++l) {
          const float d = fabsf(s - kLevels[l]);
          if (d < best_d) {
            best_d = d;
            best = l;
          }
        }
        q[j] = (uint8_t)best;
      }
      uint8_t *dst = codes + r * (cols / 2) + b * 32;
      /* per group of 8 elements: byte i = element i | element (i + 4) << 4 */
      for (int j = 0; j < 32; ++j) {
        const int e = 8 * (j / 4) + j % 4;
        dst[j] = (uint8_t)(q[e] | (q[e + 4] << 4));
      }
    }
  }
}

void oracle_nf4_dequantize(const uint8_t *codes, const uint16_t *absmax, int64_t rows,
                           int64_t cols, uint16_t *out) {
  const int64_t half = cols / 2;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < half; ++i) {
      const uint8_t byte = codes[r * half + i];
      const int64_t e = 8 * (i / 4) + i % 4; /* element of the low nibble */
      const float a = bf16_to_f32(absmax[r * (cols / 64) + e / 64]);
      const float lo = kLevels[byte & 15] * a;
      const float hi = kLevels[byte >> 4] * a;
      out[r * cols + e] = f32_to_bf16(lo);
      out[r * cols + e + 4] = f32_to_bf16(hi);
    }
  }
}

void oracle_int8_quantize(const uint16_t *w, int64_t rows, int64_t cols, int8_t *q,
                          uint16_t *scale) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t *src = w + r * cols;
    float amax = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      const float a = fabsf(bf16_to_f32(src[c]));
      if (a > amax) amax = a;
    }
    float s32 = amax / 127.0f;
    const float floor_v = 1e-30f;
    if (s32 < floor_v) s32 = floor_v;
    const uint16_t sb = f32_to_bf16(s32);
    const float s = bf16_to_f32(sb);
    for (int64_t c = 0; c < cols; ++c) {
      float v = rintf(bf16_to_f32(src[c]) / s);
      if (v > 127.0f) v = 127.0f;
      if (v < -127.0f) v = -127.0f;
      q[r * cols + c] = (int8_t)v;
    }
    scale[r] = sb;
  }
}

void oracle_int8_dequantize(const int8_t *q, const uint16_t *scale, int64_t rows, int64_t cols,
                            uint16_t *out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float s = bf16_to_f32(scale[r]);
    for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = f32_to_bf16((float)q[r * cols + c] * s);
  }
}
