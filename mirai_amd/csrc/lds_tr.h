// LDS layout and MFMA operand reads for tiles stored k-major ([k rows][n]),
// shared by the transposed-B grouped GEMMs and the LoRA weight gradients.
#pragma once

#include "common.h"

namespace mx {

// Transposed B stage: [64 k rows][256 n] bf16 (512-byte rows, 32 chunks). The
// chunk index is XOR-ed with a permutation of the row's low 4 bits so that
//  * a row-owner ds_write_b128 (16 lanes = 16 consecutive rows, one logical
//    chunk) hits 16 distinct 16-byte bank groups, and
//  * a ds_read_b64_tr_b16 half-wave (4 consecutive rows x 4 chunks) does too.
__device__ __forceinline__ int swz_t(int row, int chunk) {
  const int x = ((row & 3) << 2) | ((row >> 2) & 3);
  return row * 512 + ((chunk ^ x) << 4);
}

// The same layout over [k rows][128 n] (256-byte rows, 16 chunks): the row
// key only permutes chunks within the row, so the properties above hold.
__device__ __forceinline__ int swz_t128(int row, int chunk) {
  const int x = ((row & 3) << 2) | ((row >> 2) & 3);
  return row * 256 + ((chunk ^ x) << 4);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));

// B fragment of v_mfma_f32_32x32x16_bf16 (lane: column lane%32, k = 8*(lane/32)
// + 0..7) read from a transposed stage. ds_read_b64_tr_b16 hands lane j of a
// 16-lane group the elements j, 16+j, 32+j, 48+j of the group's concatenated
// 8-byte chunks; lane i of the group therefore fetches row k0 + i/4, columns
// c0 + 4*(i%4) .. +3, and receives column c0 + j of rows k0 .. k0+3.
template <int ROW_BYTES = 512>
__device__ __forceinline__ bf16x8 read_b_trans(const uint8_t *sB, int ncol0, int kk, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int row = 16 * kk + 8 * (g >> 1) + (i >> 2);
  const int col = ncol0 + 16 * (g & 1) + 4 * (i & 3);
  const int chunk = col >> 3, half = ((col >> 2) & 1) * 8;
  auto at = [](int r, int c) { return ROW_BYTES == 512 ? swz_t(r, c) : swz_t128(r, c); };
  // An address-space cast of the stage pointer (not an integer round trip)
  // keeps the LDS object the read comes from visible to the compiler, so a
  // read of one stage does not wait for an LDS DMA into the other.
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)(const_cast<uint8_t *>(sB) + at(row, chunk) + half));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)(const_cast<uint8_t *>(sB) + at(row + 4, chunk) + half));
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

}  // namespace mx
