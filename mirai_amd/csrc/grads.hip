// LoRA factor transposes and per-expert LoRA weight gradients of the layer
// backward. The weight gradients follow the autograd of the reference's LoRA
// composition (ActiveExpertLoRA.forward,
// mirai/core/models/compressed_weights/execution/active_expert_lora.py:316-346,
// linear(linear(x, A_e), B_e) * scale):
//   dB_e = sum_rows dOut^T (s * x A_e^T)      dA_e = sum_rows dz^T x,
// with dz = s * dOut B_e, each a sum over the expert's sorted rows.
#include "grads.h"
#include "lds_tr.h"

namespace mx {
namespace {

// Several [E, rows, cols] -> [E, cols, rows] transposes in one launch. One of
// rows / cols is a LoRA rank (at most 256): a thread moves the rank-long run
// at one position of the other (long) dimension, 32 ranks at a time, so the
// long dimension runs across the lanes of a wave and both the loads and the
// stores are coalesced. Runs are moved as 16-byte vectors when the rank is a
// multiple of 8 and both buffers are 16-byte aligned. Workgroups
// [block0[j], block0[j + 1]) serve job j.
// Jobs whose rank is a multiple of 8, whose long dimension is a multiple of 8
// and whose buffers are 16-byte aligned go through LDS instead, a block of 32
// ranks x 128 positions per workgroup: 16-byte loads along the source rows,
// 16-byte stores along the destination rows (for a rank of 16 the block's
// destination is one contiguous 4 KB run).
struct TransposeLaunch {
  FactorTranspose job[6];
  int64_t block0[7];
  int vec[6];
  int tiled[6];
  int n;
};

constexpr int kTileL = 128, kTileS = 32;

__device__ void transpose_block(const FactorTranspose &t, bool small_rows, uint32_t S, uint32_t Lg,
                                int64_t local, uint16_t *tile) {
  const int64_t lblocks = (Lg + kTileL - 1) / kTileL, sblocks = (S + kTileS - 1) / kTileS;
  const int64_t e = local / (lblocks * sblocks), rem = local - e * lblocks * sblocks;
  const uint32_t l0 = static_cast<uint32_t>(rem / sblocks) * kTileL;
  const uint32_t s0 = static_cast<uint32_t>(rem % sblocks) * kTileS;
  const uint32_t nl = min(static_cast<uint32_t>(kTileL), Lg - l0);
  const uint32_t ns = min(static_cast<uint32_t>(kTileS), S - s0);
  const int64_t base = e * S * Lg;
  const uint16_t *src = t.src + base;
  uint16_t *dst = t.dst + base;
  const int tid = threadIdx.x;
  if (small_rows) {
    // src [S][Lg] -> tile [s][l] -> dst [Lg][S].
    for (int i = tid; i < kTileS * (kTileL / 8); i += 256) {
      const uint32_t sr = i / (kTileL / 8), lp = i % (kTileL / 8);
      if (sr < ns && lp * 8 < nl)
        *reinterpret_cast<u32x4 *>(tile + sr * kTileL + lp * 8) =
            *reinterpret_cast<const u32x4 *>(src + static_cast<int64_t>(s0 + sr) * Lg + l0 + lp * 8);
    }
    __syncthreads();
    for (int i = tid; i < kTileL * (kTileS / 8); i += 256) {
      const uint32_t l = i / (kTileS / 8), sp = i % (kTileS / 8);
      if (l < nl && sp * 8 < ns) {
        u32x4 w;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          w[q] = static_cast<uint32_t>(tile[(sp * 8 + 2 * q) * kTileL + l]) |
                 (static_cast<uint32_t>(tile[(sp * 8 + 2 * q + 1) * kTileL + l]) << 16);
        *reinterpret_cast<u32x4 *>(dst + static_cast<int64_t>(l0 + l) * S + s0 + sp * 8) = w;
      }
    }
  } else {
    // src [Lg][S] -> tile [l][s] -> dst [S][Lg].
    for (int i = tid; i < kTileL * (kTileS / 8); i += 256) {
      const uint32_t l = i / (kTileS / 8), sp = i % (kTileS / 8);
      if (l < nl && sp * 8 < ns)
        *reinterpret_cast<u32x4 *>(tile + l * kTileS + sp * 8) =
            *reinterpret_cast<const u32x4 *>(src + static_cast<int64_t>(l0 + l) * S + s0 + sp * 8);
    }
    __syncthreads();
    for (int i = tid; i < kTileS * (kTileL / 8); i += 256) {
      const uint32_t sr = i / (kTileL / 8), lp = i % (kTileL / 8);
      if (sr < ns && lp * 8 < nl) {
        u32x4 w;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          w[q] = static_cast<uint32_t>(tile[(lp * 8 + 2 * q) * kTileS + sr]) |
                 (static_cast<uint32_t>(tile[(lp * 8 + 2 * q + 1) * kTileS + sr]) << 16);
        *reinterpret_cast<u32x4 *>(dst + static_cast<int64_t>(s0 + sr) * Lg + l0 + lp * 8) = w;
      }
    }
  }
}

__global__ __launch_bounds__(256) void transpose_factors_multi_kernel(TransposeLaunch L) {
  int j = 0;
  while (j + 1 < L.n && static_cast<int64_t>(blockIdx.x) >= L.block0[j + 1]) ++j;
  const FactorTranspose &t = L.job[j];
  const bool small_rows = t.rows <= t.cols;
  const uint32_t S = static_cast<uint32_t>(small_rows ? t.rows : t.cols);
  const uint32_t Lg = static_cast<uint32_t>(small_rows ? t.cols : t.rows);
  if (L.tiled[j]) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[kTileS * kTileL];
    transpose_block(t, small_rows, S, Lg, static_cast<int64_t>(blockIdx.x) - L.block0[j], tile);
    return;
  }
  const uint32_t idx = static_cast<uint32_t>(
      (static_cast<int64_t>(blockIdx.x) - L.block0[j]) * 256 + threadIdx.x);
  if (static_cast<int64_t>(idx) * S >= t.total) return;
  const uint32_t e = idx / Lg, l = idx - e * Lg;
  const int64_t base = static_cast<int64_t>(e) * S * Lg;
  const uint16_t *src = t.src + base;
  uint16_t *dst = t.dst + base;
  const bool vec = L.vec[j] != 0;
  for (uint32_t s0 = 0; s0 < S; s0 += 32) {
    const int n = static_cast<int>(S - s0 < 32 ? S - s0 : 32);  // ranks of this pass
    uint16_t v[32];
    if (small_rows) {  // src [S][Lg] -> dst [Lg][S]: gather the column, store the run
#pragma unroll
      for (int q = 0; q < 32; ++q)
        if (q < n) v[q] = src[static_cast<int64_t>(s0 + q) * Lg + l];
      uint16_t *run = dst + static_cast<int64_t>(l) * S + s0;
      if (vec) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (q * 8 < n) {
            u32x4 w;
#pragma unroll
            for (int i = 0; i < 4; ++i)
              w[i] = static_cast<uint32_t>(v[q * 8 + 2 * i]) |
                     (static_cast<uint32_t>(v[q * 8 + 2 * i + 1]) << 16);
            *reinterpret_cast<u32x4 *>(run + q * 8) = w;
          }
      } else {
#pragma unroll
        for (int q = 0; q < 32; ++q)
          if (q < n) run[q] = v[q];
      }
    } else {  // src [Lg][S] -> dst [S][Lg]: load the run, scatter it down the column
      const uint16_t *run = src + static_cast<int64_t>(l) * S + s0;
      if (vec) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (q * 8 < n) {
            const u32x4 w = *reinterpret_cast<const u32x4 *>(run + q * 8);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              v[q * 8 + 2 * i] = static_cast<uint16_t>(w[i] & 0xFFFFu);
              v[q * 8 + 2 * i + 1] = static_cast<uint16_t>(w[i] >> 16);
            }
          }
      } else {
#pragma unroll
        for (int q = 0; q < 32; ++q)
          if (q < n) v[q] = run[q];
      }
#pragma unroll
      for (int q = 0; q < 32; ++q)
        if (q < n) dst[static_cast<int64_t>(s0 + q) * Lg + l] = v[q];
    }
  }
}

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

// V-tile read for v_mfma_f32_32x32x16_bf16's B operand from [64 rows][32]
// bf16 (64-byte rows): lane j of each 16-lane group receives column
// 16*(group&1) + j of four consecutive rows (see read_b_trans).
__device__ __forceinline__ bf16x8 read_v_trans(const uint8_t *sV, int kk, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const int row = 16 * kk + 8 * (g >> 1) + (i >> 2);
  const int col = 16 * (g & 1) + 4 * (i & 3);
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)(const_cast<uint8_t *>(sV) + row * 64 + col * 2));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_i16x4 *)(const_cast<uint8_t *>(sV) + (row + 4) * 64 + col * 2));
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8, v);
}

// Jobs of one lora_weight_grads launch; workgroups [block0[j], block0[j + 1])
// serve job j, expert-major (the column slices of one expert are adjacent, so
// they meet the expert's V rows in L2).
struct GradLaunch {
  WeightGradJob job[kMaxGradJobs];
  int64_t block0[kMaxGradJobs + 1];
  int col_blocks[kMaxGradJobs];
  int n;
  const int64_t *seg_start, *seg_end;
};

// One workgroup (4 waves) per (job, expert, 128-column slice): G_b[c, j] = sum
// over the expert's rows of M[row, c] * V_b[row, j] for the job's one or two V
// blocks, on bf16 MFMA with fp32 accumulation. Both operands arrive row-major
// (the reduction runs along rows), so 64-row chunks of M and V go to LDS as
// they are and the MFMA fragments are read with ds_read_b64_tr_b16; the M
// fragment of a K step feeds both V blocks. Each wave owns 32 columns x 32
// ranks of each V block (one 32 x 32 block each). Rows past the segment and
// columns past `cols` are zero-filled. The kernel streams M once, so it is
// bound by load latency: each thread keeps two chunks of its loads in flight
// (register sets A and B, alternating), the row map of the chunk after them
// is fetched one chunk ahead, and two LDS stages alternate, so a chunk's
// loads are issued two chunks before its MFMAs. The narrow slice keeps the
// kernel within 256 registers (194) and 48 KB of LDS, so two workgroups share
// a CU and their load chains overlap (a 256-column slice needs 288 registers
// and runs one workgroup per CU).
__global__ __launch_bounds__(256) void lora_weight_grad_kernel(GradLaunch L) {
  __shared__ __attribute__((aligned(16))) uint8_t sM0[64 * 256];
  __shared__ __attribute__((aligned(16))) uint8_t sM1[64 * 256];
  __shared__ __attribute__((aligned(16))) uint8_t sV0[2 * 64 * 64];
  __shared__ __attribute__((aligned(16))) uint8_t sV1[2 * 64 * 64];
  int jn = 0;
  while (jn + 1 < L.n && static_cast<int64_t>(blockIdx.x) >= L.block0[jn + 1]) ++jn;
  const WeightGradJob &J = L.job[jn];
  const int local = static_cast<int>(static_cast<int64_t>(blockIdx.x) - L.block0[jn]);
  const int e = local / L.col_blocks[jn];
  const int64_t c0 = static_cast<int64_t>(local - e * L.col_blocks[jn]) * 128;
  const uint16_t *m = J.m;
  const int32_t *map = J.map;
  const int64_t ldm = J.ldm, ldv = J.ldv, cols = J.cols;
  const int nv = J.nv;
  const uint16_t *const vsrc[2] = {J.v[0], J.v[nv > 1 ? 1 : 0]};
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t start = L.seg_start[e], end = L.seg_end[e];
  f32x16 acc[2];
#pragma unroll
  for (int vb = 0; vb < 2; ++vb)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[vb][j] = 0.0f;

  // This thread's share of a chunk: M pieces q = tid + 256*i (row q/16,
  // 16-byte chunk q%16) and one 16-byte piece of each V block (row tid/4,
  // chunk tid%4).
  struct Loads {
    u32x4 mr[4];
    u32x4 vr[2];
  };
  const int vrow = tid >> 2, vch = tid & 3;
  // Every lane issues every load of a step, from an address clamped into the
  // segment and the slice; rows past the segment end and columns past `cols`
  // are zeroed when the chunk is staged. (With loads under a lane or
  // workgroup condition some paths through a step issue none, and the
  // compiler's wait counting then drains the whole queue before each use.)
  // A chunk's source rows: the row map's entries for its rows, clamped to the
  // segment's last row (without a map, a dummy load keeps the count even and
  // the row index is used as it is).
  const int32_t *const mbase = map ? map : reinterpret_cast<const int32_t *>(L.seg_start);
  const int64_t mstep = map ? 1 : 0;
  auto rows_of = [&](int64_t r0, int32_t *src) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t grow = min(r0 + ((tid + 256 * i) >> 4), end - 1);
      src[i] = mbase[grow * mstep];
    }
  };
  auto load = [&](int64_t r0, const int32_t *src, Loads &Ld) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t grow = min(r0 + ((tid + 256 * i) >> 4), end - 1);
      const int64_t row = map ? static_cast<int64_t>(src[i]) : grow;
      const int64_t col = min(c0 + ((tid + 256 * i) & 15) * 8, cols - 8);
      Ld.mr[i] = *reinterpret_cast<const u32x4 *>(m + row * ldm + col);
    }
    const int64_t grow = min(r0 + vrow, end - 1);
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
      Ld.vr[vb] = *reinterpret_cast<const u32x4 *>(vsrc[vb] + grow * ldv + vch * 8);
  };
  auto store = [&](int64_t r0, uint8_t *sM, uint8_t *sV, const Loads &Ld) {
    const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = tid + 256 * i;
      const bool ok = r0 + (q >> 4) < end && c0 + (q & 15) * 8 < cols;
      *reinterpret_cast<u32x4 *>(sM + swz_t128(q >> 4, q & 15)) = ok ? Ld.mr[i] : zero;
    }
    const bool vok = r0 + vrow < end;
#pragma unroll
    for (int vb = 0; vb < 2; ++vb)
      if (vb < nv)
        *reinterpret_cast<u32x4 *>(sV + vb * 4096 + vrow * 64 + vch * 16) = vok ? Ld.vr[vb] : zero;
  };
  auto compute = [&](const uint8_t *sM, const uint8_t *sV) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const bf16x8 bm = read_b_trans<256>(sM, wave * 32, kk, lane);
#pragma unroll
      for (int vb = 0; vb < 2; ++vb) {
        if (vb >= nv) continue;
        const bf16x8 bv = read_v_trans(sV + vb * 4096, kk, lane);
        acc[vb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bm, bv, acc[vb], 0, 0, 0);
      }
    }
  };
  // Chunk c (rows start + 64c) is loaded in step c-2 (set c % 2), stored to
  // stage c % 2 after the MFMAs of step c-1, and multiplied in step c; its
  // source rows are fetched in step c-3 into row set c % 2. Every step issues
  // the same loads (rows past the segment end re-read its last row and stage
  // zeros),
  // so the waits stay counted: the chunk loaded in step c-1 stays in flight
  // through step c's MFMAs.
  auto step = [&](int64_t r0, const uint8_t *cM, const uint8_t *cV, uint8_t *nM, uint8_t *nV,
                  Loads &next, Loads &after, const int32_t *src_after, int32_t *src_later) {
    rows_of(r0 + 192, src_later);
    load(r0 + 128, src_after, after);
    compute(cM, cV);
    store(r0 + 64, nM, nV, next);
    __syncthreads();
  };
  if (start < end) {
    Loads la, lb;
    int32_t s0[4], s1[4];
    rows_of(start, s0);
    load(start, s0, la);
    rows_of(start + 64, s1);
    load(start + 64, s1, lb);
    rows_of(start + 128, s0);
    store(start, sM0, sV0, la);
    __syncthreads();
    // Steps run in pairs, so the loop has one path: with an odd number of
    // chunks the last step multiplies the zeros staged past the segment end,
    // which leaves every fp32 sum as it was (a sum is never -0).
    for (int64_t r0 = start; r0 < end; r0 += 128) {
      step(r0, sM0, sV0, sM1, sV1, lb, la, s0, s1);
      step(r0 + 64, sM1, sV1, sM0, sV0, la, lb, s1, s0);
    }
  }
  // Accumulator value jj of a lane: column c = 8*(jj/4) + 4*(lane/32) + jj%4 of
  // the wave's 32 columns, rank j = lane % 32.
  const int j = lane & 31;
#pragma unroll
  for (int vb = 0; vb < 2; ++vb) {
    if (vb >= nv) continue;
    float *o = J.out[vb] + e * J.stride_e[vb];
    const int rank = J.rank[vb];
    if (J.stride_c[vb] == 1) {
      // Rank-major rows of `cols` (dA): a store of the accumulators would
      // scatter 4-byte writes over 32 rows. The [32 ranks][128 columns] block
      // goes through LDS instead (16-byte chunks XOR-swizzled by the rank; the
      // K loop's last barrier has retired every read of the stage) and leaves
      // in 16-byte runs of whole rows.
      uint8_t *st = vb ? sM1 : sM0;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int q = wave * 8 + 2 * g + (lane >> 5);
        *reinterpret_cast<u32x4 *>(st + j * 512 + ((q ^ j) << 4)) =
            u32x4{__float_as_uint(acc[vb][4 * g]), __float_as_uint(acc[vb][4 * g + 1]),
                  __float_as_uint(acc[vb][4 * g + 2]), __float_as_uint(acc[vb][4 * g + 3])};
      }
      __syncthreads();
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        const int r = pass * 8 + (tid >> 5), q = tid & 31;
        const int64_t c = c0 + 4 * q;
        if (r < rank && c < cols)
          *reinterpret_cast<u32x4 *>(o + r * J.stride_j[vb] + c) =
              *reinterpret_cast<const u32x4 *>(st + r * 512 + ((q ^ r) << 4));
      }
    } else if (j < rank) {
      float *oj = o + j * J.stride_j[vb];
      const int64_t sc = J.stride_c[vb];
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int64_t c = c0 + wave * 32 + 8 * (jj >> 2) + 4 * (lane >> 5) + (jj & 3);
        if (c < cols) oj[c * sc] = acc[vb][jj];
      }
    }
  }
}

// One thread per 8 columns of one row.
// MX_ACT_SILU: each op is rounded to bf16 as the autograd of the bf16
// reference composition h = bf16(silu(g)) * u does (experts.py:289-317); the
// silu derivative is formed in fp32, as silu_backward does.
// MX_ACT_SWIGLU7: the fp32 derivative of _memory_bounded_swiglu7_backward
// (grouped_moe.py:309-335), rounded once per gradient:
//   dG = dh * (s + 1.702 gc s (1 - s)) [g <= 7] * (uc + 1),
//   dU = dh * gc s [-7 <= u <= 7], s = sigmoid(1.702 gc).
template <int ACT>
__global__ __launch_bounds__(256) void swiglu_backward_kernel(uint16_t *dgu, const uint16_t *g,
                                                              const uint16_t *u, int64_t rows,
                                                              int64_t f) {
  const int64_t chunks = f / 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * chunks) return;
  const int64_t r = i / chunks, c = (i - r * chunks) * 8;
  uint16_t *dg_row = dgu + r * 2 * f + c;
  const uint4 dv = *reinterpret_cast<const uint4 *>(dg_row);
  const uint4 gv = *reinterpret_cast<const uint4 *>(g + r * f + c);
  const uint4 uv = *reinterpret_cast<const uint4 *>(u + r * f + c);
  const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w}, gw[4] = {gv.x, gv.y, gv.z, gv.w};
  const uint32_t uw[4] = {uv.x, uv.y, uv.z, uv.w};
  uint32_t og[4], ou[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float dgo[2], duo[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float dh = bf16_bits_to_f32(h ? dw[q] >> 16 : dw[q] & 0xffffu);
      const float gg = bf16_bits_to_f32(h ? gw[q] >> 16 : gw[q] & 0xffffu);
      const float uu = bf16_bits_to_f32(h ? uw[q] >> 16 : uw[q] & 0xffffu);
      if (ACT == MX_ACT_SWIGLU7) {
        const float gc = fminf(gg, 7.0f), uc = fminf(fmaxf(uu, -7.0f), 7.0f);
        const float s7 = 1.0f / (1.0f + expf(-(1.702f * gc)));
        const float gd = gg <= 7.0f ? s7 + ((1.702f * gc) * s7) * (1.0f - s7) : 0.0f;
        dgo[h] = (dh * gd) * (uc + 1.0f);
        duo[h] = uu >= -7.0f && uu <= 7.0f ? dh * (gc * s7) : 0.0f;
        continue;
      }
      const float sig = __builtin_amdgcn_rcpf(1.0f + __expf(-gg));
      const float sg = round_bf16(gg * sig);
      const float dsg = round_bf16(dh * uu);
      duo[h] = dh * sg;
      dgo[h] = dsg * (sig * (1.0f + gg * (1.0f - sig)));
    }
    og[q] = pack_bf16x2(dgo[0], dgo[1]);
    ou[q] = pack_bf16x2(duo[0], duo[1]);
  }
  *reinterpret_cast<uint4 *>(dg_row) = make_uint4(og[0], og[1], og[2], og[3]);
  *reinterpret_cast<uint4 *>(dg_row + f) = make_uint4(ou[0], ou[1], ou[2], ou[3]);
}

}  // namespace

int swiglu_backward(uint16_t *dgu, const uint16_t *g, const uint16_t *u, int64_t rows,
                    int64_t f, int act, hipStream_t s) {
  const int64_t total = rows * (f / 8);
  if (total <= 0) return MX_OK;
  const dim3 grid(static_cast<unsigned>(ceil_div(total, 256)));
  if (act == MX_ACT_SWIGLU7)
    hipLaunchKernelGGL(swiglu_backward_kernel<MX_ACT_SWIGLU7>, grid, dim3(256), 0, s, dgu, g, u,
                       rows, f);
  else
    hipLaunchKernelGGL(swiglu_backward_kernel<MX_ACT_SILU>, grid, dim3(256), 0, s, dgu, g, u,
                       rows, f);
  return check_launch("SwiGLU backward");
}

int transpose_factors_multi(const FactorTransposes &jobs, hipStream_t s) {
  TransposeLaunch L = {};
  int64_t blocks = 0;
  for (int j = 0; j < jobs.n; ++j) {
    const FactorTranspose &t = jobs.job[j];
    const int64_t small = t.rows < t.cols ? t.rows : t.cols;
    if (t.total < 0 || (t.total > 0 && (small < 1 || small > 256 || t.total / small >= (int64_t{1} << 31)))) {
      set_error("LoRA factor transposes: one dimension must be a rank in [1, 256] and the other "
                "times the experts below 2^31 (got %lld x %lld)",
                static_cast<long long>(t.rows), static_cast<long long>(t.cols));
      return MX_ERR_INVALID;
    }
    L.job[L.n] = t;
    L.block0[L.n] = blocks;
    L.vec[L.n] = small % 8 == 0 && reinterpret_cast<uintptr_t>(t.src) % 16 == 0 &&
                 reinterpret_cast<uintptr_t>(t.dst) % 16 == 0;
    const int64_t lg = small == t.rows ? t.cols : t.rows;
    L.tiled[L.n] = L.vec[L.n] && lg % 8 == 0;
    if (t.total > 0)
      blocks += L.tiled[L.n]
                    ? t.total / (small * lg) * ceil_div(lg, kTileL) * ceil_div(small, kTileS)
                    : ceil_div(t.total / small, 256);
    ++L.n;
  }
  L.block0[L.n] = blocks;
  if (blocks <= 0) return MX_OK;
  hipLaunchKernelGGL(transpose_factors_multi_kernel, dim3(static_cast<unsigned>(blocks)),
                     dim3(256), 0, s, L);
  return check_launch("LoRA factor transposes");
}

int lora_weight_grads(const WeightGradJobs &jobs, const int64_t *seg_start,
                      const int64_t *seg_end, int experts, hipStream_t s) {
  if (jobs.n < 0 || jobs.n > kMaxGradJobs) {
    set_error("LoRA weight gradients: %d jobs (at most %d per launch)", jobs.n, kMaxGradJobs);
    return MX_ERR_INVALID;
  }
  GradLaunch L = {};
  int64_t blocks = 0;
  for (int i = 0; i < jobs.n; ++i) {
    const WeightGradJob &j = jobs.job[i];
    bool ok = j.m && j.cols > 0 && j.cols % 8 == 0 && j.nv >= 1 && j.nv <= 2;
    for (int b = 0; ok && b < j.nv; ++b)
      ok = j.v[b] && j.out[b] && j.rank[b] >= 1 && j.rank[b] <= 32;
    if (!ok) {
      set_error("LoRA weight gradients: job %d needs M, cols a multiple of 8, and 1-2 V blocks "
                "with outputs and ranks in [1, 32]", i);
      return MX_ERR_INVALID;
    }
    L.job[i] = j;
    L.block0[i] = blocks;
    L.col_blocks[i] = static_cast<int>(ceil_div(j.cols, 128));
    blocks += static_cast<int64_t>(L.col_blocks[i]) * experts;
  }
  L.n = jobs.n;
  L.block0[jobs.n] = blocks;
  L.seg_start = seg_start;
  L.seg_end = seg_end;
  if (blocks <= 0) return MX_OK;
  hipLaunchKernelGGL(lora_weight_grad_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     s, L);
  return check_launch("LoRA weight gradients");
}

}  // namespace mx
