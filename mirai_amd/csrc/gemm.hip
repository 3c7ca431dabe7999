// Grouped expert GEMMs on bf16 MFMA (v_mfma_f32_32x32x16_bf16, gfx950) over
// expert-sorted rows, with the frozen weights decoded from NF4 / INT8 on the
// way into LDS, the per-expert LoRA up-projection fused into the epilogue, and
// five epilogues. Forward (B = W^T, K along the weight rows' `in` axis):
//   EPI_SWIGLU  : h = silu(x w1^T + dA1) * (x w3^T + dA3)   (gate/up pair)
//   EPI_STORE   : y = x w^T + dA, rows written through a row map (down proj.)
//   EPI_LORA_A  : p = bf16(s * bf16(x a^T))  (LoRA down-projection, rank <= 32)
// Backward (B = W, K along the weights' `out` axis; the decoded rows land in
// LDS n-major and reach the MFMA through ds_read_b64_tr_b16):
//   EPI_STORE2  : dh = dy w2 + dz2 a2, and dx = [dG | dU] [w1; w3] + dz1 a1 +
//                 dz3 a3 through a row map (one or two LoRA terms)
//
// Work decomposition: the dispatch plan lists row tiles (expert, first row) of
// kTileM rows; a workgroup computes one (row tile, column tile) pair. The
// blockIdx -> tile mapping gives each of the 8 XCDs a contiguous run of tiles
// (workgroups are dispatched round-robin over XCDs), ordered row-tile major,
// so the column tiles sharing an activation tile, and the row tiles sharing an
// expert's weights, run on the same XCD and hit its L2.
#include <stdlib.h>

#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <type_traits>

#include "common.h"
#include "grads.h"
#include "lds_tr.h"
#include "plan.h"
#include "rows.h"

namespace mx {
namespace gemm {

constexpr int kNf4Block = 64;   // NF4 absmax block along K
constexpr int kLoraK = 32;        // one LDS-staged LoRA K chunk: two MFMA K steps
constexpr int kLoraMaxRank = 256; // largest LoRA rank the layer takes

enum { EPI_SWIGLU = 0, EPI_STORE = 1, EPI_LORA_A = 2, EPI_STORE2 = 4 };

// NF4 codes with a bf16 absmax (the build's own quantiser), an fp32 absmax
// (bitsandbytes payloads, the double-quantised absmax decoded at load) or the
// payload's two-level absmax decoded per K step (NF4_DQ: a uint8 code into a
// 256-entry table, a nested fp32 scale per 256 blocks, an fp32 offset per
// expert).
constexpr bool is_dq(int fmt) { return fmt == MX_FMT_NF4_DQ || fmt == MX_FMT_NF4_DQ_KN; }
constexpr bool is_nf4(int fmt) {
  return fmt == MX_FMT_NF4 || fmt == MX_FMT_NF4_F32 || fmt == MX_FMT_NF4_F32_KN || is_dq(fmt);
}
constexpr bool f32_absmax(int fmt) { return fmt == MX_FMT_NF4_F32 || fmt == MX_FMT_NF4_F32_KN; }
// Bytes of one block's absmax entry (DQ: the uint8 code).
constexpr int absmax_bytes(int fmt) { return f32_absmax(fmt) ? 4 : is_dq(fmt) ? 1 : 2; }
// Weights stored [E, in, out] with the NF4 blocks along out (a MAGI-2 packed
// group, x @ W[g]): the forward reads them as the backward reads [E, out, in]
// weights (B = W, transposed decode) and the backward as the forward does.
constexpr bool is_kn(int fmt) { return fmt == MX_FMT_NF4_F32_KN || fmt == MX_FMT_NF4_DQ_KN; }

// Block absmax i of a row as raw bits (a bf16 in the low half, fp32 bits, or
// the DQ absmax code).
template <int FMT>
__device__ __forceinline__ uint32_t load_absmax(const void *row, int64_t i) {
  if (f32_absmax(FMT)) return static_cast<const uint32_t *>(row)[i];
  if (is_dq(FMT)) return static_cast<const uint8_t *>(row)[i];
  return static_cast<const uint16_t *>(row)[i];
}
// The two-level absmax of a DQ block: fp32(fp32(code * nested) + offset), two
// roundings as in the payload's dequantisation (no fused multiply-add).
__device__ __forceinline__ float dq_absmax(float code, float nested, float offset) {
#pragma clang fp contract(off)
  const float scaled = code * nested;
  return scaled + offset;
}
template <int FMT>
__device__ __forceinline__ float absmax_value(uint32_t raw) {
  return f32_absmax(FMT) ? __uint_as_float(raw) : bf16_bits_to_f32(raw);
}

// Backward epilogues multiply by W itself rather than W^T; with weights stored
// [E, in, out] the forward does.
constexpr bool trans_b(int epi, int fmt) { return (epi == EPI_STORE2) != is_kn(fmt); }
// Launches whose tiles may run in K parts (Params::k_parts).
constexpr bool has_k_parts(int fmt, int epi) {
  return (fmt == MX_FMT_F32X3 && epi == EPI_STORE) || epi == EPI_LORA_A;
}

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

// Macro tile BM x BN x BK on a WAVES_M x WAVES_N grid of wavefronts; each
// wave owns a (BM/WAVES_M) x (BN/WAVES_N) sub-tile made of 32 x 32 MFMA blocks
// (v_mfma_f32_32x32x16_bf16). BK is 64 (one NF4 block per stage) or 32.
template <int BM_, int BN_, int WAVES_M, int WAVES_N, int BK_, int WAVES_PER_SIMD_ = 1>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_;
  // Occupancy the register budget is sized for (waves per SIMD).
  static constexpr int WAVES_PER_SIMD = WAVES_PER_SIMD_;
  static constexpr int NT = 64 * WAVES_M * WAVES_N;
  static constexpr int WAVES_N_ = WAVES_N;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int MB = WM / 32, NB = WN / 32;
  static constexpr int KSUB = BK / 16;           // MFMA K steps per stage
  static constexpr int CPR = BK / 8;             // 16-byte chunks per tile row
  static constexpr int A_CHUNKS = BM * CPR / NT; // A chunks per thread per stage
  static constexpr int A_ROW_STEP = NT / CPR;    // rows between a thread's A chunks
  static constexpr int B_TPR = NT / BN;          // threads per B row (1, 2 or 4)
  static constexpr int B_ELEMS = BK / B_TPR;     // B elements decoded per thread per stage
  static constexpr int STAGE_A = BM * BK * 2;
  static constexpr int STAGE_B = BN * BK * 2;
  static constexpr int LDS = 2 * STAGE_A + 2 * STAGE_B;
};

struct Params {
  const uint16_t *x;
  int64_t ldx;
  const int32_t *row_token;  // sorted row -> activation row (null: identity)
  int64_t K;
  const void *w[4];          // per B-row group: weight data
  const void *wscale[4];     // NF4 absmax (bf16 or fp32) / INT8 scale (bf16)
  int64_t wn[4];             // rows per expert of each weight
  int64_t k_split;           // transposed B: K rows taken from w[0], the rest from w[1]
  int64_t N;                 // output columns
  int n_tiles_n;
  const uint16_t *lora_p;    // [R, ldp] scaled low-rank activations, adapter i at column i * lora_rc
  int64_t ldp;
  int lora_rc;               // width of one adapter's low-rank columns (a multiple of 32)
  const uint16_t *lora_b[2]; // [E, N, r]
  int lora_r[2];
  int64_t lora_stride[4];    // EPI_LORA_A: factor rows per expert of each sub-adapter's factor
  const int2 *tiles;
  const int32_t *num_tiles;
  const int2 *tiles_r;       // dual launch: the 128-row remainder tiles
  const int32_t *num_tiles_r;
  int slots_tall;            // dual launch: per-XCD slots of the 256-row tiles
  int stagger;               // dual launch: leading per-XCD slots given to remainder tiles
  const int64_t *seg_end;
  uint16_t *out;
  int64_t ldo;
  const int32_t *out_row;    // sorted row -> output row (null: identity)
  uint16_t *save_gate;
  uint16_t *save_up;
  float scale[4];
  int split_r[4];            // MX_FMT_F32X3 LoRA down-projection: rank of each adapter
  // EPI_LORA_A: two adapters of rank <= 16 share one 32-column block, 16
  // factor rows each (columns [16a, 16a + 16) hold adapter a, written to its
  // own 32-column output block with zeros above).
  int lora_pack;
  int act;                   // EPI_SWIGLU: MX_ACT_SILU or MX_ACT_SWIGLU7
  // MX_FMT_NF4_DQ*: per weight group (as w[0], w[1]) the nested scales [E,
  // dq_npe], the offsets [E] and the 256-entry code table; wscale holds the
  // uint8 absmax codes.
  const float *dq_nested[2];
  const float *dq_offset[2];
  const float *dq_code[2];
  int64_t dq_npe[2];
  // MX_FMT_F32X3 down projection: K parts per tile (1: none) of k_part_len
  // columns each; part q writes its [hi | lo] planes at column 2 N q.
  // EPI_LORA_A: k_part_len is the canonical part of its K sum (0: one part);
  // with k_parts > 1 each part runs in its own workgroup and leaves its fp32
  // sums in part_out [k_parts][part_rows][part_ld].
  int k_parts;
  int64_t k_part_len;
  float *part_out;
  int64_t part_rows;
  int part_ld;
};

// Per-thread choice among the small kernel-argument arrays by explicit
// selects: indexing them with a thread-dependent value would copy the
// argument block to private (scratch) memory.
template <class V>
__device__ __forceinline__ V pick(const V (&a)[4], int i) {
  return i == 0 ? a[0] : i == 1 ? a[1] : i == 2 ? a[2] : a[3];
}
template <class V>
__device__ __forceinline__ V pick2(const V (&a)[2], int i) {
  return i == 0 ? a[0] : a[1];
}

// B-tile row j -> (weight group, output column / row of that weight).
template <int EPI, class T>
__device__ __forceinline__ void b_row(int j, int nt, int &which, int64_t &n) {
  if (EPI == EPI_SWIGLU) {
    // Each wave's WN columns hold WN/2 gate rows then the WN/2 up rows of the
    // same ffn columns, so every SwiGLU pair meets in one lane.
    constexpr int H = T::WN / 2;
    which = (j / H) & 1;
    n = static_cast<int64_t>(nt) * (T::BN / 2) + (j / T::WN) * H + (j % H);
  } else if (EPI == EPI_STORE || EPI == EPI_STORE2) {
    which = 0;
    n = static_cast<int64_t>(nt) * T::BN + j;
  } else {
    which = j >> 5;
    n = j & 31;
  }
}

// EPI_LORA_A rows of a packed block: sub-adapter j / 16, factor row j % 16.
__device__ __forceinline__ void b_row_packed(int j, int &which, int64_t &n) {
  which = j >> 4;
  n = j & 15;
}

// Row key of the 128-byte-row stage swizzle: any 16 consecutive rows at one
// logical chunk land on 16 distinct 16-byte slots of a 256-byte bank line (the
// MFMA fragment reads run conflict free), and any 8 consecutive rows on 8
// distinct slots of a 128-byte half.
__device__ __forceinline__ int swz_key64(int row) { return ((row >> 1) ^ (row << 2)) & 7; }

// Tile rows of BK bf16 = 8 (BK 64) or 4 (BK 32) 16-byte chunks, the chunk
// XOR-ed with a row key (above for BK 64).
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
  if (BK == 64) return row * 128 + ((chunk ^ swz_key64(row)) << 4);
  return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4);
}
__device__ __forceinline__ int swz64(int row, int chunk) {  // 64-byte rows (LoRA tiles)
  return row * 64 + ((chunk ^ ((row >> 1) & 3)) << 4);
}

// MAGI-2 swiglu7 of one fp32 gate / up pair (grouped_moe.py:287-306,
// magi2_preview.py:2785-2787): min(g, 7) * sigmoid(1.702 min(g, 7)) *
// (clamp(u, -7, 7) + 1), evaluated in fp32 in the reference's order.
__device__ __forceinline__ float swiglu7(float g, float u) {
  const float gc = fminf(g, 7.0f);
  const float uc = fminf(fmaxf(u, -7.0f), 7.0f);
  const float sig = 1.0f / (1.0f + expf(-(1.702f * gc)));
  return (gc * sig) * (uc + 1.0f);
}

// Rounds two fp32 values to bf16 precision, one conversion each.
__device__ __forceinline__ void round2(float &a, float &b) {
  a = round_bf16(a);
  b = round_bf16(b);
}

// The calling wave's index in its workgroup, as a value the compiler keeps in
// a scalar register.
__device__ __forceinline__ int uniform_wave_index() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

// Raw buffer over [base, base + bytes): accesses at offsets >= bytes are
// dropped (stores) or read zero (loads) by the hardware range check. Tile
// buffers stay far below 2 GiB.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const uint16_t *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(base), 0,
                                           static_cast<int32_t>(bytes > 0 ? bytes : 0), 0x00020000);
}


// NF4 decode in registers. `lo`/`hi` hold the low / high bytes of the 16
// decoded bf16 values bf16(level[q] * absmax) of the current block, 4 per
// register; v_perm_b32 looks four codes up at once.
// Signed byte N of w as fp32 in one VALU instruction: v_cvt_f32_i32 with an
// SDWA byte select and sign extension. (From the C++ conversion the compiler
// emits a bit-field extract and then the conversion: two instructions.)
template <int N>
__device__ __forceinline__ float sbyte_to_f32(uint32_t w) {
  float r;
  if constexpr (N == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0"
        : "=v"(r) : "v"(w));
  else if constexpr (N == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1"
        : "=v"(r) : "v"(w));
  else if constexpr (N == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2"
        : "=v"(r) : "v"(w));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3"
        : "=v"(r) : "v"(w));
  return r;
}

struct Nf4Table {
  uint32_t lo[4], hi[4];
};

__device__ __forceinline__ Nf4Table nf4_table(float a) {
  uint32_t p[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) p[j] = pack_bf16x2(kNF4Levels[2 * j] * a, kNF4Levels[2 * j + 1] * a);
  Nf4Table t;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // p[2j] = [lo(4j) hi(4j) lo(4j+1) hi(4j+1)], p[2j+1] likewise for 4j+2, 4j+3.
    t.lo[j] = __builtin_amdgcn_perm(p[2 * j + 1], p[2 * j], 0x06040200u);
    t.hi[j] = __builtin_amdgcn_perm(p[2 * j + 1], p[2 * j], 0x07050301u);
  }
  return t;
}

// Table lookup of four 4-bit codes. `s7` holds the low three bits of each code
// (one per byte), `pick` the byte selector i + 4 * bit3 of byte i's code: the
// halves of the table (codes 0..7 and 8..15) are looked up apart and merged
// byte by byte with one more v_perm_b32 each, so no per-byte mask is formed.
__device__ __forceinline__ void nf4_lookup4(const Nf4Table &t, uint32_t s7, uint32_t pick,
                                            uint32_t &lo, uint32_t &hi) {
  const uint32_t lo_a = __builtin_amdgcn_perm(t.lo[1], t.lo[0], s7);
  const uint32_t lo_b = __builtin_amdgcn_perm(t.lo[3], t.lo[2], s7);
  const uint32_t hi_a = __builtin_amdgcn_perm(t.hi[1], t.hi[0], s7);
  const uint32_t hi_b = __builtin_amdgcn_perm(t.hi[3], t.hi[2], s7);
  lo = __builtin_amdgcn_perm(lo_b, lo_a, pick);
  hi = __builtin_amdgcn_perm(hi_b, hi_a, pick);
}

// Eight codes (one packed dword: byte i holds element i in its low nibble and
// element i + 4 in its high nibble) -> four dwords of bf16 pairs in element
// order. The low nibbles give elements 0..3 and the high nibbles 4..7, so one
// v_perm_b32 per output dword interleaves the looked-up low and high bytes.
__device__ __forceinline__ void nf4_decode8(const Nf4Table &t, uint32_t c, uint32_t *out) {
  uint32_t le, he, lo_, ho;
  // Low nibbles: bit 3 of the code sits at bit 3 of each byte.
  nf4_lookup4(t, c & 0x07070707u, ((c >> 1) & 0x04040404u) | 0x03020100u, le, he);
  // High nibbles: bit 3 of the code is bit 7 of the byte.
  nf4_lookup4(t, (c >> 4) & 0x07070707u, ((c >> 5) & 0x04040404u) | 0x03020100u, lo_, ho);
  out[0] = __builtin_amdgcn_perm(he, le, 0x05010400u);   // e0, e1
  out[1] = __builtin_amdgcn_perm(he, le, 0x07030602u);   // e2, e3
  out[2] = __builtin_amdgcn_perm(ho, lo_, 0x05010400u);  // e4, e5
  out[3] = __builtin_amdgcn_perm(ho, lo_, 0x07030602u);  // e6, e7
}

// LoRA factor tiles of the epilogue (one [BN][32] tile per adapter).
template <int EPI, bool LORA, class T>
constexpr int lora_tile_bytes() {
  return LORA ? (EPI == EPI_STORE2 ? 2 : 1) * T::BN * 64 : 16;
}

// Gate / up run of 4 columns -> the packed bf16 h run. gv / uv (the fp32
// projections) end rounded as the reference's bf16 gate / up with the bf16
// LoRA deltas a / b added (experts.py:3370-3374), then the gated activation:
// silu(g) rounded to bf16 times u (experts.py:289-317), or swiglu7 in fp32
// rounded once (grouped_moe.py:287-306).
template <bool LORA>
__device__ __forceinline__ void gated_run(float (&gv)[4], float (&uv)[4], float (&a)[4],
                                          float (&b)[4], int act, uint32_t &h0, uint32_t &h1) {
  round2(gv[0], gv[1]);
  round2(gv[2], gv[3]);
  round2(uv[0], uv[1]);
  round2(uv[2], uv[3]);
  if (LORA) {
    round2(a[0], a[1]);
    round2(a[2], a[3]);
    round2(b[0], b[1]);
    round2(b[2], b[3]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      gv[q] += a[q];
      uv[q] += b[q];
    }
    round2(gv[0], gv[1]);
    round2(gv[2], gv[3]);
    round2(uv[0], uv[1]);
    round2(uv[2], uv[3]);
  }
  if (act == MX_ACT_SWIGLU7) {
    float hq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) hq[q] = swiglu7(gv[q], uv[q]);
    h0 = pack_bf16x2(hq[0], hq[1]);
    h1 = pack_bf16x2(hq[2], hq[3]);
  } else {
    float sv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) sv[q] = gv[q] * __builtin_amdgcn_rcpf(1.0f + __expf(-gv[q]));
    round2(sv[0], sv[1]);
    round2(sv[2], sv[3]);
    h0 = pack_bf16x2(sv[0] * uv[0], sv[1] * uv[1]);
    h1 = pack_bf16x2(sv[2] * uv[2], sv[3] * uv[3]);
  }
}

// Down / backward run of 4 columns: the bf16 projection plus the bf16 LoRA
// delta a, rounded again (experts.py:3370-3374).
template <bool LORA>
__device__ __forceinline__ void projection_run(float (&v)[4], float (&a)[4], uint32_t &w0,
                                               uint32_t &w1) {
  round2(v[0], v[1]);
  round2(v[2], v[3]);
  if (LORA) {
    round2(a[0], a[1]);
    round2(a[2], a[3]);
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] += a[q];
  }
  w0 = pack_bf16x2(v[0], v[1]);
  w1 = pack_bf16x2(v[2], v[3]);
}

// One (row tile, column tile) of the grouped GEMM: `tile` = (expert, first
// sorted row), `nt` the column tile. The LDS stages are the caller's four
// distinct __shared__ arrays (two stages of A and of B): once this is
// inlined the compiler sees those objects and can prove that the A DMA into
// one stage never aliases the LDS reads and B writes of the other, so it
// inserts no wait between them.
template <int FMT, int EPI, bool LORA, class T>
__device__ __forceinline__ void gemm_tile(Params p, int2 tile, int nt, uint8_t *sA0,
                                          uint8_t *sA1, uint8_t *sB0, uint8_t *sB1,
                                          uint8_t *sLt, const float *sCode, int part = 0) {
  constexpr int kLTile = lora_tile_bytes<EPI, LORA, T>();
  const int tid = threadIdx.x;
  // MX_FMT_F32X3: bf16 planes with K = 3 * in (loaded as bf16); the
  // epilogues keep fp32 and write split outputs.
  constexpr bool kSplit = FMT == MX_FMT_F32X3;
  // Its down projection in K parts (launches with too few tiles to fill the
  // GPU): part q multiplies K columns [q k_part_len, (q + 1) k_part_len) and
  // writes its own planes; the LoRA delta goes with part 0. The LoRA
  // down-projection likewise, its parts leaving fp32 sums (see below).
  constexpr bool kKParts = has_k_parts(FMT, EPI);
  int64_t k_off = 0;
  if constexpr (kKParts) {
    if (p.k_parts > 1) {
      k_off = static_cast<int64_t>(part) * p.k_part_len;
      if constexpr (EPI == EPI_STORE) {
        p.out += 2 * p.N * part;
        if (part != 0) p.lora_r[0] = p.lora_r[1] = 0;
      }
    }
  }
  const int e = tile.x;
  const int64_t row0 = tile.y;
  const int64_t row_end = p.seg_end[e];

  // ----------------------------------------------------- A (activations)
  // Rows past the segment end re-read the segment's last row: an A row only
  // feeds its own output row, which the epilogue discards, so the loads need
  // no guard (and the K loop no branches).
  constexpr int BK = T::BK;
  // A goes global -> LDS by DMA (global_load_lds_dwordx4): one wave
  // instruction fills 1 KB of the stage, lane l landing at byte 16*l. The lane
  // that lands on (row, physical chunk) loads the logical chunk the swizzle
  // maps there, so the stage ends up in the same swizzled layout.
  // The wave index is uniform: kept in scalar registers (LDS DMA bases, M0).
  const int wave = uniform_wave_index(), lane_id = tid & 63;
  constexpr int kRowsPerDma = 1024 / (BK * 2);
  const uint16_t *a_ptr[T::A_CHUNKS];
  int a_lds[T::A_CHUNKS];  // wave-uniform LDS byte offset of each DMA inside a stage
  int64_t a_src[T::A_CHUNKS];
  int a_col[T::A_CHUNKS];
#pragma unroll
  for (int i = 0; i < T::A_CHUNKS; ++i) {
    const int region = wave * T::A_CHUNKS + i;
    const int row = region * kRowsPerDma + lane_id / T::CPR;
    const int phys = lane_id % T::CPR;
    a_col[i] = 8 * (BK == 64 ? (phys ^ swz_key64(row)) : (phys ^ ((row >> 2) & 3)));
    a_src[i] = min(row0 + row, row_end - 1);
    a_lds[i] = region * 1024;
  }
  // The row map is read under one uniform branch, so the chunks' loads are
  // in flight together (one wait, not one per chunk).
  if (p.row_token) {
#pragma unroll
    for (int i = 0; i < T::A_CHUNKS; ++i) a_src[i] = p.row_token[a_src[i]];
  }
#pragma unroll
  for (int i = 0; i < T::A_CHUNKS; ++i) a_ptr[i] = p.x + a_src[i] * p.ldx + a_col[i] + k_off;

  // ------------------------------------------------------- B (weights)
  constexpr bool TRANS = trans_b(EPI, FMT);
  static_assert(!TRANS || (T::NT == 512 && T::BK == 64 && T::BN == 256),
                "transposed B assumes 8 waves, BK 64 and BN 256");
  const int bj = tid / T::B_TPR, bh = tid % T::B_TPR;
  int which = 0;
  int64_t bn = 0;
  if (!TRANS) b_row<EPI, T>(bj, nt, which, bn);
  if (EPI == EPI_LORA_A && p.lora_pack) b_row_packed(bj, which, bn);
  // Transposed B: lane = k row of the stage, wave = 32-column slice. Columns
  // past N re-read the last full 32-column slice (discarded by the epilogue).
  // SwiGLU with transposed B (weights [E, in, out]): slice tc holds 32 gate
  // columns (tc even) or the 32 up columns of the same ffn columns (tc odd),
  // the order b_row gives the B rows of the other layout.
  const int tk = tid & 63, tc = wave;
  const int t_which = (TRANS && EPI == EPI_SWIGLU) ? (tc & 1) : 0;
  const int64_t t_col_raw = (TRANS && EPI == EPI_SWIGLU)
                                ? static_cast<int64_t>(nt) * (T::BN / 2) + 32 * (tc >> 1)
                                : static_cast<int64_t>(nt) * T::BN + 32 * tc;
  const int64_t t_col0 = TRANS ? min(t_col_raw, p.N - 32) : 0;
  // Weight rows past N (a partial column tile) re-read row N-1: they only
  // feed output columns the epilogue discards. The LoRA down-projection
  // keeps explicit zeros, as its absent adapters have no rows at all.
  const int64_t wn_rows = pick(p.wn, which);
  const bool b_valid = EPI == EPI_LORA_A ? bn < wn_rows : !TRANS;
  if (EPI != EPI_LORA_A) bn = min(bn, wn_rows - 1);
  const int64_t wrow =
      static_cast<int64_t>(e) * (EPI == EPI_LORA_A ? pick(p.lora_stride, which) : wn_rows) + bn;
  const uint8_t *b_base = nullptr;
  const void *b_absmax = nullptr;  // the row's absmax entries
  // The backward over [E, in, out] weights reads its K rows from w[0] up to
  // k_split and from w[1] after it (dx = [dG | dU] [W1; W3]): two row bases.
  constexpr bool kSplitK = EPI == EPI_STORE2 && !TRANS;
  const int64_t row_k = kSplitK ? p.k_split : p.K;  // K extent of one weight row
  const uint8_t *b_base1 = nullptr;
  const void *b_absmax1 = nullptr;
  float b_scale = 0.0f;
  if (b_valid) {
    const uint8_t *w = static_cast<const uint8_t *>(pick(p.w, which));
    if (is_nf4(FMT)) {
      b_base = w + wrow * (row_k / 2) + bh * (T::B_ELEMS / 2);
      b_absmax = static_cast<const uint8_t *>(pick(p.wscale, which)) +
                 wrow * (row_k / kNf4Block) * absmax_bytes(FMT);
      if (kSplitK && p.k_split < p.K) {
        const int64_t wrow1 = static_cast<int64_t>(e) * p.wn[1] + bn;
        b_base1 = static_cast<const uint8_t *>(p.w[1]) + wrow1 * (row_k / 2) + bh * (T::B_ELEMS / 2);
        b_absmax1 = static_cast<const uint8_t *>(p.wscale[1]) +
                    wrow1 * (row_k / kNf4Block) * absmax_bytes(FMT);
      }
    } else if (FMT == MX_FMT_INT8) {
      b_base = w + wrow * p.K + bh * T::B_ELEMS;
      b_scale = bf16_bits_to_f32(static_cast<const uint16_t *>(pick(p.wscale, which))[wrow]);
    } else {
      b_base = w + (wrow * p.K + k_off) * 2 + bh * T::B_ELEMS * 2;
    }
  }
  // NF4_DQ, row decode: the nested scales of this thread's row. With K <= 16384
  // a row's blocks span at most two 256-block groups: `lo` up to block `sw` of
  // the row, `hi` after it (the same value when the row stays in one group).
  struct DqRow {
    float lo = 0.0f, hi = 0.0f, off = 0.0f;
    int sw = 0;
  };
  auto dq_row = [&](int wsel, int64_t row_in_expert, int64_t kblocks) -> DqRow {
    DqRow r;
    const float *nest = pick2(p.dq_nested, wsel) + static_cast<int64_t>(e) * pick2(p.dq_npe, wsel);
    const int64_t b0 = row_in_expert * kblocks;
    r.lo = nest[b0 >> 8];
    r.hi = nest[(b0 + kblocks - 1) >> 8];
    r.sw = static_cast<int>((((b0 >> 8) + 1) << 8) - b0);
    r.off = pick2(p.dq_offset, wsel)[e];
    return r;
  };
  DqRow dq0, dq1;
  if (is_dq(FMT) && !TRANS && b_valid) {
    dq0 = dq_row(which, bn, row_k / kNf4Block);
    if (kSplitK && p.k_split < p.K) dq1 = dq_row(1, bn, row_k / kNf4Block);
  }

  // Bytes of B per thread per stage, in 16-byte registers.
  constexpr int kBBytes = is_nf4(FMT) ? T::B_ELEMS / 2
                                            : (FMT == MX_FMT_INT8 ? T::B_ELEMS : T::B_ELEMS * 2);
  constexpr int kBRegs = kBBytes / 16;
  constexpr int kBStageBytes = is_nf4(FMT) ? BK / 2 : (FMT == MX_FMT_INT8 ? BK : BK * 2);
  // B packed data: two register sets (stage kt+1 is decoded while kt+2 loads).
  struct BRegs {
    u32x4 q[kBRegs];
    uint32_t abs;
    uint32_t nest;  // NF4_DQ, transposed decode: the block's nested scale (fp32 bits)
  };
  BRegs rb0, rb1;

  // DMA of A for step kt into the LDS stage sA.
  auto load_a = [&](int kt, uint8_t *sA) __attribute__((always_inline)) {
    const int64_t k0 = static_cast<int64_t>(kt) * BK;
#pragma unroll
    for (int i = 0; i < T::A_CHUNKS; ++i)
      __builtin_amdgcn_global_load_lds(
          reinterpret_cast<const void *>(a_ptr[i] + k0),
          reinterpret_cast<__attribute__((address_space(3))) void *>(
              reinterpret_cast<uintptr_t>(sA + a_lds[i])),
          16, 0, 0);
  };
  auto load_b = [&](int kt, BRegs &rb) __attribute__((always_inline)) {
    if (TRANS) {
      const int64_t kb = static_cast<int64_t>(kt) * BK;
      // K split (backward dx) or, for the SwiGLU pair, the slice's weight.
      const bool second = EPI == EPI_SWIGLU ? t_which != 0 : (EPI == EPI_STORE2 && kb >= p.k_split);
      const int64_t krow = kb - ((EPI == EPI_STORE2 && second) ? p.k_split : 0) + tk;
      const uint8_t *w = static_cast<const uint8_t *>(second ? p.w[1] : p.w[0]);
      const void *ws = second ? p.wscale[1] : p.wscale[0];
      const int64_t wrow = static_cast<int64_t>(e) * (second ? p.wn[1] : p.wn[0]) + krow;
      if (is_nf4(FMT)) {
        rb.q[0] = *reinterpret_cast<const u32x4 *>(w + wrow * (p.N / 2) + t_col0 / 2);
        rb.abs = load_absmax<FMT>(ws, wrow * (p.N / kNf4Block) + t_col0 / kNf4Block);
        if (is_dq(FMT)) {
          const int wsel = second ? 1 : 0;
          const int64_t blk = krow * (p.N / kNf4Block) + t_col0 / kNf4Block;  // within the expert
          rb.nest = __float_as_uint(
              pick2(p.dq_nested, wsel)[static_cast<int64_t>(e) * pick2(p.dq_npe, wsel) + (blk >> 8)]);
        }
      } else if (FMT == MX_FMT_INT8) {
#pragma unroll
        for (int q = 0; q < kBRegs; ++q)
          rb.q[q] = *reinterpret_cast<const u32x4 *>(w + wrow * p.N + t_col0 + 16 * q);
        rb.abs = static_cast<const uint16_t *>(ws)[wrow];
      } else {
#pragma unroll
        for (int q = 0; q < kBRegs; ++q)
          rb.q[q] = *reinterpret_cast<const u32x4 *>(w + (wrow * p.N + t_col0) * 2 + 16 * q);
        rb.abs = 0;
      }
    } else if (b_valid) {
      const uint8_t *bb = b_base;
      const void *ba = b_absmax;
      int ks = kt;
      if (kSplitK && static_cast<int64_t>(kt) * BK >= p.k_split) {
        bb = b_base1;
        ba = b_absmax1;
        ks = kt - static_cast<int>(p.k_split / BK);
      }
#pragma unroll
      for (int q = 0; q < kBRegs; ++q)
        rb.q[q] = *reinterpret_cast<const u32x4 *>(bb + static_cast<int64_t>(ks) * kBStageBytes + 16 * q);
      rb.abs = is_nf4(FMT) ? load_absmax<FMT>(ba, ks * BK / kNf4Block) : 0u;
    } else {
#pragma unroll
      for (int q = 0; q < kBRegs; ++q) rb.q[q] = u32x4{0u, 0u, 0u, 0u};
      rb.abs = 0;
    }
  };
  // The decode table of K stage `stage`'s block: level x absmax, the absmax
  // from the loaded bits (DQ: the code through its weight's table in LDS, times
  // the block's nested scale, plus the expert's offset).
  auto block_table = [&](const BRegs &rb, int stage) __attribute__((always_inline)) -> Nf4Table {
    if constexpr (is_dq(FMT)) {
      int wsel;
      float nested, off;
      if (TRANS) {
        const int64_t kb = static_cast<int64_t>(stage) * BK;
        const bool second = EPI == EPI_SWIGLU ? t_which != 0 : (EPI == EPI_STORE2 && kb >= p.k_split);
        wsel = second ? 1 : 0;
        nested = __uint_as_float(rb.nest);
        off = pick2(p.dq_offset, wsel)[e];
      } else {
        int ks = stage;
        DqRow d = dq0;
        wsel = which;
        if (kSplitK && static_cast<int64_t>(stage) * BK >= p.k_split) {
          ks = stage - static_cast<int>(p.k_split / BK);
          d = dq1;
          wsel = 1;
        }
        nested = ks < d.sw ? d.lo : d.hi;
        off = d.off;
      }
      return nf4_table(dq_absmax(sCode[wsel * 256 + rb.abs], nested, off));
    } else {
      return is_nf4(FMT) ? nf4_table(absmax_value<FMT>(rb.abs)) : Nf4Table{};
    }
  };
  // Decode part `part` (of KSUB) of this thread's B elements into LDS stage st.
  constexpr int kChunks = T::B_ELEMS / 8;  // 16-byte output chunks per thread
  constexpr int kChunksPerPart = kChunks / T::KSUB > 0 ? kChunks / T::KSUB : 1;
  const int chunk0 = bh * kChunks;
  auto decode_b = [&](const BRegs &rb, const Nf4Table &t, uint8_t *sB, int part) __attribute__((always_inline)) {
    if (part * kChunksPerPart >= kChunks) return;
#pragma unroll
    for (int cc = 0; cc < kChunksPerPart; ++cc) {
      const int c = part * kChunksPerPart + cc;  // output chunk: 8 elements
      uint32_t d[4];
      const float sc = TRANS ? bf16_bits_to_f32(rb.abs) : b_scale;
      if (is_nf4(FMT)) {
        // chunk c = code bytes 4c..4c+3 = dword c of the packed registers
        const u32x4 v = rb.q[c >> 2];
        const uint32_t word = (c & 3) == 0 ? v[0] : (c & 3) == 1 ? v[1] : (c & 3) == 2 ? v[2] : v[3];
        nf4_decode8(t, word, d);
      } else if (FMT == MX_FMT_INT8) {
        // chunk c = int8 bytes 8c..8c+7 = dwords 2c, 2c+1
        const u32x4 v = rb.q[c >> 1];
        const uint32_t w0 = (c & 1) ? v[2] : v[0];
        const uint32_t w1 = (c & 1) ? v[3] : v[1];
        const uint32_t ws[2] = {w0, w1};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t w = ws[h];
          const float q0 = sbyte_to_f32<0>(w);
          const float q1 = sbyte_to_f32<1>(w);
          const float q2 = sbyte_to_f32<2>(w);
          const float q3 = sbyte_to_f32<3>(w);
          d[2 * h] = pack_bf16x2(q0 * sc, q1 * sc);
          d[2 * h + 1] = pack_bf16x2(q2 * sc, q3 * sc);
        }
      } else {
        const u32x4 v = rb.q[c];
        d[0] = v[0];
        d[1] = v[1];
        d[2] = v[2];
        d[3] = v[3];
      }
      const int addr = TRANS ? swz_t(tk, 4 * tc + c) : swz<BK>(bj, chunk0 + c);
      *reinterpret_cast<u32x4 *>(sB + addr) = u32x4{d[0], d[1], d[2], d[3]};
    }
  };

  // -------------------------------------------------------------- MFMA
  const int lane = tid & 63, wid = wave;
  const int wm = wid / T::WAVES_N_, wn = wid % T::WAVES_N_;
  f32x16 acc[T::MB][T::NB];
#pragma unroll
  for (int mb = 0; mb < T::MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[mb][nb][j] = 0.0f;
  // EPI_LORA_A: its K sum runs in canonical parts of p.k_part_len columns, a
  // function of K alone. Each part's MFMA chain starts from zero and the parts
  // are added in order, ((0 + s0) + s1) + ..., whether one workgroup runs them
  // all (folding each finished part into tot) or each part runs in its own
  // workgroup (k_parts > 1) and a pass adds their fp32 sums in the same order.
  // So the result does not depend on how many rows a launch has, and a
  // token-chunked layer stays bit-identical to the whole one. (The 128-column
  // tile of ranks above 64 sums K in one part: tot would cost it occupancy;
  // the 32- and 64-column tiles fold.)
  constexpr bool kFold = EPI == EPI_LORA_A && T::BN <= 64;
  f32x16 tot[kFold ? T::MB : 1][kFold ? T::NB : 1];
  // Steps per part here (the whole K loop when this workgroup runs one part),
  // counted down to each fold.
  int fold_steps = 1, fold_left = 1;
  if constexpr (kFold) {
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
        for (int j = 0; j < 16; ++j) tot[mb][nb][j] = 0.0f;
    fold_steps = fold_left = static_cast<int>((p.k_part_len > 0 ? p.k_part_len : p.K) / T::BK);
  }
  auto fold = [&]() __attribute__((always_inline)) {
    if constexpr (kFold) {
#pragma unroll
      for (int mb = 0; mb < T::MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < T::NB; ++nb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            tot[mb][nb][j] += acc[mb][nb][j];
            acc[mb][nb][j] = 0.0f;
          }
    }
  };

  // MFMA operand fragments of one K sub-step, double-buffered so the reads
  // of sub-step kk+1 are in flight while sub-step kk multiplies.
  struct Frags {
    bf16x8 a[T::MB], b[T::NB];
  };
  auto read_frags = [&](Frags &f, const uint8_t *sA, const uint8_t *sB, int kk) __attribute__((always_inline)) {
    const int ch = kk * 2 + (lane >> 5);
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb)
      f.a[mb] = *reinterpret_cast<const bf16x8 *>(sA + swz<BK>(wm * T::WM + mb * 32 + (lane & 31), ch));
#pragma unroll
    for (int nb = 0; nb < T::NB; ++nb)
      f.b[nb] = TRANS ? read_b_trans(sB, wn * T::WN + nb * 32, kk, lane)
                      : *reinterpret_cast<const bf16x8 *>(sB + swz<BK>(wn * T::WN + nb * 32 + (lane & 31), ch));
  };
  auto mfma_frags = [&](const Frags &f) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < T::NB; ++nb)
        // Weight fragment first: the accumulator block is the transposed
        // product (see the epilogue), which lets a lane store 4 columns at once.
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[nb], f.a[mb], acc[mb][nb], 0, 0, 0);
  };
  Frags f0, f1;

  // One K step: MFMAs on stage `cur` interleaved with the decode of the next
  // stage's B (loaded one iteration earlier) into the other buffer; the next
  // A tile and the B tile two steps ahead are in flight meanwhile. Loads past
  // the end are clamped to the last step, so the body is branch free.
  const int KT = static_cast<int>((kKParts && p.k_parts > 1 ? p.k_part_len : p.K) / BK);
  // Stage (sA, sB) is multiplied while stage (nA, nB) is produced. f0 holds
  // the first sub-step's fragments of (sA, sB) on entry, and of (nA, nB) on
  // exit (read right after the barrier).
  // LoRA up-projection tiles for the epilogue: n_adapt low-rank activation
  // tiles [BM][32] (gate and up for EPI_SWIGLU, dz1 and dz3 for EPI_STORE2)
  // and n_lb factor tiles [BN][32], both in the swz64 layout. They are DMA'd
  // during the last K step: the activation tiles into the A stage that step
  // does not refill, the factor tiles into their own buffer (the last step
  // still decodes a B stage, so that no branch splits the step body).
  constexpr int n_adapt = (EPI == EPI_SWIGLU || EPI == EPI_STORE2) ? 2 : 1;
  constexpr int n_lb = EPI == EPI_STORE2 ? 2 : 1;
  constexpr int kWaves = T::NT / 64;
  constexpr int kPDma = n_adapt * T::BM * 64 / 1024, kLDma = n_lb * T::BN * 64 / 1024;
  static_assert(n_adapt * T::BM * 64 <= T::STAGE_A && (!LORA || n_lb * T::BN * 64 <= kLTile),
                "LoRA tiles must fit their buffers");
  static_assert(!LORA || (kPDma % kWaves == 0 && kLDma % kWaves == 0),
                "LoRA tiles split evenly over waves");
  auto dma16 = [&](const uint16_t *src, uint8_t *dst) __attribute__((always_inline)) {
    __builtin_amdgcn_global_load_lds(
        reinterpret_cast<const void *>(src),
        reinterpret_cast<__attribute__((address_space(3))) void *>(reinterpret_cast<uintptr_t>(dst)),
        16, 0, 0);
  };
  // `zero` is 0 at the call; it is derived from the step index so that the
  // address arithmetic stays in the last step instead of being hoisted out of
  // the K loop, where it would hold registers for the whole loop.
  auto load_lora = [&](uint8_t *dP, uint8_t *dL, int zero) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kPDma / kWaves; ++i) {
      const int g = i * kWaves + wave;
      const int pos = g * 1024 + 16 * lane_id + zero;
      const int ad = pos / (T::BM * 64), rem = pos - ad * T::BM * 64;
      // Each DMA covers 1 KB inside one adapter's tile; absent adapters'
      // columns are not staged (they may lie past the end of the buffer).
      if (pick2(p.lora_r, ad) == 0) continue;
      const int row = rem >> 6, c = ((rem >> 4) & 3) ^ ((row >> 1) & 3);
      // Rows past the segment end repeat its last row: they feed dropped outputs.
      const int64_t grow = min(row0 + row, row_end - 1);
      dma16(p.lora_p + grow * p.ldp + ad * p.lora_rc + c * 8, dP + g * 1024);
    }
#pragma unroll
    for (int i = 0; i < kLDma / kWaves; ++i) {
      const int g = i * kWaves + wave;
      const int pos = g * 1024 + 16 * lane_id + zero;
      const int ad = pos / (T::BN * 64), rem = pos - ad * T::BN * 64;
      const int j = rem >> 6, c = ((rem >> 4) & 3) ^ ((j >> 1) & 3);
      int lw = ad;
      int64_t n = static_cast<int64_t>(nt) * T::BN + j;
      if (EPI == EPI_SWIGLU) b_row<EPI, T>(j, nt, lw, n);
      n = min(n, p.N - 1);
      const int r = pick2(p.lora_r, lw);
      const uint16_t *lb = pick2(p.lora_b, lw);
      // Chunks past the rank re-read an in-rank chunk: the matching columns
      // of the activation tile are zero. Absent adapters are skipped by the
      // epilogue and read any valid row.
      const uint16_t *src = p.lora_p;
      if (lb && r > 0) src = lb + (static_cast<int64_t>(e) * p.N + n) * r + (c * 8 < r ? c : c % (r >> 3)) * 8;
      dma16(src, dL + g * 1024);
    }
  };
  auto step = [&](int kt, const uint8_t *sA, const uint8_t *sB, uint8_t *nA, uint8_t *nB,
                  BRegs &b_next, BRegs &b_after) __attribute__((always_inline)) {
    const bool last = LORA && kt + 1 == KT;
    if (last)
      load_lora(nA, sLt, kt + 1 - KT);
    else
      load_a(min(kt + 1, KT - 1), nA);
    load_b(min(kt + 2, KT - 1), b_after);
    const Nf4Table t = block_table(b_next, min(kt + 1, KT - 1));
#pragma unroll
    for (int kk = 0; kk < T::KSUB; ++kk) {
      Frags &cur = (kk & 1) ? f1 : f0;
      Frags &nxt = (kk & 1) ? f0 : f1;
      if (kk + 1 < T::KSUB) read_frags(nxt, sA, sB, kk + 1);
      mfma_frags(cur);
      decode_b(b_next, t, nB, kk);
    }
    if (kFold && --fold_left == 0) {
      fold();
      fold_left = fold_steps;
    }
    __syncthreads();
    read_frags(f0, nA, nB, 0);
  };

  load_a(0, sA0);
  load_b(0, rb0);
  load_b(min(1, KT - 1), rb1);
  {
    const Nf4Table t = block_table(rb0, 0);
#pragma unroll
    for (int part = 0; part < T::KSUB; ++part) decode_b(rb0, t, sB0, part);
  }
  __syncthreads();
  read_frags(f0, sA0, sB0, 0);
  // Steps alternate the two stages; the final step ends in stage KT & 1.
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    step(kt, sA0, sB0, sA1, sB1, rb1, rb0);
    step(kt + 1, sA1, sB1, sA0, sB0, rb0, rb1);
  }
  if (kt < KT) step(kt, sA0, sB0, sA1, sB1, rb1, rb0);
  if constexpr (kFold) {
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < T::NB; ++nb) acc[mb][nb] = tot[mb][nb];
  }

  // ------------------------------------------- LoRA up-projection (K = 32)
  // Multiplied block by block in the epilogue, into accumulators kept apart
  // from the frozen projection so the epilogue can round both to bf16 before
  // adding them, as the reference adds a bf16 LoRA delta to a bf16
  // projection output (experts.py:3370-3374). The tiles arrived with the last
  // K step, in the stage it left free.
  const uint8_t *sP = (KT & 1) ? sA1 : sA0;
  const uint8_t *sL = sLt;
  auto lora_block = [&](int mb, int nb) -> f32x16 {
    f32x16 t;
#pragma unroll
    for (int j = 0; j < 16; ++j) t[j] = 0.0f;
#pragma unroll
    for (int a2 = 0; a2 < n_lb; ++a2) {
      const int ad = EPI == EPI_SWIGLU ? (nb / (T::NB / 2)) : a2;
      const int r = pick2(p.lora_r, ad);
      if (r == 0) continue;  // absent adapter: its tiles are not staged
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        // Ranks up to 16 leave the second K step's activations zero: the
        // step would add exact zeros to a sum that is not -0.
        if (kk == 1 && r <= 16) break;
        const int ch = kk * 2 + (lane >> 5);
        const bf16x8 a = *reinterpret_cast<const bf16x8 *>(
            sP + ad * T::BM * 64 + swz64(wm * T::WM + mb * 32 + (lane & 31), ch));
        const bf16x8 b = *reinterpret_cast<const bf16x8 *>(
            sL + a2 * T::BN * 64 + swz64(wn * T::WN + nb * 32 + (lane & 31), ch));
        t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, t, 0, 0, 0);
      }
      if (r <= kLoraK) continue;
      // Ranks above 32: the further 32-wide K chunks read their fragments
      // straight from global memory (the tile's low-rank rows and factor rows
      // stay in L2) into the same fp32 sum, so the delta is still rounded
      // once. The factor row is the one the staged tile holds for this lane.
      const int j = wn * T::WN + nb * 32 + (lane & 31);
      int lw = ad;
      int64_t n = static_cast<int64_t>(nt) * T::BN + j;
      if (EPI == EPI_SWIGLU) b_row<EPI, T>(j, nt, lw, n);
      n = min(n, p.N - 1);
      const uint16_t *frow = pick2(p.lora_b, ad) + (static_cast<int64_t>(e) * p.N + n) * r;
      const int64_t prow = min(row0 + wm * T::WM + mb * 32 + (lane & 31), row_end - 1);
      const uint16_t *arow = p.lora_p + prow * p.ldp + ad * p.lora_rc;
      for (int c0 = kLoraK; c0 < r; c0 += kLoraK) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int col = c0 + kk * 16 + (lane >> 5) * 8;
          // Columns past the rank hold zero activations; their factor read
          // stays inside the row.
          const bf16x8 a = *reinterpret_cast<const bf16x8 *>(arow + col);
          const bf16x8 b = *reinterpret_cast<const bf16x8 *>(frow + (col < r ? col : 0));
          t = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, t, 0, 0, 0);
        }
      }
    }
    return t;
  };

  // ------------------------------------------------------------ epilogue
  // The MFMAs take the weight fragment first, so each 32 x 32 accumulator
  // block holds the transposed product: value j of a lane is output row
  // lane % 32 of the block, column 8 * (j / 4) + 4 * (lane / 32) + j % 4. A lane
  // thus owns runs of 4 consecutive columns of one row (values 4g .. 4g + 3)
  // and writes each run with one 8-byte store. Outputs whose rows are this
  // tile's own sorted rows go through buffer stores over exactly the tile's
  // valid rows: rows past the segment end fall outside the buffer and are
  // dropped by the hardware, and columns past N are sent out of range on
  // purpose, so no store needs a branch. Offsets are 32-bit byte offsets
  // inside one tile.
  const int lrow = lane & 31;       // row of the lane inside a block
  const int lcol = 4 * (lane >> 5); // first column of the lane's run in group 0
  const int64_t tile_rows = min(row_end - row0, static_cast<int64_t>(T::BM));
  constexpr uint32_t kDrop = 0x80000000u;  // beyond any tile buffer
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  auto st8 = [&](const __amdgpu_buffer_rsrc_t &rs, uint32_t off, uint32_t w0, uint32_t w1)
      __attribute__((always_inline)) {
    __builtin_amdgcn_raw_buffer_store_b64(u32x2{w0, w1}, rs, off, 0, 0);
  };
  // Gate / up run of 4 columns (values 4g..4g+3 of blocks (mb, nbp) and
  // (mb, nbp + NB/2)) -> the packed bf16 h run; gv / uv end rounded as the
  // reference's bf16 gate / up (with the bf16 LoRA deltas added).
  auto swiglu_run = [&](float (&gv)[4], float (&uv)[4], const f32x16 &lg, const f32x16 &lu, int g,
                        uint32_t &h0, uint32_t &h1, int act) __attribute__((always_inline)) {
    float a[4], b[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[q] = LORA ? lg[4 * g + q] : 0.0f;
      b[q] = LORA ? lu[4 * g + q] : 0.0f;
    }
    gated_run<LORA>(gv, uv, a, b, act, h0, h1);
  };
  // Down / backward run of 4 columns of block (mb, nb): the bf16 projection
  // plus the bf16 LoRA delta, rounded again (experts.py:3370-3374).
  auto store_run = [&](float (&v)[4], const f32x16 &l2, int g, uint32_t &w0, uint32_t &w1)
      __attribute__((always_inline)) {
    float a[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) a[q] = LORA ? l2[4 * g + q] : 0.0f;
    projection_run<LORA>(v, a, w0, w1);
  };
  // Staged stores: a lane's runs are 8 bytes of one row, 32 rows per store
  // instruction, which the memory system takes as partial-line writes. The
  // rounded tile goes to LDS first (the B stages are free after the K loop)
  // and leaves in 16-byte pieces of whole row runs. Staged rows are 16-byte
  // chunks XOR-swizzled by the row, so the 32 rows a wave writes at once
  // spread over the banks.
  const bool saves = EPI == EPI_SWIGLU && p.save_gate != nullptr;
  if (EPI == EPI_SWIGLU && !kSplit && !saves) {
    // Inference h: the whole [BM][BN/2] tile is staged (BM/2 rows per B
    // stage), then every wave stores BM/waves rows, 16 lanes per 256-byte row.
    constexpr int HC = T::BN / 2;
    constexpr int RSB = HC * 2;
    constexpr int CPRH = RSB / 16;
    static_assert(EPI != EPI_SWIGLU || (CPRH == 16 && (T::BM / 2) * RSB <= T::STAGE_B),
                  "h tile must fit the B stages");
    auto h_stage = [&](int r) -> uint8_t * {
      return (r < T::BM / 2 ? sB0 : sB1) + (r & (T::BM / 2 - 1)) * RSB;
    };
    // The activation is chosen once per tile, outside the unrolled runs.
    auto stage_h = [&](auto act_c) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb) {
      const int r = wm * T::WM + mb * 32 + lrow;
      uint8_t *srow = h_stage(r);
#pragma unroll
      for (int nbp = 0; nbp < T::NB / 2; ++nbp) {
        f32x16 lg, lu;
        if (LORA) {
          lg = lora_block(mb, nbp);
          lu = lora_block(mb, nbp + T::NB / 2);
        }
        const int hc0 = wn * (T::WN / 2) + nbp * 32 + lcol;  // h column of the run, g = 0
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float gv[4], uv[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            gv[q] = acc[mb][nbp][4 * g + q];
            uv[q] = acc[mb][nbp + T::NB / 2][4 * g + q];
          }
          uint32_t h0, h1;
          swiglu_run(gv, uv, lg, lu, g, h0, h1, decltype(act_c)::value);
          const int hc = hc0 + 8 * g;
          *reinterpret_cast<u32x2 *>(srow + (((hc >> 3) ^ (r & 15)) << 4) + ((hc & 7) << 1)) =
              u32x2{h0, h1};
        }
      }
    }
    };
    if (p.act == MX_ACT_SWIGLU7)
      stage_h(std::integral_constant<int, MX_ACT_SWIGLU7>{});
    else
      stage_h(std::integral_constant<int, MX_ACT_SILU>{});
    __syncthreads();
    constexpr int RPW = T::BM / kWaves;  // rows stored per wave
    const int c = lane & 15;
    const int64_t col = static_cast<int64_t>(nt) * HC + c * 8;
#pragma unroll
    for (int it = 0; it < RPW / 4; ++it) {
      const int r = wid * RPW + it * 4 + (lane >> 4);
      const u32x4 v = *reinterpret_cast<const u32x4 *>(h_stage(r) + ((c ^ (r & 15)) << 4));
      if (row0 + r < row_end && col < p.N)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(p.out + (row0 + r) * p.ldo + col));
    }
  } else if (EPI == EPI_SWIGLU) {
    const uint32_t ld2 = static_cast<uint32_t>(p.ldo) * 2u, n2 = static_cast<uint32_t>(p.N) * 2u;
    const auto rs_h = tile_rsrc(p.out + row0 * p.ldo, tile_rows * p.ldo * 2);
    const auto rs_g = tile_rsrc(saves ? p.save_gate + row0 * p.N : p.out, saves ? tile_rows * p.N * 2 : 0);
    const auto rs_u = tile_rsrc(saves ? p.save_up + row0 * p.N : p.out, saves ? tile_rows * p.N * 2 : 0);
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb) {
      const uint32_t r = static_cast<uint32_t>(wm * T::WM + mb * 32 + lrow);
#pragma unroll
      for (int nbp = 0; nbp < T::NB / 2; ++nbp) {
        f32x16 lg, lu;
        if (LORA) {
          lg = lora_block(mb, nbp);
          lu = lora_block(mb, nbp + T::NB / 2);
        }
        const int64_t f0 = static_cast<int64_t>(nt) * (T::BN / 2) + wn * (T::WN / 2) + nbp * 32 + lcol;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          // N is a multiple of 8: a run of 4 columns is wholly valid or not.
          const bool fok = f0 + 8 * g < p.N;
          const uint32_t fc = static_cast<uint32_t>(f0 + 8 * g) * 2u;
          const uint32_t off_h = fok ? r * ld2 + fc : kDrop;
          const uint32_t off_s = fok ? r * n2 + fc : kDrop;
          float gv[4], uv[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            gv[q] = acc[mb][nbp][4 * g + q];
            uv[q] = acc[mb][nbp + T::NB / 2][4 * g + q];
          }
          if constexpr (kSplit) {
            // fp32 layer: no intermediate rounding; h goes out as bf16 planes
            // [hi | hi | lo] (row stride 3N), the down projection's split A.
            float h[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              if (LORA) {
                gv[q] += lg[4 * g + q];
                uv[q] += lu[4 * g + q];
              }
              h[q] = p.act == MX_ACT_SWIGLU7 ? swiglu7(gv[q], uv[q])
                                             : gv[q] * __builtin_amdgcn_rcpf(1.0f + __expf(-gv[q])) * uv[q];
            }
            const uint32_t hi0 = pack_bf16x2(h[0], h[1]), hi1 = pack_bf16x2(h[2], h[3]);
            const uint32_t lo0 = pack_bf16x2(h[0] - bf16_bits_to_f32(hi0 & 0xffffu), h[1] - bf16_bits_to_f32(hi0 >> 16));
            const uint32_t lo1 = pack_bf16x2(h[2] - bf16_bits_to_f32(hi1 & 0xffffu), h[3] - bf16_bits_to_f32(hi1 >> 16));
            st8(rs_h, off_h, hi0, hi1);
            st8(rs_h, off_h + n2, hi0, hi1);
            st8(rs_h, off_h + 2 * n2, lo0, lo1);
            continue;
          }
          uint32_t h0, h1;
          swiglu_run(gv, uv, lg, lu, g, h0, h1, p.act);
          st8(rs_h, off_h, h0, h1);
          if (saves) {
            st8(rs_g, off_s, pack_bf16x2(gv[0], gv[1]), pack_bf16x2(gv[2], gv[3]));
            st8(rs_u, off_s, pack_bf16x2(uv[0], uv[1]), pack_bf16x2(uv[2], uv[3]));
          }
        }
      }
    }
  } else if ((EPI == EPI_STORE || EPI == EPI_STORE2) && !kSplit) {
    // Each wave stages its own [32][WN] rows of one row block at a time in a
    // private slice of the B stages, then stores them 16 bytes per lane,
    // WN / 8 lanes per row, through the row map.
    constexpr int CH = T::WN / 8;       // 16-byte chunks per staged row
    constexpr int RPI = 64 / CH;        // rows per store instruction
    constexpr int WSB = 32 * T::WN * 2; // staged bytes per wave
    static_assert((EPI != EPI_STORE && EPI != EPI_STORE2) || (4 * WSB <= T::STAGE_B && (CH == 8 || CH == 16)),
                  "wave slices must fit a B stage");
    uint8_t *stg = (wid < 4 ? sB0 : sB1) + (wid & 3) * WSB;
    const int c = lane % CH;
    const int64_t col = static_cast<int64_t>(nt) * T::BN + wn * T::WN + c * 8;
    // Output row of each of the lane's stores (-1: past the segment end),
    // read through the row map before any store: as far as the compiler
    // knows a store may alias the map, so a map load between stores would
    // wait for every store before it to complete.
    constexpr int NIT = 32 / RPI;
    int32_t orow[T::MB][NIT];
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb)
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int64_t rr = row0 + wm * T::WM + mb * 32 + it * RPI + lane / CH;
        const int64_t rc = min(rr, row_end - 1);
        const int32_t o = p.out_row ? p.out_row[rc] : static_cast<int32_t>(rc);
        orow[mb][it] = rr < row_end ? o : -1;
      }
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb) {
#pragma unroll
      for (int nb = 0; nb < T::NB; ++nb) {
        f32x16 l2;
        if (LORA) l2 = lora_block(mb, nb);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = acc[mb][nb][4 * g + q];
          uint32_t w0, w1;
          store_run(v, l2, g, w0, w1);
          const int wc = nb * 32 + 8 * g + lcol;  // column inside the wave's slice
          *reinterpret_cast<u32x2 *>(stg + lrow * (T::WN * 2) + (((wc >> 3) ^ (lrow & (CH - 1))) << 4) +
                                     ((wc & 7) << 1)) = u32x2{w0, w1};
        }
      }
      // The slice is private to the wave: its own LDS writes are ordered
      // before these reads.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int r = it * RPI + lane / CH;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(stg + r * (T::WN * 2) + ((c ^ (r & (CH - 1))) << 4));
        if (orow[mb][it] >= 0 && col < p.N)
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(p.out + static_cast<int64_t>(orow[mb][it]) * p.ldo + col));
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  } else if (EPI == EPI_STORE || EPI == EPI_STORE2) {
    // fp32 layer: y leaves as planes [hi | lo] (row stride 2N), straight from
    // the accumulators.
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb) {
      const int64_t rr = row0 + wm * T::WM + mb * 32 + lrow;
      const bool rok = rr < row_end;
      const int64_t r = min(rr, row_end - 1);
      const int64_t o = p.out_row ? static_cast<int64_t>(p.out_row[r]) : r;
      uint16_t *orow = p.out + o * p.ldo;
#pragma unroll
      for (int nb = 0; nb < T::NB; ++nb) {
        f32x16 l2;
        if (LORA) l2 = lora_block(mb, nb);
        const int64_t n0 = static_cast<int64_t>(nt) * T::BN + wn * T::WN + nb * 32 + lcol;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          // N is a multiple of 8: a run of 4 columns is wholly valid or not.
          const bool ok = rok && n0 + 8 * g < p.N;
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = acc[mb][nb][4 * g + q];
          if (LORA) {  // one rounding of the sum
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] += l2[4 * g + q];
          }
          const uint32_t w0 = pack_bf16x2(v[0], v[1]), w1 = pack_bf16x2(v[2], v[3]);
          uint16_t *dst = orow + n0 + 8 * g;
          const uint32_t l0 = pack_bf16x2(v[0] - bf16_bits_to_f32(w0 & 0xffffu), v[1] - bf16_bits_to_f32(w0 >> 16));
          const uint32_t l1 = pack_bf16x2(v[2] - bf16_bits_to_f32(w1 & 0xffffu), v[3] - bf16_bits_to_f32(w1 >> 16));
          if (ok) {
            *reinterpret_cast<u32x2 *>(dst) = u32x2{w0, w1};
            *reinterpret_cast<u32x2 *>(dst + p.N) = u32x2{l0, l1};
          }
        }
      }
    }
  } else if (EPI == EPI_LORA_A && p.k_parts > 1) {
    // EPI_LORA_A, one K part of the tile: its fp32 sums, rows and columns as
    // the output's, to part_out (the finishing pass adds the parts and rounds).
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb) {
      const int r = wm * T::WM + mb * 32 + lrow;
      if (r >= tile_rows) continue;
      float *prow = p.part_out + (static_cast<int64_t>(part) * p.part_rows + row0 + r) * p.part_ld;
#pragma unroll
      for (int nb = 0; nb < T::NB; ++nb) {
        const int nblk = wn * T::WN + nb * 32;
        if (nblk >= p.N) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int jc = 8 * g + lcol;
          *reinterpret_cast<f32x4 *>(prow + nblk + jc) =
              f32x4{acc[mb][nb][4 * g], acc[mb][nb][4 * g + 1], acc[mb][nb][4 * g + 2],
                    acc[mb][nb][4 * g + 3]};
        }
      }
    }
  } else {
    // EPI_LORA_A: p = bf16(s * bf16(x a^T)), as low_rank.to(bf16) * scale. A
    // 32-column block is one adapter.
    const uint32_t ld2 = static_cast<uint32_t>(p.ldo) * 2u;
    const auto rs_o = tile_rsrc(p.out + row0 * p.ldo, tile_rows * p.ldo * 2);
#pragma unroll
    for (int mb = 0; mb < T::MB; ++mb) {
      const uint32_t r = static_cast<uint32_t>(wm * T::WM + mb * 32 + lrow);
#pragma unroll
      for (int nb = 0; nb < T::NB; ++nb) {
        const int nblk = wn * T::WN + nb * 32;
        const float sc = pick(p.scale, nblk >> 5);
        const uint32_t base = nblk < p.N ? r * ld2 + static_cast<uint32_t>(nblk) * 2u : kDrop;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int jc = 8 * g + lcol;  // column of the run inside the adapter's block
          float v[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = acc[mb][nb][4 * g + q];
          if constexpr (!kSplit) {
            if (p.lora_pack) {
              // Packed block (nblk == 0): columns 16a.. hold adapter a, which
              // leaves at its own block a * 32, zeros in its upper 16 columns.
              const int a = jc >> 4, c = jc & 15;
              const float psc = pick(p.scale, a);
              round2(v[0], v[1]);
              round2(v[2], v[3]);
              const uint32_t o = nblk < p.N ? r * ld2 + static_cast<uint32_t>(32 * a + c) * 2u : kDrop;
              st8(rs_o, o, pack_bf16x2(v[0] * psc, v[1] * psc), pack_bf16x2(v[2] * psc, v[3] * psc));
              st8(rs_o, o == kDrop ? kDrop : o + 32u, 0u, 0u);
              continue;
            }
          }
          if constexpr (kSplit) {
            // fp32 layer: column j < r of an adapter block leaves as planes
            // [hi | hi | lo] at columns j, r + j, 2r + j (3r <= 32); columns
            // from 3r on are zero. The rank-side LoRA factor is split [hi | lo |
            // hi] likewise, so the epilogue's K = 32 product is fp32-accurate.
            // r is a multiple of 8, so a run of 4 columns is wholly inside one
            // of these ranges.
            const int rk = pick(p.split_r, nblk >> 5);
            const bool own = jc < rk, zero = jc >= 3 * rk;
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] *= sc;
            const uint32_t hi0 = pack_bf16x2(v[0], v[1]), hi1 = pack_bf16x2(v[2], v[3]);
            const uint32_t lo0 = own ? pack_bf16x2(v[0] - bf16_bits_to_f32(hi0 & 0xffffu), v[1] - bf16_bits_to_f32(hi0 >> 16)) : 0u;
            const uint32_t lo1 = own ? pack_bf16x2(v[2] - bf16_bits_to_f32(hi1 & 0xffffu), v[3] - bf16_bits_to_f32(hi1 >> 16)) : 0u;
            const uint32_t o_hi = own ? base + static_cast<uint32_t>(jc) * 2u : kDrop;
            const uint32_t o_hi2 = own ? base + static_cast<uint32_t>(rk + jc) * 2u : kDrop;
            const uint32_t o_lo = own ? base + static_cast<uint32_t>(2 * rk + jc) * 2u
                                      : (zero ? base + static_cast<uint32_t>(jc) * 2u : kDrop);
            st8(rs_o, o_hi, hi0, hi1);
            st8(rs_o, o_hi2, hi0, hi1);
            st8(rs_o, o_lo, lo0, lo1);
            continue;
          }
          round2(v[0], v[1]);
          round2(v[2], v[3]);
          st8(rs_o, base + static_cast<uint32_t>(jc) * 2u, pack_bf16x2(v[0] * sc, v[1] * sc),
              pack_bf16x2(v[2] * sc, v[3] * sc));
        }
      }
    }
  }
}

// ------------------------------------------------------------ light tiles
// An expert with at most kLightRows rows in a launch (skewed routing leaves
// many such) would pay a whole 128-row tile: the decode of its 256 x K weight
// tile into LDS plus 128-row MFMA work, for a few rows. Its light tile keeps
// the work per weight at one decode: all of the expert's token rows are staged
// in LDS once (the four stage buffers, one barrier), and each wave decodes its
// 32 weight rows straight into MFMA operands, each lane one whole 64-element
// NF4 block per 128-wide K step, with no B stage and no per-step barrier.
//
// K permutation: in K step b a lane of half h (lane / 32) supplies, for MFMA
// sub-step s, the 8 elements 128 b + 64 h + 8 s .. + 7 of its row, for the
// weight operand and the token operand alike; the sum over K is the same sum.
constexpr int kLightRows = 32;
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int FMT, int EPI>
constexpr bool light_capable() {
  return (FMT == MX_FMT_NF4 || FMT == MX_FMT_NF4_F32 || FMT == MX_FMT_NF4_DQ) &&
         (EPI == EPI_SWIGLU || EPI == EPI_STORE);
}

// Columns of K the four stage buffers hold for 32 rows (two of SA bytes, two of SB).
template <int SA, int SB>
constexpr int light_max_k() {
  return (2 * SA + 2 * SB) / (32 * 2);
}

// K in whole 128-wide steps (a lane takes one 64-block per step) that the
// stage buffers hold.
template <int SA, int SB>
__device__ __forceinline__ bool light_tile_fits(const Params &p, int2 tile) {
  return p.seg_end[tile.x] - tile.y <= kLightRows && p.K % 128 == 0 &&
         p.K <= light_max_k<SA, SB>();
}

template <int FMT, int EPI, bool LORA, int SA, int SB>
__device__ __forceinline__ void light_tile(const Params &p, int2 tile, int nt, uint8_t *sA0,
                                           uint8_t *sA1, uint8_t *sB0, uint8_t *sB1,
                                           const float *sCode) {
  static_assert(SA % 8192 == 0 && SB % 8192 == 0, "stage rows must be whole 256-byte groups");
  const int e = tile.x;
  const int64_t row0 = tile.y;
  const int64_t row_end = p.seg_end[e];
  const int m = static_cast<int>(row_end - row0);  // 1 .. kLightRows
  const int wave = uniform_wave_index(), lane = threadIdx.x & 63;
  const int K = static_cast<int>(p.K);
  // Stage region q holds K columns [kq0, kq0 + kq) of the 32 rows, row stride
  // 2 kq bytes, 16-byte chunks XOR-swizzled by (row & 15) inside each 256-byte
  // group so the 32 rows a fragment read touches spread over the banks.
  constexpr int kA = SA / 64, kB = SB / 64;  // K columns per region
  auto region = [&](int q) __attribute__((always_inline)) -> uint8_t * {
    return q == 0 ? sA0 : q == 1 ? sA1 : q == 2 ? sB0 : sB1;
  };
  auto region_k0 = [](int q) { return q < 2 ? q * kA : 2 * kA + (q - 2) * kB; };
  auto region_k = [](int q) { return q < 2 ? kA : kB; };

  // ------------------------------------------- token rows -> LDS (by DMA)
  // One DMA instruction fills 1 KB of a region (lane l at byte 16 l): rows of
  // that region whose K range starts inside the layer's K. Rows past the
  // segment are not loaded: they only feed output rows that are dropped.
  {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int kq = region_k(q), kq0 = region_k0(q);
      if (kq0 >= K) break;
      const int rows_per_dma = 1024 / (2 * kq);  // 1 (kq = 512) or 2 (kq = 256)
      const int n_dma = 32 / rows_per_dma;
      for (int d = wave; d < n_dma; d += 8) {
        if (d * rows_per_dma >= m) break;  // wave-uniform: the DMA's rows are past the segment
        const int row = d * rows_per_dma + (lane * 16) / (2 * kq);
        const int phys = ((lane * 16) % (2 * kq)) >> 4;
        const int chunk = phys ^ (row & 15);
        const int k = kq0 + 8 * chunk;
        if (row < m && k < K) {
          const int64_t sr = row0 + row;
          const int64_t src = p.row_token ? static_cast<int64_t>(p.row_token[sr]) : sr;
          __builtin_amdgcn_global_load_lds(
              reinterpret_cast<const void *>(p.x + src * p.ldx + k),
              reinterpret_cast<__attribute__((address_space(3))) void *>(
                  reinterpret_cast<uintptr_t>(region(q) + d * 1024)),
              16, 0, 0);
        }
      }
    }
  }

  // ----------------------------------------------------- the wave's weights
  const int li = lane & 31, h = lane >> 5;
  int which = 0;
  int64_t n;
  if (EPI == EPI_SWIGLU) {
    // Rows 0..15 of the wave's block: gate rows of ffn columns f0 .. f0 + 15;
    // rows 16..31: the up rows of the same columns, so value v and v + 8 of a
    // lane's accumulator are one (gate, up) pair.
    which = li >> 4;
    n = static_cast<int64_t>(nt) * 128 + 16 * wave + (li & 15);
  } else {
    n = static_cast<int64_t>(nt) * 256 + 32 * wave + li;
  }
  const int64_t n_row = min(n, p.N - 1);  // rows past N feed dropped columns
  const int64_t wrow = static_cast<int64_t>(e) * pick(p.wn, which) + n_row;
  const uint8_t *codes = static_cast<const uint8_t *>(pick(p.w, which)) + wrow * (p.K / 2);
  const uint8_t *absrow = static_cast<const uint8_t *>(pick(p.wscale, which)) +
                          wrow * (p.K / kNf4Block) * absmax_bytes(FMT);
  // NF4_DQ: the row's nested scales (K <= 2048 here: at most two groups).
  float dq_lo = 0.0f, dq_hi = 0.0f, dq_off = 0.0f;
  int dq_sw = 0;
  if constexpr (is_dq(FMT)) {
    const int64_t kblocks = p.K / kNf4Block, b0 = n_row * kblocks;
    const float *nest = pick2(p.dq_nested, which) + static_cast<int64_t>(e) * pick2(p.dq_npe, which);
    dq_lo = nest[b0 >> 8];
    dq_hi = nest[(b0 + kblocks - 1) >> 8];
    dq_sw = static_cast<int>((((b0 >> 8) + 1) << 8) - b0);
    dq_off = pick2(p.dq_offset, which)[e];
  }
  const int KS = K / 128;  // K steps
  struct Codes {
    u32x4 q[2];
    uint32_t abs;
  };
  auto load_codes = [&](int b, Codes &c) __attribute__((always_inline)) {
    const int blk = 2 * b + h;
    c.q[0] = *reinterpret_cast<const u32x4 *>(codes + blk * 32);
    c.q[1] = *reinterpret_cast<const u32x4 *>(codes + blk * 32 + 16);
    c.abs = load_absmax<FMT>(absrow, blk);
  };

  f32x16 acc;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
  Codes c0, c1;
  load_codes(0, c0);
  __syncthreads();  // the staged token rows of every wave

  auto kstep = [&](int b, const Codes &c) __attribute__((always_inline)) {
    const int k = 128 * b + 64 * h;
    int q = 0;
#pragma unroll
    for (int r = 1; r < 4; ++r) q += k >= region_k0(r) ? 1 : 0;
    const int kq = region_k(q);
    const uint8_t *arow = region(q) + li * (2 * kq);
    const int c0k = (k - region_k0(q)) >> 3;  // first 16-byte chunk of the lane's 64 elements
    Nf4Table t;
    if constexpr (is_dq(FMT)) {
      const int blk = 2 * b + h;
      t = nf4_table(dq_absmax(sCode[which * 256 + c.abs], blk < dq_sw ? dq_lo : dq_hi, dq_off));
    } else {
      t = nf4_table(absmax_value<FMT>(c.abs));
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int chunk = c0k + s;
      const int phys = (chunk & ~15) | ((chunk & 15) ^ (li & 15));
      const bf16x8 a = *reinterpret_cast<const bf16x8 *>(arow + phys * 16);
      uint32_t d[4];
      const u32x4 v = c.q[s >> 2];
      const uint32_t word = (s & 3) == 0 ? v[0] : (s & 3) == 1 ? v[1] : (s & 3) == 2 ? v[2] : v[3];
      nf4_decode8(t, word, d);
      const bf16x8 w = __builtin_bit_cast(bf16x8, u32x4{d[0], d[1], d[2], d[3]});
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w, a, acc, 0, 0, 0);
    }
  };
  // The codes of step b + 1 load while step b decodes.
  int b = 0;
  for (; b + 1 < KS; b += 2) {
    load_codes(b + 1, c1);
    kstep(b, c0);
    load_codes(min(b + 2, KS - 1), c0);
    kstep(b + 1, c1);
  }
  if (b < KS) kstep(b, c0);

  // --------------------------------------------------- LoRA up-projection
  // The low-rank row holds [gate rc | up rc] (SwiGLU) or the down adapter's
  // rc columns; one MFMA chain over them with each lane's factor row zero
  // outside its own adapter gives the gate and up deltas of the block apart.
  const int lrow = li;
  const int64_t prow_i = min(row0 + lrow, row_end - 1);
  f32x16 lacc;
#pragma unroll
  for (int j = 0; j < 16; ++j) lacc[j] = 0.0f;
  if (LORA) {
    constexpr int n_ad = EPI == EPI_SWIGLU ? 2 : 1;
#pragma unroll
    for (int ad = 0; ad < n_ad; ++ad) {
      const int r = pick2(p.lora_r, ad);
      if (r == 0) continue;
      const bool own = EPI == EPI_SWIGLU ? (which == ad) : true;
      const uint16_t *frow = pick2(p.lora_b, ad) + (static_cast<int64_t>(e) * p.N + n_row) * r;
      const uint16_t *arow = p.lora_p + prow_i * p.ldp + ad * p.lora_rc;
      for (int c = 0; c < r; c += 16) {
        const int col = c + 8 * h;
        // Columns past the rank hold zero activations; their factor read
        // stays inside the row.
        const bf16x8 a = *reinterpret_cast<const bf16x8 *>(arow + col);
        bf16x8 f = *reinterpret_cast<const bf16x8 *>(frow + (col < r ? col : 0));
        if (!own) f = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
        lacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f, a, lacc, 0, 0, 0);
      }
    }
  }

  // ------------------------------------------------------------ epilogue
  // Value v of a lane is output row lane % 32 of the block and block row
  // 8 (v / 4) + 4 h + v % 4: runs of 4 consecutive columns.
  if (lrow >= m) return;
  if (EPI == EPI_SWIGLU) {
    const int64_t r = row0 + lrow;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int64_t f0 = static_cast<int64_t>(nt) * 128 + 16 * wave + 8 * g + 4 * h;
      float gv[4], uv[4], a[4], bb[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        gv[q] = acc[4 * g + q];
        uv[q] = acc[8 + 4 * g + q];
        a[q] = LORA ? lacc[4 * g + q] : 0.0f;
        bb[q] = LORA ? lacc[8 + 4 * g + q] : 0.0f;
      }
      uint32_t h0, h1;
      gated_run<LORA>(gv, uv, a, bb, p.act, h0, h1);
      if (f0 < p.N) {
        *reinterpret_cast<u32x2 *>(p.out + r * p.ldo + f0) = u32x2{h0, h1};
        if (p.save_gate != nullptr) {
          *reinterpret_cast<u32x2 *>(p.save_gate + r * p.N + f0) =
              u32x2{pack_bf16x2(gv[0], gv[1]), pack_bf16x2(gv[2], gv[3])};
          *reinterpret_cast<u32x2 *>(p.save_up + r * p.N + f0) =
              u32x2{pack_bf16x2(uv[0], uv[1]), pack_bf16x2(uv[2], uv[3])};
        }
      }
    }
  } else {
    const int64_t sr = row0 + lrow;
    const int64_t o = p.out_row ? static_cast<int64_t>(p.out_row[sr]) : sr;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t n0 = static_cast<int64_t>(nt) * 256 + 32 * wave + 8 * g + 4 * h;
      float v[4], a[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] = acc[4 * g + q];
        a[q] = LORA ? lacc[4 * g + q] : 0.0f;
      }
      uint32_t w0, w1;
      projection_run<LORA>(v, a, w0, w1);
      if (n0 < p.N) *reinterpret_cast<u32x2 *>(p.out + o * p.ldo + n0) = u32x2{w0, w1};
    }
  }
}

// NF4_DQ: the code tables of the launch's weights (w[0], w[1]) into LDS,
// published by a barrier before any tile builds a decode table from them.
template <int FMT>
__device__ __forceinline__ void load_code_tables(const Params &p, float *sCode) {
  if constexpr (is_dq(FMT)) {
    for (int t = threadIdx.x; t < 512; t += blockDim.x) {
      const float *code = t < 256 ? p.dq_code[0] : p.dq_code[1];
      sCode[t] = code ? code[t & 255] : 0.0f;
    }
    __syncthreads();
  }
}

// One launch over one tile list (p.tiles, *p.num_tiles row tiles). The
// blockIdx -> tile map gives each of the 8 XCDs (workgroups go to XCDs
// round-robin) a contiguous run of tiles, row-tile major, so the column tiles
// that share an activation tile, and the row tiles that share an expert's
// weights, meet in one L2.
template <int FMT, int EPI, bool LORA, class T>
__global__ __launch_bounds__(T::NT) __attribute__((amdgpu_waves_per_eu(T::WAVES_PER_SIMD)))
void grouped_gemm_kernel(Params p) {
  // 128-row tiles of the layer GEMMs: A stages of 32 KB, so that the light
  // tile stages up to 2048 K columns (the kernel runs one workgroup per CU
  // by its registers, so the LDS costs no occupancy).
  constexpr bool kLight = light_capable<FMT, EPI>() && T::BM == 128;
  constexpr int kStageA = kLight && T::STAGE_A < 32768 ? 32768 : T::STAGE_A;
  __shared__ __attribute__((aligned(16))) uint8_t sA0[kStageA];
  __shared__ __attribute__((aligned(16))) uint8_t sA1[kStageA];
  __shared__ __attribute__((aligned(16))) uint8_t sB0[T::STAGE_B];
  __shared__ __attribute__((aligned(16))) uint8_t sB1[T::STAGE_B];
  __shared__ __attribute__((aligned(16))) uint8_t sLt[lora_tile_bytes<EPI, LORA, T>()];
  __shared__ float sCode[is_dq(FMT) ? 512 : 1];
  const int parts = has_k_parts(FMT, EPI) && p.k_parts > 1 ? p.k_parts : 1;
  const int total = *p.num_tiles * p.n_tiles_n * parts;
  const int per_xcd = (total + 7) >> 3;
  const int slot = blockIdx.x >> 3;
  if (slot >= per_xcd) return;
  const int job = (blockIdx.x & 7) * per_xcd + slot;
  if (job >= total) return;
  const int logical = job / parts, part = job - logical * parts;
  const int mt = logical / p.n_tiles_n;
  const int2 tile = p.tiles[mt];
  load_code_tables<FMT>(p, sCode);
  if constexpr (kLight) {
    if (light_tile_fits<kStageA, T::STAGE_B>(p, tile)) {
      light_tile<FMT, EPI, LORA, kStageA, T::STAGE_B>(p, tile, logical - mt * p.n_tiles_n, sA0,
                                                      sA1, sB0, sB1, sCode);
      return;
    }
  }
  gemm_tile<FMT, EPI, LORA, T>(p, tile, logical - mt * p.n_tiles_n, sA0, sA1, sB0, sB1, sLt, sCode,
                               part);
}

// 256-row tiles (p.tiles) and the 128-row remainder tiles (p.tiles_r) in one
// launch. Each XCD runs its share of the tall tiles (slots p.stagger ..
// p.stagger + p.slots_tall - 1, in the map above) and then the rest of its
// share of the remainder tiles, which so fill the tail of the tall ones
// instead of running as a launch of their own after it. The first p.stagger
// slots of an XCD take remainder tiles: those CUs start their tall tiles half
// a tile later, so the CUs' epilogues (the output stores) stop coinciding.
template <int FMT, int EPI, bool LORA, class Tall, class Short>
__global__ __launch_bounds__(Tall::NT) __attribute__((amdgpu_waves_per_eu(Tall::WAVES_PER_SIMD)))
void grouped_gemm_dual_kernel(Params p) {
  static_assert(Tall::NT == Short::NT && Tall::BN == Short::BN && Tall::BK == Short::BK &&
                    Short::STAGE_A <= Tall::STAGE_A && Short::STAGE_B == Tall::STAGE_B,
                "both tile heights share one workgroup shape and its LDS");
  __shared__ __attribute__((aligned(16))) uint8_t sA0[Tall::STAGE_A];
  __shared__ __attribute__((aligned(16))) uint8_t sA1[Tall::STAGE_A];
  __shared__ __attribute__((aligned(16))) uint8_t sB0[Tall::STAGE_B];
  __shared__ __attribute__((aligned(16))) uint8_t sB1[Tall::STAGE_B];
  __shared__ __attribute__((aligned(16))) uint8_t sLt[lora_tile_bytes<EPI, LORA, Tall>()];
  __shared__ float sCode[is_dq(FMT) ? 512 : 1];
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const bool tall = slot >= p.stagger && slot < p.stagger + p.slots_tall;
  if (tall) {
    const int total = *p.num_tiles * p.n_tiles_n;
    const int per_xcd = (total + 7) >> 3;
    const int st = slot - p.stagger;
    if (st >= per_xcd) return;
    const int logical = xcd * per_xcd + st;
    if (logical >= total) return;
    const int mt = logical / p.n_tiles_n;
    load_code_tables<FMT>(p, sCode);
    gemm_tile<FMT, EPI, LORA, Tall>(p, p.tiles[mt], logical - mt * p.n_tiles_n, sA0, sA1, sB0,
                                    sB1, sLt, sCode);
  } else {
    const int total = *p.num_tiles_r * p.n_tiles_n;
    const int per_xcd = (total + 7) >> 3;
    const int s2 = slot < p.stagger ? slot : slot - p.slots_tall;
    if (s2 >= per_xcd) return;
    const int logical = xcd * per_xcd + s2;
    if (logical >= total) return;
    const int mt = logical / p.n_tiles_n;
    const int2 tile = p.tiles_r[mt];
    load_code_tables<FMT>(p, sCode);
    // An expert's only tile, when it has at most kLightRows rows.
    if constexpr (light_capable<FMT, EPI>()) {
      if (light_tile_fits<Tall::STAGE_A, Tall::STAGE_B>(p, tile)) {
        light_tile<FMT, EPI, LORA, Tall::STAGE_A, Tall::STAGE_B>(p, tile, logical - mt * p.n_tiles_n,
                                                               sA0, sA1, sB0, sB1, sCode);
        return;
      }
    }
    gemm_tile<FMT, EPI, LORA, Short>(p, tile, logical - mt * p.n_tiles_n, sA0, sA1, sB0, sB1, sLt,
                                     sCode);
  }
}

template <int FMT, int EPI, bool LORA, class T>
int launch(const Params &p, int64_t max_row_tiles, hipStream_t s) {
  const int64_t total =
      max_row_tiles * p.n_tiles_n * (has_k_parts(FMT, EPI) && p.k_parts > 1 ? p.k_parts : 1);
  if (total <= 0) return MX_OK;
  const int64_t grid = 8 * ceil_div(total, 8);
  if (grid > 0x7fffffff) {
    set_error("grouped GEMM grid too large");
    return MX_ERR_INVALID;
  }
  hipLaunchKernelGGL((grouped_gemm_kernel<FMT, EPI, LORA, T>), dim3(static_cast<unsigned>(grid)),
                     dim3(T::NT), 0, s, p);
  return check_launch("grouped GEMM launch");
}

// The dual launch: room for max_tall 256-row tiles and max_short remainder
// tiles (upper bounds; the kernel reads the plan's counts).
template <int FMT, int EPI, bool LORA, class Tall, class Short>
int launch_dual(Params p, int64_t max_tall, int64_t max_short, hipStream_t s) {
  const int64_t slots_tall = ceil_div(max_tall * p.n_tiles_n, 8);
  const int64_t slots_short = ceil_div(max_short * p.n_tiles_n, 8);
  const int64_t grid = 8 * (slots_tall + slots_short);
  if (grid <= 0) return MX_OK;
  if (grid > 0x7fffffff) {
    set_error("grouped GEMM grid too large");
    return MX_ERR_INVALID;
  }
  p.slots_tall = static_cast<int>(slots_tall);
  p.stagger = static_cast<int>(std::min<int64_t>(p.stagger, slots_short));
  hipLaunchKernelGGL((grouped_gemm_dual_kernel<FMT, EPI, LORA, Tall, Short>),
                     dim3(static_cast<unsigned>(grid)), dim3(Tall::NT), 0, s, p);
  return check_launch("grouped GEMM launch");
}

// Row-tile height: 256-row tiles when experts average at least 256 rows (the
// taller tile's better MFMA / LDS ratio outweighs its tail waste from there
// on, measured at C2, C3 and C5), else 128-row tiles.
inline bool use_tall_tiles(int64_t rows, int experts) { return rows >= 256 * static_cast<int64_t>(experts); }

// fp32 layer, down projection on 128-row tiles: K parts per tile, so that a
// launch with few tiles (C1: at most 32 tiles of 48 K steps for 256 CUs)
// still spreads over the chip. Up to 6 parts, each of at least 8 K steps,
// while the launch stays within one workgroup per CU.
constexpr int kChipCUs = 256;
inline int f32x3_down_parts(int64_t rows, int experts, int64_t hidden, int64_t ffn) {
  if (use_tall_tiles(rows, experts)) return 1;
  const int64_t slots = (ceil_div(rows, kPlanTileM) + experts) * ceil_div(hidden, 256);
  const int64_t steps = 3 * ffn / 64;
  int best = 1;
  for (int kp = 2; kp <= 6; ++kp)
    if (steps % kp == 0 && steps / kp >= 8 && slots * kp <= kChipCUs) best = kp;
  return best;
}

// 128-row tiles only (experts averaging under 256 rows).
template <int EPI, bool LORA, class Short>
int launch_tile(int fmt, const Params &p, int64_t max_tiles, hipStream_t s) {
  switch (fmt) {
    case MX_FMT_BF16:
      return launch<MX_FMT_BF16, EPI, LORA, Short>(p, max_tiles, s);
    case MX_FMT_NF4:
      return launch<MX_FMT_NF4, EPI, LORA, Short>(p, max_tiles, s);
    case MX_FMT_NF4_F32:
      return launch<MX_FMT_NF4_F32, EPI, LORA, Short>(p, max_tiles, s);
    case MX_FMT_NF4_F32_KN:
      return launch<MX_FMT_NF4_F32_KN, EPI, LORA, Short>(p, max_tiles, s);
    case MX_FMT_NF4_DQ:
      return launch<MX_FMT_NF4_DQ, EPI, LORA, Short>(p, max_tiles, s);
    case MX_FMT_NF4_DQ_KN:
      return launch<MX_FMT_NF4_DQ_KN, EPI, LORA, Short>(p, max_tiles, s);
    case MX_FMT_INT8:
      return launch<MX_FMT_INT8, EPI, LORA, Short>(p, max_tiles, s);
    case MX_FMT_F32X3:
      if constexpr (EPI == EPI_SWIGLU || EPI == EPI_STORE)
        return launch<MX_FMT_F32X3, EPI, LORA, Short>(p, max_tiles, s);
      break;
  }
  set_error("unknown weight format %d", fmt);
  return MX_ERR_INVALID;
}

template <int EPI, bool LORA, class Tall, class Short>
int launch_tile_dual(int fmt, const Params &p, int64_t max_tall, int64_t max_short,
                     hipStream_t s) {
  switch (fmt) {
    case MX_FMT_BF16:
      return launch_dual<MX_FMT_BF16, EPI, LORA, Tall, Short>(p, max_tall, max_short, s);
    case MX_FMT_NF4:
      return launch_dual<MX_FMT_NF4, EPI, LORA, Tall, Short>(p, max_tall, max_short, s);
    case MX_FMT_NF4_F32:
      return launch_dual<MX_FMT_NF4_F32, EPI, LORA, Tall, Short>(p, max_tall, max_short, s);
    case MX_FMT_NF4_F32_KN:
      return launch_dual<MX_FMT_NF4_F32_KN, EPI, LORA, Tall, Short>(p, max_tall, max_short, s);
    // The backward's dual launch with LoRA fills the 160 KB of LDS without the
    // DQ code tables: DQ backward GEMMs take the 128-row launch (launch_fmt).
    case MX_FMT_NF4_DQ:
      if constexpr (EPI != EPI_STORE2)
        return launch_dual<MX_FMT_NF4_DQ, EPI, LORA, Tall, Short>(p, max_tall, max_short, s);
      break;
    case MX_FMT_NF4_DQ_KN:
      if constexpr (EPI != EPI_STORE2)
        return launch_dual<MX_FMT_NF4_DQ_KN, EPI, LORA, Tall, Short>(p, max_tall, max_short, s);
      break;
    case MX_FMT_INT8:
      return launch_dual<MX_FMT_INT8, EPI, LORA, Tall, Short>(p, max_tall, max_short, s);
    case MX_FMT_F32X3:
      if constexpr (EPI == EPI_SWIGLU || EPI == EPI_STORE)
        return launch_dual<MX_FMT_F32X3, EPI, LORA, Tall, Short>(p, max_tall, max_short, s);
      break;
  }
  set_error("unknown weight format %d", fmt);
  return MX_ERR_INVALID;
}

template <int EPI, bool LORA>
int launch_fmt(int fmt, Params p, const PlanLayout &PL, const PlanView &v, bool tall, hipStream_t s) {
  // Column tiles are 256 wide (EPI_SWIGLU: 128 ffn columns of gate and of up).
  // The forward down projection (store epilogue) runs faster with its 8
  // waves as 4 x 2 (64 x 128 per wave); the others as 2 x 4 (measured).
  using Tall = typename std::conditional<EPI == EPI_STORE, Tile<256, 256, 4, 2, 64>,
                                         Tile<256, 256, 2, 4, 64>>::type;
  using Short = Tile<128, 256, 2, 4, 64>;
  p.n_tiles_n = static_cast<int>(EPI == EPI_SWIGLU ? ceil_div(p.N, 128) : ceil_div(p.N, 256));
  if (EPI == EPI_STORE2 && (fmt == MX_FMT_NF4_DQ || fmt == MX_FMT_NF4_DQ_KN)) tall = false;
  if (!tall) {
    p.tiles = v.tiles;
    p.num_tiles = v.num_tiles;
    return launch_tile<EPI, LORA, Short>(fmt, p, PL.max_tiles, s);
  }
  // 256-row tiles over each expert's rows except a final remainder of at most
  // 128 rows, which gets a 128-row tile (a short remainder costs about half a
  // tall tile instead of a whole one); both kinds in one launch.
  p.tiles = v.tiles2m;
  p.num_tiles = v.num_tiles2m;
  p.tiles_r = v.tilesr;
  p.num_tiles_r = v.num_tilesr;
  // Half of the 32 CUs of an XCD (gfx950: 256 CUs in 8 XCDs) start on a
  // remainder tile when experts average under 1024 rows, where remainder
  // tiles are a large share of the work (A/B: C5 -2.6 %, C3 -1.3 %), and in
  // the forward down projection, whose epilogue is mostly output stores that
  // then stop coinciding across the chip (C4 down -1.8 %). At about 2048 rows
  // per expert the gate/up GEMM gained nothing from it and lost 1.2 % at C4.
  p.stagger = (EPI == EPI_STORE || PL.rows < 1024 * static_cast<int64_t>(PL.experts)) ? 16 : 0;
  return launch_tile_dual<EPI, LORA, Tall, Short>(fmt, p, PL.max_tiles2, PL.experts, s);
}

template <int EPI>
int launch_any(int fmt, bool lora, const Params &p, const PlanLayout &PL, const PlanView &v,
               hipStream_t s) {
  const bool tall = use_tall_tiles(PL.rows, PL.experts);
  return lora ? launch_fmt<EPI, true>(fmt, p, PL, v, tall, s)
              : launch_fmt<EPI, false>(fmt, p, PL, v, tall, s);
}

// ------------------------------------------------------------ host helpers
constexpr int kStageEvents = 7;
// Process-wide, not per thread: the autograd backward calls the library from
// another host thread than the forward.
void *g_stage_events[kStageEvents] = {};
int g_stage_count = 0;

void mark_stage(int i, hipStream_t s) {
  if (g_stage_count == kStageEvents && g_stage_events[i])
    (void)hipEventRecord(static_cast<hipEvent_t>(g_stage_events[i]), s);
}

// Columns of one adapter's low-rank plane: the rank rounded up to a whole
// LoRA K chunk (32).
int lora_width(int rank) {
  return rank <= kLoraK ? kLoraK : (rank + kLoraK - 1) / kLoraK * kLoraK;
}

struct LayerLayout {
  PlanLayout plan;
  size_t off_lora = 0, off_h = 0, off_y = 0, off_x = 0, off_sum = 0, bytes = 0;
};

// Scratch of the layer: plan | low-rank activations [R, 3 rc] (planes of rc
// columns for gate, up and down, rc = lora_width of the largest rank) |
// h [R, f] | y [R, d]. The fp32 (MX_FMT_F32X3) layer holds h as planes
// [R, 3f] and y as planes [R, 2d] per K part of its down projection, and adds
// the split tokens [T, 3d] and the fp32 combine of all y planes.
LayerLayout layer_layout(int64_t rows, int num_experts, int64_t hidden, int64_t ffn,
                         bool split = false, int64_t tokens = 0, int rc = kLoraK) {
  LayerLayout L;
  L.plan = plan_layout(rows, num_experts);
  size_t off = align_up(L.plan.bytes, 256);
  L.off_lora = off;
  off = align_up(off + sizeof(uint16_t) * rows * 3 * rc, 256);
  L.off_h = off;
  off = align_up(off + sizeof(uint16_t) * rows * ffn * (split ? 3 : 1), 256);
  L.off_y = off;
  const int64_t y_planes = split ? 2 * f32x3_down_parts(rows, num_experts, hidden, ffn) : 1;
  off = align_up(off + sizeof(uint16_t) * rows * hidden * y_planes, 256);
  L.off_x = off;
  if (split) {
    off = align_up(off + sizeof(uint16_t) * tokens * hidden * 3, 256);
    L.off_sum = off;  // fp32 [T, y_planes d]: the combine of the y planes
    off = align_up(off + sizeof(float) * tokens * hidden * y_planes, 256);
  }
  L.bytes = off;
  return L;
}

bool has_lora(const mx_lora *l) { return l && l->rank > 0; }

// Rows per expert of a stored weight: its out rows, or its in rows when it is
// stored [E, in, out] (MX_FMT_NF4_F32_KN).
int64_t wn_of(const mx_weight *w) {
  return w->format == MX_FMT_NF4_F32_KN || w->format == MX_FMT_NF4_DQ_KN ? w->in_features
                                                                           : w->out_features;
}

// Weight group i (0 or 1) of a launch: its data, rows per expert and absmax
// (NF4_DQ: the uint8 codes, with the nested scales, offsets and code table).
void set_weight(Params &p, int i, const mx_weight *w) {
  p.w[i] = w->data;
  p.wn[i] = wn_of(w);
  if (w->format == MX_FMT_NF4_DQ || w->format == MX_FMT_NF4_DQ_KN) {
    const mx_nf4_dq *dq = static_cast<const mx_nf4_dq *>(w->scale);
    p.wscale[i] = dq->absmax_q;
    p.dq_nested[i] = dq->nested_absmax;
    p.dq_offset[i] = dq->offsets;
    p.dq_code[i] = dq->code;
    p.dq_npe[i] = dq->nested_per_expert;
  } else {
    p.wscale[i] = w->scale;
  }
}

__global__ __launch_bounds__(256) void zero_f32_kernel(float *p, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
    p[i] = 0.0f;
}

// The LoRA gradients of a backward that sees no routed rows: the gradient of
// an empty sum, zero in every present buffer (dA [E, r, in], dB [E, out, r]),
// written here since the weight-gradient kernels never run.
int zero_lora_grads(const char *name, int64_t experts, int64_t hidden, int64_t ffn,
                    const mx_lora *l1, const mx_lora *l3, const mx_lora *l2, float *ga1,
                    float *gb1, float *ga3, float *gb3, float *ga2, float *gb2, hipStream_t s) {
  auto rank = [](const mx_lora *l) { return has_lora(l) ? static_cast<int64_t>(l->rank) : 0; };
  const struct {
    float *p;
    int64_t n;
  } bufs[6] = {{ga1, experts * rank(l1) * hidden}, {gb1, experts * ffn * rank(l1)},
               {ga3, experts * rank(l3) * hidden}, {gb3, experts * ffn * rank(l3)},
               {ga2, experts * rank(l2) * ffn},    {gb2, experts * hidden * rank(l2)}};
  for (const auto &b : bufs) {
    if (!b.p || b.n <= 0) continue;
    const int64_t blocks = std::min<int64_t>(ceil_div(b.n, 256), 4096);
    hipLaunchKernelGGL(zero_f32_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, b.p,
                       b.n);
  }
  return check_launch(name);
}

int lora_width(const mx_lora *a, const mx_lora *b, const mx_lora *c) {
  int r = 0;
  for (const mx_lora *l : {a, b, c})
    if (has_lora(l) && l->rank > r) r = l->rank;
  return lora_width(r);
}

int check_weight(const char *name, const char *key, const mx_weight *w, int64_t out_f,
                 int64_t in_f) {
  if (!w || !w->data) {
    set_error("%s: weight %s is missing", name, key);
    return MX_ERR_INVALID;
  }
  if (w->out_features != out_f || w->in_features != in_f) {
    set_error("%s: weight %s has shape [%lld, %lld], expected [%lld, %lld]", name, key,
              static_cast<long long>(w->out_features), static_cast<long long>(w->in_features),
              static_cast<long long>(out_f), static_cast<long long>(in_f));
    return MX_ERR_INVALID;
  }
  if (w->format < MX_FMT_BF16 || w->format > MX_FMT_NF4_DQ_KN) {
    set_error("%s: weight %s has unknown format %d", name, key, w->format);
    return MX_ERR_INVALID;
  }
  if (w->format != MX_FMT_BF16 && w->format != MX_FMT_F32X3 && !w->scale) {
    set_error("%s: weight %s needs its scale / absmax buffer", name, key);
    return MX_ERR_INVALID;
  }
  if (w->format == MX_FMT_NF4_DQ || w->format == MX_FMT_NF4_DQ_KN) {
    const mx_nf4_dq *dq = static_cast<const mx_nf4_dq *>(w->scale);
    // The stored rows: [out, in] or, for _KN, [in, out]; blocks of 64 along them.
    const int64_t row_len = w->format == MX_FMT_NF4_DQ ? in_f : out_f;
    const int64_t blocks = out_f * in_f / kNf4Block;
    if (!dq->absmax_q || !dq->nested_absmax || !dq->offsets || !dq->code ||
        dq->nested_per_expert < ceil_div(blocks, 256)) {
      set_error("%s: weight %s: the two-level absmax needs its codes, nested scales (%lld per "
                "expert), offsets and code table", name, key,
                static_cast<long long>(ceil_div(blocks, 256)));
      return MX_ERR_INVALID;
    }
    if (row_len % kNf4Block != 0 || row_len > 16384) {
      set_error("%s: weight %s: two-level absmax rows hold a multiple of 64 and at most 16384 "
                "elements, got %lld", name, key, static_cast<long long>(row_len));
      return MX_ERR_INVALID;
    }
  }
  return MX_OK;
}

int check_lora(const char *name, const char *key, const mx_lora *l) {
  if (!l || l->rank == 0) return MX_OK;
  if (l->rank < 0 || l->rank > kLoraMaxRank || l->rank % 8 != 0 || !l->a || !l->b) {
    set_error("%s: LoRA on %s needs a rank that is a multiple of 8 up to %d and both factors "
              "(got rank %d)", name, key, kLoraMaxRank, l->rank);
    return MX_ERR_INVALID;
  }
  return MX_OK;
}

Params base_params(const PlanView &v) {
  Params p = {};
  p.tiles = v.tiles;
  p.num_tiles = v.num_tiles;
  return p;
}

// The canonical part of a LoRA down-projection's K sum: the split of its K
// steps into the most equal parts, at most 6, of at least 8 steps each. It
// depends on K alone, so every launch over the same K sums alike.
int64_t lora_a_part_len(int64_t K) {
  const int64_t steps = K / 64;
  int best = 1;
  for (int d = 2; d <= 6; ++d)
    if (steps % d == 0 && steps / d >= 8) best = d;
  return K / best;
}

// The finishing pass of a LoRA down-projection run in K parts: the parts'
// fp32 sums added in part order (the order one workgroup folds them in), then
// the epilogue of the unsplit tile, per run of 4 columns of a sorted row.
struct LoraFinish {
  const float *part;
  int parts;
  int64_t rows;
  int ld;
  int N;
  uint16_t *out;
  int64_t ldo;
  float scale[4];
  int split_r[4];
  int pack;  // Params::lora_pack: two 16-column adapters in a 32-column block
};

template <bool SPLIT>
__global__ __launch_bounds__(256) void lora_a_finish_kernel(LoraFinish f) {
  const int runs = f.N / 4;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= f.rows * runs) return;
  const int64_t r = i / runs;
  const int c = static_cast<int>(i - r * runs) * 4;
  const float *src = f.part + r * f.ld + c;
  f32x4 a = *reinterpret_cast<const f32x4 *>(src);
  for (int q = 1; q < f.parts; ++q) {
    const f32x4 b = *reinterpret_cast<const f32x4 *>(src + q * f.rows * f.ld);
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = a[j] + b[j];
  }
  float v[4] = {a[0], a[1], a[2], a[3]};
  typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
  if (!SPLIT && f.pack) {
    // Adapter c / 16 leaves at its own 32-column block, zeros above its 16.
    const int ad = c >> 4, jp = c & 15;
    const float psc = pick(f.scale, ad);
    round2(v[0], v[1]);
    round2(v[2], v[3]);
    uint16_t *prow = f.out + r * f.ldo + 32 * ad + jp;
    *reinterpret_cast<u32x2v *>(prow) =
        u32x2v{pack_bf16x2(v[0] * psc, v[1] * psc), pack_bf16x2(v[2] * psc, v[3] * psc)};
    *reinterpret_cast<u32x2v *>(prow + 16) = u32x2v{0u, 0u};
    return;
  }
  const int blk = c >> 5, jc = c & 31;
  const float sc = pick(f.scale, blk);
  uint16_t *orow = f.out + r * f.ldo + (c - jc);
  if constexpr (SPLIT) {
    // The fp32 layer's planes [hi | hi | lo] at columns j, r + j, 2r + j.
    const int rk = pick(f.split_r, blk);
    const bool own = jc < rk, zero = jc >= 3 * rk;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] *= sc;
    const uint32_t hi0 = pack_bf16x2(v[0], v[1]), hi1 = pack_bf16x2(v[2], v[3]);
    if (own) {
      const uint32_t lo0 = pack_bf16x2(v[0] - bf16_bits_to_f32(hi0 & 0xffffu), v[1] - bf16_bits_to_f32(hi0 >> 16));
      const uint32_t lo1 = pack_bf16x2(v[2] - bf16_bits_to_f32(hi1 & 0xffffu), v[3] - bf16_bits_to_f32(hi1 >> 16));
      *reinterpret_cast<u32x2v *>(orow + jc) = u32x2v{hi0, hi1};
      *reinterpret_cast<u32x2v *>(orow + rk + jc) = u32x2v{hi0, hi1};
      *reinterpret_cast<u32x2v *>(orow + 2 * rk + jc) = u32x2v{lo0, lo1};
    } else if (zero) {
      *reinterpret_cast<u32x2v *>(orow + jc) = u32x2v{0u, 0u};
    }
  } else {
    round2(v[0], v[1]);
    round2(v[2], v[3]);
    *reinterpret_cast<u32x2v *>(orow + jc) =
        u32x2v{pack_bf16x2(v[0] * sc, v[1] * sc), pack_bf16x2(v[2] * sc, v[3] * sc)};
  }
}

// LoRA down-projection p = bf16(s * bf16(x a^T)) for adapters that share the
// same input rows: adapter i lands in columns [i rc, (i + 1) rc) of `out`,
// zero past its rank. A rank-r adapter runs as ceil(r / 32) sub-adapters of
// at most 32 factor rows (rows [32c, 32c + 32) of every expert's [r, K]
// factor), up to four sub-adapters per launch. With `part_buf` (fp32 scratch
// of part_bytes, free for the call) and few tiles for the chip, each tile's
// K parts run in workgroups of their own: a launch of `rows` sorted rows.
int lora_down(const PlanView &v, int experts, int64_t max_tiles, const uint16_t *x, int64_t ldx,
              const int32_t *row_token, int64_t K, const mx_lora *const *adapters, int n_adapt,
              int rc, uint16_t *out, int64_t ldo, hipStream_t s, bool split = false,
              int64_t rows = 0, float *part_buf = nullptr, size_t part_bytes = 0) {
  struct Sub {
    const uint16_t *a = nullptr;
    int rows = 0, stride = 0;
    float scale = 0.0f;
  };
  constexpr int kMaxSubs = 2 * kLoraMaxRank / kLoraK;
  const int per = rc / kLoraK;
  if (n_adapt < 1 || n_adapt * per > kMaxSubs) {
    set_error("LoRA down-projection: %d adapters of width %d exceed %d sub-adapters", n_adapt, rc,
              kMaxSubs);
    return MX_ERR_INVALID;
  }
  Sub subs[kMaxSubs];
  const int n_sub = n_adapt * per;
  for (int i = 0; i < n_adapt; ++i) {
    const mx_lora *l = adapters[i];
    for (int c = 0; c < per && has_lora(l) && kLoraK * c < l->rank; ++c) {
      Sub &u = subs[i * per + c];
      u.a = static_cast<const uint16_t *>(l->a) + static_cast<int64_t>(kLoraK) * c * K;
      u.rows = std::min(kLoraK, l->rank - kLoraK * c);
      u.stride = l->rank;
      u.scale = l->scale;
    }
  }
  // Two adapters of rank <= 16 (one sub-adapter each) share one 32-column
  // block of 16 factor rows apiece.
  const bool pack = !split && n_sub == 2 && per == 1 && subs[0].rows <= 16 && subs[1].rows <= 16;
  for (int first = 0; first < n_sub; first += 4) {
    const int cnt = std::min(4, n_sub - first);
    Params p = base_params(v);
    p.lora_pack = pack ? 1 : 0;
    p.x = x;
    p.ldx = ldx;
    p.row_token = row_token;
    p.K = K;
    for (int i = 0; i < cnt; ++i) {
      const Sub &u = subs[first + i];
      p.w[i] = u.a;
      p.wn[i] = u.rows;
      p.lora_stride[i] = u.stride;
      p.scale[i] = u.scale;
      p.split_r[i] = u.rows;
    }
    p.N = pack ? kLoraK : kLoraK * cnt;
    p.n_tiles_n = 1;
    p.seg_end = v.seg + experts;
    p.out = out + kLoraK * first;
    p.ldo = ldo;
    // The tile width of the launch below; the 32- and 64-column tiles sum K
    // in its canonical parts, and run them in workgroups of their own when
    // the launch would not give three workgroups to each CU.
    const int bn = (!split && (cnt == 1 || pack)) ? 32 : (split || cnt <= 2) ? 64 : 128;
    const int64_t part_len = bn <= 64 ? lora_a_part_len(K) : K;
    const int kpc = static_cast<int>(K / part_len);
    p.k_part_len = kpc > 1 ? part_len : 0;
    const bool parts = kpc > 1 && part_buf && rows > 0 && max_tiles * kpc <= 3 * kChipCUs &&
                       static_cast<size_t>(kpc) * rows * bn * sizeof(float) <= part_bytes;
    if (parts) {
      p.k_parts = kpc;
      p.part_out = part_buf;
      p.part_rows = rows;
      p.part_ld = bn;
    }
    // Up to two sub-adapters fill a 64-column tile, one a 32-column tile;
    // the kernel is bound by the activation reads, so the narrowest tile
    // (more workgroups per CU, less MFMA and factor traffic) is the fastest
    // (one adapter on 32 columns against 64: C4's h launch 139 -> 136 us, the
    // C5 backward 1.10 -> 1.09 ms; K stages of 32, for more resident
    // workgroups, measured slower: 112 vs 92 us at the target shape). The
    // fp32 layer (split planes, K = 3 * in) writes split outputs.
    int rc2;
    if (split)
      rc2 = launch<MX_FMT_F32X3, EPI_LORA_A, false, Tile<128, 64, 4, 1, 64>>(p, max_tiles, s);
    else if (cnt == 1 || pack)
      rc2 = launch<MX_FMT_BF16, EPI_LORA_A, false, Tile<128, 32, 4, 1, 64>>(p, max_tiles, s);
    else if (cnt <= 2)
      rc2 = launch<MX_FMT_BF16, EPI_LORA_A, false, Tile<128, 64, 4, 1, 64>>(p, max_tiles, s);
    else
      rc2 = launch<MX_FMT_BF16, EPI_LORA_A, false, Tile<128, 128, 2, 2, 64>>(p, max_tiles, s);
    if (rc2) return rc2;
    if (parts) {
      LoraFinish f = {};
      f.part = part_buf;
      f.parts = kpc;
      f.rows = rows;
      f.ld = bn;
      f.N = static_cast<int>(p.N);
      f.pack = p.lora_pack;
      f.out = p.out;
      f.ldo = ldo;
      for (int i = 0; i < 4; ++i) {
        f.scale[i] = p.scale[i];
        f.split_r[i] = p.split_r[i];
      }
      const dim3 grid(static_cast<unsigned>(ceil_div(rows * (p.N / 4), 256)));
      if (split)
        hipLaunchKernelGGL(lora_a_finish_kernel<true>, grid, dim3(256), 0, s, f);
      else
        hipLaunchKernelGGL(lora_a_finish_kernel<false>, grid, dim3(256), 0, s, f);
      if ((rc2 = check_launch("LoRA down-projection parts"))) return rc2;
    }
  }
  return MX_OK;
}

// gate/up grouped GEMM with SwiGLU epilogue, then the down grouped GEMM.
int expert_mlp(const PlanLayout &PL, const PlanView &v, int experts, const uint16_t *x,
               int64_t ldx, const int32_t *row_token, int64_t hidden, int64_t ffn, int act,
               const mx_weight *w1, const mx_weight *w3, const mx_weight *w2,
               const mx_lora *l1, const mx_lora *l3, const mx_lora *l2, uint16_t *lora_buf,
               int lrc, uint16_t *h, uint16_t *save_gate, uint16_t *save_up, uint16_t *y, int64_t ldy,
               const int32_t *out_row, hipStream_t s) {
  const bool lora13 = has_lora(l1) || has_lora(l3);
  const bool lora2 = has_lora(l2);
  // fp32 layer (MX_FMT_F32X3): K runs over three bf16 planes, h is written as
  // planes, and the LoRA factors carry 3r split columns.
  const bool split = w1->format == MX_FMT_F32X3;
  const int64_t kx = split ? 3 : 1;
  const int rx = split ? 3 : 1;
  int rc;
  // A LoRA down-projection run in K parts keeps its fp32 sums in the buffer
  // the next GEMM writes: h before the gate/up GEMM, y before the down GEMM.
  const int64_t R = PL.rows;
  if (lora13) {
    const mx_lora *ad[2] = {l1, l3};
    rc = lora_down(v, experts, PL.max_tiles, x, ldx, row_token, kx * hidden, ad, 2, lrc,
                   lora_buf, 3 * lrc, s, split, R, reinterpret_cast<float *>(h),
                   sizeof(uint16_t) * R * kx * ffn);
    if (rc) return rc;
  }
  mark_stage(2, s);
  {
    Params p = base_params(v);
    p.x = x;
    p.ldx = ldx;
    p.row_token = row_token;
    p.K = kx * hidden;
    set_weight(p, 0, w1);
    set_weight(p, 1, w3);
    p.N = ffn;
    p.lora_p = lora_buf;
    p.ldp = 3 * lrc;
    p.lora_rc = lrc;
    p.lora_b[0] = has_lora(l1) ? static_cast<const uint16_t *>(l1->b) : nullptr;
    p.lora_b[1] = has_lora(l3) ? static_cast<const uint16_t *>(l3->b) : nullptr;
    p.lora_r[0] = has_lora(l1) ? rx * l1->rank : 0;
    p.lora_r[1] = has_lora(l3) ? rx * l3->rank : 0;
    p.seg_end = v.seg + experts;
    p.out = h;
    p.ldo = kx * ffn;
    p.save_gate = save_gate;
    p.save_up = save_up;
    p.act = act;
    rc = launch_any<EPI_SWIGLU>(w1->format, lora13, p, PL, v, s);
    if (rc) return rc;
  }
  mark_stage(3, s);
  if (lora2) {
    const mx_lora *ad[1] = {l2};
    rc = lora_down(v, experts, PL.max_tiles, h, kx * ffn, nullptr, kx * ffn, ad, 1, lrc,
                   lora_buf + 2 * lrc, 3 * lrc, s, split, R, reinterpret_cast<float *>(y),
                   sizeof(uint16_t) * R * ldy);
    if (rc) return rc;
  }
  mark_stage(4, s);
  Params p = base_params(v);
  p.x = h;
  p.ldx = kx * ffn;
  p.row_token = nullptr;
  p.K = kx * ffn;
  set_weight(p, 0, w2);
  p.N = hidden;
  p.lora_p = lora_buf + 2 * lrc;
  p.ldp = 3 * lrc;
  p.lora_rc = lrc;
  p.lora_b[0] = lora2 ? static_cast<const uint16_t *>(l2->b) : nullptr;
  p.lora_r[0] = lora2 ? rx * l2->rank : 0;
  p.seg_end = v.seg + experts;
  p.out = y;
  p.ldo = ldy;
  p.out_row = out_row;
  if (split) {
    p.k_parts = f32x3_down_parts(PL.rows, experts, hidden, ffn);
    p.k_part_len = 3 * ffn / p.k_parts;
  }
  return launch_any<EPI_STORE>(w2->format, lora2, p, PL, v, s);
}

int check_layer(const char *name, int64_t hidden, int64_t ffn, const mx_weight *w1,
                const mx_weight *w3, const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                const mx_lora *l2) {
  if (hidden <= 0 || ffn <= 0 || hidden % 64 != 0 || ffn % 64 != 0) {
    set_error("%s: hidden and ffn must be positive multiples of 64 (got %lld, %lld)", name,
              static_cast<long long>(hidden), static_cast<long long>(ffn));
    return MX_ERR_INVALID;
  }
  int rc;
  if ((rc = check_weight(name, "w1", w1, ffn, hidden))) return rc;
  if ((rc = check_weight(name, "w3", w3, ffn, hidden))) return rc;
  if ((rc = check_weight(name, "w2", w2, hidden, ffn))) return rc;
  if (w1->format != w3->format) {
    set_error("%s: w1 and w3 must share one storage format", name);
    return MX_ERR_INVALID;
  }
  if ((rc = check_lora(name, "w1", l1))) return rc;
  if ((rc = check_lora(name, "w3", l3))) return rc;
  if ((rc = check_lora(name, "w2", l2))) return rc;
  const bool split = w1->format == MX_FMT_F32X3;
  if (split != (w2->format == MX_FMT_F32X3)) {
    set_error("%s: MX_FMT_F32X3 (fp32) weights must be used for all three projections", name);
    return MX_ERR_INVALID;
  }
  if (split) {
    const mx_lora *ls[3] = {l1, l3, l2};
    for (const mx_lora *l : ls)
      if (has_lora(l) && l->rank != 8) {
        set_error("%s: the fp32 (MX_FMT_F32X3) layer takes LoRA factors padded to rank 8 "
                  "(split into 24 columns); got rank %d", name, l->rank);
        return MX_ERR_INVALID;
      }
  }
  return MX_OK;
}

// ------------------------------------------------------------ backward
struct BackLayout {
  PlanLayout plan;
  size_t off_dy = 0, off_dgu = 0, off_dz = 0, off_fact[6] = {}, bytes = 0;
  int rc = kLoraK;
};

// Scratch of the backward: plan, dy [R, d] (slot order; reused for the per-
// slot dx rows), [dG | dU] [R, 2f] and dz [R, 3 rc] (sorted order; planes of
// rc columns as the forward's low-rank activations), and the six transposed
// LoRA factors (B2^T, A2^T, B1^T, A1^T, B3^T, A3^T) at rank <= rc.
BackLayout back_layout(int64_t rows, int num_experts, int64_t hidden, int64_t ffn,
                       int rc = kLoraK) {
  BackLayout L;
  L.rc = rc;
  L.plan = plan_layout(rows, num_experts);
  size_t off = align_up(L.plan.bytes, 256);
  L.off_dy = off;
  off = align_up(off + sizeof(uint16_t) * rows * hidden, 256);
  L.off_dgu = off;
  off = align_up(off + sizeof(uint16_t) * rows * 2 * ffn, 256);
  L.off_dz = off;
  off = align_up(off + sizeof(uint16_t) * rows * 3 * rc, 256);
  const int64_t fact[6] = {hidden, ffn, ffn, hidden, ffn, hidden};
  for (int i = 0; i < 6; ++i) {
    L.off_fact[i] = off;
    off = align_up(off + sizeof(uint16_t) * num_experts * rc * fact[i], 256);
  }
  L.bytes = off;
  return L;
}

// The LoRA weight gradients that stream one M operand: M [rows, cols] (rows
// through `map`, null: identity) against the low-rank columns of one or more
// adapters, each gradient split into 32-wide rank slices. Slices that share
// M run two to a job (M is read once for both), and a phase's jobs go out in
// as few launches as the job table allows.
struct GradSource {
  const uint16_t *m;
  int64_t ldm;
  const int32_t *map;
  int64_t cols;
};

class GradPhase {
 public:
  // Gradient [E, cols, rank] (a_layout false: dB) or [E, rank, cols] (dA) of
  // one adapter, from its low-rank columns v (leading dimension ldv).
  void add(const GradSource &src, const uint16_t *v, int64_t ldv, int rank, float *out,
           bool a_layout) {
    if (!out || rank <= 0) return;
    const int64_t se = src.cols * rank;
    const int64_t sc = a_layout ? 1 : rank, sj = a_layout ? src.cols : 1;
    for (int c0 = 0; c0 < rank; c0 += kLoraK) {
      WeightGradJob *j = open_job(src, ldv);
      const int b = j->nv++;
      j->v[b] = v + c0;
      j->rank[b] = std::min(kLoraK, rank - c0);
      j->out[b] = out + c0 * sj;
      j->stride_e[b] = se;
      j->stride_c[b] = sc;
      j->stride_j[b] = sj;
    }
  }
  int run(const PlanView &v, int experts, hipStream_t s) {
    for (int first = 0; first < n_; first += kMaxGradJobs) {
      WeightGradJobs batch = {};
      batch.n = std::min(kMaxGradJobs, n_ - first);
      for (int i = 0; i < batch.n; ++i) batch.job[i] = jobs_[first + i];
      const int rc = lora_weight_grads(batch, v.seg, v.seg + experts, experts, s);
      if (rc) return rc;
    }
    n_ = 0;
    return MX_OK;
  }

 private:
  // The last job if it streams the same M and has a free V block, else a new one.
  WeightGradJob *open_job(const GradSource &src, int64_t ldv) {
    if (n_ > 0) {
      WeightGradJob &j = jobs_[n_ - 1];
      if (j.nv < 2 && j.m == src.m && j.ldm == src.ldm && j.map == src.map &&
          j.cols == src.cols && j.ldv == ldv)
        return &j;
    }
    WeightGradJob &j = jobs_[n_++];
    j = WeightGradJob{};
    j.m = src.m;
    j.ldm = src.ldm;
    j.map = src.map;
    j.cols = src.cols;
    j.ldv = ldv;
    return &j;
  }
  // A phase holds at most four gradients of up to 256 / 32 slices each, and
  // every slice adds at most one job.
  WeightGradJob jobs_[4 * kLoraMaxRank / kLoraK];
  int n_ = 0;
};

// The layer backward after the combine backward, shared by token-choice and
// expert-choice routes: from dy (per-slot grad of the expert outputs, slot
// order) and the forward's saved activations to the per-slot dx rows (written
// over dy, slot order) and the fp32 LoRA factor gradients. The plan view v
// maps sorted rows to token rows (row_token) and to slots (row_slot).
int backward_core(const BackLayout &L, const PlanView &v, int num_experts, int64_t R,
                  int64_t hidden, int64_t ffn, int act, const mx_weight *w1, const mx_weight *w3,
                  const mx_weight *w2, const mx_lora *l1, const mx_lora *l3, const mx_lora *l2,
                  const uint16_t *x, const uint16_t *g_in, const uint16_t *u_in,
                  const uint16_t *h_in, const uint16_t *lsave, uint16_t *dy, uint16_t *dgu,
                  uint16_t *dz, uint16_t *const *fact, float *grad_a1, float *grad_b1,
                  float *grad_a3, float *grad_b3, float *grad_a2, float *grad_b2, hipStream_t s) {
  const bool lora1 = has_lora(l1), lora3 = has_lora(l3), lora2 = has_lora(l2);
  const int lrc = L.rc;
  const int64_t ldz = 3 * lrc;
  int rc;
  // The six LoRA factor transposes (B2^T, A2^T, B1^T, A1^T, B3^T, A3^T) in one launch.
  {
    FactorTransposes jobs = {};
    auto add = [&](const void *src, int64_t rows, int64_t cols, uint16_t *dst) {
      jobs.job[jobs.n++] = {static_cast<const uint16_t *>(src), dst, rows, cols,
                            static_cast<int64_t>(num_experts) * rows * cols};
    };
    if (lora2) {
      add(l2->b, hidden, l2->rank, fact[0]);
      add(l2->a, l2->rank, ffn, fact[1]);
    }
    const mx_lora *l13t[2] = {l1, l3};
    for (int i = 0; i < 2; ++i)
      if (has_lora(l13t[i])) {
        add(l13t[i]->b, ffn, l13t[i]->rank, fact[2 + 2 * i]);
        add(l13t[i]->a, l13t[i]->rank, hidden, fact[3 + 2 * i]);
      }
    if ((rc = transpose_factors_multi(jobs, s))) return rc;
  }

  // Down projection: dz2 = s2 * dy B2, then dh = dy W2 + dz2 A2 into the dG
  // half of [dG | dU], and the SwiGLU backward turns it into [dG | dU].
  if (lora2) {
    const int r = l2->rank;
    const mx_lora t = {fact[0], nullptr, r, l2->scale};
    const mx_lora *ad[1] = {&t};
    if ((rc = lora_down(v, num_experts, L.plan.max_tiles, dy, hidden, v.row_slot, hidden, ad, 1,
                        lrc, dz + 2 * lrc, ldz, s)))
      return rc;
  }
  mark_stage(2, s);
  {
    Params p = base_params(v);
    p.x = dy;
    p.ldx = hidden;
    p.row_token = v.row_slot;
    p.K = hidden;
    set_weight(p, 0, w2);
    p.k_split = hidden;
    p.N = ffn;
    p.lora_p = dz + 2 * lrc;
    p.ldp = ldz;
    p.lora_rc = lrc;
    p.lora_b[0] = lora2 ? fact[1] : nullptr;
    p.lora_r[0] = lora2 ? l2->rank : 0;
    p.seg_end = v.seg + num_experts;
    p.out = dgu;
    p.ldo = 2 * ffn;
    if ((rc = launch_any<EPI_STORE2>(w2->format, lora2, p, L.plan, v, s))) return rc;
  }
  mark_stage(3, s);
  if (lora2) {
    // dB2 = sum dy^T p2 and dA2 = sum dz2^T h, one launch, right after the dh
    // GEMM has streamed dy (much of it still in the memory-side cache) and
    // before the SwiGLU backward leaves [dG | dU] dirty in it.
    GradPhase ph;
    ph.add({dy, hidden, v.row_slot, hidden}, lsave + 2 * lrc, ldz, l2->rank, grad_b2, false);
    ph.add({h_in, ffn, nullptr, ffn}, dz + 2 * lrc, ldz, l2->rank, grad_a2, true);
    if ((rc = ph.run(v, num_experts, s))) return rc;
  }
  if ((rc = swiglu_backward(dgu, g_in, u_in, R, ffn, act, s))) return rc;

  // Gate / up projections: dz1 = s1 * dG B1, dz3 = s3 * dU B3, the gate / up
  // LoRA weight gradients, then per-slot dx = dG W1 + dU W3 + dz1 A1 + dz3 A3
  // (written over dy, slot order).
  const mx_lora *l13[2] = {l1, l3};
  for (int i = 0; i < 2; ++i) {
    const mx_lora *l = l13[i];
    if (!has_lora(l)) continue;
    const int r = l->rank;
    uint16_t *bt = fact[2 + 2 * i];
    const mx_lora t = {bt, nullptr, r, l->scale};
    const mx_lora *ad[1] = {&t};
    if ((rc = lora_down(v, num_experts, L.plan.max_tiles, dgu + i * ffn, 2 * ffn, nullptr, ffn, ad,
                        1, lrc, dz + lrc * i, ldz, s)))
      return rc;
  }
  // dB1 / dB3 = sum dG^T p1 / dU^T p3, and dA1 / dA3 = sum dz1^T x / dz3^T x
  // from one pass over the gathered token rows, one launch, while [dG | dU]
  // is still in the memory-side cache from the SwiGLU backward and the dz
  // passes (nothing here reads what the dx GEMM overwrites).
  {
    // The dA job (two V blocks per gathered row, the heaviest workgroups)
    // is dispatched first, so the lighter dB workgroups fill the launch's tail.
    GradPhase ph;
    for (int i = 0; i < 2; ++i)
      if (has_lora(l13[i]))
        ph.add({x, hidden, v.row_token, hidden}, dz + lrc * i, ldz, l13[i]->rank,
               i ? grad_a3 : grad_a1, true);
    for (int i = 0; i < 2; ++i)
      if (has_lora(l13[i]))
        ph.add({dgu + i * ffn, 2 * ffn, nullptr, ffn}, lsave + lrc * i, ldz, l13[i]->rank,
               i ? grad_b3 : grad_b1, false);
    if ((rc = ph.run(v, num_experts, s))) return rc;
  }
  mark_stage(4, s);
  {
    Params p = base_params(v);
    p.x = dgu;
    p.ldx = 2 * ffn;
    p.row_token = nullptr;
    p.K = 2 * ffn;
    set_weight(p, 0, w1);
    set_weight(p, 1, w3);
    p.k_split = ffn;
    p.N = hidden;
    p.lora_p = dz;
    p.ldp = ldz;
    p.lora_rc = lrc;
    p.lora_b[0] = lora1 ? fact[3] : nullptr;
    p.lora_b[1] = lora3 ? fact[5] : nullptr;
    p.lora_r[0] = lora1 ? l1->rank : 0;
    p.lora_r[1] = lora3 ? l3->rank : 0;
    p.seg_end = v.seg + num_experts;
    p.out = dy;
    p.ldo = hidden;
    p.out_row = v.row_slot;
    if ((rc = launch_any<EPI_STORE2>(w1->format, lora1 || lora3, p, L.plan, v, s))) return rc;
  }
  mark_stage(5, s);
  return MX_OK;
}

}  // namespace gemm
}  // namespace mx

using namespace mx;
using namespace mx::gemm;

extern "C" size_t mx_moe_backward_workspace_size(int64_t num_tokens, int top_k, int num_experts,
                                                 int64_t hidden, int64_t ffn, int lora_rank) {
  if (num_tokens < 0 || top_k <= 0 || num_experts <= 0 || hidden <= 0 || ffn <= 0 ||
      lora_rank < 0 || lora_rank > kLoraMaxRank)
    return 0;
  return back_layout(num_tokens * top_k, num_experts, hidden, ffn, lora_width(lora_rank)).bytes;
}

extern "C" int mx_moe_backward_act(const void *grad_out, int grad_dtype, const void *tokens,
                               const int64_t *top_idx, const void *top_scores, int score_dtype,
                               int64_t num_tokens, int top_k, int num_experts, int64_t hidden,
                               int64_t ffn, int act, const mx_weight *w1, const mx_weight *w3,
                               const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                               const mx_lora *l2, const void *save_gate, const void *save_up,
                               const void *save_h, const void *save_y, const void *save_lora,
                               void *grad_tokens, int grad_tokens_dtype, float *grad_scores,
                               float *grad_a1, float *grad_b1, float *grad_a3, float *grad_b3,
                               float *grad_a2, float *grad_b2, void *workspace, void *stream) {
  clear_error();
  const char *name = "mx_moe_backward";
  int rc = validate_plan_args(name, num_tokens, top_k, num_experts);
  if (rc) return rc;
  const bool bf16_combine = (act & MX_ACT_FLAG_BF16_COMBINE) != 0;
  act &= ~MX_ACT_FLAG_BF16_COMBINE;
  if (act != MX_ACT_SILU && act != MX_ACT_SWIGLU7) {
    set_error("%s: unknown activation %d", name, act);
    return MX_ERR_INVALID;
  }
  if ((rc = check_layer(name, hidden, ffn, w1, w3, w2, l1, l3, l2))) return rc;
  if (w1->format == MX_FMT_F32X3) {
    set_error("%s: the fp32 (MX_FMT_F32X3) layer is inference-only", name);
    return MX_ERR_INVALID;
  }
  if (num_tokens == 0)
    return zero_lora_grads(name, num_experts, hidden, ffn, l1, l3, l2, grad_a1, grad_b1, grad_a3,
                           grad_b3, grad_a2, grad_b2, as_stream(stream));
  const bool lora1 = has_lora(l1), lora3 = has_lora(l3), lora2 = has_lora(l2);
  if (!grad_out || !tokens || !top_idx || !top_scores || !save_gate || !save_up || !save_h ||
      !save_y || !grad_tokens || !grad_scores || !workspace ||
      ((lora1 || lora3 || lora2) && !save_lora)) {
    set_error("%s: gradients, routes, saved activations and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  if ((grad_dtype != MX_DTYPE_BF16 && grad_dtype != MX_DTYPE_F32) ||
      (grad_tokens_dtype != MX_DTYPE_BF16 && grad_tokens_dtype != MX_DTYPE_F32)) {
    set_error("%s: gradients must be bf16 or fp32", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const int64_t R = num_tokens * top_k;
  const BackLayout L = back_layout(R, num_experts, hidden, ffn, lora_width(l1, l3, l2));
  char *ws = static_cast<char *>(workspace);
  const PlanView v = plan_view(ws, L.plan);
  uint16_t *dy = reinterpret_cast<uint16_t *>(ws + L.off_dy);
  uint16_t *dgu = reinterpret_cast<uint16_t *>(ws + L.off_dgu);
  uint16_t *dz = reinterpret_cast<uint16_t *>(ws + L.off_dz);
  uint16_t *fact[6];
  for (int i = 0; i < 6; ++i) fact[i] = reinterpret_cast<uint16_t *>(ws + L.off_fact[i]);
  const uint16_t *x = static_cast<const uint16_t *>(tokens);
  const uint16_t *lsave = static_cast<const uint16_t *>(save_lora);
  const uint16_t *g_in = static_cast<const uint16_t *>(save_gate);
  const uint16_t *u_in = static_cast<const uint16_t *>(save_up);
  const uint16_t *h_in = static_cast<const uint16_t *>(save_h);

  // Plan (the forward's, rebuilt: the counting sort is deterministic).
  mark_stage(0, s);
  rc = build_plan(top_idx, nullptr, score_dtype, num_tokens, top_k, num_experts, nullptr, nullptr,
                  nullptr, nullptr, nullptr, nullptr, nullptr, ws, s);
  if (rc) return rc;
  // dy = grad_out * score per slot, and the score gradients.
  rc = mx_combine_backward(grad_out, grad_dtype, save_y, top_idx, top_scores, score_dtype,
                           num_tokens, top_k, num_experts, hidden, dy, grad_scores, stream);
  if (rc) return rc;
  mark_stage(1, s);

  rc = backward_core(L, v, num_experts, R, hidden, ffn, act, w1, w3, w2, l1, l3, l2, x, g_in,
                     u_in, h_in, lsave, dy, dgu, dz, fact, grad_a1, grad_b1, grad_a3, grad_b3,
                     grad_a2, grad_b2, s);
  if (rc) return rc;
  // grad_tokens[t] = sum of its slots' dx rows (fp32, ascending expert order).
  rc = mx_combine(dy, top_idx, nullptr, score_dtype, num_tokens, top_k, num_experts, hidden,
                  grad_tokens, grad_tokens_dtype, stream);
  mark_stage(6, s);
  return rc;
}

extern "C" int mx_moe_backward(const void *grad_out, int grad_dtype, const void *tokens,
                               const int64_t *top_idx, const void *top_scores, int score_dtype,
                               int64_t num_tokens, int top_k, int num_experts, int64_t hidden,
                               int64_t ffn, const mx_weight *w1, const mx_weight *w3,
                               const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                               const mx_lora *l2, const void *save_gate, const void *save_up,
                               const void *save_h, const void *save_y, const void *save_lora,
                               void *grad_tokens, int grad_tokens_dtype, float *grad_scores,
                               float *grad_a1, float *grad_b1, float *grad_a3, float *grad_b3,
                               float *grad_a2, float *grad_b2, void *workspace, void *stream) {
  return mx_moe_backward_act(grad_out, grad_dtype, tokens, top_idx, top_scores, score_dtype,
                             num_tokens, top_k, num_experts, hidden, ffn, MX_ACT_SILU, w1, w3,
                             w2, l1, l3, l2, save_gate, save_up, save_h, save_y, save_lora,
                             grad_tokens, grad_tokens_dtype, grad_scores, grad_a1, grad_b1,
                             grad_a3, grad_b3, grad_a2, grad_b2, workspace, stream);
}

extern "C" size_t mx_moe_workspace_size(int64_t num_tokens, int top_k, int num_experts,
                                        int64_t hidden, int64_t ffn, int lora_rank) {
  if (num_tokens < 0 || top_k <= 0 || num_experts <= 0 || hidden <= 0 || ffn <= 0 ||
      lora_rank < 0 || lora_rank > kLoraMaxRank)
    return 0;
  return layer_layout(num_tokens * top_k, num_experts, hidden, ffn, false, 0,
                      lora_width(lora_rank)).bytes;
}

extern "C" size_t mx_moe_f32x3_workspace_size(int64_t num_tokens, int top_k, int num_experts,
                                              int64_t hidden, int64_t ffn) {
  if (num_tokens < 0 || top_k <= 0 || num_experts <= 0 || hidden <= 0 || ffn <= 0) return 0;
  return layer_layout(num_tokens * top_k, num_experts, hidden, ffn, true, num_tokens).bytes;
}

extern "C" int mx_moe_forward_ex(const void *tokens, const int64_t *top_idx,
                                 const void *top_scores, int score_dtype, int64_t num_tokens,
                                 int top_k, int num_experts, int64_t hidden, int64_t ffn, int act,
                                 const mx_weight *w1, const mx_weight *w3, const mx_weight *w2,
                                 const mx_lora *l1, const mx_lora *l3, const mx_lora *l2,
                                 void *out, int out_dtype, const void *addend,
                                 void *addend_ready, void *save_gate, void *save_up,
                                 void *save_h, void *save_y, void *save_lora, void *workspace,
                                 void *stream) {
  clear_error();
  const char *name = "mx_moe_forward";
  int rc = validate_plan_args(name, num_tokens, top_k, num_experts);
  if (rc) return rc;
  const bool bf16_combine = (act & MX_ACT_FLAG_BF16_COMBINE) != 0;
  act &= ~MX_ACT_FLAG_BF16_COMBINE;
  if (act != MX_ACT_SILU && act != MX_ACT_SWIGLU7) {
    set_error("%s: unknown activation %d", name, act);
    return MX_ERR_INVALID;
  }
  if ((rc = check_layer(name, hidden, ffn, w1, w3, w2, l1, l3, l2))) return rc;
  if (num_tokens == 0) return MX_OK;
  if (!tokens || !top_idx || !top_scores || !out || !workspace) {
    set_error("%s: tokens, routes, output and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const int64_t R = num_tokens * top_k;
  const bool split = w1->format == MX_FMT_F32X3;
  if (split && (save_gate || save_up || save_h || save_y || save_lora)) {
    set_error("%s: the fp32 (MX_FMT_F32X3) layer is inference-only and saves no activations",
              name);
    return MX_ERR_INVALID;
  }
  if (split && addend) {
    set_error("%s: an addend is supported with bf16 / NF4 / INT8 weights only", name);
    return MX_ERR_INVALID;
  }
  if (addend_ready && !addend) {
    set_error("%s: addend_ready needs an addend", name);
    return MX_ERR_INVALID;
  }
  const int lrc = lora_width(l1, l3, l2);
  const LayerLayout L = layer_layout(R, num_experts, hidden, ffn, split, num_tokens, lrc);
  char *ws = static_cast<char *>(workspace);
  const PlanView v = plan_view(ws, L.plan);
  mark_stage(0, s);
  // fp32 tokens -> [hi | hi | lo] bf16 planes, the A side of the split GEMMs.
  const uint16_t *x = static_cast<const uint16_t *>(tokens);
  if (split) {
    uint16_t *xs = reinterpret_cast<uint16_t *>(ws + L.off_x);
    if ((rc = split_f32(static_cast<const float *>(tokens), num_tokens, hidden, MX_SPLIT_ACT, xs,
                        s)))
      return rc;
    x = xs;
  }
  rc = build_plan(top_idx, nullptr, score_dtype, num_tokens, top_k, num_experts, nullptr, nullptr,
                  nullptr, nullptr, nullptr, nullptr, nullptr, ws, s);
  if (rc) return rc;
  mark_stage(1, s);
  uint16_t *lora_buf = save_lora ? static_cast<uint16_t *>(save_lora)
                                 : reinterpret_cast<uint16_t *>(ws + L.off_lora);
  uint16_t *h = save_h ? static_cast<uint16_t *>(save_h) : reinterpret_cast<uint16_t *>(ws + L.off_h);
  uint16_t *y = save_y ? static_cast<uint16_t *>(save_y) : reinterpret_cast<uint16_t *>(ws + L.off_y);
  const int y_planes = split ? 2 * f32x3_down_parts(R, num_experts, hidden, ffn) : 1;
  rc = expert_mlp(L.plan, v, num_experts, x, (split ? 3 : 1) * hidden,
                  v.row_token, hidden, ffn, act, w1, w3, w2, l1, l3, l2, lora_buf, lrc, h,
                  static_cast<uint16_t *>(save_gate), static_cast<uint16_t *>(save_up), y,
                  y_planes * hidden, v.row_slot, s);
  if (rc) return rc;
  mark_stage(5, s);
  if (split) {
    // fp32 layer: combine every y plane in fp32, then add them.
    float *sum = reinterpret_cast<float *>(ws + L.off_sum);
    rc = mx_combine(y, top_idx, top_scores, score_dtype, num_tokens, top_k, num_experts,
                    y_planes * hidden, sum, MX_DTYPE_F32, stream);
    if (!rc) rc = sum_planes(sum, num_tokens, hidden, y_planes, out, out_dtype, s);
  } else {
    // The addend (e.g. a shared expert computed on another stream) is needed
    // only here: the routed path above runs concurrently with its producer.
    if (addend_ready) {
      const hipError_t err = hipStreamWaitEvent(s, static_cast<hipEvent_t>(addend_ready), 0);
      if (err != hipSuccess) {
        set_error("%s: hipStreamWaitEvent: %s", name, hipGetErrorString(err));
        return MX_ERR_HIP;
      }
    }
    rc = combine_ex(y, top_idx, top_scores, score_dtype, num_tokens, top_k, num_experts, hidden,
                    out, out_dtype, addend, stream, bf16_combine);
  }
  mark_stage(6, s);
  return rc;
}

extern "C" int mx_moe_forward_act(const void *tokens, const int64_t *top_idx,
                                  const void *top_scores, int score_dtype, int64_t num_tokens,
                                  int top_k, int num_experts, int64_t hidden, int64_t ffn,
                                  int act, const mx_weight *w1, const mx_weight *w3,
                                  const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                                  const mx_lora *l2, void *out, int out_dtype, void *save_gate,
                                  void *save_up, void *save_h, void *save_y, void *save_lora,
                                  void *workspace, void *stream) {
  return mx_moe_forward_ex(tokens, top_idx, top_scores, score_dtype, num_tokens, top_k,
                           num_experts, hidden, ffn, act, w1, w3, w2, l1, l3, l2, out, out_dtype,
                           nullptr, nullptr, save_gate, save_up, save_h, save_y, save_lora,
                           workspace, stream);
}

extern "C" int mx_moe_forward(const void *tokens, const int64_t *top_idx, const void *top_scores,
                              int score_dtype, int64_t num_tokens, int top_k, int num_experts,
                              int64_t hidden, int64_t ffn, const mx_weight *w1,
                              const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
                              const mx_lora *l3, const mx_lora *l2, void *out, int out_dtype,
                              void *save_gate, void *save_up, void *save_h, void *save_y,
                              void *save_lora, void *workspace, void *stream) {
  return mx_moe_forward_act(tokens, top_idx, top_scores, score_dtype, num_tokens, top_k,
                            num_experts, hidden, ffn, MX_ACT_SILU, w1, w3, w2, l1, l3, l2, out,
                            out_dtype, save_gate, save_up, save_h, save_y, save_lora, workspace,
                            stream);
}

// ------------------------------------------------- allocation-free forward
// mx_moe_forward_static runs mx_moe_forward_act on a file-scope device array
// instead of a caller workspace, for callers that cannot allocate. Each GPU
// holds its own copy of the array (loaded with the code object, freed at
// process exit); its address on a device is looked up once, with that device
// current, and kept. Calls that overlap on one GPU share the array and race.
namespace {

constexpr size_t kStaticScratchBytes = size_t(MX_STATIC_SCRATCH_BYTES);
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the stream's device (the current device for
// the null stream). The array's name is only a host-side stand-in: kernels
// and copies get this pointer.
int static_scratch(const char *name, hipStream_t s, void **out) {
  int dev = -1;
  hipError_t err = s ? hipStreamGetDevice(s, &dev) : hipGetDevice(&dev);
  if (err != hipSuccess) {
    set_error("%s: cannot resolve the stream's device: %s", name, hipGetErrorString(err));
    return MX_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) {
    set_error("%s: device %d is beyond the %d devices the static scratch tracks", name, dev,
              kMaxScratchDevices);
    return MX_ERR_INVALID;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if ((err = hipGetDevice(&cur)) != hipSuccess) {
      set_error("%s: hipGetDevice: %s", name, hipGetErrorString(err));
      return MX_ERR_HIP;
    }
    if (cur != dev && (err = hipSetDevice(dev)) != hipSuccess) {
      set_error("%s: hipSetDevice(%d): %s", name, dev, hipGetErrorString(err));
      return MX_ERR_HIP;
    }
    void *ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (err != hipSuccess || !ptr) {
      set_error("%s: hipGetSymbolAddress(scratch) on device %d: %s", name, dev,
                hipGetErrorString(err));
      return MX_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MX_OK;
}

}  // namespace

extern "C" int mx_moe_forward_static(const void *tokens, const int64_t *top_idx,
                                     const void *top_scores, int score_dtype, int64_t num_tokens,
                                     int top_k, int num_experts, int64_t hidden, int64_t ffn,
                                     int act, const mx_weight *w1, const mx_weight *w3,
                                     const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                                     const mx_lora *l2, void *out, int out_dtype, void *stream) {
  clear_error();
  const char *name = "mx_moe_forward_static";
  int rc = validate_plan_args(name, num_tokens, top_k, num_experts);
  if (rc) return rc;
  if ((rc = check_layer(name, hidden, ffn, w1, w3, w2, l1, l3, l2))) return rc;
  if (num_tokens == 0) return MX_OK;
  const bool split = w1->format == MX_FMT_F32X3;
  const size_t need = layer_layout(num_tokens * top_k, num_experts, hidden, ffn, split,
                                   num_tokens, lora_width(l1, l3, l2)).bytes;
  if (need > kStaticScratchBytes) {
    set_error("%s: this layer call needs %zu bytes of scratch, more than the %zu of the static "
              "array; use mx_moe_forward with a workspace", name, need, kStaticScratchBytes);
    return MX_ERR_INVALID;
  }
  void *ws = nullptr;
  if ((rc = static_scratch(name, as_stream(stream), &ws))) return rc;
  // Every buffer of the layout is written before it is read in this call;
  // the plan clears its own counters with a kernel.
  return mx_moe_forward_ex(tokens, top_idx, top_scores, score_dtype, num_tokens, top_k,
                           num_experts, hidden, ffn, act, w1, w3, w2, l1, l3, l2, out, out_dtype,
                           nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, ws,
                           stream);
}

extern "C" int mx_set_stage_events(void **events, int count) {
  clear_error();
  if (count != 0 && (count != kStageEvents || !events)) {
    set_error("mx_set_stage_events: pass %d events or none", kStageEvents);
    return MX_ERR_INVALID;
  }
  for (int i = 0; i < kStageEvents; ++i) g_stage_events[i] = count ? events[i] : nullptr;
  g_stage_count = count;
  return MX_OK;
}

extern "C" int mx_moe_for_loop_act(const void *tokens_sorted, const int64_t *counts,
                                   int64_t num_rows, int num_experts, int64_t hidden, int64_t ffn,
                                   int act, const mx_weight *w1, const mx_weight *w3,
                                   const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                                   const mx_lora *l2, void *out, void *workspace, void *stream) {
  clear_error();
  const char *name = "mx_moe_for_loop";
  int rc = validate_plan_args(name, num_rows, 1, num_experts);
  if (rc) return rc;
  const bool bf16_combine = (act & MX_ACT_FLAG_BF16_COMBINE) != 0;
  act &= ~MX_ACT_FLAG_BF16_COMBINE;
  if (act != MX_ACT_SILU && act != MX_ACT_SWIGLU7) {
    set_error("%s: unknown activation %d", name, act);
    return MX_ERR_INVALID;
  }
  if ((rc = check_layer(name, hidden, ffn, w1, w3, w2, l1, l3, l2))) return rc;
  if (w1->format == MX_FMT_F32X3) {
    set_error("%s: MX_FMT_F32X3 (fp32) weights are supported by mx_moe_forward only", name);
    return MX_ERR_INVALID;
  }
  if (num_rows == 0) return MX_OK;
  if (!tokens_sorted || !counts || !out || !workspace) {
    set_error("%s: tokens, counts, output and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const int lrc = lora_width(l1, l3, l2);
  const LayerLayout L = layer_layout(num_rows, num_experts, hidden, ffn, false, 0, lrc);
  char *ws = static_cast<char *>(workspace);
  const PlanView v = plan_view(ws, L.plan);
  if ((rc = plan_from_counts(counts, num_rows, num_experts, ws, s))) return rc;
  return expert_mlp(L.plan, v, num_experts, static_cast<const uint16_t *>(tokens_sorted), hidden,
                    nullptr, hidden, ffn, act, w1, w3, w2, l1, l3, l2,
                    reinterpret_cast<uint16_t *>(ws + L.off_lora), lrc,
                    reinterpret_cast<uint16_t *>(ws + L.off_h), nullptr, nullptr,
                    static_cast<uint16_t *>(out), hidden, nullptr, s);
}

extern "C" int mx_moe_for_loop(const void *tokens_sorted, const int64_t *counts, int64_t num_rows,
                               int num_experts, int64_t hidden, int64_t ffn, const mx_weight *w1,
                               const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
                               const mx_lora *l3, const mx_lora *l2, void *out, void *workspace,
                               void *stream) {
  return mx_moe_for_loop_act(tokens_sorted, counts, num_rows, num_experts, hidden, ffn,
                             MX_ACT_SILU, w1, w3, w2, l1, l3, l2, out, workspace, stream);
}

extern "C" int mx_grouped_linear(const void *x, const int64_t *counts, int64_t num_rows,
                                 int num_experts, const mx_weight *w, const mx_lora *lora,
                                 void *out, void *workspace, void *stream) {
  clear_error();
  const char *name = "mx_grouped_linear";
  int rc = validate_plan_args(name, num_rows, 1, num_experts);
  if (rc) return rc;
  if (!w) {
    set_error("%s: weight is missing", name);
    return MX_ERR_INVALID;
  }
  const int64_t in_f = w->in_features, out_f = w->out_features;
  if (in_f <= 0 || in_f % 64 != 0 || out_f <= 0 || out_f % 8 != 0) {
    set_error("%s: in_features must be a multiple of 64 and out_features of 8", name);
    return MX_ERR_INVALID;
  }
  if ((rc = check_weight(name, "w", w, out_f, in_f))) return rc;
  if ((rc = check_lora(name, "w", lora))) return rc;
  if (w->format == MX_FMT_F32X3) {
    set_error("%s: MX_FMT_F32X3 (fp32) weights are supported by mx_moe_forward only", name);
    return MX_ERR_INVALID;
  }
  if (num_rows == 0) return MX_OK;
  if (!x || !counts || !out || !workspace) {
    set_error("%s: x, counts, output and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const int lrc = lora_width(lora, nullptr, nullptr);
  const LayerLayout L = layer_layout(num_rows, num_experts, in_f, out_f, false, 0, lrc);
  char *ws = static_cast<char *>(workspace);
  const PlanView v = plan_view(ws, L.plan);
  if ((rc = plan_from_counts(counts, num_rows, num_experts, ws, s))) return rc;
  uint16_t *lora_buf = reinterpret_cast<uint16_t *>(ws + L.off_lora);
  const bool lr = has_lora(lora);
  if (lr) {
    const mx_lora *ad[1] = {lora};
    rc = lora_down(v, num_experts, L.plan.max_tiles, static_cast<const uint16_t *>(x), in_f,
                   nullptr, in_f, ad, 1, lrc, lora_buf, 3 * lrc, s);
    if (rc) return rc;
  }
  Params p = base_params(v);
  p.x = static_cast<const uint16_t *>(x);
  p.ldx = in_f;
  p.K = in_f;
  set_weight(p, 0, w);
  p.N = out_f;
  p.lora_p = lora_buf;
  p.ldp = 3 * lrc;
  p.lora_rc = lrc;
  p.lora_b[0] = lr ? static_cast<const uint16_t *>(lora->b) : nullptr;
  p.lora_r[0] = lr ? lora->rank : 0;
  p.seg_end = v.seg + num_experts;
  p.out = static_cast<uint16_t *>(out);
  p.ldo = out_f;
  return launch_any<EPI_STORE>(w->format, lr, p, L.plan, v, s);
}

namespace mx {
namespace gemm {

// Scratch of the grouped-linear backward: plan | p [S, rc] (the forward's
// low-rank rows, recomputed) | dz [S, rc] | B^T [E, rc, out] | A^T [E, in, rc].
struct LinearBackLayout {
  PlanLayout plan;
  size_t off_p = 0, off_dz = 0, off_bt = 0, off_at = 0, bytes = 0;
};

LinearBackLayout linear_back_layout(int64_t rows, int num_experts, int64_t in_f, int64_t out_f,
                                    int rc) {
  LinearBackLayout L;
  L.plan = plan_layout(rows, num_experts);
  size_t off = align_up(L.plan.bytes, 256);
  L.off_p = off;
  off = align_up(off + sizeof(uint16_t) * rows * rc, 256);
  L.off_dz = off;
  off = align_up(off + sizeof(uint16_t) * rows * rc, 256);
  L.off_bt = off;
  off = align_up(off + sizeof(uint16_t) * num_experts * rc * out_f, 256);
  L.off_at = off;
  off = align_up(off + sizeof(uint16_t) * num_experts * rc * in_f, 256);
  L.bytes = off;
  return L;
}

}  // namespace gemm
}  // namespace mx

extern "C" size_t mx_grouped_linear_backward_workspace_size(int64_t num_rows, int num_experts,
                                                           int64_t in_features,
                                                           int64_t out_features, int lora_rank) {
  if (num_rows < 0 || num_experts <= 0 || in_features <= 0 || out_features <= 0 ||
      lora_rank < 0 || lora_rank > kLoraMaxRank)
    return 0;
  return linear_back_layout(num_rows, num_experts, in_features, out_features,
                            lora_width(lora_rank)).bytes;
}

extern "C" int mx_grouped_linear_backward(const void *grad_out, const void *x,
                                          const int64_t *counts, int64_t num_rows,
                                          int num_experts, const mx_weight *w,
                                          const mx_lora *lora, void *grad_x, float *grad_a,
                                          float *grad_b, void *workspace, void *stream) {
  clear_error();
  const char *name = "mx_grouped_linear_backward";
  int rc = validate_plan_args(name, num_rows, 1, num_experts);
  if (rc) return rc;
  if (!w) {
    set_error("%s: weight is missing", name);
    return MX_ERR_INVALID;
  }
  const int64_t in_f = w->in_features, out_f = w->out_features;
  if (in_f <= 0 || in_f % 64 != 0 || out_f <= 0 || out_f % 64 != 0) {
    set_error("%s: in_features and out_features must be multiples of 64 (got %lld, %lld)", name,
              static_cast<long long>(in_f), static_cast<long long>(out_f));
    return MX_ERR_INVALID;
  }
  if ((rc = check_weight(name, "w", w, out_f, in_f))) return rc;
  if ((rc = check_lora(name, "w", lora))) return rc;
  if (w->format == MX_FMT_F32X3) {
    set_error("%s: MX_FMT_F32X3 (fp32) weights are inference-only", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const bool lr = has_lora(lora);
  if (num_rows == 0) {
    // The gradient of an empty sum: zero LoRA gradients, nothing else to write.
    if (!lr) return MX_OK;
    return zero_lora_grads(name, num_experts, in_f, out_f, lora, nullptr, nullptr, grad_a,
                           grad_b, nullptr, nullptr, nullptr, nullptr, s);
  }
  if (!grad_out || !x || !counts || !workspace || (!grad_x && !lr)) {
    set_error("%s: gradient, x, counts and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  const int lrc = lora_width(lora, nullptr, nullptr);
  const LinearBackLayout L = linear_back_layout(num_rows, num_experts, in_f, out_f, lrc);
  char *ws = static_cast<char *>(workspace);
  const PlanView v = plan_view(ws, L.plan);
  if ((rc = plan_from_counts(counts, num_rows, num_experts, ws, s))) return rc;
  const uint16_t *dy = static_cast<const uint16_t *>(grad_out);
  const uint16_t *xr = static_cast<const uint16_t *>(x);
  uint16_t *prow = reinterpret_cast<uint16_t *>(ws + L.off_p);
  uint16_t *dz = reinterpret_cast<uint16_t *>(ws + L.off_dz);
  uint16_t *bt = reinterpret_cast<uint16_t *>(ws + L.off_bt);
  uint16_t *at = reinterpret_cast<uint16_t *>(ws + L.off_at);
  if (lr) {
    const int r = lora->rank;
    FactorTransposes jobs = {};
    jobs.job[jobs.n++] = {static_cast<const uint16_t *>(lora->b), bt, out_f, r,
                          static_cast<int64_t>(num_experts) * out_f * r};
    jobs.job[jobs.n++] = {static_cast<const uint16_t *>(lora->a), at, r, in_f,
                          static_cast<int64_t>(num_experts) * r * in_f};
    if ((rc = transpose_factors_multi(jobs, s))) return rc;
    // p = bf16(s bf16(x A^T)) as the forward formed it, and dz = bf16(s bf16(dy B)).
    const mx_lora *fwd[1] = {lora};
    if ((rc = lora_down(v, num_experts, L.plan.max_tiles, xr, in_f, nullptr, in_f, fwd, 1, lrc,
                        prow, lrc, s)))
      return rc;
    const mx_lora t = {bt, nullptr, r, lora->scale};
    const mx_lora *bwd[1] = {&t};
    if ((rc = lora_down(v, num_experts, L.plan.max_tiles, dy, out_f, nullptr, out_f, bwd, 1, lrc,
                        dz, lrc, s)))
      return rc;
  }
  if (grad_x) {
    // dx = dy W + dz A, W re-decoded (B = W, K along the weight's out rows).
    Params p = base_params(v);
    p.x = dy;
    p.ldx = out_f;
    p.K = out_f;
    set_weight(p, 0, w);
    p.k_split = out_f;
    p.N = in_f;
    p.lora_p = dz;
    p.ldp = lrc;
    p.lora_rc = lrc;
    p.lora_b[0] = lr ? at : nullptr;
    p.lora_r[0] = lr ? lora->rank : 0;
    p.seg_end = v.seg + num_experts;
    p.out = static_cast<uint16_t *>(grad_x);
    p.ldo = in_f;
    if ((rc = launch_any<EPI_STORE2>(w->format, lr, p, L.plan, v, s))) return rc;
  }
  if (!lr) return MX_OK;
  // dB = sum dy^T p and dA = sum dz^T x per expert, one launch.
  GradPhase ph;
  ph.add({dy, out_f, nullptr, out_f}, prow, lrc, lora->rank, grad_b, false);
  ph.add({xr, in_f, nullptr, in_f}, dz, lrc, lora->rank, grad_a, true);
  return ph.run(v, num_experts, s);
}

// ------------------------------------------------------------ expert choice
// Expert-choice routes [B, L, C] (each of L logical experts picks C tokens of
// each sample) through the same plan and grouped GEMMs: the flat slots
// s = (b, l, c) are counting-sorted by physical expert (k = 1), each sorted
// row reads token idx[s] + b * tokens_per_sample, and the combine adds every
// token's contributions in ascending (physical expert, logical expert) order.
namespace mx {
namespace gemm {

struct EcLayout {
  LayerLayout layer;
  size_t off_phys = 0, off_tok = 0, off_map = 0, bytes = 0;
};

EcLayout ec_layout(int64_t slots, int num_experts, int64_t hidden, int64_t ffn, int64_t tokens,
                   int logical, int rc) {
  EcLayout L;
  L.layer = layer_layout(slots, num_experts, hidden, ffn, false, 0, rc);
  size_t off = align_up(L.layer.bytes, 256);
  L.off_phys = off;
  off = align_up(off + sizeof(int64_t) * slots, 256);
  L.off_tok = off;
  off = align_up(off + sizeof(int64_t) * slots, 256);
  L.off_map = off;
  off = align_up(off + sizeof(int32_t) * tokens * logical, 256);
  L.bytes = off;
  return L;
}

// phys[s] = logical_to_physical[l] (or l), tok[s] = idx[s] + b * tps.
__global__ __launch_bounds__(256) void ec_slots_kernel(const int64_t *idx, int64_t slots, int L,
                                                       int C, int64_t tps, const int32_t *l2p,
                                                       int64_t *phys, int64_t *tok) {
  const int64_t s = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (s >= slots) return;
  const int64_t b = s / (static_cast<int64_t>(L) * C);
  const int l = static_cast<int>((s / C) % L);
  phys[s] = l2p ? l2p[l] : l;
  tok[s] = idx[s] + b * tps;
}

// dst[r] = tok[src[r]] (sorted token indices / sorted-row tokens) for slot
// indices src[r] in [0, rows); with clamp, tokens outside [0, T) read token 0
// (their slots are not combined).
template <typename D, typename S>
__global__ __launch_bounds__(256) void ec_gather_tok_kernel(const S *src, const int64_t *tok,
                                                            int64_t rows, int64_t T, bool clamp,
                                                            D *dst) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= rows) return;
  const int64_t i = static_cast<int64_t>(src[r]);
  int64_t t = (i >= 0 && i < rows) ? tok[i] : -1;
  if (clamp && (t < 0 || t >= T)) t = 0;
  dst[r] = static_cast<D>(t);
}

__global__ __launch_bounds__(256) void ec_map_kernel(const int64_t *tok, int64_t slots, int L,
                                                     int C, int64_t T, int32_t *map) {
  const int64_t s = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (s >= slots) return;
  const int64_t t = tok[s];
  if (t < 0 || t >= T) return;
  map[t * L + (s / C) % L] = static_cast<int32_t>(s);
}

__global__ __launch_bounds__(256) void ec_fill_kernel(int32_t *p, int64_t n, int32_t v) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

// One wave per token: the token's slots are collected in the given logical
// order into LDS, then each 512-column span sums score * y over them in fp32
// (product and sum each rounded once, as index_add_(y.float() * score)); with
// no scores the rows are summed as they are (the backward's dx rows).
__global__ __launch_bounds__(256) void ec_combine_kernel(const uint16_t *y, const void *scores,
                                                         int score_dtype, const int32_t *map,
                                                         const int32_t *order, int64_t T, int L,
                                                         int64_t cols, void *out, int out_dtype) {
  __shared__ int32_t s_slot[4][1024];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + w;
  if (t >= T) return;
  int n = 0;
  for (int i0 = 0; i0 < L; i0 += 64) {
    const int i = i0 + lane;
    int32_t s = -1;
    if (i < L) s = map[t * L + (order ? order[i] : i)];
    const uint64_t present = __ballot(s >= 0);
    const int pos = n + __popcll(present & ((1ull << lane) - 1ull));
    if (s >= 0) s_slot[w][pos] = s;
    n += __popcll(present);
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  for (int64_t c0 = static_cast<int64_t>(lane) * 8; c0 < cols; c0 += 512) {
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    for (int j = 0; j < n; ++j) {
      const int32_t s = s_slot[w][j];
      const float sc = scores ? load_score(scores, s, score_dtype) : 1.0f;
      const uint4 v = *reinterpret_cast<const uint4 *>(y + static_cast<int64_t>(s) * cols + c0);
      const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = __fadd_rn(acc[2 * i], __fmul_rn(bf16_bits_to_f32(q[i] & 0xffffu), sc));
        acc[2 * i + 1] = __fadd_rn(acc[2 * i + 1], __fmul_rn(bf16_bits_to_f32(q[i] >> 16), sc));
      }
    }
    if (out_dtype == MX_DTYPE_BF16) {
      uint4 o;
      o.x = pack_bf16x2(acc[0], acc[1]);
      o.y = pack_bf16x2(acc[2], acc[3]);
      o.z = pack_bf16x2(acc[4], acc[5]);
      o.w = pack_bf16x2(acc[6], acc[7]);
      *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + t * cols + c0) = o;
    } else {
      float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + t * cols + c0);
      o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
  }
}

// One wave per slot s of token t = tok[s]: grad_y[s] = bf16(score[s] *
// grad_out[t]) and grad_scores[s] = sum_c grad_out[t, c] * y[s, c] in fp32, as
// the token-choice combine backward does per route; slots whose token lies
// outside [0, T) (they were not combined) get zero gradients.
__global__ __launch_bounds__(256) void ec_combine_backward_kernel(
    const void *grad_out, int grad_dtype, const uint16_t *y, const int64_t *tok,
    const void *scores, int score_dtype, int64_t slots, int64_t T, int64_t cols,
    uint16_t *grad_y, float *grad_scores) {
  const int64_t sl = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (sl >= slots) return;
  const int lane = threadIdx.x & 63;
  const int64_t t = tok[sl];
  const bool ok = t >= 0 && t < T;
  const float sc = ok ? load_score(scores, sl, score_dtype) : 0.0f;
  float part = 0.0f;
  for (int64_t c0 = static_cast<int64_t>(lane) * 8; c0 < cols; c0 += 512) {
    float g[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    uint4 yv = make_uint4(0, 0, 0, 0);
    if (ok) {
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
      yv = *reinterpret_cast<const uint4 *>(y + sl * cols + c0);
    }
    const uint32_t w[4] = {yv.x, yv.y, yv.z, yv.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      part += g[2 * i] * bf16_bits_to_f32(w[i] & 0xffffu) + g[2 * i + 1] * bf16_bits_to_f32(w[i] >> 16);
      o[i] = pack_bf16x2(g[2 * i] * sc, g[2 * i + 1] * sc);
    }
    *reinterpret_cast<uint4 *>(grad_y + sl * cols + c0) = make_uint4(o[0], o[1], o[2], o[3]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
  if (lane == 0) grad_scores[sl] = ok ? part : 0.0f;
}

// Scratch of the expert-choice backward: the layer backward's over the slots,
// then the slot -> physical expert / token arrays and the token -> slot map.
struct EcBackLayout {
  BackLayout back;
  size_t off_phys = 0, off_tok = 0, off_map = 0, bytes = 0;
};

EcBackLayout ec_back_layout(int64_t slots, int num_experts, int64_t hidden, int64_t ffn,
                            int64_t tokens, int logical, int rc) {
  EcBackLayout L;
  L.back = back_layout(slots, num_experts, hidden, ffn, rc);
  size_t off = align_up(L.back.bytes, 256);
  L.off_phys = off;
  off = align_up(off + sizeof(int64_t) * slots, 256);
  L.off_tok = off;
  off = align_up(off + sizeof(int64_t) * slots, 256);
  L.off_map = off;
  off = align_up(off + sizeof(int32_t) * tokens * logical, 256);
  L.bytes = off;
  return L;
}

int validate_ec(const char *name, int batch, int logical, int capacity, int64_t tps,
                int num_experts, const int32_t *l2p) {
  if (batch < 0 || logical <= 0 || logical > 1024 || capacity <= 0 || tps <= 0 ||
      num_experts <= 0 || num_experts > kPlanMaxExperts) {
    set_error("%s: need batch >= 0, 1 <= logical experts <= 1024, capacity > 0, "
              "tokens_per_sample > 0 and 1 <= num_experts <= %d", name, kPlanMaxExperts);
    return MX_ERR_INVALID;
  }
  if (!l2p && logical != num_experts) {
    set_error("%s: logical and physical expert counts differ without an alias map", name);
    return MX_ERR_INVALID;
  }
  const int64_t slots = static_cast<int64_t>(batch) * logical * capacity;
  if (slots >= (int64_t(1) << 31)) {
    set_error("%s: expert-choice slot count exceeds the int32 range", name);
    return MX_ERR_INVALID;
  }
  return MX_OK;
}

}  // namespace gemm
}  // namespace mx

extern "C" size_t mx_expert_choice_plan_workspace_size(int batch, int logical_experts,
                                                       int capacity, int num_experts) {
  if (batch < 0 || logical_experts <= 0 || capacity <= 0 || num_experts <= 0) return 0;
  const int64_t slots = static_cast<int64_t>(batch) * logical_experts * capacity;
  return align_up(plan_layout(slots, num_experts).bytes, 256) + 2 * align_up(8 * slots, 256);
}

extern "C" int mx_build_expert_choice_plan(
    const int64_t *expert_token_indices, const void *expert_token_scores, int score_dtype,
    int batch, int logical_experts, int capacity, int64_t tokens_per_sample,
    const int32_t *logical_to_physical, int num_experts, int64_t *counts, int64_t *starts,
    int32_t *offsets, int64_t *sort_positions, int64_t *sorted_token_indices,
    void *sorted_scores, int64_t *inverse_order, void *workspace, void *stream) {
  clear_error();
  const char *name = "mx_build_expert_choice_plan";
  int rc = validate_ec(name, batch, logical_experts, capacity, tokens_per_sample, num_experts,
                       logical_to_physical);
  if (rc) return rc;
  const int64_t slots = static_cast<int64_t>(batch) * logical_experts * capacity;
  if (slots > 0 && (!expert_token_indices || !expert_token_scores || !workspace ||
                    !sort_positions || !sorted_token_indices)) {
    set_error("%s: routes, workspace, sort_positions and sorted_token_indices must be non-null",
              name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  char *ws = static_cast<char *>(workspace);
  const size_t plan_bytes = align_up(plan_layout(slots, num_experts).bytes, 256);
  int64_t *phys = reinterpret_cast<int64_t *>(ws + plan_bytes);
  int64_t *tok = reinterpret_cast<int64_t *>(ws + plan_bytes + align_up(8 * slots, 256));
  const dim3 grid(static_cast<unsigned>(ceil_div(slots > 0 ? slots : 1, 256)));
  if (slots > 0) {
    hipLaunchKernelGGL(ec_slots_kernel, grid, dim3(256), 0, s, expert_token_indices, slots,
                       logical_experts, capacity, tokens_per_sample, logical_to_physical, phys,
                       tok);
    if ((rc = check_launch(name))) return rc;
  }
  rc = build_plan(phys, expert_token_scores, score_dtype, slots, 1, num_experts, counts, starts,
                  offsets, sort_positions, sorted_token_indices, sorted_scores, inverse_order,
                  workspace, s);
  if (rc || slots == 0) return rc;
  hipLaunchKernelGGL((ec_gather_tok_kernel<int64_t, int64_t>), grid, dim3(256), 0, s,
                     sort_positions, tok, slots, int64_t(0), false, sorted_token_indices);
  return check_launch(name);
}

extern "C" size_t mx_moe_expert_choice_workspace_size(int batch, int logical_experts,
                                                      int capacity, int64_t tokens_per_sample,
                                                      int num_experts, int64_t hidden,
                                                      int64_t ffn, int lora_rank) {
  if (batch < 0 || logical_experts <= 0 || capacity <= 0 || tokens_per_sample <= 0 ||
      num_experts <= 0 || hidden <= 0 || ffn <= 0 || lora_rank < 0 || lora_rank > kLoraMaxRank)
    return 0;
  const int64_t slots = static_cast<int64_t>(batch) * logical_experts * capacity;
  return ec_layout(slots, num_experts, hidden, ffn, batch * tokens_per_sample, logical_experts,
                   lora_width(lora_rank))
      .bytes;
}

extern "C" int mx_moe_forward_expert_choice_ex(
    const void *tokens, const int64_t *expert_token_indices, const void *expert_token_scores,
    int score_dtype, int batch, int logical_experts, int capacity, int64_t tokens_per_sample,
    const int32_t *logical_to_physical, const int32_t *combine_order, int num_experts,
    int64_t hidden, int64_t ffn, int act, const mx_weight *w1, const mx_weight *w3,
    const mx_weight *w2, const mx_lora *l1, const mx_lora *l3, const mx_lora *l2, void *out,
    int out_dtype, void *save_gate, void *save_up, void *save_h, void *save_y, void *save_lora,
    void *workspace, void *stream) {
  clear_error();
  const char *name = "mx_moe_forward_expert_choice";
  int rc = validate_ec(name, batch, logical_experts, capacity, tokens_per_sample, num_experts,
                       logical_to_physical);
  if (rc) return rc;
  const bool bf16_combine = (act & MX_ACT_FLAG_BF16_COMBINE) != 0;
  act &= ~MX_ACT_FLAG_BF16_COMBINE;
  if (act != MX_ACT_SILU && act != MX_ACT_SWIGLU7) {
    set_error("%s: unknown activation %d", name, act);
    return MX_ERR_INVALID;
  }
  if ((rc = check_layer(name, hidden, ffn, w1, w3, w2, l1, l3, l2))) return rc;
  if (w1->format == MX_FMT_F32X3) {
    set_error("%s: MX_FMT_F32X3 (fp32) weights are supported by mx_moe_forward only", name);
    return MX_ERR_INVALID;
  }
  const int64_t T = static_cast<int64_t>(batch) * tokens_per_sample;
  const int64_t slots = static_cast<int64_t>(batch) * logical_experts * capacity;
  if (T == 0) return MX_OK;
  if (!tokens || !out || !workspace || (slots > 0 && (!expert_token_indices ||
                                                      !expert_token_scores))) {
    set_error("%s: tokens, routes, output and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const int lrc = lora_width(l1, l3, l2);
  const EcLayout L = ec_layout(slots, num_experts, hidden, ffn, T, logical_experts, lrc);
  char *ws = static_cast<char *>(workspace);
  int64_t *phys = reinterpret_cast<int64_t *>(ws + L.off_phys);
  int64_t *tok = reinterpret_cast<int64_t *>(ws + L.off_tok);
  int32_t *map = reinterpret_cast<int32_t *>(ws + L.off_map);
  const dim3 sgrid(static_cast<unsigned>(ceil_div(slots > 0 ? slots : 1, 256)));
  hipLaunchKernelGGL(ec_fill_kernel, dim3(static_cast<unsigned>(ceil_div(T * logical_experts, 256))),
                     dim3(256), 0, s, map, T * logical_experts, -1);
  if (slots > 0) {
    hipLaunchKernelGGL(ec_slots_kernel, sgrid, dim3(256), 0, s, expert_token_indices, slots,
                       logical_experts, capacity, tokens_per_sample, logical_to_physical, phys,
                       tok);
    hipLaunchKernelGGL(ec_map_kernel, sgrid, dim3(256), 0, s, tok, slots, logical_experts,
                       capacity, T, map);
    if ((rc = check_launch(name))) return rc;
    rc = build_plan(phys, nullptr, score_dtype, slots, 1, num_experts, nullptr, nullptr, nullptr,
                    nullptr, nullptr, nullptr, nullptr, ws, s);
    if (rc) return rc;
    const PlanView v = plan_view(ws, L.layer.plan);
    // Sorted rows carry slots (k = 1); the GEMM reads each slot's token.
    hipLaunchKernelGGL((ec_gather_tok_kernel<int32_t, int32_t>), sgrid, dim3(256), 0, s,
                       v.row_token, tok, slots, T, true, v.row_token);
    if ((rc = check_launch(name))) return rc;
    uint16_t *y = save_y ? static_cast<uint16_t *>(save_y)
                         : reinterpret_cast<uint16_t *>(ws + L.layer.off_y);
    uint16_t *lora_buf = save_lora ? static_cast<uint16_t *>(save_lora)
                                   : reinterpret_cast<uint16_t *>(ws + L.layer.off_lora);
    uint16_t *h = save_h ? static_cast<uint16_t *>(save_h)
                         : reinterpret_cast<uint16_t *>(ws + L.layer.off_h);
    rc = expert_mlp(L.layer.plan, v, num_experts, static_cast<const uint16_t *>(tokens), hidden,
                    v.row_token, hidden, ffn, act, w1, w3, w2, l1, l3, l2, lora_buf, lrc, h,
                    static_cast<uint16_t *>(save_gate), static_cast<uint16_t *>(save_up), y,
                    hidden, v.row_slot, s);
    if (rc) return rc;
  }
  hipLaunchKernelGGL(ec_combine_kernel, dim3(static_cast<unsigned>(ceil_div(T, 4))), dim3(256), 0,
                     s, save_y ? static_cast<const uint16_t *>(save_y)
                               : reinterpret_cast<const uint16_t *>(ws + L.layer.off_y),
                     expert_token_scores, score_dtype, map, combine_order, T, logical_experts,
                     hidden, out, out_dtype);
  return check_launch(name);
}

extern "C" int mx_moe_forward_expert_choice(
    const void *tokens, const int64_t *expert_token_indices, const void *expert_token_scores,
    int score_dtype, int batch, int logical_experts, int capacity, int64_t tokens_per_sample,
    const int32_t *logical_to_physical, const int32_t *combine_order, int num_experts,
    int64_t hidden, int64_t ffn, int act, const mx_weight *w1, const mx_weight *w3,
    const mx_weight *w2, const mx_lora *l1, const mx_lora *l3, const mx_lora *l2, void *out,
    int out_dtype, void *workspace, void *stream) {
  return mx_moe_forward_expert_choice_ex(
      tokens, expert_token_indices, expert_token_scores, score_dtype, batch, logical_experts,
      capacity, tokens_per_sample, logical_to_physical, combine_order, num_experts, hidden, ffn,
      act, w1, w3, w2, l1, l3, l2, out, out_dtype, nullptr, nullptr, nullptr, nullptr, nullptr,
      workspace, stream);
}

extern "C" size_t mx_moe_backward_expert_choice_workspace_size(int batch, int logical_experts,
                                                               int capacity,
                                                               int64_t tokens_per_sample,
                                                               int num_experts, int64_t hidden,
                                                               int64_t ffn, int lora_rank) {
  if (batch < 0 || logical_experts <= 0 || capacity <= 0 || tokens_per_sample <= 0 ||
      num_experts <= 0 || hidden <= 0 || ffn <= 0 || lora_rank < 0 || lora_rank > kLoraMaxRank)
    return 0;
  const int64_t slots = static_cast<int64_t>(batch) * logical_experts * capacity;
  return ec_back_layout(slots, num_experts, hidden, ffn, batch * tokens_per_sample,
                        logical_experts, lora_width(lora_rank)).bytes;
}

extern "C" int mx_moe_backward_expert_choice(
    const void *grad_out, int grad_dtype, const void *tokens, const int64_t *expert_token_indices,
    const void *expert_token_scores, int score_dtype, int batch, int logical_experts,
    int capacity, int64_t tokens_per_sample, const int32_t *logical_to_physical,
    const int32_t *combine_order, int num_experts, int64_t hidden, int64_t ffn, int act,
    const mx_weight *w1, const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
    const mx_lora *l3, const mx_lora *l2, const void *save_gate, const void *save_up,
    const void *save_h, const void *save_y, const void *save_lora, void *grad_tokens,
    int grad_tokens_dtype, float *grad_scores, float *grad_a1, float *grad_b1, float *grad_a3,
    float *grad_b3, float *grad_a2, float *grad_b2, void *workspace, void *stream) {
  clear_error();
  const char *name = "mx_moe_backward_expert_choice";
  int rc = validate_ec(name, batch, logical_experts, capacity, tokens_per_sample, num_experts,
                       logical_to_physical);
  if (rc) return rc;
  const bool bf16_combine = (act & MX_ACT_FLAG_BF16_COMBINE) != 0;
  act &= ~MX_ACT_FLAG_BF16_COMBINE;
  if (act != MX_ACT_SILU && act != MX_ACT_SWIGLU7) {
    set_error("%s: unknown activation %d", name, act);
    return MX_ERR_INVALID;
  }
  if ((rc = check_layer(name, hidden, ffn, w1, w3, w2, l1, l3, l2))) return rc;
  if (w1->format == MX_FMT_F32X3) {
    set_error("%s: MX_FMT_F32X3 (fp32) weights are inference-only", name);
    return MX_ERR_INVALID;
  }
  const int64_t T = static_cast<int64_t>(batch) * tokens_per_sample;
  const int64_t slots = static_cast<int64_t>(batch) * logical_experts * capacity;
  if (T == 0)
    return zero_lora_grads(name, num_experts, hidden, ffn, l1, l3, l2, grad_a1, grad_b1, grad_a3,
                           grad_b3, grad_a2, grad_b2, as_stream(stream));
  const bool lora = has_lora(l1) || has_lora(l3) || has_lora(l2);
  if (!grad_out || !tokens || !grad_tokens || !workspace ||
      (slots > 0 && (!expert_token_indices || !expert_token_scores || !grad_scores ||
                     !save_gate || !save_up || !save_h || !save_y || (lora && !save_lora)))) {
    set_error("%s: gradients, routes, saved activations and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  if ((grad_dtype != MX_DTYPE_BF16 && grad_dtype != MX_DTYPE_F32) ||
      (grad_tokens_dtype != MX_DTYPE_BF16 && grad_tokens_dtype != MX_DTYPE_F32)) {
    set_error("%s: gradients must be bf16 or fp32", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const EcBackLayout L = ec_back_layout(slots, num_experts, hidden, ffn, T, logical_experts,
                                        lora_width(l1, l3, l2));
  char *ws = static_cast<char *>(workspace);
  int64_t *phys = reinterpret_cast<int64_t *>(ws + L.off_phys);
  int64_t *tok = reinterpret_cast<int64_t *>(ws + L.off_tok);
  int32_t *map = reinterpret_cast<int32_t *>(ws + L.off_map);
  uint16_t *dy = reinterpret_cast<uint16_t *>(ws + L.back.off_dy);
  hipLaunchKernelGGL(ec_fill_kernel, dim3(static_cast<unsigned>(ceil_div(T * logical_experts, 256))),
                     dim3(256), 0, s, map, T * logical_experts, -1);
  if (slots > 0) {
    const dim3 sgrid(static_cast<unsigned>(ceil_div(slots, 256)));
    hipLaunchKernelGGL(ec_slots_kernel, sgrid, dim3(256), 0, s, expert_token_indices, slots,
                       logical_experts, capacity, tokens_per_sample, logical_to_physical, phys,
                       tok);
    hipLaunchKernelGGL(ec_map_kernel, sgrid, dim3(256), 0, s, tok, slots, logical_experts,
                       capacity, T, map);
    if ((rc = check_launch(name))) return rc;
    // The forward's plan over the slots (k = 1), rebuilt.
    rc = build_plan(phys, nullptr, score_dtype, slots, 1, num_experts, nullptr, nullptr, nullptr,
                    nullptr, nullptr, nullptr, nullptr, ws, s);
    if (rc) return rc;
    const PlanView v = plan_view(ws, L.back.plan);
    hipLaunchKernelGGL((ec_gather_tok_kernel<int32_t, int32_t>), sgrid, dim3(256), 0, s,
                       v.row_token, tok, slots, T, true, v.row_token);
    hipLaunchKernelGGL(ec_combine_backward_kernel, dim3(static_cast<unsigned>(ceil_div(slots, 4))),
                       dim3(256), 0, s, grad_out, grad_dtype,
                       static_cast<const uint16_t *>(save_y), tok, expert_token_scores,
                       score_dtype, slots, T, hidden, dy, grad_scores);
    if ((rc = check_launch(name))) return rc;
    uint16_t *fact[6];
    for (int i = 0; i < 6; ++i) fact[i] = reinterpret_cast<uint16_t *>(ws + L.back.off_fact[i]);
    rc = backward_core(L.back, v, num_experts, slots, hidden, ffn, act, w1, w3, w2, l1, l3, l2,
                       static_cast<const uint16_t *>(tokens),
                       static_cast<const uint16_t *>(save_gate),
                       static_cast<const uint16_t *>(save_up),
                       static_cast<const uint16_t *>(save_h),
                       static_cast<const uint16_t *>(save_lora), dy,
                       reinterpret_cast<uint16_t *>(ws + L.back.off_dgu),
                       reinterpret_cast<uint16_t *>(ws + L.back.off_dz), fact, grad_a1, grad_b1,
                       grad_a3, grad_b3, grad_a2, grad_b2, s);
    if (rc) return rc;
  } else if ((rc = zero_lora_grads(name, num_experts, hidden, ffn, l1, l3, l2, grad_a1, grad_b1,
                                   grad_a3, grad_b3, grad_a2, grad_b2, s))) {
    return rc;
  }
  // grad_tokens[t] = sum of its slots' dx rows (fp32, ascending (physical,
  // logical) order; zero for tokens no expert picked).
  hipLaunchKernelGGL(ec_combine_kernel, dim3(static_cast<unsigned>(ceil_div(T, 4))), dim3(256), 0,
                     s, dy, nullptr, MX_DTYPE_F32, map, combine_order, T, logical_experts,
                     hidden, grad_tokens, grad_tokens_dtype);
  return check_launch(name);
}
