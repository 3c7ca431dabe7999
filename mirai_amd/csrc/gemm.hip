// Grouped expert GEMMs on bf16 MFMA (v_mfma_f32_16x16x32_bf16, gfx950) over
// expert-sorted rows, with the frozen weights decoded from NF4 / INT8 on the
// way into LDS, the per-expert LoRA up-projection fused as a K-extension of
// the same accumulators, and three epilogues:
//   EPI_SWIGLU : h = silu(x w1^T + dA1) * (x w3^T + dA3)   (gate/up pair)
//   EPI_STORE  : y = x w^T + dA, rows written through a row map (down proj.)
//   EPI_LORA_A : p = bf16(s * bf16(x a^T))  (LoRA down-projection, rank <= 32)
//
// Work decomposition: the dispatch plan lists row tiles (expert, first row) of
// kTileM rows; a workgroup computes one (row tile, column tile) pair. The
// blockIdx -> tile mapping gives each of the 8 XCDs a contiguous run of tiles
// (workgroups are dispatched round-robin over XCDs), ordered row-tile major,
// so the column tiles sharing an activation tile, and the row tiles sharing an
// expert's weights, run on the same XCD and hit its L2.
#include "common.h"
#include "plan.h"

namespace mx {
namespace gemm {

constexpr int BM = kPlanTileM;  // rows per tile
constexpr int BN = 128;         // B rows (output columns) per tile
constexpr int BK = 64;          // K per pipeline stage (= one NF4 block)
constexpr int NT = 256;         // 4 wavefronts, 2 x 2, each 64 x 64
constexpr int kLoraK = 32;      // LoRA rank padded for one MFMA K step
constexpr int kLoraLd = 96;     // low-rank activation row: [gate 32 | up 32 | down 32]

enum { EPI_SWIGLU = 0, EPI_STORE = 1, EPI_LORA_A = 2 };

constexpr int kStageA = BM * BK * 2;
constexpr int kStageB = BN * BK * 2;
constexpr int kLdsBytes = 2 * kStageA + 2 * kStageB + NT * 32;

struct Params {
  const uint16_t *x;
  int64_t ldx;
  const int32_t *row_token;  // sorted row -> activation row (null: identity)
  int64_t K;
  const void *w[4];          // per B-row group: weight data
  const uint16_t *wscale[4]; // NF4 absmax / INT8 scale
  int64_t wn[4];             // rows per expert of each weight
  int64_t N;                 // output columns
  int n_tiles_n;
  const uint16_t *lora_p;    // [R, ldp] scaled low-rank activations
  int64_t ldp;
  const uint16_t *lora_b[2]; // [E, N, r]
  int lora_r[2];
  const int2 *tiles;
  const int32_t *num_tiles;
  const int64_t *seg_end;
  uint16_t *out;
  int64_t ldo;
  const int32_t *out_row;    // sorted row -> output row (null: identity)
  uint16_t *save_gate;
  uint16_t *save_up;
  float scale[4];
};

// B-tile row j -> (weight group, output column / row of that weight).
template <int EPI>
__device__ __forceinline__ void b_row(int j, int nt, int &which, int64_t &n) {
  if (EPI == EPI_SWIGLU) {
    // 64 ffn columns per tile; each wave's 64 B rows hold 32 gate then 32 up
    // rows of the same ffn columns, so the SwiGLU pairs land in one lane.
    which = (j >> 5) & 1;
    n = static_cast<int64_t>(nt) * 64 + (j >> 6) * 32 + (j & 31);
  } else if (EPI == EPI_STORE) {
    which = 0;
    n = static_cast<int64_t>(nt) * BN + j;
  } else {
    which = j >> 5;
    n = j & 31;
  }
}

__device__ __forceinline__ int swz128(int row, int chunk) {  // 8 x 16 B chunks per row
  return row * 128 + ((chunk ^ (row & 7)) << 4);
}
__device__ __forceinline__ int swz64(int row, int chunk) {  // 4 x 16 B chunks per row
  return row * 64 + ((chunk ^ (row & 3)) << 4);
}

template <int FMT, int EPI, bool LORA>
__global__ __launch_bounds__(NT) void grouped_gemm_kernel(Params p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t *sA0 = smem;
  uint8_t *sB0 = smem + 2 * kStageA;
  const int tid = threadIdx.x;
  uint16_t *lut = reinterpret_cast<uint16_t *>(smem + 2 * kStageA + 2 * kStageB) + tid * 16;

  // ---------------------------------------------------------------- tile
  const int num_m = *p.num_tiles;
  const int total = num_m * p.n_tiles_n;
  const int per_xcd = (total + 7) >> 3;
  const int slot = blockIdx.x >> 3;
  if (slot >= per_xcd) return;
  const int logical = (blockIdx.x & 7) * per_xcd + slot;
  if (logical >= total) return;
  const int mt = logical / p.n_tiles_n;
  const int nt = logical - mt * p.n_tiles_n;
  const int2 tile = p.tiles[mt];
  const int e = tile.x;
  const int64_t row0 = tile.y;
  const int64_t row_end = p.seg_end[e];

  // ----------------------------------------------------- A (activations)
  const int a_chunk = tid & 7;
  const uint16_t *a_ptr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t grow = row0 + (tid >> 3) + 32 * i;
    a_ptr[i] = nullptr;
    if (grow < row_end) {
      const int64_t src = p.row_token ? static_cast<int64_t>(p.row_token[grow]) : grow;
      a_ptr[i] = p.x + src * p.ldx + a_chunk * 8;
    }
  }

  // ------------------------------------------------------- B (weights)
  const int bj = tid >> 1, bh = tid & 1;
  int which;
  int64_t bn;
  b_row<EPI>(bj, nt, which, bn);
  const bool b_valid = bn < p.wn[which];
  const int64_t wrow = static_cast<int64_t>(e) * p.wn[which] + bn;
  const uint8_t *b_base = nullptr;
  const uint16_t *b_absmax = nullptr;
  float b_scale = 0.0f;
  if (b_valid) {
    const uint8_t *w = static_cast<const uint8_t *>(p.w[which]);
    if (FMT == MX_FMT_NF4) {
      b_base = w + wrow * (p.K / 2) + bh * 16;
      b_absmax = p.wscale[which] + wrow * (p.K / BK);
    } else if (FMT == MX_FMT_INT8) {
      b_base = w + wrow * p.K + bh * 32;
      b_scale = bf16_bits_to_f32(p.wscale[which][wrow]);
    } else {
      b_base = w + wrow * p.K * 2 + bh * 64;
    }
  }

  constexpr int kBRegs = FMT == MX_FMT_BF16 ? 4 : (FMT == MX_FMT_INT8 ? 2 : 1);
  uint4 ra[4];
  uint4 rb[kBRegs];
  uint32_t rabs = 0;

  auto load_stage = [&](int kt) {
    const int64_t k0 = static_cast<int64_t>(kt) * BK;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ra[i] = a_ptr[i] ? *reinterpret_cast<const uint4 *>(a_ptr[i] + k0) : make_uint4(0, 0, 0, 0);
    if (b_valid) {
      if (FMT == MX_FMT_NF4) {
        rb[0] = *reinterpret_cast<const uint4 *>(b_base + kt * 32);
        rabs = b_absmax[kt];
      } else if (FMT == MX_FMT_INT8) {
#pragma unroll
        for (int q = 0; q < 2; ++q) rb[q] = *reinterpret_cast<const uint4 *>(b_base + kt * 64 + 16 * q);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) rb[q] = *reinterpret_cast<const uint4 *>(b_base + kt * 128 + 16 * q);
      }
    } else {
#pragma unroll
      for (int q = 0; q < kBRegs; ++q) rb[q] = make_uint4(0, 0, 0, 0);
      rabs = 0;
    }
  };

  auto store_stage = [&](int st) {
    uint8_t *sA = sA0 + st * kStageA;
    uint8_t *sB = sB0 + st * kStageB;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<uint4 *>(sA + swz128((tid >> 3) + 32 * i, a_chunk)) = ra[i];
    uint32_t dec[16];
    if (FMT == MX_FMT_NF4) {
      // Private 16-entry table of this block's decoded values, exactly
      // bf16(fp32(level) * fp32(absmax)), then one LDS lookup per element.
      const float a = bf16_bits_to_f32(rabs);
      uint4 t0, t1;
      t0.x = pack_bf16x2(kNF4Levels[0] * a, kNF4Levels[1] * a);
      t0.y = pack_bf16x2(kNF4Levels[2] * a, kNF4Levels[3] * a);
      t0.z = pack_bf16x2(kNF4Levels[4] * a, kNF4Levels[5] * a);
      t0.w = pack_bf16x2(kNF4Levels[6] * a, kNF4Levels[7] * a);
      t1.x = pack_bf16x2(kNF4Levels[8] * a, kNF4Levels[9] * a);
      t1.y = pack_bf16x2(kNF4Levels[10] * a, kNF4Levels[11] * a);
      t1.z = pack_bf16x2(kNF4Levels[12] * a, kNF4Levels[13] * a);
      t1.w = pack_bf16x2(kNF4Levels[14] * a, kNF4Levels[15] * a);
      reinterpret_cast<uint4 *>(lut)[0] = t0;
      reinterpret_cast<uint4 *>(lut)[1] = t1;
      const uint32_t words[4] = {rb[0].x, rb[0].y, rb[0].z, rb[0].w};
#pragma unroll
      for (int wi = 0; wi < 4; ++wi) {
#pragma unroll
        for (int by = 0; by < 4; ++by) {
          const uint32_t code = (words[wi] >> (8 * by)) & 0xffu;
          dec[wi * 4 + by] = static_cast<uint32_t>(lut[code & 15u]) |
                             (static_cast<uint32_t>(lut[code >> 4]) << 16);
        }
      }
    } else if (FMT == MX_FMT_INT8) {
      const uint32_t words[8] = {rb[0].x, rb[0].y, rb[0].z, rb[0].w,
                                 rb[1].x, rb[1].y, rb[1].z, rb[1].w};
#pragma unroll
      for (int wi = 0; wi < 8; ++wi) {
        const uint32_t w = words[wi];
        const float q0 = static_cast<float>(static_cast<int8_t>(w & 0xffu));
        const float q1 = static_cast<float>(static_cast<int8_t>((w >> 8) & 0xffu));
        const float q2 = static_cast<float>(static_cast<int8_t>((w >> 16) & 0xffu));
        const float q3 = static_cast<float>(static_cast<int8_t>(w >> 24));
        dec[2 * wi] = pack_bf16x2(q0 * b_scale, q1 * b_scale);
        dec[2 * wi + 1] = pack_bf16x2(q2 * b_scale, q3 * b_scale);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        dec[4 * q] = rb[q].x;
        dec[4 * q + 1] = rb[q].y;
        dec[4 * q + 2] = rb[q].z;
        dec[4 * q + 3] = rb[q].w;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *reinterpret_cast<uint4 *>(sB + swz128(bj, 4 * bh + q)) =
          make_uint4(dec[4 * q], dec[4 * q + 1], dec[4 * q + 2], dec[4 * q + 3]);
  };

  // -------------------------------------------------------------- MFMA
  const int lane = tid & 63, wid = tid >> 6;
  const int wm = wid >> 1, wn = wid & 1;
  f32x4 acc[4][4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute_stage = [&](int st) {
    const uint8_t *sA = sA0 + st * kStageA;
    const uint8_t *sB = sB0 + st * kStageB;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int ch = kk * 4 + (lane >> 4);
      bf16x8 a[4], b[4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        a[mb] = *reinterpret_cast<const bf16x8 *>(sA + swz128(wm * 64 + mb * 16 + (lane & 15), ch));
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
        b[nb] = *reinterpret_cast<const bf16x8 *>(sB + swz128(wn * 64 + nb * 16 + (lane & 15), ch));
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[mb], b[nb], acc[mb][nb], 0, 0, 0);
    }
  };

  const int KT = static_cast<int>(p.K / BK);
  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_stage(kt + 1);
    compute_stage(cur);
    if (kt + 1 < KT) store_stage(cur ^ 1);
    __syncthreads();
  }

  // ------------------------------------------- LoRA up-projection (K = 32)
  // Accumulated apart from the frozen projection so the epilogue can round
  // both to bf16 before adding them, as the reference adds a bf16 LoRA delta
  // to a bf16 projection output (experts.py:3370-3374).
  f32x4 acc2[4][4];
  if (LORA) {
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc2[mb][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int n_adapt = EPI == EPI_SWIGLU ? 2 : 1;
    uint8_t *sP = sA0;  // n_adapt x [BM][32] bf16
    uint8_t *sL = sB0;  // [BN][32] bf16
    for (int idx = tid; idx < BM * 4 * n_adapt; idx += NT) {
      const int ad = idx / (BM * 4);
      const int rem = idx - ad * BM * 4;
      const int r = rem >> 2, c = rem & 3;
      const int64_t grow = row0 + r;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (grow < row_end)
        v = *reinterpret_cast<const uint4 *>(p.lora_p + grow * p.ldp + ad * 32 + c * 8);
      *reinterpret_cast<uint4 *>(sP + ad * BM * 64 + swz64(r, c)) = v;
    }
    {
      const int lw = EPI == EPI_SWIGLU ? which : 0;
      const int r = p.lora_r[lw];
      const uint16_t *lb = p.lora_b[lw];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int c = 2 * bh + q;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (b_valid && lb && c * 8 < r)
          v = *reinterpret_cast<const uint4 *>(lb + (static_cast<int64_t>(e) * p.N + bn) * r + c * 8);
        *reinterpret_cast<uint4 *>(sL + swz64(bj, c)) = v;
      }
    }
    __syncthreads();
    const int ch = lane >> 4;
    bf16x8 a[n_adapt][4], b[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
      b[nb] = *reinterpret_cast<const bf16x8 *>(sL + swz64(wn * 64 + nb * 16 + (lane & 15), ch));
#pragma unroll
    for (int ad = 0; ad < n_adapt; ++ad)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        a[ad][mb] = *reinterpret_cast<const bf16x8 *>(sP + ad * BM * 64 +
                                                      swz64(wm * 64 + mb * 16 + (lane & 15), ch));
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) {
        const int ad = EPI == EPI_SWIGLU ? (nb >> 1) : 0;
        acc2[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[ad][mb], b[nb], acc2[mb][nb], 0, 0, 0);
      }
  }
  // Projection output as the reference forms it: bf16(x W^T), plus the bf16
  // LoRA delta, rounded again.
  auto proj = [&](int mb, int nb, int i) -> float {
    const float base = round_bf16(acc[mb][nb][i]);
    if (!LORA) return base;
    return round_bf16(base + round_bf16(acc2[mb][nb][i]));
  };

  // ------------------------------------------------------------ epilogue
  // Accumulator layout of v_mfma_f32_16x16x32_bf16: lane holds rows
  // 4*(lane/16) + i (i = 0..3) of column lane%16.
  const int64_t rbase = row0 + wm * 64 + 4 * (lane >> 4);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = rbase + mb * 16 + i;
      if (r >= row_end) continue;
      if (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int nbp = 0; nbp < 2; ++nbp) {
          const int64_t f = static_cast<int64_t>(nt) * 64 + wn * 32 + nbp * 16 + (lane & 15);
          const float g = proj(mb, nbp, i);
          const float u = proj(mb, nbp + 2, i);
          // silu(g) rounded to bf16, then the bf16 product (experts.py:289-317).
          const float sg = round_bf16(g / (1.0f + __expf(-g)));
          p.out[r * p.ldo + f] = f32_to_bf16_bits(sg * u);
          if (p.save_gate) p.save_gate[r * p.N + f] = f32_to_bf16_bits(g);
          if (p.save_up) p.save_up[r * p.N + f] = f32_to_bf16_bits(u);
        }
      } else if (EPI == EPI_STORE) {
        const int64_t orow = p.out_row ? static_cast<int64_t>(p.out_row[r]) : r;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const int64_t n = static_cast<int64_t>(nt) * BN + wn * 64 + nb * 16 + (lane & 15);
          if (n < p.N) p.out[orow * p.ldo + n] = f32_to_bf16_bits(proj(mb, nb, i));
        }
      } else {
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
          const int n = wn * 64 + nb * 16 + (lane & 15);
          if (n < p.N) {
            // bf16(x a^T) first, then the LoRA scale, as low_rank.to(bf16) * scale.
            const float lr = round_bf16(acc[mb][nb][i]);
            p.out[r * p.ldo + n] = f32_to_bf16_bits(lr * p.scale[n >> 5]);
          }
        }
      }
    }
  }
}

template <int FMT, int EPI, bool LORA>
int launch(const Params &p, int64_t max_row_tiles, hipStream_t s) {
  const int64_t total = max_row_tiles * p.n_tiles_n;
  if (total <= 0) return MX_OK;
  const int64_t grid = 8 * ceil_div(total, 8);
  if (grid > 0x7fffffff) {
    set_error("grouped GEMM grid too large");
    return MX_ERR_INVALID;
  }
  auto kern = grouped_gemm_kernel<FMT, EPI, LORA>;
  static bool configured = false;
  if (!configured) {
    // Dynamic LDS above 64 KiB; a runtime that needs no opt-in may refuse the
    // attribute, which is harmless, so its status is consumed and dropped.
    if (hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes) != hipSuccess)
      (void)hipGetLastError();
    configured = true;
  }
  hipLaunchKernelGGL(kern, dim3(static_cast<unsigned>(grid)), dim3(NT), kLdsBytes, s, p);
  return check_launch("grouped GEMM launch");
}

template <int EPI, bool LORA>
int launch_fmt(int fmt, const Params &p, int64_t max_row_tiles, hipStream_t s) {
  switch (fmt) {
    case MX_FMT_BF16: return launch<MX_FMT_BF16, EPI, LORA>(p, max_row_tiles, s);
    case MX_FMT_NF4: return launch<MX_FMT_NF4, EPI, LORA>(p, max_row_tiles, s);
    case MX_FMT_INT8: return launch<MX_FMT_INT8, EPI, LORA>(p, max_row_tiles, s);
  }
  set_error("unknown weight format %d", fmt);
  return MX_ERR_INVALID;
}

template <int EPI>
int launch_any(int fmt, bool lora, const Params &p, int64_t max_row_tiles, hipStream_t s) {
  return lora ? launch_fmt<EPI, true>(fmt, p, max_row_tiles, s)
              : launch_fmt<EPI, false>(fmt, p, max_row_tiles, s);
}

// ------------------------------------------------------------ host helpers
constexpr int kStageEvents = 7;
thread_local void *g_stage_events[kStageEvents] = {};
thread_local int g_stage_count = 0;

void mark_stage(int i, hipStream_t s) {
  if (g_stage_count == kStageEvents && g_stage_events[i])
    (void)hipEventRecord(static_cast<hipEvent_t>(g_stage_events[i]), s);
}

struct LayerLayout {
  PlanLayout plan;
  size_t off_lora = 0, off_h = 0, off_y = 0, bytes = 0;
};

LayerLayout layer_layout(int64_t rows, int num_experts, int64_t hidden, int64_t ffn) {
  LayerLayout L;
  L.plan = plan_layout(rows, num_experts);
  size_t off = align_up(L.plan.bytes, 256);
  L.off_lora = off;
  off = align_up(off + sizeof(uint16_t) * rows * kLoraLd, 256);
  L.off_h = off;
  off = align_up(off + sizeof(uint16_t) * rows * ffn, 256);
  L.off_y = off;
  off = align_up(off + sizeof(uint16_t) * rows * hidden, 256);
  L.bytes = off;
  return L;
}

bool has_lora(const mx_lora *l) { return l && l->rank > 0; }

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
  if (w->format != MX_FMT_BF16 && w->format != MX_FMT_NF4 && w->format != MX_FMT_INT8) {
    set_error("%s: weight %s has unknown format %d", name, key, w->format);
    return MX_ERR_INVALID;
  }
  if (w->format != MX_FMT_BF16 && !w->scale) {
    set_error("%s: weight %s needs its scale / absmax buffer", name, key);
    return MX_ERR_INVALID;
  }
  return MX_OK;
}

int check_lora(const char *name, const char *key, const mx_lora *l) {
  if (!l || l->rank == 0) return MX_OK;
  if (l->rank < 0 || l->rank > kLoraK || l->rank % 8 != 0 || !l->a || !l->b) {
    set_error("%s: LoRA on %s needs rank in {8,16,24,32} and both factors (got rank %d)", name,
              key, l->rank);
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

// LoRA down-projection p = bf16(s * bf16(x a^T)) for up to 4 adapters that
// share the same input rows; adapter i lands in columns [32i, 32i+32).
int lora_down(const PlanView &v, int experts, int64_t max_tiles, const uint16_t *x, int64_t ldx,
              const int32_t *row_token, int64_t K, const mx_lora *const *adapters, int n_adapt,
              uint16_t *out, int64_t ldo, hipStream_t s) {
  Params p = base_params(v);
  p.x = x;
  p.ldx = ldx;
  p.row_token = row_token;
  p.K = K;
  for (int i = 0; i < 4; ++i) {
    const mx_lora *l = i < n_adapt ? adapters[i] : nullptr;
    p.w[i] = has_lora(l) ? l->a : nullptr;
    p.wn[i] = has_lora(l) ? l->rank : 0;
    p.scale[i] = has_lora(l) ? l->scale : 0.0f;
  }
  p.N = 32 * n_adapt;
  p.n_tiles_n = 1;
  p.seg_end = v.seg + experts;
  p.out = out;
  p.ldo = ldo;
  return launch<MX_FMT_BF16, EPI_LORA_A, false>(p, max_tiles, s);
}

// gate/up grouped GEMM with SwiGLU epilogue, then the down grouped GEMM.
int expert_mlp(const PlanLayout &PL, const PlanView &v, int experts, const uint16_t *x,
               int64_t ldx, const int32_t *row_token, int64_t hidden, int64_t ffn,
               const mx_weight *w1, const mx_weight *w3, const mx_weight *w2,
               const mx_lora *l1, const mx_lora *l3, const mx_lora *l2, uint16_t *lora_buf,
               uint16_t *h, uint16_t *save_gate, uint16_t *save_up, uint16_t *y, int64_t ldy,
               const int32_t *out_row, hipStream_t s) {
  const bool lora13 = has_lora(l1) || has_lora(l3);
  const bool lora2 = has_lora(l2);
  int rc;
  if (lora13) {
    const mx_lora *ad[2] = {l1, l3};
    rc = lora_down(v, experts, PL.max_tiles, x, ldx, row_token, hidden, ad, 2, lora_buf, kLoraLd, s);
    if (rc) return rc;
  }
  mark_stage(2, s);
  {
    Params p = base_params(v);
    p.x = x;
    p.ldx = ldx;
    p.row_token = row_token;
    p.K = hidden;
    p.w[0] = w1->data;
    p.w[1] = w3->data;
    p.wscale[0] = static_cast<const uint16_t *>(w1->scale);
    p.wscale[1] = static_cast<const uint16_t *>(w3->scale);
    p.wn[0] = p.wn[1] = ffn;
    p.N = ffn;
    p.n_tiles_n = static_cast<int>(ffn / 64);
    p.lora_p = lora_buf;
    p.ldp = kLoraLd;
    p.lora_b[0] = has_lora(l1) ? static_cast<const uint16_t *>(l1->b) : nullptr;
    p.lora_b[1] = has_lora(l3) ? static_cast<const uint16_t *>(l3->b) : nullptr;
    p.lora_r[0] = has_lora(l1) ? l1->rank : 0;
    p.lora_r[1] = has_lora(l3) ? l3->rank : 0;
    p.seg_end = v.seg + experts;
    p.out = h;
    p.ldo = ffn;
    p.save_gate = save_gate;
    p.save_up = save_up;
    rc = launch_any<EPI_SWIGLU>(w1->format, lora13, p, PL.max_tiles, s);
    if (rc) return rc;
  }
  mark_stage(3, s);
  if (lora2) {
    const mx_lora *ad[1] = {l2};
    rc = lora_down(v, experts, PL.max_tiles, h, ffn, nullptr, ffn, ad, 1, lora_buf + 64, kLoraLd, s);
    if (rc) return rc;
  }
  mark_stage(4, s);
  Params p = base_params(v);
  p.x = h;
  p.ldx = ffn;
  p.row_token = nullptr;
  p.K = ffn;
  p.w[0] = w2->data;
  p.wscale[0] = static_cast<const uint16_t *>(w2->scale);
  p.wn[0] = hidden;
  p.N = hidden;
  p.n_tiles_n = static_cast<int>(ceil_div(hidden, BN));
  p.lora_p = lora_buf + 64;
  p.ldp = kLoraLd;
  p.lora_b[0] = lora2 ? static_cast<const uint16_t *>(l2->b) : nullptr;
  p.lora_r[0] = lora2 ? l2->rank : 0;
  p.seg_end = v.seg + experts;
  p.out = y;
  p.ldo = ldy;
  p.out_row = out_row;
  return launch_any<EPI_STORE>(w2->format, lora2, p, PL.max_tiles, s);
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
  return MX_OK;
}

}  // namespace gemm
}  // namespace mx

using namespace mx;
using namespace mx::gemm;

extern "C" size_t mx_moe_workspace_size(int64_t num_tokens, int top_k, int num_experts,
                                        int64_t hidden, int64_t ffn) {
  if (num_tokens < 0 || top_k <= 0 || num_experts <= 0 || hidden <= 0 || ffn <= 0) return 0;
  return layer_layout(num_tokens * top_k, num_experts, hidden, ffn).bytes;
}

extern "C" int mx_moe_forward(const void *tokens, const int64_t *top_idx, const void *top_scores,
                              int score_dtype, int64_t num_tokens, int top_k, int num_experts,
                              int64_t hidden, int64_t ffn, const mx_weight *w1,
                              const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
                              const mx_lora *l3, const mx_lora *l2, void *out, int out_dtype,
                              void *save_gate, void *save_up, void *save_h, void *save_y,
                              void *save_lora, void *workspace, void *stream) {
  clear_error();
  const char *name = "mx_moe_forward";
  int rc = validate_plan_args(name, num_tokens, top_k, num_experts);
  if (rc) return rc;
  if ((rc = check_layer(name, hidden, ffn, w1, w3, w2, l1, l3, l2))) return rc;
  if (num_tokens == 0) return MX_OK;
  if (!tokens || !top_idx || !top_scores || !out || !workspace) {
    set_error("%s: tokens, routes, output and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const int64_t R = num_tokens * top_k;
  const LayerLayout L = layer_layout(R, num_experts, hidden, ffn);
  char *ws = static_cast<char *>(workspace);
  const PlanView v = plan_view(ws, L.plan);
  mark_stage(0, s);
  rc = build_plan(top_idx, nullptr, score_dtype, num_tokens, top_k, num_experts, nullptr, nullptr,
                  nullptr, nullptr, nullptr, nullptr, nullptr, ws, s);
  if (rc) return rc;
  mark_stage(1, s);
  uint16_t *lora_buf = save_lora ? static_cast<uint16_t *>(save_lora)
                                 : reinterpret_cast<uint16_t *>(ws + L.off_lora);
  uint16_t *h = save_h ? static_cast<uint16_t *>(save_h) : reinterpret_cast<uint16_t *>(ws + L.off_h);
  uint16_t *y = save_y ? static_cast<uint16_t *>(save_y) : reinterpret_cast<uint16_t *>(ws + L.off_y);
  rc = expert_mlp(L.plan, v, num_experts, static_cast<const uint16_t *>(tokens), hidden,
                  v.row_token, hidden, ffn, w1, w3, w2, l1, l3, l2, lora_buf, h,
                  static_cast<uint16_t *>(save_gate), static_cast<uint16_t *>(save_up), y, hidden,
                  v.row_slot, s);
  if (rc) return rc;
  mark_stage(5, s);
  rc = mx_combine(y, top_idx, top_scores, score_dtype, num_tokens, top_k, num_experts, hidden,
                  out, out_dtype, stream);
  mark_stage(6, s);
  return rc;
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

extern "C" int mx_moe_for_loop(const void *tokens_sorted, const int64_t *counts, int64_t num_rows,
                               int num_experts, int64_t hidden, int64_t ffn, const mx_weight *w1,
                               const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
                               const mx_lora *l3, const mx_lora *l2, void *out, void *workspace,
                               void *stream) {
  clear_error();
  const char *name = "mx_moe_for_loop";
  int rc = validate_plan_args(name, num_rows, 1, num_experts);
  if (rc) return rc;
  if ((rc = check_layer(name, hidden, ffn, w1, w3, w2, l1, l3, l2))) return rc;
  if (num_rows == 0) return MX_OK;
  if (!tokens_sorted || !counts || !out || !workspace) {
    set_error("%s: tokens, counts, output and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const LayerLayout L = layer_layout(num_rows, num_experts, hidden, ffn);
  char *ws = static_cast<char *>(workspace);
  const PlanView v = plan_view(ws, L.plan);
  if ((rc = plan_from_counts(counts, num_rows, num_experts, ws, s))) return rc;
  return expert_mlp(L.plan, v, num_experts, static_cast<const uint16_t *>(tokens_sorted), hidden,
                    nullptr, hidden, ffn, w1, w3, w2, l1, l3, l2,
                    reinterpret_cast<uint16_t *>(ws + L.off_lora),
                    reinterpret_cast<uint16_t *>(ws + L.off_h), nullptr, nullptr,
                    static_cast<uint16_t *>(out), hidden, nullptr, s);
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
  if (num_rows == 0) return MX_OK;
  if (!x || !counts || !out || !workspace) {
    set_error("%s: x, counts, output and workspace must be non-null", name);
    return MX_ERR_INVALID;
  }
  hipStream_t s = as_stream(stream);
  const LayerLayout L = layer_layout(num_rows, num_experts, in_f, out_f);
  char *ws = static_cast<char *>(workspace);
  const PlanView v = plan_view(ws, L.plan);
  if ((rc = plan_from_counts(counts, num_rows, num_experts, ws, s))) return rc;
  uint16_t *lora_buf = reinterpret_cast<uint16_t *>(ws + L.off_lora);
  const bool lr = has_lora(lora);
  if (lr) {
    const mx_lora *ad[1] = {lora};
    rc = lora_down(v, num_experts, L.plan.max_tiles, static_cast<const uint16_t *>(x), in_f,
                   nullptr, in_f, ad, 1, lora_buf, kLoraLd, s);
    if (rc) return rc;
  }
  Params p = base_params(v);
  p.x = static_cast<const uint16_t *>(x);
  p.ldx = in_f;
  p.K = in_f;
  p.w[0] = w->data;
  p.wscale[0] = static_cast<const uint16_t *>(w->scale);
  p.wn[0] = out_f;
  p.N = out_f;
  p.n_tiles_n = static_cast<int>(ceil_div(out_f, BN));
  p.lora_p = lora_buf;
  p.ldp = kLoraLd;
  p.lora_b[0] = lr ? static_cast<const uint16_t *>(lora->b) : nullptr;
  p.lora_r[0] = lr ? lora->rank : 0;
  p.seg_end = v.seg + num_experts;
  p.out = static_cast<uint16_t *>(out);
  p.ldo = out_f;
  return launch_any<EPI_STORE>(w->format, lr, p, L.plan.max_tiles, s);
}
