// Fused router front end: router GEMM, scores, selection and renormalisation
// in one kernel (LingBotVideoRouter.forward,
// mirai/vendors/lingbot_video/transformer_lingbot_video.py:962-1033).
//
// The reference computes fp32 logits = tokens.float() @ W.T (W [E, d] fp32),
// scores = softmax(logits) or sigmoid(logits), picks the top-k experts by
// scores + e_score_correction_bias (optionally restricted to the topk_group
// best expert groups, :865-890), gathers the bias-free scores of the picks,
// divides them by (sum + 1e-20) when k > 1 and norm_topk_prob, and multiplies
// by route_scale.
//
// Logits at fp32 accuracy on bf16 MFMA: the fp32 weight is stored as three
// bf16 planes hi + mid + lo that sum to it exactly (mx_router_weight_planes).
// bf16 tokens are exact bf16 values, so each product x*hi, x*mid, x*lo is
// exact in fp32 and the MFMA's fp32 accumulation is the only rounding, as in
// an fp32 GEMM. fp32 tokens are split the same way in registers and the six
// products of plane order <= 2 are summed (the dropped terms are below 2^-24
// of the product).
//
// Work decomposition: a workgroup of 4 waves takes 128 tokens and all E
// experts (E padded to EP = 32, 64, 128 or 256). Each wave owns 32 tokens and
// loads their rows straight from HBM into registers, several K stages ahead;
// the weight planes of one K stage are staged in LDS (double-buffered) and
// shared by the 4 waves. The MFMA takes the weight fragment first, so the
// accumulators of a lane hold ONE token (lane % 32) and half of its experts
// (lanes l and l ^ 32 together hold all EP): the softmax, the selection and
// the renormalisation run on register values with one cross-lane exchange per
// step, 32 tokens per wave at once.
#include <math.h>

#include "common.h"

namespace mx {
namespace {

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kRouterTokens = 128;  // tokens per workgroup (4 blocks of 32)

// Waves per 32-token block, per padded expert count (see router_fused_kernel).
#ifndef ROUTER_KS_32
#define ROUTER_KS_32 2
#endif
#ifndef ROUTER_KS_64
#define ROUTER_KS_64 2
#endif
#ifndef ROUTER_KS_128
#define ROUTER_KS_128 2
#endif
#ifndef ROUTER_KS_256
#define ROUTER_KS_256 1
#endif
constexpr int kRouterMaxTopK = 16;
constexpr int kRouterMaxGroups = 32;

__host__ __device__ constexpr int router_padded_experts(int E) {
  return E <= 32 ? 32 : E <= 64 ? 64 : E <= 128 ? 128 : 256;
}

// Byte offset of 16-byte chunk `chunk` of plane row `row` in a stage of rows
// of BK bf16 values, XOR-swizzled so that the 16 rows read by one quarter
// wave at one logical chunk land in 16 distinct bank groups.
template <int BK>
__device__ __forceinline__ int rswz(int row, int chunk) {
  if (BK == 64) return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4);
  return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4);
}

__device__ __forceinline__ bool better(float v, int e, float bv, int be) {
  return v > bv || (v == bv && e < be);
}

// fp32 -> three bf16 planes with x == hi + mid + lo (each residual is exact in fp32).
__device__ __forceinline__ void split3(float x, float &hi, float &mid, float &lo) {
  hi = round_bf16(x);
  const float r = x - hi;
  mid = round_bf16(r);
  lo = round_bf16(r - mid);
}

// Weight planes [3][EP][d] bf16 from fp32 W [E, d]; rows E..EP-1 are zero.
__global__ __launch_bounds__(256) void router_planes_kernel(const float *w, int E, int EP,
                                                            int64_t d, uint16_t *planes) {
  const int64_t chunks = d / 4;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(EP) * chunks) return;
  const int64_t e = i / chunks, c = i - e * chunks;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (e < E) v = reinterpret_cast<const float4 *>(w + e * d)[c];
  const float x[4] = {v.x, v.y, v.z, v.w};
  float hi[4], mid[4], lo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) split3(x[j], hi[j], mid[j], lo[j]);
  const int64_t plane = static_cast<int64_t>(EP) * d;
  uint2 *o = reinterpret_cast<uint2 *>(planes + e * d + 4 * c);
  o[0] = make_uint2(pack_bf16x2(hi[0], hi[1]), pack_bf16x2(hi[2], hi[3]));
  o[plane / 4] = make_uint2(pack_bf16x2(mid[0], mid[1]), pack_bf16x2(mid[2], mid[3]));
  o[2 * plane / 4] = make_uint2(pack_bf16x2(lo[0], lo[1]), pack_bf16x2(lo[2], lo[3]));
}

struct RouterArgs {
  const void *tokens;
  int64_t T, d;
  int E;
  const uint16_t *planes;  // [3][EP][d]
  const float *bias;       // [E] or null (selection only)
  const float *logit_delta;  // [T, E] fp32 or null, added to the logits
  int k, score_func, n_group, topk_group, norm;
  float route_scale;
  float *logits_out;  // [T, E] or null
  float *scores_out;  // [T, E] or null
  int64_t *top_idx;   // [T, k]
  void *top_scores;   // [T, k]
  int score_dtype;
};

// KS waves share each 32-token block and split every K stage between them
// (KS = 2 runs two waves per SIMD, so one wave's LDS waits overlap the other's
// MFMAs); their partial sums are added in a fixed order before the epilogue.
template <int NB, bool XF32, int KS>
__global__ __launch_bounds__(256 * KS) void router_fused_kernel(RouterArgs a) {
  constexpr int NT = 256 * KS;
  constexpr int BK = NB > 4 ? 32 : 64;  // k per stage
  constexpr int EP = 32 * NB;
  constexpr int CPR = BK / 8;            // 16-byte chunks per plane row per stage
  constexpr int SUB = BK / 16;           // MFMA k-steps per stage (= chunks per lane half)
  constexpr int SUBK = SUB / KS;         // k-steps per stage of one wave
  static_assert(SUBK >= 1, "each wave needs at least one k-step per stage");
  constexpr int W_CHUNKS = 3 * EP * CPR;
  constexpr int W_LOADS = (W_CHUNKS + NT - 1) / NT;
  constexpr int XB = XF32 ? 4 : 2;
  constexpr int X_REGS = SUBK * XB / 2;  // 16-byte registers per lane per stage
  constexpr int DEPTH = 4;               // token stages in flight
  constexpr int W_STAGE = W_CHUNKS * 16;
  constexpr int V = NB * 16;             // values per lane
  constexpr int KEY_BYTES = kRouterTokens * EP * 4;
  constexpr int SEL_BYTES = kRouterTokens * kRouterMaxTopK * 4;
  constexpr int GRP_BYTES = kRouterTokens * kRouterMaxGroups * 4;
  constexpr int EPI_BYTES = KEY_BYTES + SEL_BYTES + GRP_BYTES;
  constexpr int RED_BYTES = KS > 1 ? 4 * V * 64 * 4 : 0;
  constexpr int SMEM0 = 2 * W_STAGE > EPI_BYTES ? 2 * W_STAGE : EPI_BYTES;
  constexpr int SMEM = SMEM0 > RED_BYTES ? SMEM0 : RED_BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5;
  const int tb = wave & 3, kq = wave >> 2;   // token block, k part
  const int slot = tb * 32 + (lane & 31);    // token of this lane within the workgroup
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * kRouterTokens + slot;
  const int64_t trow = tok < a.T ? tok : a.T - 1;  // tail lanes re-read the last token
  const int KT = static_cast<int>(a.d / BK);

  // Token rows: lane half h covers k in [h*BK/2, (h+1)*BK/2) of each stage,
  // k part kq the SUBK consecutive 8-element chunks from kq*SUBK of that. The
  // weight fragments use the same k order, so the permutation of k inside the
  // MFMA is immaterial to the dot product.
  const uint8_t *xrow = static_cast<const uint8_t *>(a.tokens) +
                        (trow * a.d + h * (BK / 2) + kq * SUBK * 8) * XB;
  auto load_x = [&](int kt, u32x4 (&r)[X_REGS]) __attribute__((always_inline)) {
    const u32x4 *p = reinterpret_cast<const u32x4 *>(xrow + static_cast<int64_t>(kt) * BK * XB);
#pragma unroll
    for (int j = 0; j < X_REGS; ++j) r[j] = p[j];
  };

  // Weight stage: thread tid moves 16-byte chunks q = i*NT + tid.
  uint32_t w_src[W_LOADS];
  int w_dst[W_LOADS];
#pragma unroll
  for (int i = 0; i < W_LOADS; ++i) {
    const int q = (i * NT + tid) % W_CHUNKS, row = q / CPR, c = q % CPR;
    w_src[i] = static_cast<uint32_t>(row * a.d + c * 8);
    w_dst[i] = rswz<BK>(row, c);
  }
  auto w_live = [&](int i) __attribute__((always_inline)) {
    return W_CHUNKS % NT == 0 || i * NT + tid < W_CHUNKS;
  };
  auto load_w = [&](int kt, u32x4 (&r)[W_LOADS]) __attribute__((always_inline)) {
    const uint16_t *base = a.planes + static_cast<int64_t>(kt) * BK;
#pragma unroll
    for (int i = 0; i < W_LOADS; ++i) r[i] = *reinterpret_cast<const u32x4 *>(base + w_src[i]);
  };
  auto store_w = [&](int buf, const u32x4 (&r)[W_LOADS]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < W_LOADS; ++i)
      if (w_live(i)) *reinterpret_cast<u32x4 *>(smem + buf * W_STAGE + w_dst[i]) = r[i];
  };

  f32x16 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[nb][j] = 0.0f;

  auto compute = [&](int buf, const u32x4 (&xr)[X_REGS]) __attribute__((always_inline)) {
    const uint8_t *sw = smem + buf * W_STAGE;
    bf16x8 wf[SUBK][NB][3];
#pragma unroll
    for (int s = 0; s < SUBK; ++s) {
      const int c = h * SUB + kq * SUBK + s;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int p = 0; p < 3; ++p)
          wf[s][nb][p] =
              *reinterpret_cast<const bf16x8 *>(sw + rswz<BK>(p * EP + nb * 32 + (lane & 31), c));
    }
#pragma unroll
    for (int s = 0; s < SUBK; ++s) {
      bf16x8 xa[XF32 ? 3 : 1];
      if constexpr (!XF32) {
        xa[0] = __builtin_bit_cast(bf16x8, xr[s]);
      } else {
        const u32x4 p0 = xr[2 * s], p1 = xr[2 * s + 1];
        const float v[8] = {__uint_as_float(p0[0]), __uint_as_float(p0[1]), __uint_as_float(p0[2]),
                            __uint_as_float(p0[3]), __uint_as_float(p1[0]), __uint_as_float(p1[1]),
                            __uint_as_float(p1[2]), __uint_as_float(p1[3])};
        u32x4 ph, pm, pl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float h0, m0, l0, h1, m1, l1;
          split3(v[2 * j], h0, m0, l0);
          split3(v[2 * j + 1], h1, m1, l1);
          ph[j] = pack_bf16x2(h0, h1);
          pm[j] = pack_bf16x2(m0, m1);
          pl[j] = pack_bf16x2(l0, l1);
        }
        xa[0] = __builtin_bit_cast(bf16x8, ph);
        xa[1] = __builtin_bit_cast(bf16x8, pm);
        xa[2] = __builtin_bit_cast(bf16x8, pl);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[s][nb][0], xa[0], acc[nb], 0, 0, 0);
        acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[s][nb][1], xa[0], acc[nb], 0, 0, 0);
        acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[s][nb][2], xa[0], acc[nb], 0, 0, 0);
        if constexpr (XF32) {
          acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[s][nb][0], xa[1], acc[nb], 0, 0, 0);
          acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[s][nb][1], xa[1], acc[nb], 0, 0, 0);
          acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[s][nb][0], xa[2], acc[nb], 0, 0, 0);
        }
      }
    }
  };

  // ------------------------------------------------------------ K loop
  // Token stages run DEPTH ahead in registers; weight stages are loaded into
  // registers three steps ahead, written to LDS one step ahead.
  u32x4 xr[DEPTH][X_REGS];
  u32x4 wr[2][W_LOADS];
  const int last = KT - 1;
  load_w(0, wr[0]);
#pragma unroll
  for (int u = 0; u < DEPTH; ++u) load_x(u < last ? u : last, xr[u]);
  load_w(1 < last ? 1 : last, wr[1]);
  store_w(0, wr[0]);
  load_w(2 < last ? 2 : last, wr[0]);
  __syncthreads();
  for (int kb = 0; kb < KT; kb += DEPTH) {
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      const int kt = kb + u;
      if (kt < KT) {
        compute(u & 1, xr[u]);
        load_x(kt + DEPTH < last ? kt + DEPTH : last, xr[u]);
        store_w((u + 1) & 1, wr[(u + 1) & 1]);
        load_w(kt + 3 < last ? kt + 3 : last, wr[(u + 1) & 1]);
        __syncthreads();
      }
    }
  }
  if constexpr (KS > 1) {
    // k part 1 hands its partial sums to k part 0 (sum order: part 0 + part 1).
    float *red = reinterpret_cast<float *>(smem);
    if (kq == 1) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 16; ++j) red[((tb * NB + nb) * 16 + j) * 64 + lane] = acc[nb][j];
    }
    __syncthreads();
    if (kq == 0) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[nb][j] += red[((tb * NB + nb) * 16 + j) * 64 + lane];
    }
    __syncthreads();
    if (kq != 0) return;
  }

  // ------------------------------------------------------------ epilogue
  // Value j of acc[nb] is expert 32*nb + 8*(j/4) + 4*h + j%4 of token `tok`.
  const int E = a.E;
  const bool live = tok < a.T;
  float v[V];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int j = 0; j < 16; ++j) v[nb * 16 + j] = acc[nb][j];
  auto expert_of = [&](int i) __attribute__((always_inline)) {
    return 32 * (i >> 4) + 8 * ((i & 15) >> 2) + 4 * h + (i & 3);
  };
  auto store_rows = [&](float *out) __attribute__((always_inline)) {
    if (!out || !live) return;
#pragma unroll
    for (int q = 0; q < V / 4; ++q) {
      const int e0 = expert_of(4 * q);
      if (e0 >= E) continue;
      float *p = out + tok * E + e0;
      if ((E & 3) == 0) {
        *reinterpret_cast<float4 *>(p) = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (e0 + j < E) p[j] = v[4 * q + j];
      }
    }
  };
  if (a.logit_delta) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int e = expert_of(i);
      if (e < E) v[i] += a.logit_delta[trow * E + e];
    }
  }
  store_rows(a.logits_out);

  // Scores.
  if (a.score_func == MX_SCORE_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (expert_of(i) < E) m = fmaxf(m, v[i]);
    m = fmaxf(m, __shfl_xor(m, 32, 64));
    float z = 0.0f;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      v[i] = expert_of(i) < E ? expf(v[i] - m) : 0.0f;
      z += v[i];
    }
    z += __shfl_xor(z, 32, 64);
    const float rz = 1.0f / z;
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] *= rz;
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) v[i] = 1.0f / (1.0f + expf(-v[i]));
  }
  store_rows(a.scores_out);

  // Selection keys: score + correction bias. A NaN key never compares as
  // better, so NaN marks padded and already taken experts.
  float key[V];
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int e = expert_of(i);
    key[i] = e < E ? v[i] + (a.bias ? a.bias[e] : 0.0f) : __builtin_nanf("");
  }

  float *skey = reinterpret_cast<float *>(smem);                        // [128][EP]
  float *ssel = reinterpret_cast<float *>(smem + KEY_BYTES);            // [128][16]
  float *sgrp = reinterpret_cast<float *>(smem + KEY_BYTES + SEL_BYTES);  // [128][32]
  if (a.n_group > 1) {
    // Group-limited choice (_group_limited_choice_scores, :873-886): a group's
    // score is the sum of its two largest keys; the topk_group best groups
    // (ties to the lower group) stay, the other experts' keys become -inf.
    const int epg = E / a.n_group;
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (expert_of(i) < E) skey[slot * EP + expert_of(i)] = key[i];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int g = h; g < a.n_group; g += 2) {
      float t1 = -INFINITY, t2 = -INFINITY;
      for (int e = g * epg; e < (g + 1) * epg; ++e) {
        const float x = skey[slot * EP + e];
        if (x > t1) {
          t2 = t1;
          t1 = x;
        } else if (x > t2) {
          t2 = x;
        }
      }
      sgrp[slot * kRouterMaxGroups + g] = t1 + t2;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    uint32_t keep = 0;
    for (int r = 0; r < a.topk_group; ++r) {
      float bv = -INFINITY;
      int bg = 0x7fffffff;
      for (int g = 0; g < a.n_group; ++g) {
        const float x = sgrp[slot * kRouterMaxGroups + g];
        if (!((keep >> g) & 1u) && better(x, g, bv, bg)) {
          bv = x;
          bg = g;
        }
      }
      keep |= 1u << bg;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int e = expert_of(i);
      if (e < E && !((keep >> (e / epg)) & 1u)) key[i] = -INFINITY;
    }
  }

  // Top-k: k rounds of (lane-local best, exchange with lane ^ 32). Both lanes
  // of a pair see the same winner; ties go to the lower expert id. Values are
  // scanned in increasing expert order, so a strict > keeps the lower id.
  float psum = 0.0f;
  for (int r = 0; r < a.k; ++r) {
    float bv = -INFINITY, bp = 0.0f;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < V; ++i) {
      if (key[i] > bv || (key[i] == bv && be == 0x7fffffff)) {
        bv = key[i];
        be = expert_of(i);
        bp = v[i];
      }
    }
    const float ov = __shfl_xor(bv, 32, 64), op = __shfl_xor(bp, 32, 64);
    const int oe = __shfl_xor(be, 32, 64);
    if (better(ov, oe, bv, be)) {
      bv = ov;
      be = oe;
      bp = op;
    }
#pragma unroll
    for (int i = 0; i < V; ++i)
      if (expert_of(i) == be) key[i] = __builtin_nanf("");
    if (h == 0) {
      ssel[slot * kRouterMaxTopK + r] = bp;
      if (live) a.top_idx[tok * a.k + r] = be;
    }
    psum += bp;
  }
  if (h == 0 && live) {
    const float denom = psum + 1e-20f;
    for (int r = 0; r < a.k; ++r) {
      float p = ssel[slot * kRouterMaxTopK + r];
      if (a.norm) p = p / denom;
      store_value(a.top_scores, tok * a.k + r, p * a.route_scale, a.score_dtype);
    }
  }
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_router_padded_experts(int num_experts) {
  return num_experts <= 0 || num_experts > 256 ? -1 : router_padded_experts(num_experts);
}

extern "C" size_t mx_router_planes_size(int num_experts, int64_t hidden) {
  if (num_experts <= 0 || num_experts > 256 || hidden <= 0) return 0;
  return static_cast<size_t>(3) * router_padded_experts(num_experts) * hidden * sizeof(uint16_t);
}

extern "C" int mx_router_weight_planes(const float *weight, int num_experts, int64_t hidden,
                                       void *planes, void *stream) {
  clear_error();
  if (!weight || !planes || num_experts <= 0 || num_experts > 256 || hidden <= 0 ||
      hidden % 64 != 0) {
    set_error("mx_router_weight_planes: need non-null buffers, 1 <= num_experts <= 256 and "
              "hidden a positive multiple of 64");
    return MX_ERR_INVALID;
  }
  const int EP = router_padded_experts(num_experts);
  const int64_t n = static_cast<int64_t>(EP) * (hidden / 4);
  hipLaunchKernelGGL(router_planes_kernel, dim3(static_cast<unsigned>(ceil_div(n, 256))), dim3(256),
                     0, as_stream(stream), weight, num_experts, EP, hidden,
                     static_cast<uint16_t *>(planes));
  return check_launch("mx_router_weight_planes");
}

extern "C" int mx_router_forward(const void *tokens, int token_dtype, int64_t num_tokens,
                                 int64_t hidden, int num_experts, const void *planes,
                                 const float *expert_bias, const float *logit_delta, int top_k,
                                 int score_func, int n_group, int topk_group, int norm_topk_prob,
                                 float route_scale, float *logits_out, float *scores_out,
                                 int64_t *top_idx, void *top_scores, int score_dtype,
                                 void *stream) {
  clear_error();
  if (!planes || num_tokens < 0 || (num_tokens > 0 && (!tokens || !top_idx || !top_scores))) {
    set_error("mx_router_forward: planes, tokens and outputs must be non-null, num_tokens >= 0");
    return MX_ERR_INVALID;
  }
  if (token_dtype != MX_DTYPE_BF16 && token_dtype != MX_DTYPE_F32) {
    set_error("mx_router_forward: tokens must be bf16 or fp32");
    return MX_ERR_INVALID;
  }
  if (hidden <= 0 || hidden % 64 != 0) {
    set_error("mx_router_forward: hidden must be a positive multiple of 64, got %lld",
              static_cast<long long>(hidden));
    return MX_ERR_INVALID;
  }
  if (num_experts <= 0 || num_experts > 256) {
    set_error("mx_router_forward: num_experts must be in [1, 256], got %d", num_experts);
    return MX_ERR_INVALID;
  }
  if (static_cast<int64_t>(3) * router_padded_experts(num_experts) * hidden >= (int64_t(1) << 31)) {
    set_error("mx_router_forward: the weight planes (3 x %d x %lld) exceed the 32-bit offsets of "
              "the kernel", router_padded_experts(num_experts), static_cast<long long>(hidden));
    return MX_ERR_INVALID;
  }
  if (top_k <= 0 || top_k > kRouterMaxTopK || top_k > num_experts) {
    set_error("mx_router_forward: top_k must be in [1, min(16, num_experts)], got %d", top_k);
    return MX_ERR_INVALID;
  }
  if (score_func != MX_SCORE_SOFTMAX && score_func != MX_SCORE_SIGMOID) {
    set_error("mx_router_forward: unknown score function %d", score_func);
    return MX_ERR_INVALID;
  }
  if (score_dtype != MX_DTYPE_BF16 && score_dtype != MX_DTYPE_F32) {
    set_error("mx_router_forward: scores must be bf16 or fp32");
    return MX_ERR_INVALID;
  }
  if (n_group > 1) {
    const int epg = num_experts / n_group;
    if (n_group > kRouterMaxGroups || num_experts % n_group != 0 || epg < 2 || topk_group < 1 ||
        topk_group > n_group || top_k > topk_group * epg) {
      set_error("mx_router_forward: group-limited routing needs n_group <= 32 dividing "
                "num_experts into groups of >= 2, 1 <= topk_group <= n_group and "
                "top_k <= topk_group * experts per group");
      return MX_ERR_INVALID;
    }
  }
  if (num_tokens == 0) return MX_OK;
  RouterArgs a{tokens, num_tokens, hidden, num_experts, static_cast<const uint16_t *>(planes),
               expert_bias, logit_delta, top_k, score_func, n_group > 1 ? n_group : 1,
               topk_group, (top_k > 1 && norm_topk_prob) ? 1 : 0, route_scale, logits_out,
               scores_out, top_idx, top_scores, score_dtype};
  const dim3 grid(static_cast<unsigned>(ceil_div(num_tokens, kRouterTokens)));
  hipStream_t s = as_stream(stream);
  const int EP = router_padded_experts(num_experts);
  const bool f32 = token_dtype == MX_DTYPE_F32;
#define MX_ROUTER_LAUNCH(NB, KS)                                                              \
  do {                                                                                        \
    const dim3 block(256 * KS);                                                               \
    if (f32)                                                                                  \
      hipLaunchKernelGGL((router_fused_kernel<NB, true, KS>), grid, block, 0, s, a);          \
    else                                                                                      \
      hipLaunchKernelGGL((router_fused_kernel<NB, false, KS>), grid, block, 0, s, a);         \
  } while (0)
  switch (EP) {
    case 32: MX_ROUTER_LAUNCH(1, ROUTER_KS_32); break;
    case 64: MX_ROUTER_LAUNCH(2, ROUTER_KS_64); break;
    case 128: MX_ROUTER_LAUNCH(4, ROUTER_KS_128); break;
    default: MX_ROUTER_LAUNCH(8, ROUTER_KS_256); break;
  }
#undef MX_ROUTER_LAUNCH
  return check_launch("mx_router_forward");
}
