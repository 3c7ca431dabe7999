// Top-k token-choice routing: one wavefront per token.
//
// Selection is by logit: softmax is strictly monotone, so the k largest
// probabilities belong to the k largest logits; ties go to the lower expert
// id. Scores are the softmax probabilities of the picks, renormalised and
// scaled as the router asks (routers.py:234-249,
// transformer_lingbot_video.py:1002-1033).
#include <math.h>

#include "common.h"

namespace mx {
namespace {

constexpr int kMaxTopK = 16;

__device__ __forceinline__ bool better(float v, int e, float bv, int be) {
  return v > bv || (v == bv && e < be);
}

template <int PER_LANE>
__global__ __launch_bounds__(256) void route_topk_kernel(const float *logits, int64_t T, int E,
                                                         int k, int renorm, float route_scale,
                                                         int64_t *top_idx, void *top_scores,
                                                         int score_dtype) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float *row = logits + t * E;
  float v[PER_LANE];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER_LANE; ++j) {
    const int e = lane + 64 * j;
    v[j] = e < E ? row[e] : -INFINITY;
    m = fmaxf(m, v[j]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  float z = 0.0f;
#pragma unroll
  for (int j = 0; j < PER_LANE; ++j)
    if (lane + 64 * j < E) z += __expf(v[j] - m);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) z += __shfl_xor(z, off, 64);

  uint32_t taken = 0;
  int my_e = 0;
  float my_v = -INFINITY;
  for (int s = 0; s < k; ++s) {
    float bv = -INFINITY;
    int be = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) {
      const int e = lane + 64 * j;
      if (e < E && !((taken >> j) & 1u) && better(v[j], e, bv, be)) {
        bv = v[j];
        be = e;
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oe = __shfl_xor(be, off, 64);
      if (better(ov, oe, bv, be)) {
        bv = ov;
        be = oe;
      }
    }
    if ((be & 63) == lane) taken |= 1u << (be >> 6);
    if (lane == s) {
      my_e = be;
      my_v = bv;
    }
  }
  float p = lane < k ? __expf(my_v - m) / z : 0.0f;
  float sum = p;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
  float score = p;
  if (renorm == MX_RENORM_CLAMP)
    score = p / fmaxf(sum, 1e-20f);
  else if (renorm == MX_RENORM_EPS)
    score = p / (sum + 1e-20f);
  score *= route_scale;
  if (lane < k) {
    top_idx[t * k + lane] = my_e;
    store_value(top_scores, t * k + lane, score, score_dtype);
  }
}

// The same routing with four lanes per token for 32 < E <= 64 (E a multiple
// of 4): lane q of a quad holds experts [16q, 16q + 16), one 64-byte run of the
// row, so a wave reads 16 whole rows and a token's serial chains are a quarter
// as long. The row max, the softmax sum (four partial sums added in a fixed
// tree) and each round's pick are combined across the quad by lane exchanges.
// A pick is the largest remaining value, the lowest id on ties (the serial
// scan's rule: NaN keys never win, and the first valid id stands in when all
// remaining values are -inf); the quad's owner of the pick marks it NaN.
__global__ __launch_bounds__(256) void route_topk_quad_kernel(const float *logits, int64_t T,
                                                              int E, int k, int renorm,
                                                              float route_scale, int64_t *top_idx,
                                                              void *top_scores, int score_dtype) {
  const int64_t t = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 2;
  if (t >= T) return;  // whole quads leave together
  const int q = threadIdx.x & 3, e0 = 16 * q;
  const float *row = logits + t * E + e0;
  float v[16];
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    const float4 x = e0 + i < E ? *reinterpret_cast<const float4 *>(row + i)
                                : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    v[i] = x.x;
    v[i + 1] = x.y;
    v[i + 2] = x.z;
    v[i + 3] = x.w;
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < 16; ++i) m = fmaxf(m, v[i]);
  m = fmaxf(m, __shfl_xor(m, 1));
  m = fmaxf(m, __shfl_xor(m, 2));
  float z = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (e0 + i < E) z += __expf(v[i] - m);
  z += __shfl_xor(z, 1);
  z += __shfl_xor(z, 2);
  // Lane q keeps the picks of rounds q, q + 4, q + 8, q + 12 (the ones it
  // stores); the rounds loop stays rolled, so the registers stay few.
  int my_sel[4] = {0, 0, 0, 0};
  float my_p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float sum = 0.0f;
#pragma unroll 1
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY;
    int be = -1;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (e0 + i < E && (v[i] > bv || (be < 0 && v[i] == bv))) {
        bv = v[i];
        be = e0 + i;
      }
#pragma unroll
    for (int off = 1; off <= 2; off <<= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oe = __shfl_xor(be, off);
      if (oe >= 0 && (be < 0 || ov > bv || (ov == bv && oe < be))) {
        bv = ov;
        be = oe;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (e0 + i == be) v[i] = __builtin_nanf("");
    const float pr = __expf(bv - m) / z;
    sum += pr;
    if ((r & 3) == q) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if ((r >> 2) == j) {
          my_sel[j] = be;
          my_p[j] = pr;
        }
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = 4 * j + q;
    if (r >= k) break;
    float score = my_p[j];
    if (renorm == MX_RENORM_CLAMP)
      score = my_p[j] / fmaxf(sum, 1e-20f);
    else if (renorm == MX_RENORM_EPS)
      score = my_p[j] / (sum + 1e-20f);
    score *= route_scale;
    top_idx[t * k + r] = my_sel[j];
    store_value(top_scores, t * k + r, score, score_dtype);
  }
}

// The same routing with one LANE per token for E <= 64: the lane holds its
// token's logits in registers, so the max, the softmax sum and the k selection
// rounds need no cross-lane exchange. Taken experts become NaN keys (never
// better); the scan runs in increasing expert order, so a strict > keeps the
// lower id on ties.
template <int EC>
__global__ __launch_bounds__(64) void route_topk_lane_kernel(const float *logits, int64_t T,
                                                              int E, int k, int renorm,
                                                              float route_scale, int64_t *top_idx,
                                                              void *top_scores, int score_dtype,
                                                              bool vec4) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= T) return;
  const float *row = logits + t * E;
  float v[EC];
  if (vec4) {  // 16-byte row loads: E % 4 == 0 and a 16-byte aligned base
#pragma unroll
    for (int e = 0; e < EC; e += 4) {
      const float4 q = e < E ? *reinterpret_cast<const float4 *>(row + e)
                             : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      v[e] = q.x;
      v[e + 1] = q.y;
      v[e + 2] = q.z;
      v[e + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < EC; ++e) v[e] = e < E ? row[e] : -INFINITY;
  }
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < EC; ++e) m = fmaxf(m, v[e]);
  float z = 0.0f;
#pragma unroll
  for (int e = 0; e < EC; ++e)
    if (e < E) z += __expf(v[e] - m);
  int sel[kMaxTopK];
  float p[kMaxTopK];
  float sum = 0.0f;
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    sel[r] = 0;
    p[r] = 0.0f;
    if (r < k) {
      float bv = -INFINITY;
      int be = -1;
#pragma unroll
      for (int e = 0; e < EC; ++e)
        if (e < E && (v[e] > bv || (be < 0 && v[e] == bv))) {
          bv = v[e];
          be = e;
        }
#pragma unroll
      for (int e = 0; e < EC; ++e)
        if (e == be) v[e] = __builtin_nanf("");
      sel[r] = be;
      p[r] = __expf(bv - m) / z;
      sum += p[r];
    }
  }
#pragma unroll
  for (int r = 0; r < kMaxTopK; ++r) {
    if (r >= k) break;
    float score = p[r];
    if (renorm == MX_RENORM_CLAMP)
      score = p[r] / fmaxf(sum, 1e-20f);
    else if (renorm == MX_RENORM_EPS)
      score = p[r] / (sum + 1e-20f);
    score *= route_scale;
    top_idx[t * k + r] = sel[r];
    store_value(top_scores, t * k + r, score, score_dtype);
  }
}

// d(logits) for the selected experts of each row; one wavefront per row of
// fp32 logits [rows, E]. The scores p are softmax or sigmoid of the logits
// (recomputed here); the picks' scores were renormalised by `renorm` with the
// floor `floor` (MX_RENORM_CLAMP: p / max(sum, floor); MX_RENORM_EPS:
// p / (sum + floor)) and multiplied by route_scale. The chain: dL/dp of the
// picks through the renormalisation, then the softmax Jacobian
// (dl_e = p_e (dp_e - sum_m p_m dp_m)) or the sigmoid's (dl_e = dp_e p_e (1 - p_e)).
template <int PER_LANE>
__global__ __launch_bounds__(256) void route_topk_backward_kernel(
    const float *logits, int64_t T, int E, int k, int score_func, int renorm, float floor,
    float route_scale, const int64_t *top_idx, const float *grad_scores, float *grad_logits) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float *row = logits + t * E;
  const bool softmax = score_func == MX_SCORE_SOFTMAX;
  float pr[PER_LANE];
  float m = -INFINITY, z = 1.0f;
#pragma unroll
  for (int j = 0; j < PER_LANE; ++j) {
    const int e = lane + 64 * j;
    pr[j] = e < E ? row[e] : -INFINITY;
    m = fmaxf(m, pr[j]);
  }
  if (softmax) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    z = 0.0f;
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) {
      pr[j] = lane + 64 * j < E ? expf(pr[j] - m) : 0.0f;
      z += pr[j];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) z += __shfl_xor(z, off, 64);
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) pr[j] /= z;
  } else {
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j)
      pr[j] = lane + 64 * j < E ? 1.0f / (1.0f + expf(-pr[j])) : 0.0f;
  }

  // Selected slot of this lane (lane < k): its expert, score and grad.
  int se = -1;
  float sg = 0.0f;
  if (lane < k) {
    se = static_cast<int>(top_idx[t * k + lane]);
    sg = grad_scores[t * k + lane];
  }
  const bool sel_ok = se >= 0 && se < E;
  float sp = 0.0f;
  if (sel_ok) sp = softmax ? expf(row[se] - m) / z : 1.0f / (1.0f + expf(-row[se]));
  float ssum = sp;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ssum += __shfl_xor(ssum, off, 64);
  // dL/dp for the selected experts.
  float dp;
  if (renorm == MX_RENORM_NONE) {
    dp = route_scale * sg;
  } else {
    const float denom = renorm == MX_RENORM_CLAMP ? fmaxf(ssum, floor) : ssum + floor;
    const bool denom_active = renorm == MX_RENORM_EPS || ssum >= floor;
    float gp = sg * sp;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) gp += __shfl_xor(gp, off, 64);
    dp = route_scale * (sg / denom - (denom_active ? gp / (denom * denom) : 0.0f));
  }
  if (!sel_ok) dp = 0.0f;
  float pdp = sp * dp;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) pdp += __shfl_xor(pdp, off, 64);
  // Broadcast the k selections to every lane before any lane diverges.
  int sel_e[kMaxTopK];
  float sel_dp[kMaxTopK];
#pragma unroll
  for (int s = 0; s < kMaxTopK; ++s) {
    sel_e[s] = __shfl(se, s, 64);
    sel_dp[s] = __shfl(dp, s, 64);
  }
#pragma unroll
  for (int j = 0; j < PER_LANE; ++j) {
    const int e = lane + 64 * j;
    float dpe = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxTopK; ++s)
      if (s < k && sel_e[s] == e) dpe += sel_dp[s];
    if (e < E)
      grad_logits[t * E + e] = softmax ? pr[j] * (dpe - pdp) : dpe * pr[j] * (1.0f - pr[j]);
  }
}

// Multi-head routing (MAGI-2): one wavefront per (head, token) row of fp32
// logits [H, S, E]. Scores are softmax or sigmoid of the logits; experts are
// picked by score + expert_bias[h] (the bias steers selection only), ties to
// the lower expert id; the picks' unbiased scores are renormalised to sum 1
// (p / max(sum p, floor), the L1 F.normalize of route.py:136-140) when asked
// and multiplied by route_scale (magi2_preview.py:2735-2742). Follows
// _compute_topk_probs_and_indices_torch_impl (flash_mh_moe/route.py:28-148)
// with num_virtual_group = 1.
template <int PER_LANE>
__global__ __launch_bounds__(256) void route_heads_kernel(
    const float *logits, int64_t S, int H, int E, int k, int score_func, const float *bias,
    int renorm, float renorm_floor, float route_scale, int n_vg, int topk_vg, int layout,
    int64_t *top_idx, void *top_scores, int score_dtype) {
  const int lane = threadIdx.x & 63;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);  // h * S + s
  if (q >= static_cast<int64_t>(H) * S) return;
  const int h = static_cast<int>(q / S);
  const int64_t s = q - static_cast<int64_t>(h) * S;
  const float *row = logits + q * E;
  float sc[PER_LANE], key[PER_LANE];
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < PER_LANE; ++j) {
    const int e = lane + 64 * j;
    sc[j] = e < E ? row[e] : -INFINITY;
    m = fmaxf(m, sc[j]);
  }
  if (score_func == MX_SCORE_SOFTMAX) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    float z = 0.0f;
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) {
      sc[j] = lane + 64 * j < E ? expf(sc[j] - m) : 0.0f;
      z += sc[j];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) z += __shfl_xor(z, off, 64);
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) sc[j] = sc[j] / z;
  } else {
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) sc[j] = lane + 64 * j < E ? 1.0f / (1.0f + expf(-sc[j])) : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < PER_LANE; ++j) {
    const int e = lane + 64 * j;
    key[j] = e < E ? sc[j] + (bias ? bias[static_cast<int64_t>(h) * E + e] : 0.0f) : -INFINITY;
  }
  if (n_vg > 1) {
    // Virtual groups (route.py:62-105): the E experts form n_vg groups of
    // epg consecutive ids; a group scores the sum of its two largest keys
    // (its largest when it holds one expert), the topk_vg best groups are
    // kept (ties to the lower group id), and every other expert's key becomes
    // 0.0 (masked_fill(~mask, 0.0), not -inf) before the expert selection.
    const int epg = E / n_vg;
    float gscore = -INFINITY;  // lane g < n_vg: the score of group g
    for (int g = 0; g < n_vg; ++g) {
      float m1 = -INFINITY, m2 = -INFINITY;
#pragma unroll
      for (int j = 0; j < PER_LANE; ++j) {
        const int e = lane + 64 * j;
        if (e < E && e / epg == g) {
          const float v = key[j];
          if (v > m1) {
            m2 = m1;
            m1 = v;
          } else if (v > m2) {
            m2 = v;
          }
        }
      }
      // Top two of the union of two (largest, second) pairs.
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float o1 = __shfl_xor(m1, off, 64), o2 = __shfl_xor(m2, off, 64);
        const float second = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
        m1 = fmaxf(m1, o1);
        m2 = second;
      }
      if (lane == g) gscore = epg >= 2 ? m1 + m2 : m1;
    }
    uint64_t keep = 0;
    for (int r = 0; r < topk_vg; ++r) {
      const bool cand = lane < n_vg && !((keep >> lane) & 1ull);
      float bv = cand ? gscore : -INFINITY;
      int bg = cand ? lane : 0x7fffffff;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int og = __shfl_xor(bg, off, 64);
        if (better(ov, og, bv, bg)) {
          bv = ov;
          bg = og;
        }
      }
      keep |= 1ull << (bg & 63);
    }
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) {
      const int e = lane + 64 * j;
      if (e < E && !((keep >> (e / epg)) & 1ull)) key[j] = 0.0f;
    }
  }
  uint32_t taken = 0;
  int my_e = 0;
  float my_p = 0.0f;
  for (int r = 0; r < k; ++r) {
    float bv = -INFINITY, bp = 0.0f;
    int be = 0x7fffffff;
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) {
      const int e = lane + 64 * j;
      if (e < E && !((taken >> j) & 1u) && better(key[j], e, bv, be)) {
        bv = key[j];
        be = e;
        bp = sc[j];
      }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oe = __shfl_xor(be, off, 64);
      const float op = __shfl_xor(bp, off, 64);
      if (better(ov, oe, bv, be)) {
        bv = ov;
        be = oe;
        bp = op;
      }
    }
    if ((be & 63) == lane) taken |= 1u << (be >> 6);
    if (lane == r) {
      my_e = be;
      my_p = bp;
    }
  }
  float p = lane < k ? my_p : 0.0f;
  float sum = p;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
  float score = p;
  if (renorm == MX_RENORM_CLAMP)
    score = p / fmaxf(sum, renorm_floor);
  else if (renorm == MX_RENORM_EPS)
    score = p / (sum + renorm_floor);
  score *= route_scale;
  if (lane < k) {
    int64_t o;
    int64_t id;
    if (layout == MX_ROUTE_LAYOUT_ROWS) {
      o = (s * H + h) * k + lane;
      id = static_cast<int64_t>(h) * E + my_e;
    } else {
      o = q * k + lane;
      id = my_e;
    }
    top_idx[o] = id;
    store_value(top_scores, o, score, score_dtype);
  }
}

}  // namespace
}  // namespace mx

using namespace mx;

#define MX_ROUTE_DISPATCH(KERNEL, ...)                                                          \
  do {                                                                                         \
    const int per_lane = (num_experts + 63) / 64;                                              \
    dim3 grid(ceil_div(num_tokens, 4)), block(256);                                            \
    hipStream_t s = as_stream(stream);                                                         \
    switch (per_lane) {                                                                        \
      case 1: hipLaunchKernelGGL(KERNEL<1>, grid, block, 0, s, __VA_ARGS__); break;            \
      case 2: hipLaunchKernelGGL(KERNEL<2>, grid, block, 0, s, __VA_ARGS__); break;            \
      case 3:                                                                                  \
      case 4: hipLaunchKernelGGL(KERNEL<4>, grid, block, 0, s, __VA_ARGS__); break;            \
      case 5: case 6: case 7:                                                                  \
      case 8: hipLaunchKernelGGL(KERNEL<8>, grid, block, 0, s, __VA_ARGS__); break;            \
      default: hipLaunchKernelGGL(KERNEL<16>, grid, block, 0, s, __VA_ARGS__); break;          \
    }                                                                                          \
  } while (0)

static int validate_route(const char *name, const void *logits, int64_t num_tokens,
                          int num_experts, int top_k, int renorm) {
  if (num_tokens < 0 || (!logits && num_tokens > 0)) {
    set_error("%s: need num_tokens >= 0 and non-null logits when it is positive", name);
    return MX_ERR_INVALID;
  }
  if (num_experts <= 0 || num_experts > 1024) {
    set_error("%s: num_experts must be in [1, 1024], got %d", name, num_experts);
    return MX_ERR_INVALID;
  }
  if (top_k <= 0 || top_k > kMaxTopK || top_k > num_experts) {
    set_error("%s: top_k must be in [1, min(16, num_experts)], got %d", name, top_k);
    return MX_ERR_INVALID;
  }
  if (renorm < MX_RENORM_NONE || renorm > MX_RENORM_EPS) {
    set_error("%s: unknown renorm mode %d", name, renorm);
    return MX_ERR_INVALID;
  }
  return MX_OK;
}

extern "C" int mx_route_topk(const float *logits, int64_t num_tokens, int num_experts, int top_k,
                             int renorm, float route_scale, int64_t *top_idx, void *top_scores,
                             int score_dtype, void *stream) {
  clear_error();
  int rc = validate_route("mx_route_topk", logits, num_tokens, num_experts, top_k, renorm);
  if (rc) return rc;
  if (num_tokens > 0 && (!top_idx || !top_scores)) {
    set_error("mx_route_topk: outputs must be non-null");
    return MX_ERR_INVALID;
  }
  if (num_tokens == 0) return MX_OK;
  // The quad kernel and the vector path of the lane kernel read rows as
  // float4: E % 4 == 0 and a 16-byte aligned base (a view with a storage
  // offset may not be); otherwise the lane kernel reads scalars.
  const bool vec4 = (num_experts & 3) == 0 && (reinterpret_cast<uintptr_t>(logits) & 15) == 0;
  if (num_experts > 32 && num_experts <= 64 && vec4) {
    hipLaunchKernelGGL(route_topk_quad_kernel, dim3(static_cast<unsigned>(ceil_div(num_tokens, 64))),
                       dim3(256), 0, as_stream(stream), logits, num_tokens, num_experts, top_k,
                       renorm, route_scale, top_idx, top_scores, score_dtype);
    return check_launch("mx_route_topk");
  }
  if (num_experts <= 64) {
    // One-wave workgroups spread the tokens over every CU.
    const dim3 grid(static_cast<unsigned>(ceil_div(num_tokens, 64)));
    hipStream_t s = as_stream(stream);
#define MX_ROUTE_LANE(EC)                                                                    \
  hipLaunchKernelGGL(route_topk_lane_kernel<EC>, grid, dim3(64), 0, s, logits, num_tokens,    \
                     num_experts, top_k, renorm, route_scale, top_idx, top_scores, score_dtype, \
                     vec4)
    if (num_experts <= 8)
      MX_ROUTE_LANE(8);
    else if (num_experts <= 16)
      MX_ROUTE_LANE(16);
    else if (num_experts <= 32)
      MX_ROUTE_LANE(32);
    else
      MX_ROUTE_LANE(64);
#undef MX_ROUTE_LANE
    return check_launch("mx_route_topk");
  }
  MX_ROUTE_DISPATCH(route_topk_kernel, logits, num_tokens, num_experts, top_k, renorm,
                    route_scale, top_idx, top_scores, score_dtype);
  return check_launch("mx_route_topk");
}

extern "C" int mx_route_scores_backward(const float *logits, int64_t num_rows, int num_experts,
                                        int top_k, int score_func, int renorm, float renorm_floor,
                                        float route_scale, const int64_t *top_idx,
                                        const float *grad_scores, float *grad_logits,
                                        void *stream) {
  clear_error();
  const char *name = "mx_route_scores_backward";
  const int64_t num_tokens = num_rows;
  int rc = validate_route(name, logits, num_tokens, num_experts, top_k, renorm);
  if (rc) return rc;
  if (score_func != MX_SCORE_SOFTMAX && score_func != MX_SCORE_SIGMOID) {
    set_error("%s: unknown score function %d", name, score_func);
    return MX_ERR_INVALID;
  }
  if (!(renorm_floor >= 0.0f)) {
    set_error("%s: renorm_floor must be >= 0", name);
    return MX_ERR_INVALID;
  }
  if (num_tokens > 0 && (!top_idx || !grad_scores || !grad_logits)) {
    set_error("%s: buffers must be non-null", name);
    return MX_ERR_INVALID;
  }
  if (num_tokens == 0) return MX_OK;
  MX_ROUTE_DISPATCH(route_topk_backward_kernel, logits, num_tokens, num_experts, top_k,
                    score_func, renorm, renorm_floor, route_scale, top_idx, grad_scores,
                    grad_logits);
  return check_launch(name);
}

extern "C" int mx_route_topk_backward(const float *logits, int64_t num_tokens, int num_experts,
                                      int top_k, int renorm, float route_scale,
                                      const int64_t *top_idx, const float *grad_scores,
                                      float *grad_logits, void *stream) {
  return mx_route_scores_backward(logits, num_tokens, num_experts, top_k, MX_SCORE_SOFTMAX, renorm,
                                  1e-20f, route_scale, top_idx, grad_scores, grad_logits, stream);
}

extern "C" int mx_route_topk_heads(const float *logits, int num_heads, int64_t num_tokens,
                                   int num_experts, int top_k, int score_func,
                                   const float *expert_bias, int renorm, float renorm_floor,
                                   float route_scale, int num_virtual_group,
                                   int topk_virtual_group, int layout, int64_t *top_idx,
                                   void *top_scores, int score_dtype, void *stream) {
  clear_error();
  int rc = validate_route("mx_route_topk_heads", logits, num_tokens, num_experts, top_k, renorm);
  if (rc) return rc;
  if (num_heads <= 0 || (num_tokens > 0 && (!top_idx || !top_scores))) {
    set_error("mx_route_topk_heads: need num_heads > 0 and non-null outputs");
    return MX_ERR_INVALID;
  }
  if (score_func != MX_SCORE_SOFTMAX && score_func != MX_SCORE_SIGMOID) {
    set_error("mx_route_topk_heads: unknown score function %d", score_func);
    return MX_ERR_INVALID;
  }
  if (layout != MX_ROUTE_LAYOUT_HEADS && layout != MX_ROUTE_LAYOUT_ROWS) {
    set_error("mx_route_topk_heads: unknown output layout %d", layout);
    return MX_ERR_INVALID;
  }
  if (!(renorm_floor >= 0.0f)) {
    set_error("mx_route_topk_heads: renorm_floor must be >= 0");
    return MX_ERR_INVALID;
  }
  if (num_virtual_group < 1 || num_virtual_group > 64 ||
      num_experts % num_virtual_group != 0 ||
      (num_virtual_group > 1 &&
       (topk_virtual_group < 1 || topk_virtual_group > num_virtual_group))) {
    set_error("mx_route_topk_heads: num_virtual_group must divide num_experts and lie in "
              "[1, 64], topk_virtual_group in [1, num_virtual_group] (got %d, %d)",
              num_virtual_group, topk_virtual_group);
    return MX_ERR_INVALID;
  }
  const int64_t rows = num_tokens * num_heads;
  if (rows == 0) return MX_OK;
  const int per_lane = (num_experts + 63) / 64;
  const dim3 grid(static_cast<unsigned>(ceil_div(rows, 4))), block(256);
  hipStream_t s = as_stream(stream);
#define MX_HEADS_ARGS logits, num_tokens, num_heads, num_experts, top_k, score_func, expert_bias, \
    renorm, renorm_floor, route_scale, num_virtual_group, topk_virtual_group, layout, top_idx, \
    top_scores, score_dtype
  switch (per_lane) {
    case 1: hipLaunchKernelGGL(route_heads_kernel<1>, grid, block, 0, s, MX_HEADS_ARGS); break;
    case 2: hipLaunchKernelGGL(route_heads_kernel<2>, grid, block, 0, s, MX_HEADS_ARGS); break;
    case 3:
    case 4: hipLaunchKernelGGL(route_heads_kernel<4>, grid, block, 0, s, MX_HEADS_ARGS); break;
    case 5: case 6: case 7:
    case 8: hipLaunchKernelGGL(route_heads_kernel<8>, grid, block, 0, s, MX_HEADS_ARGS); break;
    default: hipLaunchKernelGGL(route_heads_kernel<16>, grid, block, 0, s, MX_HEADS_ARGS); break;
  }
#undef MX_HEADS_ARGS
  return check_launch("mx_route_topk_heads");
}
