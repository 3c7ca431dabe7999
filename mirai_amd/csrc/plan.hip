// Dispatch plan: a stable counting sort of the R = T*k route slots by expert,
// built without any host synchronisation.
//
// The flat slot array is cut into blocks of EB consecutive slots. Inside a
// block, every expert owns an EB-bit mask in LDS marking the slots routed to
// it (OR is order independent, so the masks are deterministic). A slot's rank
// among the block's slots of the same expert is the popcount of the mask bits
// below it, which is exactly the stable order of argsort(stable=True).
// Pass 1 writes per-block expert counts (and per-block counts of invalid ids),
// pass 2 (one workgroup) scans them into per-(block, expert) bases and writes
// the plan's error count, pass 3 rebuilds the masks and scatters. Every
// counter is written, not accumulated, so a plan needs no clearing launch.
#include "common.h"
#include "plan.h"

namespace mx {
namespace {

__device__ __forceinline__ void build_masks(const int64_t *top_idx, int64_t slot0, int n_slots,
                                            int E, int words, uint32_t *mask,
                                            int32_t *lds_err) {
  for (int i = threadIdx.x; i < E * words; i += blockDim.x) mask[i] = 0;
  __syncthreads();
  for (int p = threadIdx.x; p < n_slots; p += blockDim.x) {
    const int64_t e = top_idx[slot0 + p];
    if (e >= 0 && e < E) {
      atomicOr(&mask[e * words + (p >> 5)], 1u << (p & 31));
    } else if (lds_err && e != MX_ROUTE_DROPPED) {
      atomicAdd(lds_err, 1);
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(256) void plan_count_kernel(const int64_t *top_idx, int64_t R,
                                                         int E, int EB, int32_t *block_counts,
                                                         int32_t *block_err) {
  extern __shared__ uint32_t mask[];
  __shared__ int32_t n_err;
  if (threadIdx.x == 0) n_err = 0;
  const int words = EB >> 5;
  const int64_t slot0 = static_cast<int64_t>(blockIdx.x) * EB;
  const int n_slots = static_cast<int>(min<int64_t>(EB, R - slot0));
  build_masks(top_idx, slot0, n_slots, E, words, mask, &n_err);  // syncs before and after
  if (threadIdx.x == 0) block_err[blockIdx.x] = n_err;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int c = 0;
    for (int w = 0; w < words; ++w) c += __popc(mask[e * words + w]);
    block_counts[static_cast<int64_t>(blockIdx.x) * E + e] = c;
  }
}

// Block-wide exclusive scan of one int64 per thread (blockDim.x == 1024).
__device__ int64_t block_exclusive_scan(int64_t v, int64_t *shared, int64_t *total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int64_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int64_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) shared[wid] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t run = 0;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) {
      const int64_t s = shared[w];
      shared[w] = run;
      run += s;
    }
    shared[16] = run;
  }
  __syncthreads();
  const int64_t r = shared[wid] + x - v;
  *total = shared[16];
  __syncthreads();
  return r;
}

// One workgroup of 1024 threads. Thread t owns experts t, t + 1024, ...
// (E <= kPlanMaxExperts); the exclusive scans over experts run chunk by chunk
// of 1024 in expert order, carrying the running total. With E <= 1024 the
// per-block counts are summed and turned into per-block bases by G groups of
// E threads, each over a contiguous range of blocks (G = min(16, 1024 / E));
// with more experts each thread walks all blocks for each of its experts.
// kEpt: experts per thread the kernel is compiled for (1 when E <= 1024).
template <int kEpt>
__global__ __launch_bounds__(1024) void plan_scan_kernel(
    const int32_t *block_counts, const int32_t *block_err, int n_blocks, int E, int64_t n_rows,
    int tile_m, const int64_t *counts_in, int32_t *block_base, int64_t *seg, int2 *tiles,
    int32_t *num_tiles, int2 *tiles2, int32_t *num_tiles2, int2 *tiles2m, int32_t *num_tiles2m,
    int2 *tilesr, int32_t *num_tilesr, int32_t *err_counter, int64_t *counts_out,
    int64_t *starts_out, int32_t *offsets_out) {
  __shared__ int64_t scan_tmp[32];
  __shared__ int32_t part[1024];     // [group][expert] block-range counts (E <= 1024)
  __shared__ int64_t start_s[1024];  // expert starts (E <= 1024)
  __shared__ int32_t n_err;
  const int t = threadIdx.x;
  if (t == 0) n_err = 0;
  __syncthreads();
  if (block_err) {
    int32_t c = 0;
    for (int b = t; b < n_blocks; b += blockDim.x) c += block_err[b];
    if (c) atomicAdd(&n_err, c);
  }
  const int ept = (E + 1023) / 1024;
  const bool small = E <= 1024;
  const int G = counts_in || !small ? 1 : max(1, min(16, 1024 / E));
  const int ge = small ? t / E : 0, ee = small ? t - ge * E : 0;
  const bool gact = !counts_in && small && G > 1 && ge < G;
  const int b_lo = gact ? static_cast<int>(static_cast<int64_t>(n_blocks) * ge / G) : 0;
  const int b_hi = gact ? static_cast<int>(static_cast<int64_t>(n_blocks) * (ge + 1) / G) : 0;
  if (gact) {
    // Unrolled so that several block counts are in flight at once: the loop is
    // latency bound (one workgroup, 16+ loads per thread).
    int32_t c = 0;
#pragma unroll 8
    for (int b = b_lo; b < b_hi; ++b) c += block_counts[static_cast<int64_t>(b) * E + ee];
    part[t] = c;
  }
  __syncthreads();
  int64_t count[kEpt], start[kEpt], seg_lo[kEpt], seg_hi[kEpt];
  int64_t carry = 0;
#pragma unroll
  for (int c = 0; c < kEpt; ++c) {
    count[c] = start[c] = seg_lo[c] = seg_hi[c] = 0;
    if (c >= ept) continue;  // uniform across the workgroup
    const int e = t + 1024 * c;
    if (e < E) {
      if (counts_in) {
        count[c] = counts_in[e];
        if (count[c] < 0 || count[c] > n_rows) {
          atomicAdd(&n_err, 1);
          count[c] = count[c] < 0 ? 0 : n_rows;
        }
      } else if (G > 1) {
        for (int gg = 0; gg < G; ++gg) count[c] += part[gg * E + e];
      } else {
        for (int b = 0; b < n_blocks; ++b) count[c] += block_counts[static_cast<int64_t>(b) * E + e];
      }
    }
    int64_t chunk_total = 0;
    start[c] = carry + block_exclusive_scan(count[c], scan_tmp, &chunk_total);
    carry += chunk_total;
    seg_lo[c] = start[c];
    seg_hi[c] = start[c] + count[c];
    if (counts_in) {
      // Rows beyond num_rows are never touched, even if the counts disagree.
      if (seg_lo[c] > n_rows) seg_lo[c] = n_rows;
      if (seg_hi[c] > n_rows) seg_hi[c] = n_rows;
    }
  }
  if (counts_in && t == 0 && carry != n_rows) atomicAdd(&n_err, 1);
  if (small && t < E) start_s[t] = start[0];
  __syncthreads();
  if (gact) {
    int64_t run = start_s[ee];
    for (int gg = 0; gg < ge; ++gg) run += part[gg * E + ee];
#pragma unroll 8
    for (int b = b_lo; b < b_hi; ++b) {
      const int64_t i = static_cast<int64_t>(b) * E + ee;
      block_base[i] = static_cast<int32_t>(run);
      run += block_counts[i];
    }
  }
#pragma unroll
  for (int c = 0; c < kEpt; ++c) {
    const int e = t + 1024 * c;
    if (c >= ept || e >= E) continue;
    if (!counts_in && G == 1) {
      int64_t run = start[c];
      for (int b = 0; b < n_blocks; ++b) {
        const int64_t i = static_cast<int64_t>(b) * E + e;
        block_base[i] = static_cast<int32_t>(run);
        run += block_counts[i];
      }
    }
    seg[e] = seg_lo[c];
    seg[E + e] = seg_hi[c];
    if (counts_out) counts_out[e] = count[c];
    if (starts_out) starts_out[e] = start[c];
    if (offsets_out) offsets_out[e] = static_cast<int32_t>(start[c] + count[c]);
  }
  // Lists: 0 = tile_m-row tiles, 1 = 2*tile_m-row tiles over all rows;
  // 2 = 2*tile_m-row tiles over each expert's rows but a final remainder of
  // at most tile_m rows, 3 = one tile_m-row tile for that remainder.
  for (int list = 0; list < 4; ++list) {
    const int tm = list == 0 || list == 3 ? tile_m : 2 * tile_m;
    int2 *out = list == 0 ? tiles : list == 1 ? tiles2 : list == 2 ? tiles2m : tilesr;
    int64_t tcarry = 0;
#pragma unroll
    for (int c = 0; c < kEpt; ++c) {
      if (c >= ept) continue;  // uniform
      const int e = t + 1024 * c;
      const int64_t n = e < E ? seg_hi[c] - seg_lo[c] : 0;
      const int64_t full = n / (2 * tile_m), rem = n - full * 2 * tile_m;
      int64_t my_tiles, first = seg_lo[c];
      if (list <= 1)
        my_tiles = (n + tm - 1) / tm;
      else if (list == 2)
        my_tiles = full + (rem > tile_m ? 1 : 0);
      else {
        my_tiles = rem > 0 && rem <= tile_m ? 1 : 0;
        first = seg_lo[c] + full * 2 * tile_m;
      }
      int64_t chunk_tiles = 0;
      const int64_t tile0 = tcarry + block_exclusive_scan(my_tiles, scan_tmp, &chunk_tiles);
      tcarry += chunk_tiles;
      for (int64_t j = 0; j < my_tiles; ++j)
        out[tile0 + j] = make_int2(e, static_cast<int>(first + j * tm));
    }
    if (threadIdx.x == 0) {
      int32_t *num = list == 0 ? num_tiles : list == 1 ? num_tiles2 : list == 2 ? num_tiles2m
                                                                               : num_tilesr;
      *num = static_cast<int32_t>(tcarry);
    }
  }
  __syncthreads();
  if (t == 0) *err_counter = n_err;
}

template <int SCORE_DTYPE>
__global__ __launch_bounds__(256) void plan_scatter_kernel(
    const int64_t *top_idx, const void *top_scores, int64_t R, int k, int E, int EB,
    const int32_t *block_base, int64_t *sort_positions, int64_t *sorted_token_indices,
    void *sorted_scores, int64_t *inverse_order, int32_t *row_token, int32_t *row_slot) {
  extern __shared__ uint32_t lds[];
  const int words = EB >> 5;
  uint32_t *mask = lds;
  // Per-word popcount prefixes sit in LDS when they fit next to the masks;
  // otherwise (many experts, EB <= 256: at most 7 words below a slot) each
  // slot adds up the popcounts of the words below its own.
  const bool lds_prefix = plan_prefix_in_lds(E, EB);
  uint32_t *prefix = lds + E * words;
  const int64_t slot0 = static_cast<int64_t>(blockIdx.x) * EB;
  const int n_slots = static_cast<int>(min<int64_t>(EB, R - slot0));
  build_masks(top_idx, slot0, n_slots, E, words, mask, nullptr);
  if (lds_prefix) {
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      uint32_t run = 0;
      for (int w = 0; w < words; ++w) {
        prefix[e * words + w] = run;
        run += __popc(mask[e * words + w]);
      }
    }
    __syncthreads();
  }
  const int32_t *base = block_base + static_cast<int64_t>(blockIdx.x) * E;
  for (int p = threadIdx.x; p < n_slots; p += blockDim.x) {
    const int64_t i = slot0 + p;
    const int64_t e = top_idx[i];
    if (e < 0 || e >= E) {
      if (inverse_order) inverse_order[i] = -1;
      continue;
    }
    const int w = p >> 5;
    const uint32_t below = mask[e * words + w] & ((1u << (p & 31)) - 1u);
    uint32_t pre = 0;
    if (lds_prefix) {
      pre = prefix[e * words + w];
    } else {
      for (int w2 = 0; w2 < w; ++w2) pre += __popc(mask[e * words + w2]);
    }
    const int64_t pos = base[e] + pre + __popc(below);
    const int64_t tok = i / k;
    if (sort_positions) sort_positions[pos] = i;
    if (sorted_token_indices) sorted_token_indices[pos] = tok;
    if (sorted_scores) {
      if (SCORE_DTYPE == MX_DTYPE_BF16)
        reinterpret_cast<uint16_t *>(sorted_scores)[pos] =
            reinterpret_cast<const uint16_t *>(top_scores)[i];
      else
        reinterpret_cast<float *>(sorted_scores)[pos] = reinterpret_cast<const float *>(top_scores)[i];
    }
    if (inverse_order) inverse_order[i] = pos;
    row_token[pos] = static_cast<int32_t>(tok);
    row_slot[pos] = static_cast<int32_t>(i);
  }
}

constexpr int kPlanMaxEpt = kPlanMaxExperts / 1024;

}  // namespace

int slots_per_plan_block(int num_experts, int64_t rows) {
  // Masks + prefixes of E * EB bits each must fit in 64 KiB of LDS, and large
  // route counts are cut into at least 256 blocks (one workgroup per CU).
  int eb = 4096;
  while (eb > 256 && (static_cast<int64_t>(num_experts) * eb > 262144 || ceil_div(rows, eb) < 256))
    eb >>= 1;
  if (static_cast<int64_t>(num_experts) * eb <= 262144) return eb;
  // More than 1024 experts: the masks alone fill the 64 KiB (prefixes are
  // recounted per slot), so the blocks shrink to 32..128 slots.
  while (eb > 32 && static_cast<int64_t>(num_experts) * eb > 524288) eb >>= 1;
  return eb;
}

PlanLayout plan_layout(int64_t num_rows, int num_experts) {
  PlanLayout L;
  L.rows = num_rows;
  L.experts = num_experts;
  L.slots_per_block = slots_per_plan_block(num_experts, num_rows);
  L.blocks = static_cast<int>(ceil_div(num_rows, L.slots_per_block));
  L.max_tiles = ceil_div(num_rows, kPlanTileM) + num_experts;
  L.max_tiles2 = ceil_div(num_rows, kPlanTileM2) + num_experts;
  size_t off = 256;  // header: error counter, tile count
  L.off_block_counts = off;
  off = align_up(off + sizeof(int32_t) * L.blocks * num_experts, 256);
  L.off_block_base = off;
  off = align_up(off + sizeof(int32_t) * L.blocks * num_experts, 256);
  L.off_seg = off;
  off = align_up(off + sizeof(int64_t) * 2 * num_experts, 256);
  L.off_tiles = off;
  off = align_up(off + sizeof(int2) * L.max_tiles, 256);
  L.off_tiles2 = off;
  off = align_up(off + sizeof(int2) * L.max_tiles2, 256);
  L.off_tiles2m = off;
  off = align_up(off + sizeof(int2) * L.max_tiles2, 256);
  L.off_tilesr = off;
  off = align_up(off + sizeof(int2) * num_experts, 256);
  L.off_row_token = off;
  off = align_up(off + sizeof(int32_t) * num_rows, 256);
  L.off_row_slot = off;
  off = align_up(off + sizeof(int32_t) * num_rows, 256);
  L.off_block_err = off;
  off = align_up(off + sizeof(int32_t) * L.blocks, 256);
  L.bytes = off;
  return L;
}

PlanView plan_view(void *ws, const PlanLayout &L) {
  char *b = static_cast<char *>(ws);
  PlanView v;
  v.err = reinterpret_cast<int32_t *>(b);
  v.num_tiles = reinterpret_cast<int32_t *>(b) + 1;
  v.num_tiles2 = reinterpret_cast<int32_t *>(b) + 2;
  v.num_tiles2m = reinterpret_cast<int32_t *>(b) + 3;
  v.num_tilesr = reinterpret_cast<int32_t *>(b) + 4;
  v.block_counts = reinterpret_cast<int32_t *>(b + L.off_block_counts);
  v.block_base = reinterpret_cast<int32_t *>(b + L.off_block_base);
  v.seg = reinterpret_cast<int64_t *>(b + L.off_seg);
  v.tiles = reinterpret_cast<int2 *>(b + L.off_tiles);
  v.tiles2 = reinterpret_cast<int2 *>(b + L.off_tiles2);
  v.tiles2m = reinterpret_cast<int2 *>(b + L.off_tiles2m);
  v.tilesr = reinterpret_cast<int2 *>(b + L.off_tilesr);
  v.row_token = reinterpret_cast<int32_t *>(b + L.off_row_token);
  v.row_slot = reinterpret_cast<int32_t *>(b + L.off_row_slot);
  v.block_err = reinterpret_cast<int32_t *>(b + L.off_block_err);
  return v;
}

int build_plan(const int64_t *top_idx, const void *top_scores, int score_dtype,
               int64_t num_tokens, int top_k, int num_experts, int64_t *counts, int64_t *starts,
               int32_t *offsets, int64_t *sort_positions, int64_t *sorted_token_indices,
               void *sorted_scores, int64_t *inverse_order, void *workspace, hipStream_t s) {
  const int64_t R = num_tokens * top_k;
  const PlanLayout L = plan_layout(R, num_experts);
  const PlanView v = plan_view(workspace, L);
  if (L.blocks > 0) {
    const size_t lds = sizeof(uint32_t) * num_experts * (L.slots_per_block / 32);
    hipLaunchKernelGGL(plan_count_kernel, dim3(L.blocks), dim3(256), lds, s, top_idx, R,
                       num_experts, L.slots_per_block, v.block_counts, v.block_err);
  }
  hipLaunchKernelGGL(num_experts <= 1024 ? plan_scan_kernel<1> : plan_scan_kernel<kPlanMaxEpt>,
                     dim3(1), dim3(1024), 0, s, v.block_counts,
                     L.blocks > 0 ? v.block_err : static_cast<int32_t *>(nullptr), L.blocks,
                     num_experts, R,
                     kPlanTileM, static_cast<const int64_t *>(nullptr), v.block_base, v.seg,
                     v.tiles, v.num_tiles, v.tiles2, v.num_tiles2, v.tiles2m, v.num_tiles2m,
                     v.tilesr, v.num_tilesr, v.err, counts, starts, offsets);
  if (L.blocks > 0) {
    const size_t lds = (plan_prefix_in_lds(num_experts, L.slots_per_block) ? 2 : 1) *
                       sizeof(uint32_t) * num_experts * (L.slots_per_block / 32);
    if (score_dtype == MX_DTYPE_BF16)
      hipLaunchKernelGGL(plan_scatter_kernel<MX_DTYPE_BF16>, dim3(L.blocks), dim3(256), lds, s,
                         top_idx, top_scores, R, top_k, num_experts, L.slots_per_block,
                         v.block_base, sort_positions, sorted_token_indices,
                         top_scores ? sorted_scores : nullptr, inverse_order, v.row_token,
                         v.row_slot);
    else
      hipLaunchKernelGGL(plan_scatter_kernel<MX_DTYPE_F32>, dim3(L.blocks), dim3(256), lds, s,
                         top_idx, top_scores, R, top_k, num_experts, L.slots_per_block,
                         v.block_base, sort_positions, sorted_token_indices,
                         top_scores ? sorted_scores : nullptr, inverse_order, v.row_token,
                         v.row_slot);
  }
  return check_launch("mx_build_plan");
}

int plan_from_counts(const int64_t *counts, int64_t num_rows, int num_experts, void *workspace,
                     hipStream_t s) {
  const PlanLayout L = plan_layout(num_rows, num_experts);
  const PlanView v = plan_view(workspace, L);
  hipLaunchKernelGGL(num_experts <= 1024 ? plan_scan_kernel<1> : plan_scan_kernel<kPlanMaxEpt>,
                     dim3(1), dim3(1024), 0, s,
                     static_cast<const int32_t *>(nullptr), static_cast<const int32_t *>(nullptr),
                     0, num_experts, num_rows,
                     kPlanTileM, counts, static_cast<int32_t *>(nullptr), v.seg, v.tiles,
                     v.num_tiles, v.tiles2, v.num_tiles2, v.tiles2m, v.num_tiles2m, v.tilesr,
                     v.num_tilesr, v.err, static_cast<int64_t *>(nullptr),
                     static_cast<int64_t *>(nullptr), static_cast<int32_t *>(nullptr));
  return check_launch("mx_plan_from_counts");
}

int validate_plan_args(const char *name, int64_t num_tokens, int top_k, int num_experts) {
  if (num_tokens < 0 || top_k <= 0 || top_k > 16) {
    set_error("%s: need num_tokens >= 0 and top_k in [1, 16]", name);
    return MX_ERR_INVALID;
  }
  if (num_experts <= 0 || num_experts > kPlanMaxExperts) {
    set_error("%s: num_experts must be in [1, %d], got %d", name, kPlanMaxExperts, num_experts);
    return MX_ERR_INVALID;
  }
  if (num_tokens * top_k >= (int64_t(1) << 31)) {
    set_error("%s: num_tokens * top_k must stay below 2^31", name);
    return MX_ERR_INVALID;
  }
  return MX_OK;
}

}  // namespace mx

using namespace mx;

extern "C" size_t mx_plan_workspace_size(int64_t num_tokens, int top_k, int num_experts) {
  if (num_tokens < 0 || top_k <= 0 || num_experts <= 0) return 0;
  return plan_layout(num_tokens * top_k, num_experts).bytes;
}

extern "C" int mx_build_plan(const int64_t *top_idx, const void *top_scores, int score_dtype,
                             int64_t num_tokens, int top_k, int num_experts, int64_t *counts,
                             int64_t *starts, int32_t *offsets, int64_t *sort_positions,
                             int64_t *sorted_token_indices, void *sorted_scores,
                             int64_t *inverse_order, void *workspace, void *stream) {
  clear_error();
  int rc = validate_plan_args("mx_build_plan", num_tokens, top_k, num_experts);
  if (rc) return rc;
  if (!workspace || (num_tokens > 0 && !top_idx)) {
    set_error("mx_build_plan: top_idx and workspace must be non-null");
    return MX_ERR_INVALID;
  }
  if (sorted_scores && !top_scores) {
    set_error("mx_build_plan: sorted_scores requires top_scores");
    return MX_ERR_INVALID;
  }
  return build_plan(top_idx, top_scores, score_dtype, num_tokens, top_k, num_experts, counts,
                    starts, offsets, sort_positions, sorted_token_indices, sorted_scores,
                    inverse_order, workspace, as_stream(stream));
}

extern "C" int mx_plan_from_counts(const int64_t *counts, int64_t num_rows, int num_experts,
                                   void *workspace, void *stream) {
  clear_error();
  int rc = validate_plan_args("mx_plan_from_counts", num_rows, 1, num_experts);
  if (rc) return rc;
  if (!counts || !workspace) {
    set_error("mx_plan_from_counts: counts and workspace must be non-null");
    return MX_ERR_INVALID;
  }
  return plan_from_counts(counts, num_rows, num_experts, workspace, as_stream(stream));
}

extern "C" const int32_t *mx_plan_error_counter(const void *workspace) {
  return static_cast<const int32_t *>(workspace);
}
