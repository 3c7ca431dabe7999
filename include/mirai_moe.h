/*
 * mirai_moe.h -- C-ABI of the MI355X (gfx950) sparse-MoE expert-layer library
 * (libmirai_moe.so).
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t passed
 * as void*, and returns an int status (MX_OK on success). On failure a message
 * is available from mx_last_error() (thread-local). No entry point allocates
 * device memory: scratch space is passed in by the caller, sized by the
 * matching *_workspace_size() query. All work is enqueued on `stream`; nothing
 * synchronises with the host.
 *
 * Data formats (row-major, contiguous unless a leading dimension is given):
 *   tokens          [T, d]          bf16
 *   logits          [T, E]          fp32
 *   top_idx         [T, k]          int64   expert id per route slot
 *   top_scores      [T, k]          fp32 or bf16 (score_dtype)
 *   NF4 weight      codes [E, out, in/2] uint8 (per group of 8 elements along
 *                   in, byte i holds element i in the low nibble and element
 *                   i+4 in the high nibble), absmax [E, out, in/64] bf16
 *   NF4_F32 weight  codes as NF4, absmax [E, out, in/64] fp32 (the double-quant
 *                   absmax of a bitsandbytes payload, decoded by mx_nf4_from_bnb)
 *   NF4_DQ weight   codes as NF4; `scale` points to a host-side mx_nf4_dq
 *                   holding the bitsandbytes two-level absmax as stored
 *                   (uint8 codes, fp32 nested scales, fp32 offsets, 256-entry
 *                   code table), decoded inside the GEMMs
 *   NF4_DQ_KN       NF4_DQ for a weight stored [E, in, out] (as NF4_F32_KN)
 *   NF4_F32_KN      the same codes and fp32 absmax for a weight stored
 *                   [E, in, out] (y = x @ W[e], the MAGI-2 group layout of
 *                   magi2_preview.py:2680-2704): codes [E, in, out/2] packed
 *                   along out, absmax [E, in, out/64]. out_features /
 *                   in_features keep their meaning (N and K of the forward)
 *   INT8 weight     q [E, out, in] int8, scale [E, out] bf16
 *   BF16 weight     w [E, out, in] bf16
 *   F32X3 weight    w [E, out, 3*in] bf16: an fp32 weight split into bf16
 *                   planes [hi | lo | hi] along in (see mx_split_f32)
 *   LoRA factors    A [E, r, in], B [E, out, r] bf16 (r a multiple of 8,
 *                   at most 256); with F32X3 weights A [E, r, 3*in] and
 *                   B [E, out, 3*r] in [hi | lo | hi] planes, r = 8
 *   lora_rank       argument of the *_workspace_size queries: the largest
 *                   rank of the adapters the calls will carry (0 without
 *                   LoRA). The low-rank rows hold 3 planes of
 *                   rc = max(32, lora_rank rounded up to 32) columns.
 *
 * Each declaration cites the reference interface (seruva19/mirai, path:line)
 * whose semantics it implements.
 */
#ifndef MIRAI_MOE_H
#define MIRAI_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MX_OK 0
#define MX_ERR_INVALID 1 /* bad argument (shape, dtype, null pointer) */
#define MX_ERR_HIP 2     /* a HIP runtime call failed */

#define MX_DTYPE_F32 0
#define MX_DTYPE_BF16 1

#define MX_FMT_BF16 0
#define MX_FMT_NF4 1
#define MX_FMT_INT8 2
#define MX_FMT_F32X3 3
#define MX_FMT_NF4_F32 4  /* NF4 codes with an fp32 absmax per block (ingested bitsandbytes) */
#define MX_FMT_NF4_F32_KN 5  /* NF4_F32 stored [E, in, out], blocks along out (MAGI-2 groups) */
#define MX_FMT_NF4_DQ 6      /* NF4 codes with the two-level absmax of a bitsandbytes payload */
#define MX_FMT_NF4_DQ_KN 7   /* NF4_DQ stored [E, in, out], blocks along out */

/*
 * Two-level (double-quantised) absmax of an MX_FMT_NF4_DQ / _DQ_KN weight, as a
 * bitsandbytes payload stores it (quantize_4bit with compress_statistics=True,
 * blocksize 64, nested blocksize 256; quant.py:294-302, 407-431 and
 * quantized_experts.py:325-346 of the reference): block b of expert e, the
 * blocks numbered along the stored rows in order, has the absmax
 * fp32(fp32(code[absmax_q[e][b]] * nested_absmax[e][b / 256]) + offsets[e]),
 * two roundings, as mx_nf4_from_bnb decodes it. The pointers are device
 * pointers; the struct itself is read on the host during the call.
 */
typedef struct mx_nf4_dq {
  const uint8_t *absmax_q;     /* [E, blocks per expert] */
  const float *nested_absmax;  /* [E, nested_per_expert] */
  const float *offsets;        /* [E] */
  const float *code;           /* [256] */
  int64_t nested_per_expert;   /* ceil(blocks per expert / 256) */
} mx_nf4_dq;

/* Expert id of a route slot that is left out of the layer on purpose: the
 * plan skips it without counting it as an invalid route (any other id outside
 * [0, E) is counted, see mx_plan_error_counter), and the combine skips it like
 * any id outside [0, E). Used for the zero-score slots of coalesced logical
 * expert aliases, which the reference leaves out of the dispatch
 * (experts.py:2361-2367). */
#define MX_ROUTE_DROPPED (-9223372036854775807LL - 1)

/* Plane orders of mx_split_f32. */
#define MX_SPLIT_ACT 0     /* [hi | hi | lo]: activations */
#define MX_SPLIT_WEIGHT 1  /* [hi | lo | hi]: weights and LoRA factors */

/* Router normalisation modes. */
#define MX_RENORM_NONE 0      /* scores = softmax probabilities of the picks   */
#define MX_RENORM_CLAMP 1     /* p / clamp_min(sum p, 1e-20)                   */
#define MX_RENORM_EPS 2       /* p / (sum p + 1e-20)                           */

/* Expert activations (h from the gate projection g and the up projection u). */
#define MX_ACT_SILU 0     /* h = bf16(silu(g)) * u  (SwiGLU, experts.py:289-317) */
#define MX_ACT_SWIGLU7 1  /* h = min(g,7) * sigmoid(1.702 min(g,7)) * (clamp(u,-7,7) + 1)
                             in fp32 (MAGI-2, grouped_moe.py:287-306) */
/* Flag or-ed into `act` of the token-choice layer forward: the combine forms
 * each term bf16(y * bf16(score)) and rounds the running sum to bf16 after
 * every add, in ascending expert order -- the bf16 index_add of the
 * reference's MAGI-2 backend (grouped_moe.py:750-754) -- instead of the fp32
 * sum of run_direct_routed. Entry points that do not combine ignore it. */
#define MX_ACT_FLAG_BF16_COMBINE 0x100

/* Router score functions and output layouts of mx_route_topk_heads. */
#define MX_SCORE_SOFTMAX 0
#define MX_SCORE_SIGMOID 1
#define MX_ROUTE_LAYOUT_HEADS 0  /* [H, S, k], expert ids per head in [0, E)      */
#define MX_ROUTE_LAYOUT_ROWS 1   /* [S*H, k], row s*H+h, group ids h*E+e          */

/* Last error message of the calling thread ("" when none). */
const char *mx_last_error(void);
/* ABI version; bumped on any signature change. */
int mx_abi_version(void);

/* ------------------------------------------------------------------------ */
/* Routing                                                                   */
/* ------------------------------------------------------------------------ */

/*
 * Top-k token-choice routing over fp32 router logits.
 * Replaces the softmax -> topk -> gather -> renormalise -> *route_scale
 * sequence of TokenChoiceRouter.forward
 * (mirai/core/moe/routing/routers.py:234-249, renorm MX_RENORM_CLAMP) and of
 * LingBotVideoRouter.forward with score_func="softmax" and a zero correction
 * bias (mirai/vendors/lingbot_video/transformer_lingbot_video.py:1002-1033,
 * renorm MX_RENORM_EPS when norm_topk_prob, else MX_RENORM_NONE).
 * Selection is by logit (softmax is monotone); ties go to the lower expert id;
 * slots are written in descending-score order. E <= 1024, 1 <= k <= 16.
 * `logits` needs only fp32 alignment; a 16-byte aligned base with E % 4 == 0
 * takes 16-byte row loads.
 */
int mx_route_topk(const float *logits, int64_t num_tokens, int num_experts, int top_k,
                  int renorm, float route_scale, int64_t *top_idx, void *top_scores,
                  int score_dtype, void *stream);

/*
 * Backward of mx_route_topk: d(logits) from d(top_scores) for the selected
 * experts (softmax Jacobian through the renormalisation), i.e. the router-gate
 * gradient of LingBotVideoRouter.forward
 * (transformer_lingbot_video.py:1002-1033) under autograd.
 */
int mx_route_topk_backward(const float *logits, int64_t num_tokens, int num_experts,
                           int top_k, int renorm, float route_scale,
                           const int64_t *top_idx, const float *grad_scores,
                           float *grad_logits, void *stream);

/*
 * Router-gate gradient of any of the routers above: d(logits) [rows, E] fp32
 * from d(top_scores) [rows, k] fp32 for the picks top_idx [rows, k], where the
 * scores were softmax or sigmoid (score_func) of the fp32 logits, the picks'
 * scores were renormalised by `renorm` with the floor `renorm_floor`
 * (MX_RENORM_CLAMP: p / max(sum p, floor); MX_RENORM_EPS: p / (sum p + floor))
 * and multiplied by route_scale. The bias that steered the selection carries
 * no gradient. This is the autograd of the score path of
 * LingBotVideoRouter.forward (transformer_lingbot_video.py:1002-1033: softmax /
 * sigmoid, gather, / (sum + 1e-20), * route_scale) and of CoreMultiHeadMoE._route
 * (mirai/vendors/magi2_preview/model/magi2_preview.py:2727-2743 with
 * flash_mh_moe/route.py:28-148: F.normalize(p=1, eps) is MX_RENORM_CLAMP) with
 * one logits row per (head, token). Slots whose expert id lies outside [0, E)
 * get no gradient. The gradient of the router GEMM itself (d tokens =
 * d logits . W, d W = d logits^T . tokens) is a plain fp32 GEMM left to the
 * caller. E <= 1024, 1 <= k <= 16.
 */
int mx_route_scores_backward(const float *logits, int64_t num_rows, int num_experts, int top_k,
                             int score_func, int renorm, float renorm_floor, float route_scale,
                             const int64_t *top_idx, const float *grad_scores,
                             float *grad_logits, void *stream);

/*
 * Multi-head top-k routing (MAGI-2). Replaces compute_topk_probs_and_indices
 * (mirai/vendors/magi2_preview/flash_mh_moe/route.py:28-148,157-196) followed
 * by `* route_scale` in CoreMultiHeadMoE._route
 * (mirai/vendors/magi2_preview/model/magi2_preview.py:2727-2743) and the
 * head-flattening of Magi2GroupedMoEBackend._execute_routed_chunk
 * (mirai/core/models/magi2_preview/grouped_moe.py:658-663).
 * logits [H, S, E] fp32; scores = softmax or sigmoid (score_func); experts are
 * picked by score + expert_bias[h, e] (expert_bias [H, E] fp32, may be NULL;
 * it steers selection only); ties go to the lower expert id. With
 * num_virtual_group > 1 (dividing E, at most 64) the experts form that many
 * groups of consecutive ids, each scored by the sum of its two largest biased
 * scores; only the topk_virtual_group best groups (ties to the lower group id)
 * keep their experts' keys, every other key is set to 0.0 before the expert
 * selection (route.py:62-105); num_virtual_group = 1 disables it and ignores
 * topk_virtual_group. Probabilities are
 * the picks' unbiased scores, renormalised by renorm (MX_RENORM_CLAMP:
 * p / max(sum p, renorm_floor), the L1 F.normalize with eps = renorm_floor;
 * MX_RENORM_EPS: p / (sum p + renorm_floor)), times route_scale.
 * layout MX_ROUTE_LAYOUT_HEADS writes [H, S, k] per-head expert ids (the
 * reference's output); MX_ROUTE_LAYOUT_ROWS writes [S*H, k] with row s*H+h and
 * flattened group ids h*E+e, the input of mx_build_plan / mx_moe_forward_act.
 * E <= 1024, 1 <= k <= 16.
 */
int mx_route_topk_heads(const float *logits, int num_heads, int64_t num_tokens, int num_experts,
                        int top_k, int score_func, const float *expert_bias, int renorm,
                        float renorm_floor, float route_scale, int num_virtual_group,
                        int topk_virtual_group, int layout, int64_t *top_idx, void *top_scores,
                        int score_dtype, void *stream);

/* ------------------------------------------------------------------------ */
/* Fused router front end (router GEMM + scores + selection)                 */
/* ------------------------------------------------------------------------ */

/* Experts padded to the router kernel's column tile (32, 64, 128 or 256);
 * -1 when num_experts is outside [1, 256]. */
int mx_router_padded_experts(int num_experts);
/* Bytes of the router weight planes [3][EP][hidden] bf16 (0 on bad sizes). */
size_t mx_router_planes_size(int num_experts, int64_t hidden);
/* Split the fp32 router weight W [E, hidden] (LingBotVideoRouter.weight,
 * transformer_lingbot_video.py:520) into bf16 planes hi, mid, lo with
 * W == hi + mid + lo exactly, rows E..EP-1 zero. Done once per weight value;
 * mx_router_forward reads the planes. hidden % 64 == 0. */
int mx_router_weight_planes(const float *weight, int num_experts, int64_t hidden, void *planes,
                            void *stream);
/* Replaces LingBotVideoRouter.forward (transformer_lingbot_video.py:962-1033,
 * group-limited choice :865-890) without its optional extensions:
 *   logits = tokens.float() @ W.T (+ logit_delta)      fp32 products, fp32 sums
 *   scores = softmax(logits) or sigmoid(logits)         (score_func)
 *   picks  = top_k of scores + expert_bias, optionally within the topk_group
 *            best of n_group expert groups (group score = sum of its two
 *            largest biased scores); ties go to the lower expert / group id
 *   top_scores = scores[picks] / (sum + 1e-20) if top_k > 1 && norm_topk_prob,
 *                times route_scale, stored as score_dtype
 * Picks are written in descending order of the selection key. tokens [T, hidden]
 * bf16 or fp32 (token_dtype); planes from mx_router_weight_planes; expert_bias
 * [E] fp32 and logit_delta [T, E] fp32 may be NULL; n_group <= 1 disables group
 * limiting. Optional outputs logits_out / scores_out [T, E] fp32 (may be NULL).
 * E <= 256, 1 <= top_k <= 16, hidden % 64 == 0. */
int mx_router_forward(const void *tokens, int token_dtype, int64_t num_tokens, int64_t hidden,
                      int num_experts, const void *planes, const float *expert_bias,
                      const float *logit_delta, int top_k, int score_func, int n_group,
                      int topk_group, int norm_topk_prob, float route_scale, float *logits_out,
                      float *scores_out, int64_t *top_idx, void *top_scores, int score_dtype,
                      void *stream);

/* ------------------------------------------------------------------------ */
/* Dispatch plan (stable counting sort of routes by expert)                  */
/* ------------------------------------------------------------------------ */

/* Bytes of scratch needed by mx_build_plan / mx_plan_from_counts. */
size_t mx_plan_workspace_size(int64_t num_tokens, int top_k, int num_experts);

/*
 * Device-resident dispatch plan; replaces build_dispatch_plan(backend="device")
 * (mirai/core/models/compressed_weights/execution/dispatch_preprocess.py:128-179)
 * and the argsort/bincount/cumsum block of
 * CompressedGroupedExperts._run_direct_routed_batched_vectorized
 * (mirai/core/models/compressed_weights/execution/experts.py:2369-2381).
 * Outputs (all device, any may be NULL except where noted):
 *   counts[E] int64, starts[E] int64 (exclusive), offsets[E] int32 (inclusive),
 *   sort_positions[R], sorted_token_indices[R], inverse_order[R] int64,
 *   sorted_scores[R] (score_dtype, needs top_scores).
 * R = num_tokens * top_k, E <= 8192 (MAGI-2's flattened head x expert groups
 * exceed the 1023-group cap of torch grouped_mm, which the reference works
 * around by segmenting, grouped_moe.py:1365-1370; the plan has no such cap).
 * Route slots whose expert id is outside [0, E) are dropped
 * (inverse_order = -1) and counted in the workspace error flag.
 * The plan stays in `workspace` for the grouped GEMMs of mx_moe_forward.
 */
int mx_build_plan(const int64_t *top_idx, const void *top_scores, int score_dtype,
                  int64_t num_tokens, int top_k, int num_experts, int64_t *counts,
                  int64_t *starts, int32_t *offsets, int64_t *sort_positions,
                  int64_t *sorted_token_indices, void *sorted_scores,
                  int64_t *inverse_order, void *workspace, void *stream);

/*
 * Plan for rows that are already expert-sorted (counts given on device);
 * the layout consumed by CompressedGroupedExperts.run_for_loop
 * (experts.py:1656-1747): segment e holds rows [starts[e], starts[e]+counts[e]).
 */
int mx_plan_from_counts(const int64_t *counts, int64_t num_rows, int num_experts,
                        void *workspace, void *stream);

/* Number of invalid expert ids seen by the last plan built in `workspace`
 * (device int32 pointer inside the workspace, for an optional host check). */
const int32_t *mx_plan_error_counter(const void *workspace);

/* ------------------------------------------------------------------------ */
/* Permute / combine                                                          */
/* ------------------------------------------------------------------------ */

/*
 * out[i] = tokens[index[i]] for i < rows (rows whose index is outside
 * [0, src_rows) are zero); width `cols` elements of `dtype`.
 * Replaces _PermuteRoutedTokens.forward
 * (mirai/core/models/compressed_weights/execution/dispatch_ops.py:8-13).
 */
int mx_gather_rows(const void *tokens, int64_t src_rows, const int64_t *index, int64_t rows,
                   int64_t cols, int dtype, void *out, void *stream);

/*
 * out[index[i]] += row_scale[i] * rows_in[i] in fp32 (row_scale may be NULL
 * for 1; `out` is zeroed first; indices outside [0, out_rows) are skipped).
 * Replaces _PermuteRoutedTokens.backward (dispatch_ops.py:15-20) and the
 * index_add_ of _CombineRoutedTokens.forward (dispatch_ops.py:23-33) for
 * arbitrary (duplicate-carrying) index lists.
 */
int mx_scatter_add_rows(const void *rows_in, const float *row_scale, const int64_t *index,
                        int64_t rows, int64_t cols, int dtype, int64_t out_rows, float *out,
                        void *stream);

/*
 * out[t] = sum over the k slots of token t, in ascending expert order, of
 * score[t,j] * y[t*k+j] accumulated in fp32, then cast to out_dtype.
 * Replaces the fp32 output.index_add_ of run_direct_routed
 * (experts.py:1786-1790, 2430-2438) and _CombineRoutedTokens.forward
 * (dispatch_ops.py:23-33); deterministic. top_scores may be NULL for unit
 * weights (the per-token sum of the slot rows, as the permute backward).
 */
int mx_combine(const void *y, const int64_t *top_idx, const void *top_scores,
               int score_dtype, int64_t num_tokens, int top_k, int num_experts,
               int64_t cols, void *out, int out_dtype, void *stream);

/*
 * Backward of mx_combine: grad_y[t*k+j] = bf16(grad_out[t] * score[t,j]) and
 * grad_scores[t,j] = sum_n grad_out[t,n] * y[t*k+j,n] (fp32).
 * Replaces _CombineRoutedTokens.backward (dispatch_ops.py:34-44).
 */
int mx_combine_backward(const void *grad_out, int grad_dtype, const void *y,
                        const int64_t *top_idx, const void *top_scores, int score_dtype,
                        int64_t num_tokens, int top_k, int num_experts, int64_t cols,
                        void *grad_y, float *grad_scores, void *stream);

/* ------------------------------------------------------------------------ */
/* Frozen-weight codecs                                                       */
/* ------------------------------------------------------------------------ */

/*
 * NF4, blocksize 64, bf16 absmax, no double quantisation. For each block of 64
 * consecutive `in` elements: absmax = max|w| (w taken as bf16), code =
 * argmin_j |w/absmax - NF4[j]| (fp32, first index on ties). Codebook:
 * mirai/core/models/quantization.py:100-117; packing order of NF4Linear
 * (quantization.py:171-175). Replaces the quantize_4bit call of
 * _nf4_quantize_2d (mirai/core/models/compressed_weights/quantization/quant.py:315-358)
 * in the BASELINE storage format. `rows` = E*out, `cols` = in (multiple of 64).
 */
int mx_nf4_quantize(const void *w, int w_dtype, int64_t rows, int64_t cols, uint8_t *codes,
                    void *absmax, void *stream);

/*
 * w = bf16(fp32(NF4[code]) * fp32(absmax)); replaces nf4_dequantize_stack /
 * _nf4_dequantize (quant.py:380-472) in the BASELINE storage format.
 */
int mx_nf4_dequantize(const uint8_t *codes, const void *absmax, int64_t rows, int64_t cols,
                      void *out, int out_dtype, void *stream);

/* mx_nf4_dequantize with the absmax in bf16 or fp32 (absmax_dtype MX_DTYPE_*;
 * fp32 is MX_FMT_NF4_F32): w = bf16(fp32(NF4[code]) * absmax). */
int mx_nf4_dequantize_ex(const uint8_t *codes, const void *absmax, int absmax_dtype,
                         int64_t rows, int64_t cols, void *out, int out_dtype, void *stream);

/*
 * Ingests a bitsandbytes double-quantised NF4 payload (quantize_4bit with
 * compress_statistics=True, blocksize 64, nested blocksize 256, bitsandbytes
 * 0.49.2) as the reference stores it per expert
 * (CompressedGroupedExperts._store_nf4_grouped, experts.py:998-1031; buffers
 * {key}_nf4, _nf4_absmax, _nf4_nabsmax, _nf4_offset, _nf4_ncode):
 *   packed [E, rows*cols/2] uint8 (byte j: element 2j high nibble, 2j+1 low),
 *   absmax_q [E, rows*cols/64] uint8, nested_absmax [E, ceil(rows*cols/16384)]
 *   fp32, offsets [E] fp32, nested_code [256] fp32.
 * Writes MX_FMT_NF4_F32 weights: codes [E, rows, cols/2] in this library's
 * nibble order and absmax [E, rows, cols/64] fp32 =
 * nested_code[absmax_q] * nested_absmax + offset (fp32, two roundings), the
 * absmax bitsandbytes dequantises with (quant.py:413-431), so the GEMMs decode
 * the payload's weights without re-quantisation. The 16-entry NF4 code table
 * of the payload ({key}_nf4_code) must equal the NF4 levels (checked by the
 * caller). cols a multiple of 64. With absmax NULL only the codes are written
 * (MX_FMT_NF4_DQ keeps the payload's two-level absmax as it is).
 */
int mx_nf4_from_bnb(const uint8_t *packed, const uint8_t *absmax_q, const float *nested_absmax,
                    const float *offsets, const float *nested_code, int64_t experts, int64_t rows,
                    int64_t cols, uint8_t *codes, float *absmax, void *stream);

/*
 * The fp32 block absmax of a two-level (MX_FMT_NF4_DQ) payload, as the GEMMs
 * decode it per K step: absmax[e][b] = fp32(fp32(code[absmax_q[e][b]] *
 * nested_absmax[e][b / 256]) + offsets[e]) for b < blocks_per_expert (the
 * dequantize_blockwise + offset step of quant.py:413-424). With it,
 * mx_nf4_dequantize_ex dequantises NF4_DQ weights.
 */
int mx_nf4_dq_absmax(const mx_nf4_dq *dq, int64_t experts, int64_t blocks_per_expert,
                     float *absmax, void *stream);

/*
 * Symmetric per-output-row INT8: scale = bf16(max(absmax_row/127, 1e-30)),
 * q = clamp(round_half_even(w/scale), -127, 127). Replaces _quantize_weight
 * with group_size=0 (quant.py:189-235; scale rule quant.py:227-231).
 */
int mx_int8_quantize(const void *w, int w_dtype, int64_t rows, int64_t cols, int8_t *q,
                     void *scale, void *stream);

/* w = bf16(fp32(q) * fp32(scale)); replaces _dequantize_weight with
 * group_size=0 (quant.py:238-260). */
int mx_int8_dequantize(const int8_t *q, const void *scale, int64_t rows, int64_t cols,
                       void *out, int out_dtype, void *stream);

/* ------------------------------------------------------------------------ */
/* Grouped expert GEMMs and the fused layer                                   */
/* ------------------------------------------------------------------------ */

/* Frozen projection weight in one of the MX_FMT_* formats, [E, out, in]. */

typedef struct mx_weight {
  int format;           /* MX_FMT_* */
  const void *data;     /* bf16 w | uint8 codes | int8 q */
  const void *scale;    /* NULL | absmax [E,out,in/64] (bf16, fp32) | bf16 scale [E,out]
                           | const mx_nf4_dq * (NF4_DQ formats, host memory) */
  int64_t out_features;
  int64_t in_features;
} mx_weight;

/* Per-expert LoRA factors of one projection (all NULL / rank 0 when absent). */
typedef struct mx_lora {
  const void *a;        /* bf16 [E, r, in]  */
  const void *b;        /* bf16 [E, out, r] */
  int rank;             /* 0 (no adapter), or a multiple of 8 up to 256 */
  float scale;          /* alpha / r (or alpha / sqrt(r)) times extra scales */
} mx_lora;

/*
 * Profiling hook; no counterpart in the reference (which times whole calls
 * with CUDA events, scripts/agent/probe_moe_runtime.py:113-146). While set,
 * each mx_moe_forward call on this thread records events[0..6] (hipEvent_t)
 * on its stream at the stage boundaries: start, plan, LoRA down-projection of
 * gate/up, gate/up GEMM, LoRA down-projection of down, down GEMM, combine.
 * Pass NULL / 0 to clear. count must be 0 or 7.
 */
int mx_set_stage_events(void **events, int count);

/* Bytes of scratch for mx_moe_forward / mx_moe_for_loop / mx_grouped_linear
 * (BF16, NF4, INT8 weights) with adapters of rank <= lora_rank. */
size_t mx_moe_workspace_size(int64_t num_tokens, int top_k, int num_experts,
                             int64_t hidden, int64_t ffn, int lora_rank);

/* Bytes of scratch for mx_moe_forward with MX_FMT_F32X3 weights (fp32 tokens). */
size_t mx_moe_f32x3_workspace_size(int64_t num_tokens, int top_k, int num_experts,
                                   int64_t hidden, int64_t ffn);

/* Size of the static device scratch of mx_moe_forward_static (64 MiB per GPU). */
#define MX_STATIC_SCRATCH_BYTES (64u << 20)

/*
 * mx_moe_forward_act without a workspace argument and without saved
 * activations (inference): the scratch is a static device array of
 * MX_STATIC_SCRATCH_BYTES that each GPU holds until the process ends, so the
 * call allocates nothing (no hipMalloc / hipFree, no allocating library call).
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops). Calls whose
 * mx_moe_workspace_size (mx_moe_f32x3_workspace_size for MX_FMT_F32X3
 * weights) exceeds MX_STATIC_SCRATCH_BYTES fail with MX_ERR_INVALID. Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU (on
 * different streams or threads) race. The first call on a device resolves
 * that device's array address (hipGetSymbolAddress); make it once outside
 * any stream capture (a warm-up call), after which the call can be captured
 * into a HIP graph and replayed.
 */
int mx_moe_forward_static(const void *tokens, const int64_t *top_idx, const void *top_scores,
                          int score_dtype, int64_t num_tokens, int top_k, int num_experts,
                          int64_t hidden, int64_t ffn, int act, const mx_weight *w1,
                          const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
                          const mx_lora *l3, const mx_lora *l2, void *out, int out_dtype,
                          void *stream);

/*
 * fp32 -> bf16 planes for the fp32 path on bf16 MFMA. Row i of x (cols fp32)
 * becomes 3*cols bf16 values with hi = bf16(x), lo = bf16(x - hi), in the
 * order [hi | hi | lo] (MX_SPLIT_ACT) or [hi | lo | hi] (MX_SPLIT_WEIGHT). The
 * dot product of an activation row and a weight row split this way is
 * hi*hi + hi*lo + lo*hi: the fp32 product up to the lo*lo term (relative
 * 2^-16). No reference counterpart: the reference computes its fp32 layer
 * (run_direct_routed with fp32 tokens, experts.py:1749-1912) on fp32 GEMMs;
 * this is how the MI355X path reaches the same precision on the matrix cores.
 */
int mx_split_f32(const float *x, int64_t rows, int64_t cols, int pattern, void *out,
                 void *stream);

/*
 * Full routed expert layer: plan -> gathered gate/up grouped GEMM with
 * in-register weight decode, fused LoRA and SwiGLU -> down grouped GEMM with
 * fused LoRA -> deterministic gate-weighted combine.
 * Replaces CompressedGroupedExperts.run_direct_routed (experts.py:1749-1912)
 * with the canonical gated SwiGLU spec (mirai/core/moe/runtime/specs.py:222-231):
 * gate = w1, up = w3, down = w2, h = silu(x w1^T + dA1) * (x w3^T + dA3),
 * y = h w2^T + dA2, out[t] = sum_j score[t,j] * y[t,j] (fp32) -> out_dtype.
 * hidden and ffn must be multiples of 64 (one NF4 block per K step of the
 * GEMMs); other sizes return MX_ERR_INVALID.
 * Optional saved activations for backward (any may be NULL):
 *   save_gate/save_up [R, ffn] bf16 pre-activation projections (sorted order),
 *   save_h [R, ffn] bf16, save_y [R, hidden] bf16 (flat slot order t*k+j),
 *   save_lora [R, 3, rc] bf16 scaled low-rank activations (rc as above,
 *   from the largest attached rank).
 * With MX_FMT_F32X3 weights (all three) the layer runs at fp32 precision:
 * tokens are fp32 [T, hidden], the workspace comes from
 * mx_moe_f32x3_workspace_size, no activations are saved (inference only),
 * and LoRA factors are split as the format list above describes.
 */
int mx_moe_forward(const void *tokens, const int64_t *top_idx, const void *top_scores,
                   int score_dtype, int64_t num_tokens, int top_k, int num_experts,
                   int64_t hidden, int64_t ffn, const mx_weight *w1, const mx_weight *w3,
                   const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                   const mx_lora *l2, void *out, int out_dtype, void *save_gate,
                   void *save_up, void *save_h, void *save_y, void *save_lora,
                   void *workspace, void *stream);

/*
 * mx_moe_forward with a choice of expert activation (MX_ACT_*). With
 * MX_ACT_SWIGLU7 it is the MAGI-2 routed expert MLP of
 * Magi2GroupedMoEBackend._execute_routed_chunk / Magi2QuantizedGroupedMoEBackend
 * ._routed_inference (mirai/core/models/magi2_preview/grouped_moe.py:639-756,
 * 1337-1418): rows are (token, head) pairs, experts the flattened (head,
 * expert) groups (num_experts = H*E, up to 8192), gate and up are bf16
 * projections and h = bf16(swiglu7(gate, up)) (grouped_moe.py:287-306).
 * MAGI-2's [G, in, out] weights are stored transposed, as [G, out, in].
 */
int mx_moe_forward_act(const void *tokens, const int64_t *top_idx, const void *top_scores,
                       int score_dtype, int64_t num_tokens, int top_k, int num_experts,
                       int64_t hidden, int64_t ffn, int act, const mx_weight *w1,
                       const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
                       const mx_lora *l3, const mx_lora *l2, void *out, int out_dtype,
                       void *save_gate, void *save_up, void *save_h, void *save_y,
                       void *save_lora, void *workspace, void *stream);

/*
 * mx_moe_forward_act with the block's shared-expert sum fused into the
 * combine: with addend [T, hidden] (out's dtype) the output is
 * out_dtype(out_dtype(routed sum) + addend), the `out + shared_output` of
 * LingBotVideoSparseMoeBlock (transformer_lingbot_video.py:2374-2377, shared
 * expert LingBotVideoMLP :491-499). addend_ready (a hipEvent_t, may be NULL)
 * is waited on by `stream` right before the combine, so a producer of the
 * addend on another stream overlaps the whole routed path. addend NULL gives
 * mx_moe_forward_act. Not with MX_FMT_F32X3 weights.
 */
int mx_moe_forward_ex(const void *tokens, const int64_t *top_idx, const void *top_scores,
                      int score_dtype, int64_t num_tokens, int top_k, int num_experts,
                      int64_t hidden, int64_t ffn, int act, const mx_weight *w1,
                      const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
                      const mx_lora *l3, const mx_lora *l2, void *out, int out_dtype,
                      const void *addend, void *addend_ready, void *save_gate, void *save_up,
                      void *save_h, void *save_y, void *save_lora, void *workspace,
                      void *stream);

/*
 * Expert-choice routes: expert_token_indices / expert_token_scores [B, L, C]
 * (each of L logical experts picks C tokens of each of B samples; token ids
 * in [0, tokens_per_sample)). The flat slots s = (b, l, c) map to physical
 * expert logical_to_physical[l] (NULL: l, with L == num_experts) and token
 * idx + b * tokens_per_sample.
 *
 * mx_build_expert_choice_plan replaces build_expert_choice_dispatch_plan
 * (mirai/core/models/compressed_weights/execution/dispatch_preprocess.py:182-278):
 * the plan fields of mx_build_plan over the slots sorted stably by physical
 * expert, with sorted_token_indices the slots' flat token ids.
 */
size_t mx_expert_choice_plan_workspace_size(int batch, int logical_experts, int capacity,
                                            int num_experts);
int mx_build_expert_choice_plan(const int64_t *expert_token_indices,
                                const void *expert_token_scores, int score_dtype, int batch,
                                int logical_experts, int capacity, int64_t tokens_per_sample,
                                const int32_t *logical_to_physical, int num_experts,
                                int64_t *counts, int64_t *starts, int32_t *offsets,
                                int64_t *sort_positions, int64_t *sorted_token_indices,
                                void *sorted_scores, int64_t *inverse_order, void *workspace,
                                void *stream);

/*
 * Expert-choice routed layer, replacing run_compressed_expert_choice
 * (execution/expert_choice.py:16-152, run_expert_choice_routed
 * experts.py:1954-1974): the expert MLP of every slot (same kernels as
 * mx_moe_forward_act) and out[t] = sum over t's slots of score * y in fp32,
 * in ascending order of (physical expert, logical expert) -- the order the
 * reference's index_add_ visits the sorted slots on the CPU -- cast to
 * out_dtype. combine_order [L] lists the logical experts in that order (NULL:
 * 0..L-1, right when logical_to_physical is NULL or monotone). Tokens no
 * expert picked get 0. Preconditions: a token appears at most once per
 * (sample, logical expert); token ids outside [0, tokens_per_sample) are
 * skipped. L <= 1024. mx_moe_forward_expert_choice_ex also keeps, when the
 * save pointers are non-NULL, the activations the backward needs (as
 * mx_moe_forward_ex does, with the S = B * L * C slots as the rows: gate / up /
 * h [S, ffn] in expert-sorted order, y [S, hidden] in slot order, low-rank
 * rows [S, 3, rc]).
 */
size_t mx_moe_expert_choice_workspace_size(int batch, int logical_experts, int capacity,
                                           int64_t tokens_per_sample, int num_experts,
                                           int64_t hidden, int64_t ffn, int lora_rank);
int mx_moe_forward_expert_choice(const void *tokens, const int64_t *expert_token_indices,
                                 const void *expert_token_scores, int score_dtype, int batch,
                                 int logical_experts, int capacity, int64_t tokens_per_sample,
                                 const int32_t *logical_to_physical,
                                 const int32_t *combine_order, int num_experts, int64_t hidden,
                                 int64_t ffn, int act, const mx_weight *w1, const mx_weight *w3,
                                 const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                                 const mx_lora *l2, void *out, int out_dtype, void *workspace,
                                 void *stream);
int mx_moe_forward_expert_choice_ex(
    const void *tokens, const int64_t *expert_token_indices, const void *expert_token_scores,
    int score_dtype, int batch, int logical_experts, int capacity, int64_t tokens_per_sample,
    const int32_t *logical_to_physical, const int32_t *combine_order, int num_experts,
    int64_t hidden, int64_t ffn, int act, const mx_weight *w1, const mx_weight *w3,
    const mx_weight *w2, const mx_lora *l1, const mx_lora *l3, const mx_lora *l2, void *out,
    int out_dtype, void *save_gate, void *save_up, void *save_h, void *save_y, void *save_lora,
    void *workspace, void *stream);

/*
 * Backward of the expert-choice layer: the autograd of
 * run_compressed_expert_choice (execution/expert_choice.py:16-152; its
 * gather of token rows, per-expert MLP and index_add_ of y.float() * score),
 * with frozen weights re-decoded as in mx_moe_backward. From grad_out [T,
 * hidden] and the activations saved by mx_moe_forward_expert_choice_ex:
 * grad_scores [B, L, C] fp32 (grad_out[token] . y of the slot, 0 for skipped
 * slots), grad_tokens [T, hidden] (the sum over a token's slots of their dx
 * rows, fp32 in the forward's combine order; 0 for tokens no expert picked)
 * and the fp32 LoRA factor gradients (layout as mx_moe_backward; NULL: not
 * wanted). Workspace: mx_moe_backward_expert_choice_workspace_size bytes.
 */
size_t mx_moe_backward_expert_choice_workspace_size(int batch, int logical_experts,
                                                    int capacity, int64_t tokens_per_sample,
                                                    int num_experts, int64_t hidden,
                                                    int64_t ffn, int lora_rank);
int mx_moe_backward_expert_choice(
    const void *grad_out, int grad_dtype, const void *tokens, const int64_t *expert_token_indices,
    const void *expert_token_scores, int score_dtype, int batch, int logical_experts,
    int capacity, int64_t tokens_per_sample, const int32_t *logical_to_physical,
    const int32_t *combine_order, int num_experts, int64_t hidden, int64_t ffn, int act,
    const mx_weight *w1, const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
    const mx_lora *l3, const mx_lora *l2, const void *save_gate, const void *save_up,
    const void *save_h, const void *save_y, const void *save_lora, void *grad_tokens,
    int grad_tokens_dtype, float *grad_scores, float *grad_a1, float *grad_b1, float *grad_a3,
    float *grad_b3, float *grad_a2, float *grad_b2, void *workspace, void *stream);

/*
 * Expert MLP over rows already sorted by expert (no gate weighting):
 * out[i] = (silu(x w1^T + dA1) * (x w3^T + dA3)) w2^T + dA2 for the expert that
 * owns row i. Replaces CompressedGroupedExperts.run_for_loop
 * (experts.py:1656-1747).
 */
int mx_moe_for_loop(const void *tokens_sorted, const int64_t *counts, int64_t num_rows,
                    int num_experts, int64_t hidden, int64_t ffn, const mx_weight *w1,
                    const mx_weight *w3, const mx_weight *w2, const mx_lora *l1,
                    const mx_lora *l3, const mx_lora *l2, void *out, void *workspace,
                    void *stream);

/*
 * mx_moe_for_loop with the expert activation `act` (MX_ACT_SILU or
 * MX_ACT_SWIGLU7, the MAGI-2 swiglu7 of grouped_moe.py:287-306): run_for_loop
 * of a module whose spec names either activation (experts.py:1656-1747).
 */
int mx_moe_for_loop_act(const void *tokens_sorted, const int64_t *counts, int64_t num_rows,
                        int num_experts, int64_t hidden, int64_t ffn, int act,
                        const mx_weight *w1, const mx_weight *w3, const mx_weight *w2,
                        const mx_lora *l1, const mx_lora *l3, const mx_lora *l2, void *out,
                        void *workspace, void *stream);

/*
 * One grouped projection over expert-sorted rows: out[i] = x[i] W_e^T (+LoRA)
 * for the expert e owning row i (segments from `counts`). Replaces
 * CompressedGroupedExperts.grouped_linear (experts.py:803-827) and the
 * jagged-offset grouped_mm contract (mirai/core/moe/runtime/gemm.py:433-482),
 * with no per-call group-count cap.
 */
int mx_grouped_linear(const void *x, const int64_t *counts, int64_t num_rows, int num_experts,
                      const mx_weight *w, const mx_lora *lora, void *out, void *workspace,
                      void *stream);

/* Bytes of scratch for mx_grouped_linear_backward. */
size_t mx_grouped_linear_backward_workspace_size(int64_t num_rows, int num_experts,
                                                 int64_t in_features, int64_t out_features,
                                                 int lora_rank);

/*
 * Backward of mx_grouped_linear over the same rows (x [S, in] bf16, the
 * forward's input) and grad_out [S, out] bf16: grad_x [S, in] bf16 (may be
 * NULL) = grad_out W_e + dz A_e with the frozen W_e re-decoded in-kernel and
 * dz = bf16(s bf16(grad_out B_e)); with LoRA also the fp32 factor gradients
 * grad_a [E, r, in] = sum dz^T x and grad_b [E, out, r] = sum grad_out^T p
 * per expert, p = bf16(s bf16(x A_e^T)) recomputed as the forward formed it
 * (zero when num_rows is 0). Replaces _FrozenGroupedMMLinear.backward
 * (mirai/core/models/compressed_weights/execution/torch_grouped.py:71-91:
 * dX = grouped_mm(dY, W) over the re-dequantised weight) plus the autograd of
 * ActiveExpertLoRA.grouped_forward (active_expert_lora.py:348-399), the
 * backward of CompressedGroupedExperts.grouped_linear (experts.py:803-827).
 * in_features and out_features are multiples of 64; BF16, NF4, NF4_F32 and
 * INT8 weights.
 */
int mx_grouped_linear_backward(const void *grad_out, const void *x, const int64_t *counts,
                               int64_t num_rows, int num_experts, const mx_weight *w,
                               const mx_lora *lora, void *grad_x, float *grad_a, float *grad_b,
                               void *workspace, void *stream);

/*
 * Backward of mx_moe_forward (adapter training, frozen base): given
 * grad_out [T, hidden] and the activations saved by the forward, produces
 * grad_tokens [T, hidden] (fp32 accumulation, out_dtype), grad_scores [T, k]
 * fp32, and fp32 LoRA gradients dA/dB for each adapter (NULL if absent; all
 * zero when num_tokens is 0, the gradient of an empty sum).
 * Base weights are re-decoded in-kernel, never materialised. Replaces the
 * autograd of _FrozenDequantBatchedLinear(Pair).backward (linear.py:117-125,
 * 192-203), the LoRA bmm chain (active_expert_lora.py:434-477) and
 * _CombineRoutedTokens.backward (dispatch_ops.py:34-44).
 */
int mx_moe_backward(const void *grad_out, int grad_dtype, const void *tokens,
                    const int64_t *top_idx, const void *top_scores, int score_dtype,
                    int64_t num_tokens, int top_k, int num_experts, int64_t hidden,
                    int64_t ffn, const mx_weight *w1, const mx_weight *w3,
                    const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                    const mx_lora *l2, const void *save_gate, const void *save_up,
                    const void *save_h, const void *save_y, const void *save_lora,
                    void *grad_tokens, int grad_tokens_dtype, float *grad_scores,
                    float *grad_a1, float *grad_b1, float *grad_a3, float *grad_b3,
                    float *grad_a2, float *grad_b2, void *workspace, void *stream);

/*
 * mx_moe_backward with a choice of expert activation (MX_ACT_*); the
 * MX_ACT_SWIGLU7 derivative is that of _memory_bounded_swiglu7_backward
 * (mirai/core/models/magi2_preview/grouped_moe.py:309-335).
 */
int mx_moe_backward_act(const void *grad_out, int grad_dtype, const void *tokens,
                        const int64_t *top_idx, const void *top_scores, int score_dtype,
                        int64_t num_tokens, int top_k, int num_experts, int64_t hidden,
                        int64_t ffn, int act, const mx_weight *w1, const mx_weight *w3,
                        const mx_weight *w2, const mx_lora *l1, const mx_lora *l3,
                        const mx_lora *l2, const void *save_gate, const void *save_up,
                        const void *save_h, const void *save_y, const void *save_lora,
                        void *grad_tokens, int grad_tokens_dtype, float *grad_scores,
                        float *grad_a1, float *grad_b1, float *grad_a3, float *grad_b3,
                        float *grad_a2, float *grad_b2, void *workspace, void *stream);

/* Bytes of scratch for mx_moe_backward (and mx_moe_backward_act). */
size_t mx_moe_backward_workspace_size(int64_t num_tokens, int top_k, int num_experts,
                                      int64_t hidden, int64_t ffn, int lora_rank);

#ifdef __cplusplus
}
#endif

#endif /* MIRAI_MOE_H */
