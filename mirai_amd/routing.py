"""Top-k token-choice routing on the GPU (router front end of the expert op).

``route_topk`` replaces the softmax -> topk -> gather -> renormalise ->
route_scale sequence of TokenChoiceRouter.forward
(mirai/core/moe/routing/routers.py:234-249) and LingBotVideoRouter.forward with
softmax scores and no correction bias
(mirai/vendors/lingbot_video/transformer_lingbot_video.py:1002-1033).
Gradients flow from the scores back to the logits; the indices carry none.
"""

from __future__ import annotations

import torch

from . import _native as nat

RENORM_MODES = {"none": nat.RENORM_NONE, "clamp": nat.RENORM_CLAMP, "eps": nat.RENORM_EPS}


class _RouteTopK(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, top_k, renorm, route_scale, score_dtype):
        device = nat.require_gpu(logits)
        logits = logits.detach().float().contiguous()
        T, E = (int(v) for v in logits.shape)
        idx = torch.empty((T, top_k), dtype=torch.int64, device=device)
        scores = torch.empty((T, top_k), dtype=score_dtype, device=device)
        nat.call("mx_route_topk", logits.data_ptr(), T, E, int(top_k), renorm, float(route_scale),
                 idx.data_ptr(), scores.data_ptr(), nat.dtype_code(score_dtype), nat.stream(device))
        ctx.save_for_backward(logits, idx)
        ctx.cfg = (int(top_k), renorm, float(route_scale))
        ctx.mark_non_differentiable(idx)
        return idx, scores

    @staticmethod
    def backward(ctx, grad_idx, grad_scores):
        logits, idx = ctx.saved_tensors
        top_k, renorm, route_scale = ctx.cfg
        T, E = (int(v) for v in logits.shape)
        grad_logits = torch.empty_like(logits)
        if grad_scores is None:
            return None, None, None, None, None
        g = grad_scores.float().contiguous()
        nat.call("mx_route_topk_backward", logits.data_ptr(), T, E, top_k, renorm, route_scale,
                 idx.data_ptr(), g.data_ptr(), grad_logits.data_ptr(),
                 nat.stream(logits.device))
        return grad_logits, None, None, None, None


def route_topk(logits: torch.Tensor, top_k: int, *, renorm: str = "clamp",
               route_scale: float = 1.0, score_dtype: torch.dtype = torch.float32):
    """Return ``(top_indices [T,k] int64, top_scores [T,k])`` in descending order.

    renorm: "clamp" (TokenChoiceRouter), "eps" (LingBot norm_topk_prob) or "none".
    Ties between equal logits go to the lower expert id.
    """
    if logits.ndim != 2:
        raise ValueError("router logits must be [tokens, experts].")
    if renorm not in RENORM_MODES:
        raise ValueError(f"renorm must be one of {sorted(RENORM_MODES)}.")
    E = int(logits.shape[1])
    if int(top_k) <= 0 or int(top_k) > min(E, 16):
        raise ValueError("top_k must be in [1, min(num_experts, 16)].")
    return _RouteTopK.apply(logits, int(top_k), RENORM_MODES[renorm], float(route_scale),
                            score_dtype)
