"""Softmax top-k token-choice routing, restated.

Follows TokenChoiceRouter.forward (mirai/core/moe/routing/routers.py:234-249:
softmax, topk, renormalise by clamp_min(sum, 1e-20)) and
LingBotVideoRouter.forward with score_func="softmax" and no correction bias
(mirai/vendors/lingbot_video/transformer_lingbot_video.py:1002-1033:
renormalise by sum + 1e-20 when norm_topk_prob, then * route_scale).

Canonical selection rule: the k largest logits (softmax is strictly monotone),
ties to the lower expert id, slots in descending order. torch.topk's slot
order with sorted=False is unspecified, so the slot order is fixed here.
"""

from __future__ import annotations

import numpy as np
import torch

RENORM_NONE, RENORM_CLAMP, RENORM_EPS = 0, 1, 2


def route_topk(logits: np.ndarray, top_k: int, *, renorm: int = RENORM_CLAMP,
               route_scale: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """Return (top_idx int64 [T,k], top_scores float32 [T,k])."""
    logits = np.asarray(logits, dtype=np.float32)
    order = np.argsort(-logits, axis=1, kind="stable")[:, :top_k].astype(np.int64)
    shifted = (logits - logits.max(axis=1, keepdims=True)).astype(np.float64)
    ex = np.exp(shifted)
    probs = ex / ex.sum(axis=1, keepdims=True)
    sel = np.take_along_axis(probs, order, axis=1)
    total = sel.sum(axis=1, keepdims=True)
    if renorm == RENORM_CLAMP:
        sel = sel / np.maximum(total, 1e-20)
    elif renorm == RENORM_EPS:
        sel = sel / (total + 1e-20)
    sel = sel * route_scale
    return order, sel.astype(np.float32)


def route_topk_backward(logits: np.ndarray, top_idx: np.ndarray, grad_scores: np.ndarray, *,
                        renorm: int = RENORM_CLAMP, route_scale: float = 1.0) -> np.ndarray:
    """d(logits) by float64 autograd of softmax -> gather -> renormalise -> scale."""
    lg = torch.tensor(np.asarray(logits, dtype=np.float64), requires_grad=True)
    probs = torch.softmax(lg, dim=-1)
    sel = probs.gather(1, torch.as_tensor(top_idx, dtype=torch.int64))
    total = sel.sum(dim=-1, keepdim=True)
    if renorm == RENORM_CLAMP:
        sel = sel / total.clamp_min(1e-20)
    elif renorm == RENORM_EPS:
        sel = sel / (total + 1e-20)
    sel = sel * route_scale
    sel.backward(torch.as_tensor(np.asarray(grad_scores, dtype=np.float64)))
    return lg.grad.numpy()
