"""LingBot router front end, restated (test infrastructure: only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline use oracle/).

Follows LingBotVideoRouter.forward
(mirai/vendors/lingbot_video/transformer_lingbot_video.py:962-1033) with no
extensions installed, in the reference's dtypes on the CPU:

* logits = F.linear(tokens.float(), weight) in fp32 (+ logit_delta)   :982-994
* scores = softmax(logits, -1) or sigmoid(logits)                        :1002-1005
* scores_for_choice = scores + e_score_correction_bias                   :1006
* group-limited choice when n_group > 1 (_group_limited_choice_scores,
  :873-886): group score = sum of the two largest choice scores of the group,
  the topk_group best groups stay, the rest is masked to -inf
* top_indices = topk(scores_for_choice, k)                               :1027-1029
* top_scores = scores.gather(top_indices); / (sum + 1e-20) when k > 1 and
  norm_topk_prob; * route_scale; .to(tokens.dtype)                       :1030-1033, 1132

torch.topk with sorted=False leaves the slot order and the choice among equal
keys unspecified; here picks are in descending key order and ties go to the
lower expert (and group) id.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def router_logits(tokens: torch.Tensor, weight: torch.Tensor,
                  logit_delta: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 logits [T, E] as the reference computes them (:989-999)."""
    logits = F.linear(tokens.float(), weight.float())
    if logit_delta is not None:
        logits = logits + logit_delta.float()
    return logits


def _topk_desc(keys: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest entries per row, descending, ties to the lower index."""
    return np.argsort(-keys, axis=-1, kind="stable")[..., :k]


def group_mask(keys: torch.Tensor, n_group: int, topk_group: int) -> torch.Tensor:
    """Boolean [T, E] mask of the experts in each token's topk_group best groups."""
    T, E = keys.shape
    grouped = keys.view(T, n_group, E // n_group)
    group_scores = grouped.topk(2, dim=-1)[0].sum(dim=-1)  # :875
    keep = _topk_desc(group_scores.numpy(), topk_group)
    gmask = np.zeros((T, n_group), dtype=bool)
    np.put_along_axis(gmask, keep, True, axis=1)
    return torch.from_numpy(np.repeat(gmask, E // n_group, axis=1))


def route_from_logits(logits: torch.Tensor, top_k: int, *, score_func: str = "sigmoid",
                      expert_bias: torch.Tensor | None = None, norm_topk_prob: bool = True,
                      n_group: int | None = None, topk_group: int | None = None,
                      route_scale: float = 1.0, out_dtype: torch.dtype = torch.float32,
                      picks: torch.Tensor | None = None):
    """Selection and scores from fp32 logits: (top_idx int64 [T,k], top_scores [T,k],
    scores [T,E] fp32, scores_for_choice [T,E] fp32)."""
    logits = logits.float()
    if score_func == "softmax":
        scores = F.softmax(logits, dim=-1)
    elif score_func == "sigmoid":
        scores = logits.sigmoid()
    else:
        raise ValueError(score_func)
    return route_from_scores(scores, top_k, expert_bias=expert_bias,
                             norm_topk_prob=norm_topk_prob, n_group=n_group,
                             topk_group=topk_group, route_scale=route_scale, out_dtype=out_dtype,
                             picks=picks)


def route_from_scores(scores: torch.Tensor, top_k: int, *,
                      expert_bias: torch.Tensor | None = None, norm_topk_prob: bool = True,
                      n_group: int | None = None, topk_group: int | None = None,
                      route_scale: float = 1.0, out_dtype: torch.dtype = torch.float32,
                      picks: torch.Tensor | None = None):
    """The selection and gating of :1006-1033 from fp32 scores [T, E]. With
    ``picks`` [T, k] the selection is taken as given (only the gating is
    computed): the autograd-capable path of the backward checks."""
    scores = scores.float()
    bias = torch.zeros(scores.shape[1]) if expert_bias is None else expert_bias.float()
    choice = scores + bias.unsqueeze(0)
    keys = choice.detach()
    if n_group is not None and n_group > 1:
        keep = group_mask(keys, n_group, topk_group)
        keys = keys.masked_fill(~keep, float("-inf"))
    if picks is not None:
        idx = picks.to(torch.int64)
    else:
        idx = torch.from_numpy(_topk_desc(keys.numpy(), top_k).astype(np.int64))
    top = scores.gather(1, idx)
    if top_k > 1 and norm_topk_prob:
        top = top / (top.sum(dim=-1, keepdim=True) + 1e-20)
    top = top * route_scale
    return idx, top.to(out_dtype), scores, choice


def router_forward(tokens: torch.Tensor, weight: torch.Tensor, top_k: int, *,
                   logit_delta: torch.Tensor | None = None, **kw):
    """(top_idx, top_scores in tokens' dtype, logits, scores, scores_for_choice)."""
    logits = router_logits(tokens, weight, logit_delta)
    idx, top, scores, choice = route_from_logits(logits, top_k, out_dtype=tokens.dtype, **kw)
    return idx, top, logits, scores, choice


def logits_error_bound(tokens: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Per-token bound [T] on |fp32 logit - exact logit|: 64 * 2^-24 * max_e sum_i |x_i w_ei|.

    Each fp32 addition errs by at most 2^-24 times a partial sum, and every
    partial sum is at most sum_i |x_i w_i|; 64 covers summation chains of 64
    roundings at worst, and longer chains (a sequential MFMA accumulation
    over 3*d/16 steps) in the statistical sense, with margin: their rounding
    errors are independent and their partial sums are far below the bound's
    magnitude sum.
    """
    mag = tokens.double().abs() @ weight.double().abs().t()
    return 64 * 2.0**-24 * mag.max(dim=1).values
