"""Expert-choice dispatch plan and routed layer, restated (test
infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline use oracle/).

* build_expert_choice_plan follows build_expert_choice_dispatch_plan
  (mirai/core/models/compressed_weights/execution/dispatch_preprocess.py:182-278):
  token = idx + b * tokens_per_sample, physical expert = alias[l] (or l), a
  stable sort of the flat slots (b, l, c) by physical expert, counts /
  exclusive starts / inclusive offsets, inverse permutation.
* expert_choice_forward follows run_compressed_expert_choice
  (execution/expert_choice.py:16-152) with _run_direct_routed_device_chunks
  (experts.py, the index_add_ of y.float() * score.float() into an fp32
  buffer over the sorted slots, cast to the token dtype at the end) on the
  CPU, where index_add_ adds in slot order.
"""

from __future__ import annotations

import numpy as np
import torch

from . import layer as olayer


def build_expert_choice_plan(idx: np.ndarray, scores: np.ndarray, tokens_per_sample: int,
                             num_physical: int, alias=()):
    idx = np.asarray(idx, dtype=np.int64)
    B, L, C = idx.shape
    tokens = (idx + (np.arange(B, dtype=np.int64) * int(tokens_per_sample)).reshape(B, 1, 1))
    logical = np.broadcast_to(np.arange(L, dtype=np.int64).reshape(1, L, 1), (B, L, C))
    phys = np.asarray(alias, dtype=np.int64)[logical] if len(alias) else logical
    phys = phys.reshape(-1)
    order = np.argsort(phys, kind="stable")
    counts = np.bincount(phys, minlength=num_physical).astype(np.int64)
    cum = np.cumsum(counts)
    inverse = np.empty_like(order)
    inverse[order] = np.arange(order.size)
    flat_scores = np.asarray(scores).reshape(-1)
    return dict(counts=counts, starts=cum - counts, offsets=cum.astype(np.int32),
                sort_positions=order.astype(np.int64),
                sorted_token_indices=tokens.reshape(-1)[order],
                sorted_scores=flat_scores[order], inverse_order=inverse.astype(np.int64))


def expert_choice_forward(tokens: torch.Tensor, scores: torch.Tensor, idx: torch.Tensor,
                          tokens_per_sample: int, weights: dict, loras: dict, num_physical: int,
                          alias=()) -> torch.Tensor:
    """[B * tokens_per_sample, d] output in the token dtype."""
    plan = build_expert_choice_plan(idx.numpy(), scores.detach().float().numpy(),
                                    tokens_per_sample, num_physical, alias)
    output = torch.zeros(tokens.shape, dtype=torch.float32)
    sorted_tokens = torch.from_numpy(plan["sorted_token_indices"])
    # The plan's sorted scores, gathered with torch so that autograd reaches
    # the [B, L, C] scores (the reference's plan index_selects them).
    sorted_scores = scores.reshape(-1).float()[torch.from_numpy(plan["sort_positions"])]
    for e in range(num_physical):
        a, n = int(plan["starts"][e]), int(plan["counts"][e])
        if n == 0:
            continue
        tok = sorted_tokens[a:a + n]
        y = olayer.expert_mlp(tokens.index_select(0, tok), e, weights, loras)
        output = output.index_add(0, tok, y.float() * sorted_scores[a:a + n].unsqueeze(1))
    return output.to(tokens.dtype)
