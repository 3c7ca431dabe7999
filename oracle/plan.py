"""Dispatch plan, restated from build_dispatch_plan
(mirai/core/models/compressed_weights/execution/dispatch_preprocess.py:128-179)
and the vectorized runner (experts.py:2369-2381): stable argsort of the flat
expert ids, token = position // k, bincount, inclusive/exclusive cumsum,
inverse permutation. Route slots with an expert id outside [0, E) take no
position (inverse_order = -1).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Plan:
    counts: np.ndarray               # [E] int64
    starts: np.ndarray               # [E] int64 exclusive prefix
    offsets: np.ndarray              # [E] int32 inclusive prefix
    sort_positions: np.ndarray       # [S] int64
    sorted_token_indices: np.ndarray # [S] int64
    sorted_scores: np.ndarray | None # [S]
    inverse_order: np.ndarray        # [T*k] int64 (-1 for dropped slots)


def build_dispatch_plan(top_idx: np.ndarray, top_scores: np.ndarray | None,
                        num_experts: int) -> Plan:
    top_idx = np.asarray(top_idx, dtype=np.int64)
    k = top_idx.shape[1] if top_idx.ndim == 2 else 1
    flat = top_idx.reshape(-1)
    valid = (flat >= 0) & (flat < num_experts)
    candidates = np.nonzero(valid)[0]
    order = candidates[np.argsort(flat[candidates], kind="stable")]
    counts = np.bincount(flat[valid], minlength=num_experts).astype(np.int64)
    cumsum = np.cumsum(counts)
    inverse = np.full(flat.shape[0], -1, dtype=np.int64)
    inverse[order] = np.arange(order.shape[0], dtype=np.int64)
    sorted_scores = None
    if top_scores is not None:
        sorted_scores = np.asarray(top_scores).reshape(-1)[order]
    return Plan(
        counts=counts,
        starts=(cumsum - counts).astype(np.int64),
        offsets=cumsum.astype(np.int32),
        sort_positions=order.astype(np.int64),
        sorted_token_indices=(order // k).astype(np.int64),
        sorted_scores=sorted_scores,
        inverse_order=inverse,
    )
