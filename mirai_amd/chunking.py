"""Token-chunked routed expert execution (drop-in for MoETokenChunkPolicy,
mirai/core/moe/runtime/token_chunking.py:26-118).

Routing happens once, over all tokens; in training the routed layer then runs
over contiguous token chunks so that only one chunk's per-slot activations are
alive at a time. The policy's surface (``token_chunk_size``, ``enabled``,
``chunk_count``, ``execute(tokens, top_scores, top_indices, *, runner,
training)``, the ValueError messages) is the reference's.

Execution is this build's own. A runner made by :func:`fused_chunk_runner`
(the fused routed layer of one ``CompressedGroupedExperts``) goes to a single
autograd function that checkpoints at the native call boundary: the forward
writes each chunk's output rows in place and keeps nothing but the inputs, the
backward recomputes and differentiates one chunk at a time and sums the LoRA
factor gradients in fp32 (``fused.routed_experts_chunked``). Any other runner
falls back to torch's non-reentrant checkpoint per chunk.
"""

from __future__ import annotations

import functools
from dataclasses import dataclass
from typing import Any, Callable

import torch

ChunkRunner = Callable[[Any, Any, Any, int], Any]


class FusedChunkRunner:
    """Runner ``(tokens, top_scores, top_indices, token_offset) -> out`` of the
    fused routed layer of ``experts``; the policy recognises it and chunks at
    the native call boundary."""

    def __init__(self, experts) -> None:
        self.experts = experts

    def __call__(self, tokens, top_scores, top_indices, token_offset: int = 0):
        # run_direct_routed: its checks, alias coalescing, then the fused layer.
        return self.experts.run_direct_routed(tokens, top_scores, top_indices)


def fused_chunk_runner(experts) -> FusedChunkRunner:
    return FusedChunkRunner(experts)


def _checkpointed(runner: ChunkRunner, offset: int, tokens, top_scores, top_indices):
    return runner(tokens, top_scores, top_indices, offset)


@dataclass(frozen=True)
class MoETokenChunkPolicy:
    """Contiguous token chunks of at most ``token_chunk_size`` tokens (0: off)."""

    token_chunk_size: int = 0

    def __post_init__(self) -> None:
        size = int(self.token_chunk_size)
        if size < 0:
            raise ValueError("training.moe_token_chunk_size must be >= 0.")
        object.__setattr__(self, "token_chunk_size", size)

    @property
    def enabled(self) -> bool:
        return self.token_chunk_size > 0

    def chunk_count(self, token_count: int) -> int:
        n = int(token_count)
        if n < 0:
            raise ValueError("MoE token count must be >= 0.")
        return len(self.chunk_bounds(n)) if self.enabled and n > 0 else 1

    def chunk_bounds(self, token_count: int) -> list[tuple[int, int]]:
        """[(start, end), ...] covering range(token_count) in order."""
        n, c = int(token_count), self.token_chunk_size
        return [(a, min(a + c, n)) for a in range(0, n, c)] if c > 0 else [(0, n)]

    def execute(self, tokens: torch.Tensor, top_scores: torch.Tensor,
                top_indices: torch.Tensor, *, runner: ChunkRunner,
                training: bool) -> torch.Tensor:
        if int(top_indices.ndim) != 2 or top_scores.shape != top_indices.shape:
            raise ValueError("MoE token chunking requires matching [tokens, top_k] routes.")
        if int(tokens.ndim) != 2:
            raise ValueError("MoE token chunking requires a [tokens, hidden] tensor.")
        n = int(tokens.shape[0])
        if int(top_indices.shape[0]) != n:
            raise ValueError("MoE token chunk routes do not match the token count.")
        # One pass when chunking is off, when the tokens fit one chunk, and in
        # inference (nothing is saved for a backward there).
        if not (self.enabled and bool(training)) or n <= self.token_chunk_size:
            return runner(tokens, top_scores, top_indices, 0)
        bounds = self.chunk_bounds(n)
        if isinstance(runner, FusedChunkRunner):
            from .fused import routed_experts_chunked

            # Checks and alias coalescing once over all tokens: coalescing
            # merges slots within a token, so every chunk then runs exactly
            # the physical routes of the unchunked layer.
            scores, indices = runner.experts.direct_routes(tokens, top_scores, top_indices)
            return routed_experts_chunked(runner.experts, tokens, scores, indices, bounds)
        if not torch.is_grad_enabled():
            return torch.cat([runner(tokens[a:b], top_scores[a:b], top_indices[a:b], a)
                              for a, b in bounds], dim=0)
        from torch.utils.checkpoint import checkpoint

        parts = [checkpoint(functools.partial(_checkpointed, runner, a), tokens[a:b],
                            top_scores[a:b], top_indices[a:b], use_reentrant=False)
                 for a, b in bounds]
        return torch.cat(parts, dim=0)


__all__ = ["ChunkRunner", "FusedChunkRunner", "MoETokenChunkPolicy", "fused_chunk_runner"]
