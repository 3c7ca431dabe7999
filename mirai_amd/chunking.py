"""Token-chunked routed expert execution for adapter training.

Drop-in for MoETokenChunkPolicy (mirai/core/moe/runtime/token_chunking.py:26-118):
routing is computed once for all tokens; in training with gradients the
routed layer then runs one contiguous token chunk at a time under activation
checkpointing, so the saved activations of only one chunk are alive at once
(the fused layer saves gate / up / h / y / low-rank rows per routed slot, about
(3f + d + 96) * 2 bytes per slot).

Each chunk is one call of the fused layer. Routed rows are computed
independently of the other rows of their GEMM tile and the combine sums each
token's own slots, so the chunked forward output is bit-identical to the
unchunked one; only the LoRA weight gradients, summed over chunks, differ by
fp32 summation order.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

import torch

ChunkRunner = Callable[[Any, Any, Any, int], Any]


@dataclass(frozen=True)
class MoETokenChunkPolicy:
    """Checkpoint local expert work in bounded contiguous token chunks."""

    token_chunk_size: int = 0

    def __post_init__(self) -> None:
        if int(self.token_chunk_size) < 0:
            raise ValueError("training.moe_token_chunk_size must be >= 0.")
        object.__setattr__(self, "token_chunk_size", int(self.token_chunk_size))

    @property
    def enabled(self) -> bool:
        return self.token_chunk_size > 0

    def chunk_count(self, token_count: int) -> int:
        count = int(token_count)
        if count < 0:
            raise ValueError("MoE token count must be >= 0.")
        if not self.enabled or count == 0:
            return 1
        return -(-count // self.token_chunk_size)

    def execute(self, tokens: torch.Tensor, top_scores: torch.Tensor, top_indices: torch.Tensor,
                *, runner: ChunkRunner, training: bool) -> torch.Tensor:
        """Run one route plan through chunk-local expert execution (token_chunking.py:48-118)."""
        if top_scores.shape != top_indices.shape or int(top_indices.ndim) != 2:
            raise ValueError("MoE token chunking requires matching [tokens, top_k] routes.")
        if int(tokens.ndim) != 2:
            raise ValueError("MoE token chunking requires a [tokens, hidden] tensor.")
        count = int(tokens.shape[0])
        if int(top_indices.shape[0]) != count:
            raise ValueError("MoE token chunk routes do not match the token count.")
        if not self.enabled or count <= self.token_chunk_size or not bool(training):
            return runner(tokens, top_scores, top_indices, 0)
        use_checkpoint = torch.is_grad_enabled()
        outputs = []
        for start in range(0, count, self.token_chunk_size):
            end = min(start + self.token_chunk_size, count)
            args = (tokens[start:end], top_scores[start:end], top_indices[start:end])
            if use_checkpoint:
                from torch.utils.checkpoint import checkpoint

                def run_chunk(t, s, i, *, token_offset=start):
                    return runner(t, s, i, token_offset)

                outputs.append(checkpoint(run_chunk, *args, use_reentrant=False,
                                          preserve_rng_state=True))
            else:
                outputs.append(runner(*args, start))
        return torch.cat(outputs, dim=0)


__all__ = ["MoETokenChunkPolicy"]
