"""Dispatch plan and routed permute / combine on the GPU.

Mirrors mirai/core/models/compressed_weights/execution/dispatch_preprocess.py
(DispatchPlan :22-41, build_dispatch_plan :128-179) and dispatch_ops.py
(permute_routed_tokens / combine_routed_tokens :8-63) with the same field
names, dtypes and autograd contract.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native as nat


@dataclass(frozen=True)
class DispatchPlan:
    counts: torch.Tensor                # [E] int64
    starts: torch.Tensor                # [E] int64 exclusive prefix
    offsets: torch.Tensor               # [E] int32 inclusive prefix
    sort_positions: torch.Tensor        # [S] int64
    sorted_token_indices: torch.Tensor  # [S] int64
    sorted_scores: torch.Tensor         # [S]
    inverse_order: torch.Tensor         # [S] int64
    total_slots: int
    top_k: int
    max_count_bound: int


def _empty_plan(E: int, score_dtype, device, *, k: int, bound: int) -> DispatchPlan:
    """The plan of no routed slots: every expert's segment is empty and there
    is nothing to sort (no kernel runs)."""
    def none(dtype):
        return torch.empty(0, dtype=dtype, device=device)
    return DispatchPlan(counts=torch.zeros(E, dtype=torch.int64, device=device),
                        starts=torch.zeros(E, dtype=torch.int64, device=device),
                        offsets=torch.zeros(E, dtype=torch.int32, device=device),
                        sort_positions=none(torch.int64), sorted_token_indices=none(torch.int64),
                        sorted_scores=none(score_dtype), inverse_order=none(torch.int64),
                        total_slots=0, top_k=k, max_count_bound=bound)


def build_dispatch_plan(top_indices: torch.Tensor, top_scores: torch.Tensor, num_experts: int,
                        *, backend: str = "device") -> DispatchPlan:
    """Device-resident plan (no host sync): a stable counting sort by expert.

    ``backend`` accepts the reference's names; both run the same kernels.
    """
    selected = str(backend).strip().lower()
    if selected not in {"device", "sonic"}:
        raise ValueError("dispatch-plan backend must be 'device' or 'sonic'.")
    if top_indices.ndim != 2 or tuple(top_scores.shape) != tuple(top_indices.shape):
        raise ValueError("top_indices and top_scores must both be [tokens, top_k].")
    device = nat.require_gpu(top_indices, top_scores)
    T, k = (int(v) for v in top_indices.shape)
    E = int(num_experts)
    S = T * k
    if S >= 2**31:
        raise ValueError("dispatch plan slot count exceeds int32 range")
    idx = top_indices.to(torch.int64).contiguous()
    scores = top_scores.contiguous()
    if scores.dtype not in (torch.float32, torch.bfloat16):
        scores = scores.float()
    if S == 0:
        return _empty_plan(E, scores.dtype, device, k=k, bound=T)
    counts = torch.empty(E, dtype=torch.int64, device=device)
    starts = torch.empty(E, dtype=torch.int64, device=device)
    offsets = torch.empty(E, dtype=torch.int32, device=device)
    sort_positions = torch.empty(S, dtype=torch.int64, device=device)
    sorted_tokens = torch.empty(S, dtype=torch.int64, device=device)
    sorted_scores = torch.empty(S, dtype=scores.dtype, device=device)
    inverse = torch.empty(S, dtype=torch.int64, device=device)
    ws = nat.workspace(nat.load_library().mx_plan_workspace_size(T, k, E), device)
    nat.call("mx_build_plan", idx.data_ptr(), scores.data_ptr(), nat.dtype_code(scores.dtype),
             T, k, E, counts.data_ptr(), starts.data_ptr(), offsets.data_ptr(),
             sort_positions.data_ptr(), sorted_tokens.data_ptr(), sorted_scores.data_ptr(),
             inverse.data_ptr(), ws.data_ptr(), nat.stream(device))
    return DispatchPlan(counts=counts, starts=starts, offsets=offsets,
                        sort_positions=sort_positions, sorted_token_indices=sorted_tokens,
                        sorted_scores=sorted_scores, inverse_order=inverse, total_slots=S,
                        top_k=k, max_count_bound=T)


def build_expert_choice_dispatch_plan(expert_token_indices: torch.Tensor,
                                      expert_token_scores: torch.Tensor, *,
                                      tokens_per_sample: int, num_physical_experts: int,
                                      logical_to_physical: tuple[int, ...] = ()) -> DispatchPlan:
    """Expert-contiguous plan from [batch, expert, capacity] routes
    (dispatch_preprocess.py:182-278), device-resident: the flat slots sorted
    stably by physical expert, sorted_token_indices = idx + b * tokens_per_sample."""
    if expert_token_indices.shape != expert_token_scores.shape:
        raise ValueError("Expert-choice indices and scores must have matching shapes.")
    if expert_token_indices.ndim != 3:
        raise ValueError("Expert-choice routes must have shape [batch, expert, capacity].")
    B, L, C = (int(v) for v in expert_token_indices.shape)
    if expert_token_indices.device != expert_token_scores.device:
        raise ValueError("Expert-choice indices and scores must share a device.")
    if expert_token_indices.dtype.is_floating_point:
        raise TypeError("Expert-choice token indices must use an integer dtype.")
    if L <= 0 or C <= 0:
        raise ValueError("Expert-choice routes require experts and positive capacity.")
    if int(tokens_per_sample) <= 0:
        raise ValueError("tokens_per_sample must be > 0.")
    E = int(num_physical_experts)
    if E <= 0:
        raise ValueError("num_physical_experts must be > 0.")
    aliases = tuple(int(v) for v in logical_to_physical)
    if aliases and len(aliases) != L:
        raise ValueError("Logical expert alias map does not match Expert-Choice routes.")
    if aliases and any(v < 0 or v >= E for v in aliases):
        raise ValueError("Logical expert alias map contains an invalid physical id.")
    if not aliases and L != E:
        raise ValueError("Logical and physical expert counts differ without an alias map.")
    S = B * L * C
    if S >= 2**31:
        raise ValueError("Expert-choice dispatch plan exceeds the int32 slot range.")
    device = nat.require_gpu(expert_token_indices, expert_token_scores)
    idx = expert_token_indices.to(torch.int64).contiguous()
    scores = expert_token_scores.contiguous()
    if scores.dtype not in (torch.float32, torch.bfloat16):
        scores = scores.float()
    if S == 0:
        return _empty_plan(E, scores.dtype, device, k=0, bound=0)
    l2p = torch.tensor(aliases, dtype=torch.int32, device=device) if aliases else None
    counts = torch.empty(E, dtype=torch.int64, device=device)
    starts = torch.empty(E, dtype=torch.int64, device=device)
    offsets = torch.empty(E, dtype=torch.int32, device=device)
    sort_positions = torch.empty(S, dtype=torch.int64, device=device)
    sorted_tokens = torch.empty(S, dtype=torch.int64, device=device)
    sorted_scores = torch.empty(S, dtype=scores.dtype, device=device)
    inverse = torch.empty(S, dtype=torch.int64, device=device)
    ws = nat.workspace(nat.load_library().mx_expert_choice_plan_workspace_size(B, L, C, E), device)
    nat.call("mx_build_expert_choice_plan", idx.data_ptr(), scores.data_ptr(),
             nat.dtype_code(scores.dtype), B, L, C, int(tokens_per_sample), nat.ptr(l2p), E,
             counts.data_ptr(), starts.data_ptr(), offsets.data_ptr(), sort_positions.data_ptr(),
             sorted_tokens.data_ptr(), sorted_scores.data_ptr(), inverse.data_ptr(),
             ws.data_ptr(), nat.stream(device))
    if aliases:
        bound = B * C * max(aliases.count(i) for i in range(E))
    else:
        bound = B * C
    return DispatchPlan(counts=counts, starts=starts, offsets=offsets,
                        sort_positions=sort_positions, sorted_token_indices=sorted_tokens,
                        sorted_scores=sorted_scores, inverse_order=inverse, total_slots=S,
                        top_k=0, max_count_bound=bound)


def _gather(tokens: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    device = nat.require_gpu(tokens, index)
    src = tokens.contiguous()
    idx = index.to(torch.int64).contiguous()
    out = torch.empty((int(idx.numel()), int(src.shape[-1])), dtype=src.dtype, device=device)
    nat.call("mx_gather_rows", src.data_ptr(), int(src.shape[0]), idx.data_ptr(), int(idx.numel()),
             int(src.shape[-1]), nat.dtype_code(src.dtype), out.data_ptr(), nat.stream(device))
    return out


def _scatter_add(rows: torch.Tensor, scale: torch.Tensor | None, index: torch.Tensor,
                 out_rows: int) -> torch.Tensor:
    device = nat.require_gpu(rows, index)
    src = rows.contiguous()
    if src.dtype not in (torch.float32, torch.bfloat16):
        src = src.float()
    idx = index.to(torch.int64).contiguous()
    sc = None if scale is None else scale.float().contiguous()
    out = torch.empty((int(out_rows), int(src.shape[-1])), dtype=torch.float32, device=device)
    nat.call("mx_scatter_add_rows", src.data_ptr(), nat.ptr(sc), idx.data_ptr(), int(idx.numel()),
             int(src.shape[-1]), nat.dtype_code(src.dtype), int(out_rows), out.data_ptr(),
             nat.stream(device))
    return out


class _PermuteRoutedTokens(torch.autograd.Function):
    @staticmethod
    def forward(ctx, tokens, token_indices):
        ctx.input_rows = int(tokens.shape[0])
        ctx.save_for_backward(token_indices)
        return _gather(tokens, token_indices)

    @staticmethod
    def backward(ctx, grad_output):
        (token_indices,) = ctx.saved_tensors
        grad = _scatter_add(grad_output, None, token_indices, ctx.input_rows)
        return grad.to(grad_output.dtype), None


class _CombineRoutedTokens(torch.autograd.Function):
    @staticmethod
    def forward(ctx, expert_output, scores, token_indices, output_rows):
        ctx.expert_dtype = expert_output.dtype
        ctx.score_dtype = scores.dtype
        ctx.save_for_backward(expert_output, scores, token_indices)
        return _scatter_add(expert_output, scores, token_indices, output_rows)

    @staticmethod
    def backward(ctx, grad_output):
        expert_output, scores, token_indices = ctx.saved_tensors
        gathered = _gather(grad_output.float(), token_indices)
        grad_expert = (gathered * scores.float().unsqueeze(1)).to(ctx.expert_dtype)
        grad_scores = (gathered * expert_output.float()).sum(dim=1).to(ctx.score_dtype)
        return grad_expert, grad_scores, None, None


def permute_routed_tokens(tokens: torch.Tensor, token_indices: torch.Tensor) -> torch.Tensor:
    """``tokens.index_select(0, token_indices)`` with an index_add backward."""
    return _PermuteRoutedTokens.apply(tokens, token_indices)


def combine_routed_tokens(expert_output: torch.Tensor, scores: torch.Tensor,
                          token_indices: torch.Tensor, *, output_rows: int,
                          output_dtype: torch.dtype) -> torch.Tensor:
    """fp32 ``index_add`` of ``expert_output * score`` rows into ``output_rows`` rows."""
    return _CombineRoutedTokens.apply(expert_output, scores, token_indices,
                                      int(output_rows)).to(dtype=output_dtype)
