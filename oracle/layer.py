"""The routed expert layer in the reference op order, on the CPU with torch.

Restates the per-expert reference loop of CompressedGroupedExperts.run_direct_routed
(mirai/core/models/compressed_weights/execution/experts.py:1786-1895):
for each expert with routed rows (ascending), gather its tokens, run the frozen
projections ``x @ W^T`` (_FrozenDequantExpertLinear, linear.py:74-79) plus the
expert LoRA ``linear(linear(x, A_e), B_e) * scale`` in the activation dtype
(ActiveExpertLoRA.forward, active_expert_lora.py:316-346, scale from
lora_scale, mirai/core/models/adapters/lora_allocation.py:163-168), combine
``silu(gate) * up`` (experts.py:289-317 with CANONICAL_PACKED_EXPERT_MLP_SPEC,
mirai/core/moe/runtime/specs.py:222-231), project down, and ``index_add_`` the
fp32 product ``y.float() * score`` into an fp32 buffer that is finally cast to
the token dtype. run_for_loop follows experts.py:1656-1747.

Autograd through these torch ops is the backward oracle (frozen weights are
plain tensors without grad; tokens, scores and LoRA factors carry grads).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import fastcodec


def lora_scale(alpha: float, rank: int, *, use_rslora: bool = False) -> float:
    """mirai/core/models/adapters/lora_allocation.py:163-168."""
    if int(rank) <= 0:
        raise ValueError("LoRA rank must be positive when computing scale.")
    return float(alpha) / (math.sqrt(rank) if use_rslora else float(rank))


def dense_weight(fmt: str, payload, shape, dtype=torch.bfloat16) -> torch.Tensor:
    """Dense [E, out, in] tensor of a stored weight, decoded by the oracle codec
    (the C restatement in oracle/codec.c, equal to oracle/codec.py)."""
    E, out_f, in_f = shape
    if fmt in ("bf16", "fp32"):
        return payload.to(dtype)
    if fmt == "nf4":
        codes, absmax = payload
        bits = fastcodec.nf4_dequantize(
            codes.reshape(E * out_f, in_f // 2), absmax.reshape(E * out_f, in_f // 64)
        )
    elif fmt == "int8":
        q, scale = payload
        bits = fastcodec.int8_dequantize(q.reshape(E * out_f, in_f), scale.reshape(E * out_f))
    else:
        raise ValueError(fmt)
    t = torch.from_numpy(bits.view("int16").reshape(E, out_f, in_f)).view(torch.bfloat16)
    return t.to(dtype)


def _projection(x, weight, lora, e):
    out = x @ weight[e].transpose(-2, -1)
    if lora is not None:
        a, b, scale = lora
        out = out + F.linear(F.linear(x, a[e].to(x.dtype)), b[e].to(x.dtype)) * scale
    return out


def expert_mlp(x, e, weights, loras):
    g = _projection(x, weights["w1"], loras.get("w1"), e)
    u = _projection(x, weights["w3"], loras.get("w3"), e)
    h = F.silu(g) * u
    return _projection(h, weights["w2"], loras.get("w2"), e)


def layer_forward(tokens, top_scores, top_idx, weights, loras, num_experts):
    """[T, d] output of the routed layer (autograd-capable)."""
    output = torch.zeros(tokens.shape, dtype=torch.float32)
    for e in range(num_experts):
        assignments = torch.nonzero(top_idx == e, as_tuple=False)
        if assignments.numel() == 0:
            continue
        tok, slot = assignments[:, 0], assignments[:, 1]
        y = expert_mlp(tokens.index_select(0, tok), e, weights, loras)
        weight = top_scores[tok, slot].float().unsqueeze(1)
        output = output.index_add(0, tok, y.float() * weight)
    return output.to(tokens.dtype)


def for_loop_forward(tokens_sorted, counts, weights, loras):
    """run_for_loop: expert MLP over rows already grouped by expert."""
    outputs = []
    for e, rows in enumerate(torch.split(tokens_sorted, [int(c) for c in counts], dim=0)):
        if rows.numel():
            outputs.append(expert_mlp(rows, e, weights, loras))
    if not outputs:
        return tokens_sorted.new_zeros(tokens_sorted.shape)
    return torch.cat(outputs, dim=0)


def grouped_linear(x, counts, weight, lora=None):
    """One projection over expert-grouped rows (grouped_mm per-group loop)."""
    outputs = []
    for e, rows in enumerate(torch.split(x, [int(c) for c in counts], dim=0)):
        if rows.numel():
            outputs.append(_projection(rows, weight, lora, e))
    return torch.cat(outputs, dim=0) if outputs else x.new_zeros((0, weight.shape[1]))
