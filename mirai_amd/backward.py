"""Backward of the fused routed expert layer (adapter training, frozen base).

One ``mx_moe_backward_act`` call turns grad_out into grad_tokens, grad_scores and
the fp32 LoRA factor gradients. The frozen weights are decoded again inside
the backward GEMMs (never saved on ctx, never materialised), as the reference's
_FrozenDequantBatchedLinear(Pair).backward re-dequantises
(mirai/core/models/compressed_weights/execution/linear.py:95-125, 192-203).
"""

from __future__ import annotations

import torch

from . import _native as nat


def routed_experts_backward(ctx, grad_out):
    from .fused import _lora_descriptors, _weight_descriptors, kernel_activation

    x, scores, idx, gate, up, h, y, lora_rows = ctx.saved_tensors
    module = ctx.module
    device = x.device
    T, d = (int(v) for v in x.shape)
    k = int(idx.shape[1])
    E = module.num_experts
    (w1, w3, w2), packed = _weight_descriptors(module, device)
    f = int(packed[0].shape[1])
    lora, keep = _lora_descriptors(module, device)
    g = grad_out.contiguous()
    if g.dtype not in (torch.float32, torch.bfloat16):
        g = g.float()
    tok_dtype = torch.float32 if ctx.token_dtype == torch.float32 else torch.bfloat16
    grad_tokens = torch.empty((T, d), dtype=tok_dtype, device=device)
    grad_scores = torch.empty((T, k), dtype=torch.float32, device=device)
    lora_needs = ctx.needs_input_grad[4:]
    raw = []
    for i, adapter in enumerate(module._adapters()):
        if adapter is None:
            raw += [None, None]
            continue
        r8 = adapter.padded_rank()
        ga = (torch.empty((E, r8, adapter.in_features), dtype=torch.float32, device=device)
              if lora_needs[2 * i] else None)
        gb = (torch.empty((E, adapter.out_features, r8), dtype=torch.float32, device=device)
              if lora_needs[2 * i + 1] else None)
        raw += [ga, gb]
    lib = nat.load_library()
    ws = nat.workspace(lib.mx_moe_backward_workspace_size(T, k, E, d, f), device)
    nat.call("mx_moe_backward_act", g.data_ptr(), nat.dtype_code(g.dtype), x.data_ptr(),
             idx.data_ptr(), scores.data_ptr(), nat.dtype_code(scores.dtype), T, k, E, d, f,
             kernel_activation(module), w1, w3, w2, lora[0], lora[1], lora[2], gate.data_ptr(),
             up.data_ptr(), h.data_ptr(), y.data_ptr(), lora_rows.data_ptr(),
             grad_tokens.data_ptr(),
             nat.dtype_code(grad_tokens.dtype), grad_scores.data_ptr(),
             *[nat.ptr(t) for t in raw], ws.data_ptr(), nat.stream(device))
    del keep
    lora_grads = []
    for i, adapter in enumerate(module._adapters()):
        ga, gb = raw[2 * i], raw[2 * i + 1]
        if adapter is None:
            lora_grads += [None, None]
            continue
        r = adapter.rank
        lora_grads.append(None if ga is None else ga[:, :r, :].to(adapter.lora_a.dtype))
        lora_grads.append(None if gb is None else gb[:, :, :r].contiguous().to(adapter.lora_b.dtype))
    grad_t = grad_tokens.to(ctx.token_dtype) if ctx.needs_input_grad[1] else None
    grad_s = grad_scores.to(ctx.score_dtype) if ctx.needs_input_grad[2] else None
    return (None, grad_t, grad_s, None, *lora_grads)


def sorted_experts_autograd(module, tokens, counts):
    """run_for_loop with gradients: rows already grouped by expert are the
    routed layer with top-1 routes (the row's expert) and unit scores."""
    from .fused import routed_experts

    c = counts.detach().to(device=tokens.device, dtype=torch.int64)
    if int(c.numel()) != module.num_experts:
        raise ValueError("counts must hold one entry per expert.")
    S = int(tokens.shape[0])
    idx = torch.repeat_interleave(torch.arange(module.num_experts, device=tokens.device), c)
    if int(idx.numel()) != S:
        raise ValueError(f"counts sum to {int(idx.numel())}, but {S} rows were given.")
    scores = torch.ones((S, 1), dtype=torch.float32, device=tokens.device)
    return routed_experts(module, tokens, scores, idx.view(S, 1))
