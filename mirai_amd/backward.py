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


def native_backward(module, saved, grad_out, token_dtype, *, need_tokens=True, need_scores=True,
                    lora_needs=None):
    """One mx_moe_backward_act call over the activations ``saved`` by a forward
    of the routed layer (x, scores, idx, gate, up, h, y, low-rank rows).

    Returns (grad_tokens, fp32 for fp32 tokens else bf16; fp32 grad_scores; raw fp32
    LoRA factor gradients at the padded rank: [dA, dB] per adapter, None where
    not wanted or absent)."""
    from .fused import _lora_descriptors, _weight_descriptors, kernel_activation, lora_rank

    x, scores, idx, gate, up, h, y, lora_rows = saved
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
    grad_tokens = torch.empty((T, d), dtype=torch.float32 if token_dtype == torch.float32
                              else torch.bfloat16, device=device)
    grad_scores = torch.empty((T, k), dtype=torch.float32, device=device)
    raw = []
    for i, adapter in enumerate(module._adapters()):
        if adapter is None:
            raw += [None, None]
            continue
        want_a = lora_needs is None or lora_needs[2 * i]
        want_b = lora_needs is None or lora_needs[2 * i + 1]
        r8 = adapter.padded_rank()
        raw.append(torch.empty((E, r8, adapter.in_features), dtype=torch.float32, device=device)
                   if want_a else None)
        raw.append(torch.empty((E, adapter.out_features, r8), dtype=torch.float32, device=device)
                   if want_b else None)
    lib = nat.load_library()
    ws = nat.workspace(lib.mx_moe_backward_workspace_size(T, k, E, d, f, lora_rank(module)),
                       device)
    nat.call("mx_moe_backward_act", g.data_ptr(), nat.dtype_code(g.dtype), x.data_ptr(),
             idx.data_ptr(), scores.data_ptr(), nat.dtype_code(scores.dtype), T, k, E, d, f,
             kernel_activation(module), w1, w3, w2, lora[0], lora[1], lora[2], gate.data_ptr(),
             up.data_ptr(), h.data_ptr(), y.data_ptr(), lora_rows.data_ptr(),
             grad_tokens.data_ptr(),
             nat.dtype_code(grad_tokens.dtype), grad_scores.data_ptr(),
             *[nat.ptr(t) for t in raw], ws.data_ptr(), nat.stream(device))
    del keep
    return (grad_tokens if need_tokens else None, grad_scores if need_scores else None, raw)


def lora_param_grads(module, raw):
    """Raw padded-rank fp32 LoRA gradients -> gradients shaped and typed like
    each adapter's lora_a / lora_b (None where absent)."""
    grads = []
    for i, adapter in enumerate(module._adapters()):
        ga, gb = raw[2 * i], raw[2 * i + 1]
        if adapter is None:
            grads += [None, None]
            continue
        r = adapter.rank
        grads.append(None if ga is None else ga[:, :r, :].to(adapter.lora_a.dtype))
        grads.append(None if gb is None else gb[:, :, :r].contiguous().to(adapter.lora_b.dtype))
    return grads


def routed_experts_backward(ctx, grad_out):
    gt, gs, raw = native_backward(ctx.module, ctx.saved_tensors, grad_out, ctx.token_dtype,
                                  need_tokens=ctx.needs_input_grad[1],
                                  need_scores=ctx.needs_input_grad[2],
                                  lora_needs=ctx.needs_input_grad[4:])
    grad_t = gt.to(ctx.token_dtype) if gt is not None else None
    grad_s = gs.to(ctx.score_dtype) if gs is not None else None
    return (None, grad_t, grad_s, None, *lora_param_grads(ctx.module, raw))


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
