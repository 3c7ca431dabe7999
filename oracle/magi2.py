"""MAGI-2 multi-head MoE: routing, swiglu7 and the routed expert MLP, restated
on the CPU -- TEST INFRASTRUCTURE ONLY (the checker for the HIP path; the
product package never imports it).

* Routing follows _compute_topk_probs_and_indices_torch_impl
  (mirai/vendors/magi2_preview/flash_mh_moe/route.py:28-148): scores =
  softmax or sigmoid of the [H, S, E] logits, experts picked by score +
  expert_bias[h] (selection only), within the best virtual groups when
  num_virtual_group > 1 (route.py:62-105), probabilities
  gathered from the unbiased scores and L1-normalised with eps when
  route_norm; CoreMultiHeadMoE._route then multiplies by route_scale
  (mirai/vendors/magi2_preview/model/magi2_preview.py:2727-2743). Selection
  order is canonical: larger biased score first, ties to the lower expert id.
* swiglu7 follows _memory_bounded_swiglu7 and its backward
  (mirai/core/models/magi2_preview/grouped_moe.py:287-335).
* The layer follows Magi2GroupedMoEBackend._execute_routed_chunk
  (grouped_moe.py:639-756) on the grouped bf16 path: rows are (token, head)
  pairs s*H+h, groups the flattened (head, expert) pairs h*E+e; gate and up
  are bf16 projections with the [G, in, out] weights (x @ W[g]), hidden =
  bf16(swiglu7(gate, up)), the down projection is bf16, and the output is the
  index_add of bf16(y * bf16(prob)) in bf16 over the stable expert order.
  Optional expert LoRA deltas are added to the bf16 projection outputs as in
  the SwiGLU layer oracle (oracle/layer.py).
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

SCORE_SOFTMAX, SCORE_SIGMOID = "softmax", "sigmoid"


def _scores(logits: torch.Tensor, score_func: str) -> torch.Tensor:
    if score_func == SCORE_SOFTMAX:
        return F.softmax(logits, dim=-1)
    if score_func == SCORE_SIGMOID:
        return torch.sigmoid(logits)
    raise ValueError(score_func)


def virtual_group_keys(keys: torch.Tensor, num_virtual_group: int,
                       topk_virtual_group: int) -> torch.Tensor:
    """route.py:62-105: each of the num_virtual_group groups of consecutive
    experts scores the sum of its two largest keys (its largest when it holds
    one expert); the topk_virtual_group best groups keep their keys (ties to
    the lower group id), all other keys become 0.0."""
    H, S, E = keys.shape
    G = int(num_virtual_group)
    epg = E // G
    gs = keys.reshape(H, S, G, epg).topk(min(2, epg), dim=-1)[0].sum(dim=-1)
    keep = np.argsort(-gs.numpy(), axis=-1, kind="stable")[..., :topk_virtual_group]
    gmask = np.zeros((H, S, G), dtype=bool)
    np.put_along_axis(gmask, keep, True, axis=-1)
    emask = torch.from_numpy(np.repeat(gmask, epg, axis=-1))
    return keys.masked_fill(~emask, 0.0)


def route_topk_heads(router_logits: torch.Tensor, top_k: int, *, score_func: str = "sigmoid",
                     expert_bias: torch.Tensor | None = None, route_norm: bool = True,
                     norm_eps: float = 1e-12, route_scale: float = 1.0,
                     num_virtual_group: int = 1, topk_virtual_group: int = 0):
    """Return (probs [H,S,k] fp32, indices [H,S,k] int64), slots in selection order."""
    logits = router_logits.detach().float()
    scores = _scores(logits, score_func)
    keys = scores if expert_bias is None else scores + expert_bias.float().view(
        logits.shape[0], 1, logits.shape[2])
    if num_virtual_group > 1:
        keys = virtual_group_keys(keys, num_virtual_group, topk_virtual_group)
    H, S, E = keys.shape
    kn = keys.numpy().reshape(H * S, E)
    # Canonical order: descending key, ties to the lower expert id (stable).
    order = np.argsort(-kn, axis=1, kind="stable")[:, :top_k]
    idx = torch.from_numpy(order.astype(np.int64)).view(H, S, top_k)
    probs = scores.gather(-1, idx)
    if route_norm:
        probs = F.normalize(probs, p=1, dim=-1, eps=norm_eps)
    return probs * route_scale, idx


def route_probs_for_picks(router_logits: torch.Tensor, idx: torch.Tensor, *,
                          score_func: str = "sigmoid", route_norm: bool = True,
                          norm_eps: float = 1e-12, route_scale: float = 1.0) -> torch.Tensor:
    """The probabilities of given picks idx [H,S,k] as torch ops on the logits
    (autograd-capable; route.py:115-147 and the `* route_scale` of
    magi2_preview.py:2741): the backward oracle of the routing."""
    z = router_logits.to(torch.promote_types(router_logits.dtype, torch.float32))
    probs = _scores(z, score_func).gather(-1, idx)
    if route_norm:
        probs = F.normalize(probs, p=1, dim=-1, eps=norm_eps)
    return probs * route_scale


def heads_to_rows(probs: torch.Tensor, idx: torch.Tensor, num_experts: int):
    """[H,S,k] per-head routes -> [S*H, k] rows (s*H+h) with group ids h*E+e."""
    H, S, K = idx.shape
    flat = idx + torch.arange(H).view(H, 1, 1) * num_experts
    return probs.permute(1, 0, 2).reshape(S * H, K), flat.permute(1, 0, 2).reshape(S * H, K)


def swiglu7(gate: torch.Tensor, up: torch.Tensor, out_dtype=torch.bfloat16) -> torch.Tensor:
    """bf16 (or any) gate / up -> out_dtype, computed in fp32 (grouped_moe.py:287-306)."""
    g = gate.float().clamp(max=7.0)
    u = up.float().clamp(min=-7.0, max=7.0)
    h = g * torch.sigmoid(1.702 * g)
    return (h * (u + 1.0)).to(out_dtype)


def swiglu7_backward(gate: torch.Tensor, up: torch.Tensor, grad_out: torch.Tensor):
    """(d gate, d up) in the gate / up dtype (grouped_moe.py:309-335)."""
    raw_g, raw_u = gate.float(), up.float()
    g = raw_g.clamp(max=7.0)
    u = raw_u.clamp(min=-7.0, max=7.0)
    s = torch.sigmoid(1.702 * g)
    gd = (s + (1.702 * g * s * (1.0 - s))) * (raw_g <= 7.0)
    dh = grad_out.float()
    dg = dh * gd * (u + 1.0)
    du = dh * (g * s) * ((raw_u >= -7.0) & (raw_u <= 7.0))
    return dg.to(gate.dtype), du.to(up.dtype)


class _Swiglu7(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gate, up):
        ctx.save_for_backward(gate, up)
        return swiglu7(gate, up, gate.dtype)

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        return swiglu7_backward(gate, up, grad)


def _projection(x, weight, lora, g):
    out = x @ weight[g].to(x.dtype)  # [G, in, out]: no transpose
    if lora is not None:
        a, b, scale = lora
        out = out + F.linear(F.linear(x, a[g].to(x.dtype)), b[g].to(x.dtype)) * scale
    return out


def layer_forward(x_heads: torch.Tensor, probs: torch.Tensor, idx: torch.Tensor, weights: dict,
                  num_experts: int, loras: dict | None = None) -> torch.Tensor:
    """[S, H, d_head] output of the MAGI-2 routed experts (autograd-capable).

    weights: W_gate / W_up [G, d_head, d_expert], W_down [G, d_expert, d_head]
    in the activation dtype; loras: optional {key: (A [G, r, in], B [G, out, r],
    scale)} per weight key.
    """
    loras = loras or {}
    S, H, d = x_heads.shape
    rows = x_heads.reshape(S * H, d)
    p_rows, g_rows = heads_to_rows(probs, idx, num_experts)
    K = int(g_rows.shape[1])
    out = torch.zeros((S * H, d), dtype=x_heads.dtype)
    flat = g_rows.reshape(-1)
    order = torch.argsort(flat, stable=True)
    sorted_groups = flat[order]
    for g in torch.unique(sorted_groups).tolist():
        pos = order[sorted_groups == g]
        r = pos // K
        xg = rows.index_select(0, r)
        gate = _projection(xg, weights["W_gate"], loras.get("W_gate"), g)
        up = _projection(xg, weights["W_up"], loras.get("W_up"), g)
        hidden = _Swiglu7.apply(gate, up)
        y = _projection(hidden, weights["W_down"], loras.get("W_down"), g)
        weighted = y * p_rows.reshape(-1)[pos].to(y.dtype).unsqueeze(1)
        out = out.index_add(0, r, weighted.to(out.dtype))
    return out.view(S, H, d)


def layer_forward_fp64(x_heads, probs, idx, weights, num_experts) -> torch.Tensor:
    """Independent per-(token, head, slot) formulation in fp64 without rounding."""
    S, H, d = x_heads.shape
    K = int(idx.shape[2])
    out = torch.zeros((S, H, d), dtype=torch.float64)
    wg, wu, wd = (weights[k].double() for k in ("W_gate", "W_up", "W_down"))
    for h in range(H):
        for s in range(S):
            x = x_heads[s, h].double()
            for j in range(K):
                g = h * num_experts + int(idx[h, s, j])
                gate = (x @ wg[g]).clamp(max=7.0)
                up = (x @ wu[g]).clamp(min=-7.0, max=7.0)
                hid = gate * torch.sigmoid(1.702 * gate) * (up + 1.0)
                out[s, h] += float(probs[h, s, j]) * (hid @ wd[g])
    return out
