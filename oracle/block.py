"""LingBot sparse-MoE block forward, restated (test infrastructure: only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline use oracle/).

LingBotVideoSparseMoeBlock._forward_once
(mirai/vendors/lingbot_video/transformer_lingbot_video.py:2216-2377) without
extensions, on the CPU in the reference's dtypes:

* tokens = hidden_states.view(-1, H)                                      :2228
* routes from the router (oracle.router.router_forward)                   :2267-2273
* with a padding mask: scores * mask, / (sum + 1e-9), * route_scale       :2282-2287
* out = routed expert layer (oracle.layer.layer_forward)                  :2345-2350
* out = out.view(B, -1, H) + shared_experts(hidden_states), where the
  shared expert is LingBotVideoMLP: down(silu(gate(x)) * up(x)) in the
  token dtype                                                              :491-499, 2374-2377
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import layer as olayer
from . import router as orouter


def shared_mlp(x: torch.Tensor, gate: torch.Tensor, up: torch.Tensor,
               down: torch.Tensor) -> torch.Tensor:
    """LingBotVideoMLP.forward (:498-499) with bias-free linears in x's dtype."""
    return F.linear(F.silu(F.linear(x, gate.to(x.dtype))) * F.linear(x, up.to(x.dtype)),
                    down.to(x.dtype))


def block_forward(hidden_states: torch.Tensor, router_weight: torch.Tensor, top_k: int,
                  expert_weights: dict, expert_loras: dict, num_experts: int, *,
                  shared: tuple | None = None, padding_mask: torch.Tensor | None = None,
                  routes: tuple | None = None, **router_kw):
    """[B, S, H] block output; ``routes`` = (top_idx, top_scores) overrides the
    router (to check the composition on given routes). Returns (out, top_idx)."""
    B = int(hidden_states.shape[0])
    H = int(hidden_states.shape[-1])
    tokens = hidden_states.reshape(-1, H)
    if routes is None:
        idx, top, _, _, _ = orouter.router_forward(tokens, router_weight, top_k, **router_kw)
    else:
        idx, top = routes
    if padding_mask is not None:
        pm = padding_mask.reshape(-1, 1).to(top.dtype)
        top = top * pm
        top = top / (top.sum(dim=-1, keepdim=True) + 1e-9)
        top = top * router_kw.get("route_scale", 1.0)
    out = olayer.layer_forward(tokens, top, idx, expert_weights, expert_loras, num_experts)
    out = out.view(B, -1, H)
    if shared is not None:
        out = out + shared_mlp(tokens, *shared).view(B, -1, H)
    return out, idx
