"""LingBot sparse-MoE block on the MI355X kernels: fused router front end,
routed experts and the shared expert, overlapped on two streams.

``FusedSparseMoeBlock`` mirrors LingBotVideoSparseMoeBlock
(mirai/vendors/lingbot_video/transformer_lingbot_video.py:1175-1205,
2216-2377) for its standard path (no router / expert extensions): constructor
arguments, submodule names (``router``, ``experts``, ``shared_experts``) and
forward(hidden_states, padding_mask) -> [B, S, H].

Execution in inference:
* the shared expert (a dense SwiGLU MLP over every token, LingBotVideoMLP
  :491-499) starts first on a side stream, as a one-expert layer of the
  grouped kernels;
* the fused router kernel and the routed layer run on the current stream;
* the routed layer's combine waits for the shared expert's event and adds
  its output in the same pass (out = bf16(bf16(routed) + shared), the
  reference's `out + shared_output`, :2374-2377).
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _native as nat
from .chunking import MoETokenChunkPolicy, fused_chunk_runner
from .experts import CompressedGroupedExperts
from .fused import routed_experts, routed_experts_plus, sorted_experts
from .router import FusedRouter


class SharedExpertMLP(nn.Module):
    """LingBotVideoMLP (down(silu(gate(x)) * up(x)), bf16 nn.Linear weights
    gate_proj / up_proj / down_proj) as one expert of the grouped kernels over
    rows already in order (mx_moe_for_loop with one segment of all tokens): no
    plan, no combine, and the gate/up epilogue rounds exactly where the
    reference's bf16 linears and silu do."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)
        self._packed = None
        self._packed_key = None
        self._counts = {}

    def _experts(self) -> CompressedGroupedExperts:
        projs = (self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.device) for w in projs)
        if self._packed is None or self._packed_key != key:
            m = CompressedGroupedExperts.from_empty(num_experts=1, quant_format="bf16",
                                                    expert_weight_access="fused_kernel")
            for name, w in zip(("w1", "w3", "w2"), projs):
                m.load_dense_weight(name, w.detach().to(torch.bfloat16).unsqueeze(0))
            self._packed, self._packed_key = m, key
        return self._packed

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if any(p.requires_grad for p in self.parameters()) and torch.is_grad_enabled():
            raise NotImplementedError(
                "the shared expert runs over frozen weights; freeze gate_proj / up_proj / "
                "down_proj (adapter training) or call it under torch.no_grad()")
        key = (int(x.shape[0]), x.device)
        counts = self._counts.get(key)
        if counts is None:  # one segment of all rows, kept on the device
            counts = self._counts[key] = torch.tensor([key[0]], dtype=torch.int64,
                                                      device=x.device)
        return sorted_experts(self._experts(), x, counts)


class FusedSparseMoeBlock(nn.Module):
    """LingBotVideoSparseMoeBlock's standard forward on the fused kernels."""

    def __init__(self, hidden_size, intermediate_size, num_experts, top_k, moe_intermediate_size,
                 score_func, norm_topk_prob, n_group, topk_group, routed_scaling_factor,
                 n_shared_experts, *, quant_format: str = "nf4"):
        super().__init__()
        del intermediate_size  # the dense MLP width of non-MoE layers
        self.hidden_size = int(hidden_size)
        self.num_experts = int(num_experts)
        self.router = FusedRouter(hidden_size, num_experts, top_k, score_func, norm_topk_prob,
                                  n_group, topk_group, routed_scaling_factor)
        self.experts = CompressedGroupedExperts.from_empty(
            num_experts=num_experts, quant_format=quant_format,
            expert_weight_access="fused_kernel")
        self.shared_experts = None
        if n_shared_experts is not None and n_shared_experts > 0:
            self.shared_experts = SharedExpertMLP(hidden_size,
                                                  moe_intermediate_size * n_shared_experts)
        self._mirai_token_chunk_policy = None
        self._side_streams = {}

    def set_token_chunk_policy(self, policy: MoETokenChunkPolicy | None) -> None:
        self._mirai_token_chunk_policy = policy

    def _side_stream(self, device: torch.device) -> torch.cuda.Stream:
        if device not in self._side_streams:
            self._side_streams[device] = torch.cuda.Stream(device=device)  # default priority
        return self._side_streams[device]

    def _routes(self, tokens, padding_mask, router_logit_delta):
        # Live tokens, as the reference routes them (:2259-2264): in training
        # the gating scores carry the router's gradient to the tokens and the
        # router weight.
        top_indices, top_scores, _, _, _ = self.router(tokens, logit_delta=router_logit_delta)
        if padding_mask is not None:  # :2282-2287
            pm = padding_mask.reshape(-1, 1).to(top_scores.dtype)
            top_scores = top_scores * pm
            top_scores = top_scores / (top_scores.sum(dim=-1, keepdim=True) + 1e-9)
            top_scores = top_scores * self.router.route_scale
        return top_indices, top_scores

    def forward(self, hidden_states: torch.Tensor, padding_mask: torch.Tensor | None = None,
                router_logit_delta: torch.Tensor | None = None) -> torch.Tensor:
        B = int(hidden_states.shape[0])
        tokens = hidden_states.reshape(-1, self.hidden_size)
        device = nat.require_gpu(tokens)
        grad = torch.is_grad_enabled() and (
            tokens.requires_grad or any(p.requires_grad for p in self.experts.parameters())
            or self.router.weight.requires_grad)

        shared, ready = None, None
        if self.shared_experts is not None:
            main = torch.cuda.current_stream(device)
            side = self._side_stream(device)
            side.wait_stream(main)
            with torch.cuda.stream(side):
                shared = self.shared_experts(tokens)
                ready = torch.cuda.Event()
                ready.record(side)
            tokens.record_stream(side)
            shared.record_stream(main)

        top_indices, top_scores = self._routes(tokens, padding_mask, router_logit_delta)
        policy = self._mirai_token_chunk_policy
        if policy is not None and policy.enabled and grad:
            out = policy.execute(tokens, top_scores, top_indices,
                                 runner=fused_chunk_runner(self.experts), training=self.training)
            if shared is not None:
                torch.cuda.current_stream(device).wait_event(ready)
                out = out + shared
        elif shared is not None:
            out = routed_experts_plus(self.experts, tokens, top_scores, top_indices, shared, ready)
        else:
            out = routed_experts(self.experts, tokens, top_scores, top_indices)
        return out.view(B, -1, self.hidden_size)
