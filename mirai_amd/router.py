"""Fused router front end on the MI355X kernels.

``FusedRouter`` is a drop-in for LingBotVideoRouter's standard path
(mirai/vendors/lingbot_video/transformer_lingbot_video.py:502-560, 962-1033):
same constructor arguments, parameter and buffer names (``weight`` [E, d]
fp32, ``e_score_correction_bias`` [E]), same forward signature and return
tuple. One HIP kernel (mx_router_forward) computes the fp32 router GEMM, the
softmax / sigmoid scores, the bias-steered (optionally group-limited) top-k
selection, the renormalisation and route_scale; the logits and scores come
out of the same pass. In training the gating scores carry gradients back to
the tokens, the router weight and the logit delta (``_FusedRouterFn``).
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _native as nat

SCORE_FUNCS = {"softmax": nat.SCORE_SOFTMAX, "sigmoid": nat.SCORE_SIGMOID}


def router_weight_planes(weight: torch.Tensor) -> torch.Tensor:
    """bf16 planes [3, EP, d] (as uint8 bytes) with weight == hi + mid + lo exactly."""
    if weight.ndim != 2:
        raise ValueError("router weight must be [num_experts, hidden].")
    E, d = (int(v) for v in weight.shape)
    device = nat.require_gpu(weight)
    size = int(nat.load_library().mx_router_planes_size(E, d))
    if size == 0 or d % 64:
        raise ValueError("router weight needs 1 <= num_experts <= 256 and hidden % 64 == 0.")
    w = weight.detach().to(device=device, dtype=torch.float32).contiguous()
    planes = torch.empty(size, dtype=torch.uint8, device=device)
    nat.call("mx_router_weight_planes", w.data_ptr(), E, d, planes.data_ptr(), nat.stream(device))
    return planes


def fused_router_forward(tokens: torch.Tensor, planes: torch.Tensor, num_experts: int,
                         top_k: int, *, score_func: str = "sigmoid",
                         expert_bias: torch.Tensor | None = None,
                         logit_delta: torch.Tensor | None = None, norm_topk_prob: bool = True,
                         n_group: int | None = None, topk_group: int | None = None,
                         route_scale: float = 1.0, return_logits: bool = True,
                         return_scores: bool = True, score_dtype: torch.dtype | None = None):
    """tokens [T, d] (bf16 or fp32) -> (top_idx [T, k] int64, top_scores [T, k],
    logits [T, E] fp32 or None, scores [T, E] fp32 or None)."""
    if tokens.ndim != 2:
        raise ValueError("tokens must be [num_tokens, hidden].")
    if score_func not in SCORE_FUNCS:
        raise ValueError(f"Unknown score_func: {score_func}")
    if tokens.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("router tokens must be bf16 or fp32.")
    device = nat.require_gpu(tokens)
    T, d = (int(v) for v in tokens.shape)
    E, k = int(num_experts), int(top_k)
    x = tokens.detach().contiguous()
    score_dtype = tokens.dtype if score_dtype is None else score_dtype
    idx = torch.empty((T, k), dtype=torch.int64, device=device)
    top = torch.empty((T, k), dtype=score_dtype, device=device)
    logits = torch.empty((T, E), dtype=torch.float32, device=device) if return_logits else None
    scores = torch.empty((T, E), dtype=torch.float32, device=device) if return_scores else None
    bias = None
    if expert_bias is not None:
        bias = expert_bias.detach().to(device=device, dtype=torch.float32).reshape(E).contiguous()
    delta = None
    if logit_delta is not None:
        if tuple(logit_delta.shape) != (T, E):
            raise ValueError("Router logit delta must match the native router logits shape.")
        delta = logit_delta.detach().to(device=device, dtype=torch.float32).contiguous()
    groups = int(n_group) if n_group is not None else 1
    nat.call("mx_router_forward", x.data_ptr(), nat.dtype_code(x.dtype), T, d, E,
             planes.data_ptr(), nat.ptr(bias), nat.ptr(delta), k, SCORE_FUNCS[score_func],
             groups, int(topk_group) if topk_group is not None else groups,
             int(bool(norm_topk_prob)), float(route_scale), nat.ptr(logits), nat.ptr(scores),
             idx.data_ptr(), top.data_ptr(), nat.dtype_code(score_dtype), nat.stream(device))
    return idx, top, logits, scores


def router_scores_backward(logits: torch.Tensor, top_idx: torch.Tensor, grad_top: torch.Tensor,
                           *, score_func: str, renorm: int, renorm_floor: float,
                           route_scale: float) -> torch.Tensor:
    """d(logits) [rows, E] fp32 from d(top_scores) [rows, k] (mx_route_scores_backward)."""
    device = nat.require_gpu(logits, top_idx, grad_top)
    rows, E = (int(v) for v in logits.shape)
    k = int(top_idx.shape[-1])
    lg = logits.detach().float().contiguous()
    idx = top_idx.detach().to(torch.int64).reshape(rows, k).contiguous()
    g = grad_top.detach().float().reshape(rows, k).contiguous()
    out = torch.empty((rows, E), dtype=torch.float32, device=device)
    nat.call("mx_route_scores_backward", lg.data_ptr(), rows, E, k, SCORE_FUNCS[score_func],
             int(renorm), float(renorm_floor), float(route_scale), idx.data_ptr(), g.data_ptr(),
             out.data_ptr(), nat.stream(device))
    return out


class _FusedRouterFn(torch.autograd.Function):
    """The fused router with gradients through the gating scores: d top_scores
    -> d logits (softmax / sigmoid Jacobian through the `/ (sum + 1e-20)`
    renormalisation and route_scale, mx_route_scores_backward), then the fp32
    router GEMM's d tokens = d logits . W, d W = d logits^T . tokens.float()
    and d logit_delta = d logits: the autograd of LingBotVideoRouter.forward
    (transformer_lingbot_video.py:975-1033). Indices, logits and scores are
    returned without gradients."""

    @staticmethod
    def forward(ctx, router, tokens, weight, logit_delta):
        idx, top, logits, scores = fused_router_forward(
            tokens, router.weight_planes(), router.num_experts, router.top_k,
            score_func=router.score_func, expert_bias=router.e_score_correction_bias,
            logit_delta=logit_delta, norm_topk_prob=router.norm_topk_prob, n_group=router.n_group,
            topk_group=router.topk_group, route_scale=router.route_scale)
        ctx.mark_non_differentiable(idx, logits, scores)
        ctx.cfg = (router.score_func, router.top_k > 1 and router.norm_topk_prob,
                   float(router.route_scale), tokens.dtype)
        ctx.save_for_backward(tokens, weight, logits, idx)
        return idx, top, logits, scores

    @staticmethod
    def backward(ctx, _g_idx, g_top, _g_logits, _g_scores):
        tokens, weight, logits, idx = ctx.saved_tensors
        score_func, renorm, route_scale, token_dtype = ctx.cfg
        if g_top is None:
            return None, None, None, None
        dl = router_scores_backward(logits, idx, g_top, score_func=score_func,
                                    renorm=nat.RENORM_EPS if renorm else nat.RENORM_NONE,
                                    renorm_floor=1e-20, route_scale=route_scale)
        g_tokens = g_weight = g_delta = None
        if ctx.needs_input_grad[1]:
            g_tokens = (dl @ weight.detach().float()).to(token_dtype)
        if ctx.needs_input_grad[2]:
            g_weight = (dl.t() @ tokens.detach().float()).to(weight.dtype)
        if ctx.needs_input_grad[3]:
            g_delta = dl
        return None, g_tokens, g_weight, g_delta


class FusedRouter(nn.Module):
    """LingBotVideoRouter's standard path as one kernel, with its backward.

    The asymmetry of the reference is kept: selection uses the bias-added
    score, the gating weights gather the bias-free score.
    """

    def __init__(self, hidden_size, num_experts, top_k, score_func, norm_topk_prob, n_group,
                 topk_group, route_scale):
        super().__init__()
        if score_func not in SCORE_FUNCS:
            raise ValueError(f"Unknown score_func: {score_func}")
        if int(num_experts) > nat.ROUTER_MAX_EXPERTS:
            raise ValueError(f"FusedRouter takes up to {nat.ROUTER_MAX_EXPERTS} experts.")
        self.num_experts = int(num_experts)
        self.top_k = int(top_k)
        self.score_func = score_func
        self.norm_topk_prob = bool(norm_topk_prob)
        self.n_group = n_group
        self.topk_group = topk_group
        self.route_scale = route_scale
        self.weight = nn.Parameter(torch.empty(num_experts, hidden_size))
        self.register_buffer("e_score_correction_bias", torch.zeros(num_experts), persistent=True)
        self._planes = None
        self._planes_key = None
        self.last_top_indices = None
        self.last_top_scores = None
        self.last_scores = None

    @classmethod
    def from_router(cls, router: nn.Module) -> "FusedRouter":
        """Build from a LingBotVideoRouter-like module (same attribute names)."""
        hidden = int(router.weight.shape[1])
        fused = cls(hidden, router.num_experts, router.top_k, router.score_func,
                    router.norm_topk_prob, router.n_group, router.topk_group, router.route_scale)
        fused.to(router.weight.device)
        with torch.no_grad():
            fused.weight.copy_(router.weight.float())
            fused.e_score_correction_bias.copy_(router.e_score_correction_bias.float())
        return fused

    def weight_planes(self) -> torch.Tensor:
        """The split weight, rebuilt whenever ``weight`` changes."""
        w = self.weight
        key = (w.data_ptr(), w._version, w.device)
        if self._planes is None or self._planes_key != key:
            self._planes = router_weight_planes(w)
            self._planes_key = key
        return self._planes

    def forward(self, tokens: torch.Tensor, *, logit_delta: torch.Tensor | None = None,
                valid_token_mask: torch.Tensor | None = None,
                route_scope_mask: torch.Tensor | None = None):
        """Returns (top_indices, top_scores in tokens' dtype, logits, scores,
        scores_for_choice), as the reference does (:1132). When tokens, the
        router weight or logit_delta require a gradient, top_scores carries
        one back to them (the other outputs are returned without gradients)."""
        del valid_token_mask, route_scope_mask  # consumed by extensions only
        if torch.is_grad_enabled() and any(
                t is not None and t.requires_grad for t in (tokens, self.weight, logit_delta)):
            idx, top, logits, scores = _FusedRouterFn.apply(self, tokens, self.weight,
                                                             logit_delta)
            choice = scores + self.e_score_correction_bias.float().unsqueeze(0)
            self.last_top_indices = idx
            self.last_top_scores = top.detach()
            self.last_scores = scores
            return idx, top, logits, scores, choice
        idx, top, logits, scores = fused_router_forward(
            tokens, self.weight_planes(), self.num_experts, self.top_k,
            score_func=self.score_func, expert_bias=self.e_score_correction_bias,
            logit_delta=logit_delta, norm_topk_prob=self.norm_topk_prob, n_group=self.n_group,
            topk_group=self.topk_group, route_scale=self.route_scale)
        choice = scores + self.e_score_correction_bias.float().unsqueeze(0)
        self.last_top_indices = idx
        self.last_top_scores = top
        self.last_scores = scores
        return idx, top, logits, scores, choice
