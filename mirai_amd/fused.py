"""Autograd wrappers that drive the fused HIP expert kernels.

Forward: one ``mx_moe_forward_act`` call (plan, gate/up GEMM + LoRA + SwiGLU, down
GEMM + LoRA, combine). When gradients are needed it also keeps the bf16
pre-activations, the SwiGLU output, the per-slot expert outputs and the scaled
low-rank activations for the backward; frozen weights are never saved -- the
backward re-decodes them from the packed buffers, as the reference's
_FrozenDequant*Linear.backward does (linear.py:95-125).
"""

from __future__ import annotations

import torch

from . import _native as nat



def lora_rank(module) -> int:
    """Largest padded rank of the attached adapters (0 without LoRA): the
    ``lora_rank`` the native workspace queries are sized for."""
    return max((a.padded_rank() for a in module._adapters() if a is not None), default=0)


def lora_row(module) -> int:
    """Columns of one saved low-rank row: [gate | up | down] planes of the
    largest rank rounded up to 32 (at least 32 columns each)."""
    return 3 * max(32, -(-lora_rank(module) // 32) * 32)


def kernel_activation(module) -> int:
    """Expert activation of the fused kernels: SwiGLU (the canonical packed
    expert MLP) unless a wrapper such as the MAGI-2 experts selects swiglu7;
    with ACT_FLAG_BF16_COMBINE when the module combines in bf16 like the
    reference's MAGI-2 backend (``_combine_bf16_terms``)."""
    act = int(getattr(module, "_kernel_activation", nat.ACT_SILU))
    if getattr(module, "_combine_bf16_terms", False):
        act |= nat.ACT_FLAG_BF16_COMBINE
    return act


def _lora_descriptors(module, device, split=False):
    """MxLora structs for (gate, up, down) plus the bf16 factor tensors they point to."""
    descs, keep = [], []
    for adapter in module._adapters():
        if adapter is None:
            descs.append(nat.MxLora(None, None, 0, 0.0))
            continue
        a, b = adapter.kernel_factors(device, split=split)
        keep += [a, b]
        descs.append(nat.MxLora(a.data_ptr(), b.data_ptr(), adapter.padded_rank(),
                                float(adapter.scale())))
    return descs, keep


def _weight_descriptors(module, device):
    packed = [module.packed_weight(k) for k in module._role_keys()]
    for p in packed:
        if p.data.device != device:
            raise ValueError(
                f"expert weights live on {p.data.device}, activations on {device}; "
                "move the module with .to(device)")
    return [p.descriptor() for p in packed], packed


def _lora_params(module):
    params = []
    for adapter in module._adapters():
        params += [None, None] if adapter is None else [adapter.lora_a, adapter.lora_b]
    return params


def _forward(module, tokens, top_scores, top_indices, need_grad, addend=None, addend_ready=None,
             out=None):
    """One mx_moe_forward call; returns (out, saved tensors or None). With an
    addend [T, d] (bf16) the combine adds it to the rounded routed sum, after
    waiting for the event ``addend_ready`` (torch.cuda.Event or None). ``out``
    (contiguous, the kernel's output dtype) receives the result in place."""
    device = nat.require_gpu(tokens, top_scores, top_indices)
    nat.poll_route_errors()
    # fp32 weights (quant_format "fp32") run the split-precision layer on
    # fp32 tokens; the other formats take bf16 tokens.
    split = module.quant_format == "fp32"
    x = tokens.detach().to(torch.float32 if split else torch.bfloat16).contiguous()
    scores = top_scores.detach()
    if scores.dtype not in (torch.float32, torch.bfloat16):
        scores = scores.float()
    scores = scores.contiguous()
    idx = top_indices.detach().to(torch.int64).contiguous()
    T, d = (int(v) for v in x.shape)
    k = int(idx.shape[1])
    E = module.num_experts
    (w1, w3, w2), packed = _weight_descriptors(module, device)
    f = int(packed[0].shape[1])
    lora, keep = _lora_descriptors(module, device, split)
    out_dtype = tokens.dtype if tokens.dtype == torch.float32 else torch.bfloat16
    if out is None:
        out = torch.empty((T, d), dtype=out_dtype, device=device)
    elif out.dtype != out_dtype or tuple(out.shape) != (T, d) or not out.is_contiguous():
        raise ValueError("out must be a contiguous [tokens, hidden] tensor of the kernel's dtype.")
    if need_grad and split:
        raise NotImplementedError(
            "the fp32 (quant_format='fp32') expert layer is inference-only; train adapters "
            "over bf16, nf4 or int8 weights")
    R = T * k
    saves = [None] * 5
    if need_grad:
        saves = [
            torch.empty((R, f), dtype=torch.bfloat16, device=device),  # gate
            torch.empty((R, f), dtype=torch.bfloat16, device=device),  # up
            torch.empty((R, f), dtype=torch.bfloat16, device=device),  # h
            torch.empty((R, d), dtype=torch.bfloat16, device=device),  # y (slot order)
            torch.zeros((R, lora_row(module)), dtype=torch.bfloat16, device=device),
        ]
    lib = nat.load_library()
    if split:
        ws = nat.workspace(lib.mx_moe_f32x3_workspace_size(T, k, E, d, f), device)
    else:
        ws = nat.workspace(lib.mx_moe_workspace_size(T, k, E, d, f, lora_rank(module)), device)
    if addend is not None:
        if need_grad or split or addend.dtype != out.dtype or tuple(addend.shape) != (T, d):
            raise ValueError("the fused addend is a bf16 [tokens, hidden] inference input.")
        addend = addend.contiguous()
    nat.call("mx_moe_forward_ex", x.data_ptr(), idx.data_ptr(), scores.data_ptr(),
             nat.dtype_code(scores.dtype), T, k, E, d, f, kernel_activation(module), w1, w3, w2,
             lora[0], lora[1], lora[2], out.data_ptr(), nat.dtype_code(out.dtype),
             nat.ptr(addend), addend_ready.cuda_event if addend_ready is not None else None,
             *[nat.ptr(t) for t in saves], ws.data_ptr(), nat.stream(device))
    del keep
    if T > 0:  # a call with no tokens builds no plan (and writes no error count)
        nat.watch_plan_errors(ws, device, "a routed expert layer call")
    return out.to(tokens.dtype), ((x, scores, idx, *saves) if need_grad else None)


class _RoutedExperts(torch.autograd.Function):
    @staticmethod
    def forward(ctx, module, tokens, top_scores, top_indices, *lora_params):
        out, saved = _forward(module, tokens, top_scores, top_indices, True)
        ctx.module = module
        ctx.token_dtype = tokens.dtype
        ctx.score_dtype = top_scores.dtype
        ctx.save_for_backward(*saved)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        from .backward import routed_experts_backward
        return routed_experts_backward(ctx, grad_out)


def fp32_layer_composition(module, tokens, scores, idx, loras):
    """The routed layer over fp32 weights as torch fp32 ops on the GPU, for
    its backward: per expert g = x W1^T + s1 (x A1^T) B1^T, u likewise with W3,
    h = act(g, u), y = h W2^T + s2 (h A2^T) B2^T, and out[t] the score-weighted
    sum over the token's experts (experts.py:1749-1912 on fp32 tensors, no
    intermediate rounding). The weights are the stored planes' hi + lo, the
    values the split-precision kernels multiply. ``loras``: (A, B, scale) or
    None per role (gate, up, down). Route slots outside [0, E) contribute
    nothing."""
    from . import quant

    E = module.num_experts
    w1, w3, w2 = (quant.dequantize(module.packed_weight(k), dtype=torch.float32)
                  for k in module._role_keys())
    act = int(getattr(module, "_kernel_activation", nat.ACT_SILU))
    T, k = (int(v) for v in idx.shape)
    flat = idx.reshape(-1)
    token_of = torch.arange(T * k, device=idx.device) // k
    sflat = scores.reshape(-1).float()
    x = tokens.float()
    out = torch.zeros((T, int(x.shape[1])), dtype=torch.float32, device=x.device)

    def proj(inp, w, lora, e):
        y = inp @ w[e].t()
        if lora is not None:
            a, b, sc = lora
            y = y + sc * ((inp @ a[e].t()) @ b[e].t())
        return y

    for e in range(E):
        sel = (flat == e).nonzero().squeeze(1)
        if sel.numel() == 0:
            continue
        rows = token_of[sel]
        xs = x[rows]
        g = proj(xs, w1, loras[0], e)
        u = proj(xs, w3, loras[1], e)
        if act == nat.ACT_SWIGLU7:
            # clamp(g, max=7) * sigmoid(1.702 clamp(g)) * (clamp(u, -7, 7) + 1)
            gc = g.clamp(max=7.0)
            h = gc * torch.sigmoid(1.702 * gc) * (u.clamp(-7.0, 7.0) + 1.0)
        else:
            h = torch.nn.functional.silu(g) * u
        y = proj(h, w2, loras[2], e)
        out = out.index_add(0, rows, y * sflat[sel].unsqueeze(1))
    return out


class _Fp32RoutedExperts(torch.autograd.Function):
    """The layer over fp32 weights under autograd. The forward is the
    split-precision kernel layer; the backward recomputes the layer as
    fp32_layer_composition (torch fp32 on the GPU, the same stored weights) and
    differentiates it: gradients to the tokens, the scores and the LoRA
    factors, with the reference's fp32 arithmetic."""

    @staticmethod
    def forward(ctx, module, tokens, top_scores, top_indices, *lora_params):
        out, _ = _forward(module, tokens, top_scores, top_indices, False)
        ctx.module = module
        ctx.save_for_backward(tokens, top_scores, top_indices)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        tokens, scores, idx = ctx.saved_tensors
        needs = ctx.needs_input_grad
        with torch.enable_grad():
            t = tokens.detach().float().requires_grad_(needs[1])
            s = scores.detach().float().requires_grad_(needs[2])
            leaves, loras = [], []
            for i, adapter in enumerate(ctx.module._adapters()):
                if adapter is None:
                    loras.append(None)
                    leaves += [None, None]
                    continue
                a = adapter.lora_a.detach().float().requires_grad_(needs[4 + 2 * i])
                b = adapter.lora_b.detach().float().requires_grad_(needs[5 + 2 * i])
                loras.append((a, b, float(adapter.scale())))
                leaves += [a, b]
            out = fp32_layer_composition(ctx.module, t, s, idx, loras)
            wrt = [v for v in (t, s, *leaves) if v is not None and v.requires_grad]
            got = torch.autograd.grad(out, wrt, grad_out.float(), allow_unused=True) if wrt else ()
        it = iter(got)

        def take(v, like):
            if v is None or not v.requires_grad:
                return None
            g = next(it)
            if g is None:
                g = torch.zeros_like(v)
            return g.to(like.dtype)

        grad_t = take(t, tokens)
        grad_s = take(s, scores)
        params = _lora_params(ctx.module)
        grad_l = [take(v, p) if p is not None else None for v, p in zip(leaves, params)]
        return (None, grad_t, grad_s, None, *grad_l)


def routed_experts(module, tokens, top_scores, top_indices):
    """The routed layer; with autograd only when a gradient can flow (in
    inference nothing is saved for a backward)."""
    params = _lora_params(module)
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (tokens, top_scores, *params)):
        if module.quant_format == "fp32":
            return _Fp32RoutedExperts.apply(module, tokens, top_scores, top_indices, *params)
        return _RoutedExperts.apply(module, tokens, top_scores, top_indices, *params)
    return _forward(module, tokens, top_scores, top_indices, False)[0]


class _ChunkedRoutedExperts(torch.autograd.Function):
    """The routed layer over contiguous token chunks, checkpointed at the native
    call boundary.

    The forward runs each chunk through the inference kernels (no activation
    is kept) straight into its rows of the output. The backward walks the
    chunks in order: it reruns a chunk's forward with its per-slot activations
    saved ((3f + d + 3 rc) * 2 bytes per routed slot, rc the LoRA row plane), runs that chunk's native
    backward, writes the chunk's token and score gradients into their rows and
    adds its fp32 LoRA factor gradients to running sums, then frees the chunk's
    activations. At most one chunk's activations are alive at a time; the
    layer is deterministic, so the recomputation reproduces the forward
    exactly (there is no RNG state to carry)."""

    @staticmethod
    def forward(ctx, module, bounds, tokens, top_scores, top_indices, *lora_params):
        T, d = (int(v) for v in tokens.shape)
        out_dtype = tokens.dtype if tokens.dtype == torch.float32 else torch.bfloat16
        out = torch.empty((T, d), dtype=out_dtype, device=tokens.device)
        for a, b in bounds:
            _forward(module, tokens[a:b], top_scores[a:b], top_indices[a:b], False, out=out[a:b])
        ctx.module = module
        ctx.bounds = bounds
        ctx.token_dtype = tokens.dtype
        ctx.score_dtype = top_scores.dtype
        ctx.save_for_backward(tokens, top_scores, top_indices)
        return out.to(tokens.dtype)

    @staticmethod
    def backward(ctx, grad_out):
        from .backward import lora_param_grads, native_backward

        tokens, scores, idx = ctx.saved_tensors
        need_t, need_s = ctx.needs_input_grad[2], ctx.needs_input_grad[3]
        lora_needs = ctx.needs_input_grad[5:]
        grad_t = torch.empty(tokens.shape, dtype=ctx.token_dtype, device=tokens.device) if need_t else None
        grad_s = torch.empty(scores.shape, dtype=ctx.score_dtype, device=scores.device) if need_s else None
        lora_sum = None
        for a, b in ctx.bounds:
            _, saved = _forward(ctx.module, tokens[a:b], scores[a:b], idx[a:b], True)
            gt, gs, raw = native_backward(ctx.module, saved, grad_out[a:b], ctx.token_dtype,
                                          need_tokens=need_t, need_scores=need_s,
                                          lora_needs=lora_needs)
            del saved
            if need_t:
                grad_t[a:b] = gt
            if need_s:
                grad_s[a:b] = gs
            lora_sum = raw if lora_sum is None else [
                None if x is None else x.add_(y) for x, y in zip(lora_sum, raw)]
        return (None, None, grad_t, grad_s, None, *lora_param_grads(ctx.module, lora_sum))


def routed_experts_chunked(module, tokens, top_scores, top_indices, bounds):
    """routed_experts(...) computed chunk by chunk over the token ranges
    ``bounds`` ([(start, end), ...] covering the tokens in order); with autograd
    through the chunk-checkpointed function above."""
    bounds = [(int(a), int(b)) for a, b in bounds if int(b) > int(a)]
    if not bounds:
        return routed_experts(module, tokens, top_scores, top_indices)
    params = _lora_params(module)
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (tokens, top_scores, *params)):
        if module.quant_format == "fp32":
            # Each chunk's backward recomputes only that chunk's fp32 layer.
            return torch.cat([
                _Fp32RoutedExperts.apply(module, tokens[a:b], top_scores[a:b], top_indices[a:b],
                                         *params) for a, b in bounds], dim=0)
        return _ChunkedRoutedExperts.apply(module, tuple(bounds), tokens, top_scores, top_indices,
                                           *params)
    with torch.no_grad():
        return torch.cat([routed_experts(module, tokens[a:b], top_scores[a:b], top_indices[a:b])
                          for a, b in bounds], dim=0)


def routed_experts_plus(module, tokens, top_scores, top_indices, addend, addend_ready=None):
    """routed_experts(...) + addend, the add fused into the combine in inference
    (the combine waits for ``addend_ready``); with autograd a plain add."""
    params = _lora_params(module)
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad for t in (tokens, top_scores, addend, *params)):
        if addend_ready is not None:
            torch.cuda.current_stream(tokens.device).wait_event(addend_ready)
        return routed_experts(module, tokens, top_scores, top_indices) + addend
    if tokens.dtype != torch.bfloat16 or module.quant_format == "fp32":
        if addend_ready is not None:
            torch.cuda.current_stream(tokens.device).wait_event(addend_ready)
        return routed_experts(module, tokens, top_scores, top_indices) + addend
    return _forward(module, tokens, top_scores, top_indices, False, addend, addend_ready)[0]


_EC_META: dict = {}


def _expert_choice_meta(aliases, logical, num_experts, device):
    """Device alias map and the combine's logical order (ascending (physical,
    logical)); built once per (map, device): they are static checkpoint metadata."""
    if not aliases:
        if logical != num_experts:
            raise ValueError("Logical and physical expert counts differ without an alias map.")
        return None, None
    if len(aliases) != logical:
        raise ValueError("Logical expert alias map does not match Expert-Choice routes.")
    key = (aliases, str(device))
    if key not in _EC_META:
        order = sorted(range(logical), key=lambda l: (aliases[l], l))
        _EC_META[key] = (torch.tensor(aliases, dtype=torch.int32, device=device),
                         torch.tensor(order, dtype=torch.int32, device=device))
    return _EC_META[key]


def _ec_inputs(module, tokens, expert_token_scores, expert_token_indices, tokens_per_sample,
               aliases):
    if expert_token_indices.shape != expert_token_scores.shape:
        raise ValueError("Expert-choice indices and scores must have matching shapes.")
    if expert_token_indices.ndim != 3:
        raise ValueError("Expert-choice routes must have shape [batch, expert, capacity].")
    if expert_token_indices.dtype.is_floating_point:
        raise TypeError("Expert-choice token indices must use an integer dtype.")
    if module.quant_format == "fp32":
        raise NotImplementedError("expert-choice routes run over bf16, nf4 or int8 weights")
    device = nat.require_gpu(tokens, expert_token_scores, expert_token_indices)
    B, L, C = (int(v) for v in expert_token_indices.shape)
    l2p, order = _expert_choice_meta(tuple(aliases), L, module.num_experts, device)
    x = tokens.detach().to(torch.bfloat16).contiguous()
    idx = expert_token_indices.detach().to(torch.int64).contiguous()
    scores = expert_token_scores.detach()
    if scores.dtype not in (torch.float32, torch.bfloat16):
        scores = scores.float()
    return device, (B, L, C), l2p, order, x, idx, scores.contiguous()


def _ec_forward(module, tokens, expert_token_scores, expert_token_indices, tokens_per_sample,
                aliases, need_grad):
    """One mx_moe_forward_expert_choice_ex call; returns (out, saved or None)."""
    device, (B, L, C), l2p, order, x, idx, scores = _ec_inputs(
        module, tokens, expert_token_scores, expert_token_indices, tokens_per_sample, aliases)
    T, d = (int(v) for v in x.shape)
    S = B * L * C
    (w1, w3, w2), packed = _weight_descriptors(module, device)
    f = int(packed[0].shape[1])
    lora, keep = _lora_descriptors(module, device)
    # fp32 sums are kept for fp32 tokens (the reference casts its fp32 buffer
    # to the token dtype).
    out = torch.empty((T, d), dtype=torch.float32 if tokens.dtype == torch.float32
                      else torch.bfloat16, device=device)
    saves = [None] * 5
    if need_grad:
        saves = [torch.empty((S, f), dtype=torch.bfloat16, device=device),
                 torch.empty((S, f), dtype=torch.bfloat16, device=device),
                 torch.empty((S, f), dtype=torch.bfloat16, device=device),
                 torch.empty((S, d), dtype=torch.bfloat16, device=device),
                 torch.zeros((S, lora_row(module)), dtype=torch.bfloat16, device=device)]
    lib = nat.load_library()
    ws = nat.workspace(lib.mx_moe_expert_choice_workspace_size(
        B, L, C, tokens_per_sample, module.num_experts, d, f, lora_rank(module)), device)
    nat.call("mx_moe_forward_expert_choice_ex", x.data_ptr(), idx.data_ptr(), scores.data_ptr(),
             nat.dtype_code(scores.dtype), B, L, C, int(tokens_per_sample), nat.ptr(l2p),
             nat.ptr(order), module.num_experts, d, f, kernel_activation(module), w1, w3, w2,
             lora[0], lora[1], lora[2], out.data_ptr(), nat.dtype_code(out.dtype),
             *[nat.ptr(t) for t in saves], ws.data_ptr(), nat.stream(device))
    del keep
    return out.to(tokens.dtype), ((x, scores, idx, *saves) if need_grad else None)


class _ExpertChoiceExperts(torch.autograd.Function):
    """Expert-choice layer with gradients to tokens, scores and the LoRA
    factors (the autograd of run_compressed_expert_choice,
    execution/expert_choice.py:16-152): one mx_moe_backward_expert_choice call."""

    @staticmethod
    def forward(ctx, module, tokens_per_sample, aliases, tokens, expert_token_scores,
                expert_token_indices, *lora_params):
        out, saved = _ec_forward(module, tokens, expert_token_scores, expert_token_indices,
                                 tokens_per_sample, aliases, True)
        ctx.module, ctx.tps, ctx.aliases = module, tokens_per_sample, aliases
        ctx.token_dtype, ctx.score_dtype = tokens.dtype, expert_token_scores.dtype
        ctx.save_for_backward(*saved)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        from .backward import lora_param_grads

        x, scores, idx, gate, up, h, y, lora_rows = ctx.saved_tensors
        module = ctx.module
        device = x.device
        B, L, C = (int(v) for v in idx.shape)
        T, d = (int(v) for v in x.shape)
        E = module.num_experts
        l2p, order = _expert_choice_meta(tuple(ctx.aliases), L, E, device)
        (w1, w3, w2), packed = _weight_descriptors(module, device)
        f = int(packed[0].shape[1])
        lora, keep = _lora_descriptors(module, device)
        g = grad_out.contiguous()
        if g.dtype not in (torch.float32, torch.bfloat16):
            g = g.float()
        grad_tokens = torch.empty((T, d), dtype=torch.float32 if ctx.token_dtype == torch.float32
                                  else torch.bfloat16, device=device)
        grad_scores = torch.empty((B, L, C), dtype=torch.float32, device=device)
        lora_needs = ctx.needs_input_grad[6:]
        raw = []
        for i, adapter in enumerate(module._adapters()):
            if adapter is None:
                raw += [None, None]
                continue
            r8 = adapter.padded_rank()
            raw.append(torch.empty((E, r8, adapter.in_features), dtype=torch.float32,
                                   device=device) if lora_needs[2 * i] else None)
            raw.append(torch.empty((E, adapter.out_features, r8), dtype=torch.float32,
                                   device=device) if lora_needs[2 * i + 1] else None)
        lib = nat.load_library()
        ws = nat.workspace(lib.mx_moe_backward_expert_choice_workspace_size(
            B, L, C, ctx.tps, E, d, f, lora_rank(module)), device)
        nat.call("mx_moe_backward_expert_choice", g.data_ptr(), nat.dtype_code(g.dtype),
                 x.data_ptr(), idx.data_ptr(), scores.data_ptr(), nat.dtype_code(scores.dtype),
                 B, L, C, int(ctx.tps), nat.ptr(l2p), nat.ptr(order), E, d, f,
                 kernel_activation(module), w1, w3, w2, lora[0], lora[1], lora[2],
                 gate.data_ptr(), up.data_ptr(), h.data_ptr(), y.data_ptr(), lora_rows.data_ptr(),
                 grad_tokens.data_ptr(), nat.dtype_code(grad_tokens.dtype),
                 grad_scores.data_ptr(), *[nat.ptr(t) for t in raw], ws.data_ptr(),
                 nat.stream(device))
        del keep
        grad_t = grad_tokens.to(ctx.token_dtype) if ctx.needs_input_grad[3] else None
        grad_s = grad_scores.to(ctx.score_dtype) if ctx.needs_input_grad[4] else None
        return (None, None, None, grad_t, grad_s, None, *lora_param_grads(module, raw))


def expert_choice_experts(module, tokens, expert_token_scores, expert_token_indices,
                          tokens_per_sample, aliases=()):
    """Expert-choice routed layer through mx_moe_forward_expert_choice_ex; with
    autograd (gradients to tokens, scores and the LoRA factors) when one of
    them requires a gradient."""
    params = _lora_params(module)
    if torch.is_grad_enabled() and any(
            t is not None and t.requires_grad
            for t in (tokens, expert_token_scores, *params)):
        _ec_inputs(module, tokens, expert_token_scores, expert_token_indices, tokens_per_sample,
                   aliases)  # validates before autograd records anything
        return _ExpertChoiceExperts.apply(module, int(tokens_per_sample), tuple(aliases), tokens,
                                          expert_token_scores, expert_token_indices, *params)
    return _ec_forward(module, tokens, expert_token_scores, expert_token_indices,
                       int(tokens_per_sample), aliases, False)[0]


def sorted_experts(module, tokens, counts):
    """Expert MLP over expert-grouped rows (forward kernels; run_for_loop)."""
    device = nat.require_gpu(tokens)
    if module.quant_format == "fp32":
        # The fp32 layer is the split-precision routed layer: a pre-grouped row
        # is a route of k = 1 to its own expert with a unit score, whose fp32
        # combine returns the expert output unchanged.
        c = counts.detach().to(device=device, dtype=torch.int64)
        if int(c.numel()) != module.num_experts:
            raise ValueError("counts must hold one entry per expert.")
        S = int(tokens.shape[0])
        idx = torch.repeat_interleave(torch.arange(module.num_experts, device=device), c)
        if int(idx.numel()) != S:
            raise ValueError(f"counts sum to {int(idx.numel())}, but {S} rows were given.")
        ones = torch.ones((S, 1), dtype=torch.float32, device=device)
        return routed_experts(module, tokens, ones, idx.view(S, 1))
    if torch.is_grad_enabled() and (tokens.requires_grad or any(
            p is not None and p.requires_grad for p in _lora_params(module))):
        from .backward import sorted_experts_autograd
        return sorted_experts_autograd(module, tokens, counts)
    x = tokens.detach().to(torch.bfloat16).contiguous()
    c = counts.detach().to(device=device, dtype=torch.int64).contiguous()
    if int(c.numel()) != module.num_experts:
        raise ValueError("counts must hold one entry per expert.")
    S, d = (int(v) for v in x.shape)
    (w1, w3, w2), packed = _weight_descriptors(module, device)
    f = int(packed[0].shape[1])
    lora, keep = _lora_descriptors(module, device)
    out = torch.empty((S, d), dtype=torch.bfloat16, device=device)
    lib = nat.load_library()
    ws = nat.workspace(lib.mx_moe_workspace_size(S, 1, module.num_experts, d, f,
                                                 lora_rank(module)), device)
    nat.call("mx_moe_for_loop_act", x.data_ptr(), c.data_ptr(), S, module.num_experts, d, f,
             kernel_activation(module), w1, w3, w2, lora[0], lora[1], lora[2], out.data_ptr(),
             ws.data_ptr(), nat.stream(device))
    del keep
    if S > 0:
        nat.watch_plan_errors(ws, device, "a run_for_loop call")
    return out.to(tokens.dtype)


def _grouped_inputs(module, key, x, offsets):
    """(device, counts [E] int64, bf16 rows, packed weight, adapter or None)."""
    device = nat.require_gpu(x)
    offs = offsets.detach().to(device=device, dtype=torch.int64)
    if int(offs.numel()) != module.num_experts:
        raise ValueError("offsets must hold one inclusive row end per expert.")
    counts = torch.diff(offs, prepend=offs.new_zeros(1)).contiguous()
    packed = module.packed_weight(key)
    in_f = int(packed.shape[2])
    if int(x.shape[-1]) != in_f:
        raise ValueError(f"x has {int(x.shape[-1])} features, weight '{key}' expects {in_f}.")
    xb = x.detach().to(torch.bfloat16).contiguous()
    adapter = module.expert_lora[key] if key in module.expert_lora else None
    return device, counts, xb, packed, adapter


def _single_lora(adapter, device):
    if adapter is None:
        return nat.MxLora(None, None, 0, 0.0), [], 0
    a, b = adapter.kernel_factors(device)
    return (nat.MxLora(a.data_ptr(), b.data_ptr(), adapter.padded_rank(), float(adapter.scale())),
            [a, b], adapter.padded_rank())


def _grouped_linear_forward(module, key, device, counts, xb, packed, adapter):
    S = int(xb.shape[0])
    out_f = int(packed.shape[1])
    lora, keep, rank = _single_lora(adapter, device)
    out = torch.empty((S, out_f), dtype=torch.bfloat16, device=device)
    lib = nat.load_library()
    ws = nat.workspace(lib.mx_moe_workspace_size(S, 1, module.num_experts, int(packed.shape[2]),
                                                 out_f, rank), device)
    nat.call("mx_grouped_linear", xb.data_ptr(), counts.data_ptr(), S, module.num_experts,
             packed.descriptor(), lora, out.data_ptr(), ws.data_ptr(), nat.stream(device))
    del keep
    if S > 0:
        nat.watch_plan_errors(ws, device, "a grouped_linear call")
    return out


class _GroupedLinear(torch.autograd.Function):
    """grouped_linear with gradients to x and to the projection's LoRA factors:
    the autograd of _FrozenGroupedMMLinear (torch_grouped.py:53-91, dX through
    the re-decoded frozen weight) plus ActiveExpertLoRA.grouped_forward
    (active_expert_lora.py:348-399), one mx_grouped_linear_backward call."""

    @staticmethod
    def forward(ctx, module, key, x, offsets, *lora_params):
        device, counts, xb, packed, adapter = _grouped_inputs(module, key, x, offsets)
        out = _grouped_linear_forward(module, key, device, counts, xb, packed, adapter)
        ctx.module, ctx.key, ctx.x_dtype = module, key, x.dtype
        ctx.save_for_backward(xb, counts)
        return out.to(x.dtype)

    @staticmethod
    def backward(ctx, grad_out):
        xb, counts = ctx.saved_tensors
        module, key = ctx.module, ctx.key
        device = xb.device
        packed = module.packed_weight(key)
        adapter = module.expert_lora[key] if key in module.expert_lora else None
        S, in_f = (int(v) for v in xb.shape)
        out_f = int(packed.shape[1])
        E = module.num_experts
        lora, keep, rank = _single_lora(adapter, device)
        need_x = ctx.needs_input_grad[2]
        need_a = adapter is not None and ctx.needs_input_grad[4]
        need_b = adapter is not None and ctx.needs_input_grad[5]
        if not (need_x or need_a or need_b):
            return (None,) * (4 + len(ctx.needs_input_grad[4:]))
        g = grad_out.detach().to(torch.bfloat16).contiguous()
        grad_x = torch.empty((S, in_f), dtype=torch.bfloat16, device=device) if need_x else None
        ga = gb = None
        if adapter is not None:
            # The kernel writes both factor gradients together.
            ga = torch.empty((E, rank, in_f), dtype=torch.float32, device=device)
            gb = torch.empty((E, out_f, rank), dtype=torch.float32, device=device)
        lib = nat.load_library()
        ws = nat.workspace(lib.mx_grouped_linear_backward_workspace_size(S, E, in_f, out_f, rank),
                           device)
        nat.call("mx_grouped_linear_backward", g.data_ptr(), xb.data_ptr(), counts.data_ptr(), S,
                 E, packed.descriptor(), lora, nat.ptr(grad_x), nat.ptr(ga), nat.ptr(gb),
                 ws.data_ptr(), nat.stream(device))
        del keep
        grads = [grad_x.to(ctx.x_dtype) if need_x else None, None]
        if adapter is None:
            return (None, None, *grads)
        r = adapter.rank
        grads.append(ga[:, :r, :].to(adapter.lora_a.dtype) if need_a else None)
        grads.append(gb[:, :, :r].contiguous().to(adapter.lora_b.dtype) if need_b else None)
        return (None, None, *grads)


def grouped_projection(module, key, x, offsets):
    """x [S, in] rows grouped by expert with inclusive int32 offsets -> [S, out],
    with autograd to x and the LoRA factors when either requires a gradient."""
    adapter = module.expert_lora[key] if key in module.expert_lora else None
    params = [] if adapter is None else [adapter.lora_a, adapter.lora_b]
    if torch.is_grad_enabled() and any(t.requires_grad for t in (x, *params)):
        return _GroupedLinear.apply(module, key, x, offsets, *params)
    device, counts, xb, packed, adapter = _grouped_inputs(module, key, x, offsets)
    return _grouped_linear_forward(module, key, device, counts, xb, packed, adapter).to(x.dtype)
