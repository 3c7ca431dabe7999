"""MAGI-2 multi-head MoE experts on the MI355X kernels.

MAGI-2 (mirai/vendors/magi2_preview/model/magi2_preview.py:2630-2800) splits
each token into H heads of d_head features; every head routes to k of its own
E experts. The reference's Mirai seam (Magi2GroupedMoEBackend /
Magi2QuantizedGroupedMoEBackend, mirai/core/models/magi2_preview/
grouped_moe.py:432-756, 1262-1450) flattens (token, head) onto the row axis
(row s*H+h) and (head, expert) onto one group axis (group h*E+e), sorts the
routed slots stably by group, runs gate / up projections, swiglu7 and the
down projection per group, and index-adds the probability-weighted outputs.

Here that is one fused routed layer of the HIP library with the swiglu7
epilogue: the same plan (no 1023-group cap, so no segmenting), the grouped
GEMMs with in-register NF4 / INT8 decode and optional expert LoRA, and the
deterministic combine. The [G, in, out] weights are stored transposed, as the
kernels' [G, out, in]. Routing (softmax / sigmoid scores, selection-only
expert bias, L1 renormalisation, route_scale) is one kernel as well.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from . import _native as nat
from .experts import CompressedGroupedExperts
from .quant import NF4_BLOCKSIZE
from .specs import MAGI2_EXPERT_MLP_SPEC

MAGI2_ROUTED_EXPERT_TENSOR_NAMES = ("W_gate", "W_up", "W_down")
SCORE_FUNCS = {"softmax": nat.SCORE_SOFTMAX, "sigmoid": nat.SCORE_SIGMOID}
_LAYOUTS = {"heads": nat.ROUTE_LAYOUT_HEADS, "rows": nat.ROUTE_LAYOUT_ROWS}


class Magi2QuantizedExpertError(ValueError):
    """Raised when quantized MAGI-2 expert storage cannot be built, persisted or
    restored (quantized_experts.py:63-64)."""


def _route_heads_native(logits, top_k, score_func, bias, route_norm, norm_eps, route_scale,
                        num_virtual_group, topk_virtual_group, layout, score_dtype):
    H, S, E = (int(v) for v in logits.shape)
    device = logits.device
    shape = (H, S, int(top_k)) if layout == "heads" else (S * H, int(top_k))
    idx = torch.empty(shape, dtype=torch.int64, device=device)
    probs = torch.empty(shape, dtype=score_dtype, device=device)
    nat.call("mx_route_topk_heads", logits.data_ptr(), H, S, E, int(top_k),
             SCORE_FUNCS[score_func], nat.ptr(bias),
             nat.RENORM_CLAMP if route_norm else nat.RENORM_NONE, float(norm_eps),
             float(route_scale), int(num_virtual_group), int(topk_virtual_group),
             _LAYOUTS[layout], idx.data_ptr(), probs.data_ptr(), nat.dtype_code(score_dtype),
             nat.stream(device))
    return probs, idx


class _HeadRoutes(torch.autograd.Function):
    """Per-head routing with the gradient of the probabilities back to the
    logits: the autograd of _compute_topk_probs_and_indices_torch_impl
    (route.py:28-148; softmax / sigmoid, gather, F.normalize(p=1, eps)) and
    CoreMultiHeadMoE._route's `* route_scale` (magi2_preview.py:2741), one
    mx_route_scores_backward call over the H * S logits rows."""

    @staticmethod
    def forward(ctx, logits_in, args):
        logits = logits_in.detach().float().contiguous()
        probs, idx = _route_heads_native(logits, *args)
        ctx.mark_non_differentiable(idx)
        ctx.args = args
        ctx.logits_dtype = logits_in.dtype
        ctx.save_for_backward(logits, idx)
        return probs, idx

    @staticmethod
    def backward(ctx, g_probs, _g_idx):
        logits, idx = ctx.saved_tensors
        top_k, score_func, _bias, route_norm, norm_eps, route_scale, _, _, layout, _ = ctx.args
        H, S, E = (int(v) for v in logits.shape)
        g = g_probs.float()
        if layout == "rows":
            # rows s*H+h with group ids h*E+e -> [H, S, k] per-head expert ids
            heads = torch.arange(H, device=idx.device).view(1, H, 1) * E
            idx = (idx.view(S, H, top_k) - heads).permute(1, 0, 2)
            g = g.view(S, H, top_k).permute(1, 0, 2)
        from .router import router_scores_backward

        dl = router_scores_backward(logits.view(H * S, E), idx.reshape(H * S, top_k),
                                    g.reshape(H * S, top_k), score_func=score_func,
                                    renorm=nat.RENORM_CLAMP if route_norm else nat.RENORM_NONE,
                                    renorm_floor=norm_eps, route_scale=route_scale)
        return dl.view(H, S, E).to(ctx.logits_dtype), None


def route_topk_heads(router_logits: torch.Tensor, top_k: int, *, score_func: str = "sigmoid",
                     expert_bias: torch.Tensor | None = None, route_norm: bool = True,
                     norm_eps: float = 1e-12, route_scale: float = 1.0,
                     num_virtual_group: int = 1, topk_virtual_group: int = 0,
                     layout: str = "heads", score_dtype: torch.dtype = torch.float32):
    """Multi-head top-k routing of fp32 logits [H, S, E] on the GPU.

    Returns ``(probs, indices)``: with layout "heads" both are [H, S, k] and the
    indices are per-head expert ids (compute_topk_probs_and_indices,
    flash_mh_moe/route.py:157-196, then * route_scale as CoreMultiHeadMoE._route
    does, magi2_preview.py:2735-2742); with layout "rows" both are [S*H, k], row
    s*H+h, and the indices are flattened group ids h*E+e, ready for
    Magi2GroupedExperts.run_rows. Selection is by score + expert_bias (ties to
    the lower expert id), within the topk_virtual_group best of
    num_virtual_group expert groups when num_virtual_group > 1
    (route.py:62-105). When the logits require a gradient, the probabilities
    carry one back to them.
    """
    if router_logits.ndim != 3:
        raise ValueError("router logits must be [heads, tokens, experts].")
    if score_func not in SCORE_FUNCS:
        raise ValueError(f"Unknown score_func: {score_func}")
    if layout not in _LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}.")
    H, S, E = (int(v) for v in router_logits.shape)
    if int(top_k) <= 0 or int(top_k) > min(E, 16):
        raise ValueError("top_k must be in [1, min(num_experts, 16)].")
    nvg, tvg = int(num_virtual_group), int(topk_virtual_group)
    if nvg > 1 and not (0 < tvg <= nvg):
        raise ValueError(
            f"topk_virtual_group ({tvg}) must be in (0, num_virtual_group ({nvg})]")
    if nvg > 1 and E % nvg:
        raise ValueError(f"num_experts ({E}) must be divisible by num_virtual_group ({nvg})")
    device = nat.require_gpu(router_logits)
    bias = None
    if expert_bias is not None:
        bias = expert_bias.detach().to(device=device, dtype=torch.float32).reshape(H, E)
        bias = bias.contiguous()
    args = (int(top_k), score_func, bias, bool(route_norm), float(norm_eps), float(route_scale),
            nvg, tvg, layout, score_dtype)
    if torch.is_grad_enabled() and router_logits.requires_grad:
        return _HeadRoutes.apply(router_logits, args)
    return _route_heads_native(router_logits.detach().float().contiguous(), *args)


def compute_topk_probs_and_indices(router_logits: torch.Tensor, top_k: int,
                                   score_func: str = "softmax",
                                   expert_bias: torch.Tensor | None = None,
                                   num_virtual_group: int = 1, topk_virtual_group: int = 0,
                                   route_norm: bool = True, norm_eps: float = 1e-12):
    """Drop-in for flash_mh_moe.route.compute_topk_probs_and_indices
    (flash_mh_moe/route.py:157-196)."""
    return route_topk_heads(router_logits, top_k, score_func=score_func, expert_bias=expert_bias,
                            route_norm=route_norm, norm_eps=norm_eps,
                            num_virtual_group=num_virtual_group,
                            topk_virtual_group=topk_virtual_group)


class Magi2GroupedExperts(nn.Module):
    """Packed MAGI-2 routed experts for H heads x E experts (G = H*E groups).

    ``load_dense_weight`` takes the reference layer's [G, in, out] tensors
    (W_gate, W_up [G, d_head, d_expert]; W_down [G, d_expert, d_head]) and
    stores them in ``quant_format`` ("nf4", "int8" or "bf16").
    """

    def __init__(self, *, num_heads: int, num_experts: int, quant_format: str = "nf4",
                 expert_weight_access: str = "fused_kernel", expert_dequant_chunk_size: int = 0):
        super().__init__()
        self.num_heads = int(num_heads)
        self.num_experts = int(num_experts)
        if self.num_heads <= 0 or self.num_experts <= 0:
            raise ValueError("num_heads and num_experts must be positive.")
        self.experts = CompressedGroupedExperts.from_empty(
            num_experts=self.num_heads * self.num_experts, quant_format=quant_format,
            expert_weight_access=expert_weight_access,
            expert_dequant_chunk_size=expert_dequant_chunk_size,
            execution_spec=MAGI2_EXPERT_MLP_SPEC)
        # The reference's MAGI-2 backend sums the weighted expert outputs with
        # a bf16 index_add (grouped_moe.py:750-754): each term bf16(y *
        # bf16(prob)), the running sum rounded to bf16 (expert order here).
        self.experts._combine_bf16_terms = True

        # The reference layer's [G, in, out] shape and dtype of every loaded tensor.
        self._source_shapes: dict[str, tuple[int, int, int]] = {}
        self._source_dtypes: dict[str, torch.dtype] = {}

    @property
    def num_groups(self) -> int:
        return self.num_heads * self.num_experts

    @property
    def blocksize(self) -> int:
        """NF4 block size of the stored codes (one absmax per 64 inputs)."""
        return NF4_BLOCKSIZE

    def expert_weight_shape(self, key: str) -> tuple[int, int, int]:
        """The reference layer's shape of ``key`` ([G, in, out])."""
        if key not in self._source_shapes:
            raise Magi2QuantizedExpertError(f"MAGI-2 NF4 expert tensor '{key}' has not been quantized.")
        return self._source_shapes[key]

    def expert_weight_dtype(self, key: str) -> torch.dtype:
        if key not in self._source_dtypes:
            raise Magi2QuantizedExpertError(f"MAGI-2 NF4 expert tensor '{key}' has not been quantized.")
        return self._source_dtypes[key]

    def packed_buffers(self) -> dict[str, torch.Tensor]:
        """The packed payload of the loaded tensors, by buffer name."""
        out = {}
        for key in MAGI2_ROUTED_EXPERT_TENSOR_NAMES:
            if key in self._source_shapes:
                for name in self.experts.packed_buffer_names(key):
                    out[name] = getattr(self.experts, name)
        return out

    def payload_bytes(self) -> int:
        return int(sum(t.numel() * t.element_size() for t in self.packed_buffers().values()))

    def quantized_numel(self) -> int:
        return int(sum(g * a * b for g, a, b in self._source_shapes.values()))

    def load_reference_nf4_store(self, buffers: dict, expert_shapes: dict,
                                 expert_dtypes: dict | None = None, *,
                                 two_level: bool = False) -> None:
        """Adopt the payload of the reference's Magi2Nf4ExpertStore for this layer
        without re-quantising (quantized_experts.py:275-347): per key the
        double-quantised NF4 buffers ``{key}_nf4`` (codes of each group's
        [in, out] matrix, element 2j in the high nibble of byte j),
        ``_nf4_absmax`` (uint8 codes), ``_nf4_nabsmax``, ``_nf4_offset``,
        ``_nf4_code`` (the NF4 levels) and ``_nf4_ncode`` (256 fp32), with
        ``expert_shapes[key] = (G, in, out)``. The group payloads keep their
        [in, out] orientation (64-blocks along out): the kernels read them as
        stored (MX_FMT_NF4_F32_KN), the absmax decoded once to fp32, or with
        ``two_level=True`` kept as stored and decoded by the GEMMs
        (MX_FMT_NF4_DQ_KN)."""
        if self.experts.quant_format != "nf4":
            raise Magi2QuantizedExpertError(
                "a reference NF4 store loads into a module with quant_format='nf4'.")
        for key in MAGI2_ROUTED_EXPERT_TENSOR_NAMES:
            shape = tuple(int(v) for v in expert_shapes[key])
            if len(shape) != 3 or shape[0] != self.num_groups:
                raise Magi2QuantizedExpertError(
                    f"{key} has the shape {shape}; this layer holds {self.num_groups} groups.")
            g, rows, cols = shape
            fields = {}
            for field in _NF4_FIELDS:
                name = f"{key}_{field}"
                if name not in buffers:
                    raise Magi2QuantizedExpertError(f"the NF4 store lacks '{name}'.")
                fields[field] = buffers[name]
            device = self.experts_device()
            t = {f: v.to(device) for f, v in fields.items()}
            try:
                self.experts.load_packed_nf4(
                    key, packed=t["nf4"], absmax=t["nf4_absmax"], nested_absmax=t["nf4_nabsmax"],
                    offset=t["nf4_offset"], code=t["nf4_code"], nested_code=t["nf4_ncode"],
                    shape=(g, cols, rows), layout="in_out", two_level=two_level)
            except ValueError as err:
                raise Magi2QuantizedExpertError(f"{key}: {err}") from err
            self._source_shapes[key] = shape
            dtype = (expert_dtypes or {}).get(key, torch.bfloat16)
            self._source_dtypes[key] = dtype if isinstance(dtype, torch.dtype) else getattr(
                torch, str(dtype), torch.bfloat16)

    def experts_device(self) -> torch.device:
        """The device the packed weights live on (the current GPU before any is loaded)."""
        for t in self.experts.buffers():
            return t.device
        return torch.device("cuda", torch.cuda.current_device())

    @classmethod
    def from_dense(cls, W_gate: torch.Tensor, W_up: torch.Tensor, W_down: torch.Tensor, *,
                   num_heads: int, quant_format: str = "nf4", **kwargs) -> "Magi2GroupedExperts":
        groups = int(W_gate.shape[0])
        if groups % int(num_heads):
            raise ValueError("the group axis must hold num_heads x num_experts entries.")
        module = cls(num_heads=num_heads, num_experts=groups // int(num_heads),
                     quant_format=quant_format, **kwargs)
        for key, tensor in zip(MAGI2_ROUTED_EXPERT_TENSOR_NAMES, (W_gate, W_up, W_down)):
            module.load_dense_weight(key, tensor)
        return module

    def load_dense_weight(self, key: str, source: torch.Tensor) -> None:
        if key not in MAGI2_ROUTED_EXPERT_TENSOR_NAMES:
            raise ValueError(f"Unknown MAGI-2 routed expert tensor '{key}'.")
        if source.ndim != 3 or int(source.shape[0]) != self.num_groups:
            raise ValueError(
                f"MAGI-2 tensor {key} must be [{self.num_groups}, in, out], got "
                f"{tuple(source.shape)}.")
        self.experts.load_dense_weight(key, source.detach().transpose(1, 2).contiguous())
        self._source_shapes[key] = tuple(int(v) for v in source.shape)
        self._source_dtypes[key] = source.dtype

    def attach_expert_lora(self, *, tensor_name: str, adapter_name: str, rank: int,
                           alpha: float, init: str = "kaiming", use_rslora: bool = False):
        """Per-group LoRA on W_gate / W_up / W_down (factors A [G, r, in], B [G, out, r])."""
        return self.experts.attach_expert_lora(tensor_name=tensor_name, adapter_name=adapter_name,
                                               rank=rank, alpha=alpha, init=init,
                                               use_rslora=use_rslora)

    def is_fully_loaded(self) -> bool:
        return self.experts.is_fully_loaded()

    def run_rows(self, rows: torch.Tensor, row_probs: torch.Tensor,
                 row_groups: torch.Tensor) -> torch.Tensor:
        """rows [S*H, d_head], routes [S*H, k] with group ids -> [S*H, d_head]."""
        return self.experts.run_direct_routed(rows, row_probs, row_groups)

    def execute(self, x_heads: torch.Tensor, topk_probs: torch.Tensor,
                topk_indices: torch.Tensor) -> torch.Tensor:
        """[S, H, d_head] tokens and [H, S, k] per-head routes -> [S, H, d_head]
        (Magi2GroupedMoEBackend.execute, grouped_moe.py:615-637)."""
        if x_heads.ndim != 3 or int(x_heads.shape[1]) != self.num_heads:
            raise ValueError(f"x_heads must be [tokens, {self.num_heads}, d_head].")
        S, H, d = (int(v) for v in x_heads.shape)
        if tuple(topk_indices.shape[:2]) != (H, S) or topk_probs.shape != topk_indices.shape:
            raise ValueError("topk_probs / topk_indices must be [heads, tokens, k].")
        K = int(topk_indices.shape[2])
        heads = torch.arange(H, device=topk_indices.device).view(H, 1, 1) * self.num_experts
        groups = (topk_indices.to(torch.int64) + heads).permute(1, 0, 2).reshape(S * H, K)
        probs = topk_probs.permute(1, 0, 2).reshape(S * H, K)
        out = self.run_rows(x_heads.reshape(S * H, d), probs, groups)
        return out.view(S, H, d)

    def forward(self, x_heads: torch.Tensor, router_logits: torch.Tensor, *, top_k: int,
                score_func: str = "sigmoid", expert_bias: torch.Tensor | None = None,
                route_norm: bool = True, route_scale: float = 1.0) -> torch.Tensor:
        """Route [H, S, E] logits and run the experts: [S, H, d_head] out."""
        S, H, d = (int(v) for v in x_heads.shape)
        probs, groups = route_topk_heads(router_logits, top_k, score_func=score_func,
                                         expert_bias=expert_bias, route_norm=route_norm,
                                         route_scale=route_scale, layout="rows")
        return self.run_rows(x_heads.reshape(S * H, d), probs, groups).view(S, H, d)


# Field suffixes of one weight's double-quantised NF4 payload in the
# reference's store (quantized_experts.py:325-346).
_NF4_FIELDS = ("nf4", "nf4_absmax", "nf4_nabsmax", "nf4_offset", "nf4_code", "nf4_ncode")
# The artifact format the reference writes (packed_experts.py:19-20): its
# schema name and version, and the file naming its shards.
REFERENCE_MAGI2_ARTIFACT = ("mirai.magi2_preview.nf4_experts", 2)
_ARTIFACT_MANIFEST = "manifest.json"


def read_reference_magi2_artifact(path) -> dict[str, dict]:
    """Read a MAGI-2 NF4 expert artifact as the reference writes it
    (save_magi2_nf4_packed_state, packed_experts.py:28-78): a manifest naming
    one safetensors shard per MoE layer, each shard holding the six NF4
    buffers of W_gate, W_up and W_down. Returns {layer name: {"shapes":
    {key: (G, in, out)}, "dtypes": {key: dtype}, "buffers": {name: CPU
    tensor}}}. Only the safetensors loader touches the shards (no pickle).
    Anything this build cannot ingest raises Magi2QuantizedExpertError."""
    import json
    from pathlib import Path

    from safetensors import safe_open

    root = Path(path).expanduser()
    try:
        manifest = json.loads((root / _ARTIFACT_MANIFEST).read_text(encoding="utf-8"))
    except (OSError, ValueError) as err:
        raise Magi2QuantizedExpertError(f"no readable MAGI-2 artifact manifest in {root}") from err
    found = (manifest.get("schema"), manifest.get("schema_version"))
    if found != REFERENCE_MAGI2_ARTIFACT or manifest.get("quant_format") != "nf4":
        raise Magi2QuantizedExpertError(
            f"{root} holds artifact {found} ({manifest.get('quant_format')}); this reader takes "
            f"{REFERENCE_MAGI2_ARTIFACT} NF4 experts.")
    layers = manifest.get("layers")
    if not isinstance(layers, dict) or not layers:
        raise Magi2QuantizedExpertError(f"the artifact in {root} lists no layers.")
    wanted = sorted(f"{k}_{f}" for k in MAGI2_ROUTED_EXPERT_TENSOR_NAMES for f in _NF4_FIELDS)
    out = {}
    for name, spec in layers.items():
        meta = spec.get("nf4_meta") or {}
        if int(meta.get("blocksize", -1)) != NF4_BLOCKSIZE or int(
                meta.get("nested_blocksize", -1)) != 256:
            raise Magi2QuantizedExpertError(
                f"layer '{name}': NF4 blocks {meta.get('blocksize')} / nested "
                f"{meta.get('nested_blocksize')}; the kernels take 64 / 256.")
        shard = root / str(spec.get("shard", ""))
        if shard.parent != root or not shard.is_file():
            raise Magi2QuantizedExpertError(f"layer '{name}': shard {spec.get('shard')!r} "
                                            f"is not a file of {root}.")
        with safe_open(str(shard), framework="pt", device="cpu") as handle:
            absent = sorted(set(wanted) - set(handle.keys()))
            if absent:
                raise Magi2QuantizedExpertError(f"layer '{name}': shard lacks {absent}.")
            buffers = {n: handle.get_tensor(n) for n in wanted}
        shapes = spec.get("expert_shapes") or {}
        dtypes = spec.get("expert_dtypes") or {}
        try:
            out[name] = {
                "shapes": {k: tuple(int(v) for v in shapes[k])
                           for k in MAGI2_ROUTED_EXPERT_TENSOR_NAMES},
                "dtypes": {k: getattr(torch, str(dtypes.get(k, "bfloat16")), torch.bfloat16)
                           for k in MAGI2_ROUTED_EXPERT_TENSOR_NAMES},
                "buffers": buffers,
            }
        except (KeyError, TypeError, ValueError) as err:
            raise Magi2QuantizedExpertError(f"layer '{name}': bad expert shapes {shapes}") from err
    return out


def load_reference_magi2_artifact(path, layers: dict, *, two_level: bool = False) -> dict:
    """Ingest a reference MAGI-2 NF4 artifact into ``layers`` ({layer name:
    Magi2GroupedExperts with quant_format "nf4"}, names as in the manifest)
    without re-quantising; returns ``layers``."""
    entries = read_reference_magi2_artifact(path)
    if set(entries) != set(layers):
        raise Magi2QuantizedExpertError(
            f"artifact layers {sorted(entries)} do not match the model's {sorted(layers)}.")
    for name, entry in entries.items():
        layers[name].load_reference_nf4_store(entry["buffers"], entry["shapes"], entry["dtypes"],
                                              two_level=two_level)
    return layers


class Magi2FusedMoEBackend:
    """The reference's expert-execution seam (``module._mirai_moe_kernel_backend``
    with ``execute(module, x_heads, topk_probs, topk_indices)``,
    grouped_moe.py:615-637) over packed experts attached with ``attach``."""

    name = "mi355x_fused"

    @staticmethod
    def attach(module: nn.Module, experts: Magi2GroupedExperts) -> "Magi2FusedMoEBackend":
        module._mirai_amd_experts = experts
        backend = Magi2FusedMoEBackend()
        module._mirai_moe_kernel_backend = backend
        return backend

    def execute(self, module, x_heads, topk_probs, topk_indices):
        experts = getattr(module, "_mirai_amd_experts", None)
        if experts is None:
            raise RuntimeError(
                "MAGI-2 fused execution requires packed experts attached with "
                "Magi2FusedMoEBackend.attach(module, experts).")
        return experts.execute(x_heads, topk_probs, topk_indices)
