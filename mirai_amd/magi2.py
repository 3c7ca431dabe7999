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


def _dtype_name(dtype: torch.dtype) -> str:
    return str(dtype).removeprefix("torch.")


def _parse_dtype(value: object) -> torch.dtype:
    dtype = getattr(torch, str(value), None)
    if not isinstance(dtype, torch.dtype):
        raise Magi2QuantizedExpertError(f"Packed MAGI-2 store declares unknown dtype '{value}'.")
    return dtype


def route_topk_heads(router_logits: torch.Tensor, top_k: int, *, score_func: str = "sigmoid",
                     expert_bias: torch.Tensor | None = None, route_norm: bool = True,
                     norm_eps: float = 1e-12, route_scale: float = 1.0, layout: str = "heads",
                     score_dtype: torch.dtype = torch.float32):
    """Multi-head top-k routing of fp32 logits [H, S, E] on the GPU.

    Returns ``(probs, indices)``: with layout "heads" both are [H, S, k] and the
    indices are per-head expert ids (compute_topk_probs_and_indices,
    flash_mh_moe/route.py:157-196, then * route_scale as CoreMultiHeadMoE._route
    does, magi2_preview.py:2735-2742); with layout "rows" both are [S*H, k], row
    s*H+h, and the indices are flattened group ids h*E+e, ready for
    Magi2GroupedExperts.run_rows. Selection is by score + expert_bias (ties to
    the lower expert id); the probabilities carry no gradient here.
    """
    if router_logits.ndim != 3:
        raise ValueError("router logits must be [heads, tokens, experts].")
    if score_func not in SCORE_FUNCS:
        raise ValueError(f"Unknown score_func: {score_func}")
    if layout not in _LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}.")
    if torch.is_grad_enabled() and router_logits.requires_grad:
        raise NotImplementedError(
            "route_topk_heads computes routes without a router gradient; call it under "
            "torch.no_grad() or on detached logits")
    H, S, E = (int(v) for v in router_logits.shape)
    if int(top_k) <= 0 or int(top_k) > min(E, 16):
        raise ValueError("top_k must be in [1, min(num_experts, 16)].")
    device = nat.require_gpu(router_logits)
    logits = router_logits.detach().float().contiguous()
    bias = None
    if expert_bias is not None:
        bias = expert_bias.detach().to(device=device, dtype=torch.float32).reshape(H, E)
        bias = bias.contiguous()
    shape = (H, S, int(top_k)) if layout == "heads" else (S * H, int(top_k))
    idx = torch.empty(shape, dtype=torch.int64, device=device)
    probs = torch.empty(shape, dtype=score_dtype, device=device)
    nat.call("mx_route_topk_heads", logits.data_ptr(), H, S, E, int(top_k), SCORE_FUNCS[score_func],
             nat.ptr(bias), nat.RENORM_CLAMP if route_norm else nat.RENORM_NONE, float(norm_eps),
             float(route_scale), _LAYOUTS[layout], idx.data_ptr(), probs.data_ptr(),
             nat.dtype_code(score_dtype), nat.stream(device))
    return probs, idx


def compute_topk_probs_and_indices(router_logits: torch.Tensor, top_k: int,
                                   score_func: str = "softmax",
                                   expert_bias: torch.Tensor | None = None,
                                   num_virtual_group: int = 1, topk_virtual_group: int = 0,
                                   route_norm: bool = True, norm_eps: float = 1e-12):
    """Drop-in for flash_mh_moe.route.compute_topk_probs_and_indices
    (flash_mh_moe/route.py:157-196) without virtual groups."""
    if int(num_virtual_group) != 1:
        raise NotImplementedError("virtual-group routing (num_virtual_group > 1) is not built")
    return route_topk_heads(router_logits, top_k, score_func=score_func, expert_bias=expert_bias,
                            route_norm=route_norm, norm_eps=norm_eps)


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

    def packed_state_descriptor(self) -> dict[str, object]:
        """Metadata that restores this exact payload (quantized_experts.py:140-163):
        group count, block size, the reference shapes and dtypes of the three
        tensors, the storage format and the buffer inventory. The payload is this
        build's packed layout ([G, out, in] codes or int8 values and their scales),
        restored as stored, never through dense weights."""
        if not self.is_fully_loaded():
            raise Magi2QuantizedExpertError(
                "MAGI-2 NF4 store must be complete before it can be persisted.")
        fmt = self.experts.quant_format
        meta: dict[str, object] = {"format": fmt, "blocksize": NF4_BLOCKSIZE}
        if fmt == "nf4":
            scale = getattr(self.experts, self.experts.packed_buffer_names("W_gate")[1])
            meta["absmax_dtype"] = _dtype_name(scale.dtype)
        return {
            "num_groups": self.num_groups,
            "blocksize": NF4_BLOCKSIZE,
            "expert_shapes": {k: list(self._source_shapes[k]) for k in MAGI2_ROUTED_EXPERT_TENSOR_NAMES},
            "expert_dtypes": {k: _dtype_name(self._source_dtypes[k])
                              for k in MAGI2_ROUTED_EXPERT_TENSOR_NAMES},
            "packed_meta": meta,
            "buffers": sorted(self.packed_buffers()),
        }

    def restore_packed_state(self, *, descriptor: dict[str, object],
                             buffers: dict[str, torch.Tensor]) -> None:
        """Restore a validated persisted payload without dense reconstruction
        (quantized_experts.py:165-219)."""
        if int(descriptor.get("num_groups", -1)) != self.num_groups:
            raise Magi2QuantizedExpertError("Packed MAGI-2 store has incompatible groups.")
        if int(descriptor.get("blocksize", -1)) != NF4_BLOCKSIZE:
            raise Magi2QuantizedExpertError("Packed MAGI-2 store has incompatible NF4 blocksize.")
        shapes, dtypes = descriptor.get("expert_shapes"), descriptor.get("expert_dtypes")
        if not isinstance(shapes, dict) or not isinstance(dtypes, dict):
            raise Magi2QuantizedExpertError("Packed MAGI-2 store has incomplete tensor metadata.")
        names = set(MAGI2_ROUTED_EXPERT_TENSOR_NAMES)
        if set(shapes) != names or set(dtypes) != names:
            raise Magi2QuantizedExpertError("Packed MAGI-2 store has incomplete expert metadata.")
        meta = descriptor.get("packed_meta")
        if not isinstance(meta, dict):
            raise Magi2QuantizedExpertError("Packed MAGI-2 store has no NF4 metadata.")
        if str(meta.get("format")) != self.experts.quant_format:
            raise Magi2QuantizedExpertError(
                f"Packed MAGI-2 store holds '{meta.get('format')}' weights, this module "
                f"stores '{self.experts.quant_format}'.")
        parsed_dtypes = {k: _parse_dtype(dtypes[k]) for k in names}
        parsed_shapes = {}
        for k in names:
            shape = tuple(int(v) for v in shapes[k])
            if len(shape) != 3 or shape[0] != self.num_groups:
                raise Magi2QuantizedExpertError(
                    f"Packed MAGI-2 store gives {k} the shape {shape}.")
            parsed_shapes[k] = shape
        if set(descriptor.get("buffers", [])) != set(buffers):
            raise Magi2QuantizedExpertError(
                "Packed MAGI-2 store buffer inventory does not match its descriptor.")
        for key in MAGI2_ROUTED_EXPERT_TENSOR_NAMES:
            g, rows, cols = parsed_shapes[key]
            try:
                self.experts.adopt_packed(key, buffers, (g, cols, rows))
            except ValueError as err:
                raise Magi2QuantizedExpertError(f"Packed MAGI-2 store: {err}") from err
            self._source_shapes[key] = parsed_shapes[key]
            self._source_dtypes[key] = parsed_dtypes[key]

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
        with torch.no_grad():
            probs, groups = route_topk_heads(router_logits, top_k, score_func=score_func,
                                             expert_bias=expert_bias, route_norm=route_norm,
                                             route_scale=route_scale, layout="rows")
        return self.run_rows(x_heads.reshape(S * H, d), probs, groups).view(S, H, d)


MAGI2_PACKED_SCHEMA = "mirai_amd.magi2.packed_experts"
MAGI2_PACKED_SCHEMA_VERSION = 1
_MANIFEST = "manifest.json"


class Magi2PackedExpertStateError(ValueError):
    """Raised when a packed MAGI-2 expert artifact is incompatible
    (packed_experts.py:24-25)."""


def _magi2_layers(model) -> dict[str, Magi2GroupedExperts]:
    if isinstance(model, dict):
        return dict(model)
    if isinstance(model, Magi2GroupedExperts):
        return {"": model}
    return {name: m for name, m in model.named_modules() if isinstance(m, Magi2GroupedExperts)}


def save_magi2_packed_state(path, model, *, metadata: dict | None = None):
    """Write every layer's packed payload (one safetensors shard per layer) and a
    versioned manifest holding each layer's descriptor, with no dense
    reconstruction (save_magi2_nf4_packed_state, packed_experts.py:28-78).
    ``model``: a module holding Magi2GroupedExperts layers, one such layer, or a
    {name: layer} mapping."""
    import json
    from pathlib import Path

    from safetensors.torch import save_file

    target = Path(path).expanduser()
    if target.exists() and any(target.iterdir()):
        raise FileExistsError(f"Packed MAGI-2 export directory must be empty: {target}")
    target.mkdir(parents=True, exist_ok=True)
    layers = {}
    for index, (name, layer) in enumerate(_magi2_layers(model).items()):
        if not layer.is_fully_loaded():
            raise Magi2PackedExpertStateError(
                f"MAGI-2 layer '{name}' has no complete packed expert store.")
        descriptor = layer.packed_state_descriptor()
        shard = f"layer_{index:03d}.safetensors"
        save_file({k: v.detach().cpu().contiguous() for k, v in layer.packed_buffers().items()},
                  str(target / shard))
        layers[name] = {"shard": shard, **descriptor}
    if not layers:
        raise Magi2PackedExpertStateError("MAGI-2 packed expert export matched no routed-expert layers.")
    manifest = {"schema": MAGI2_PACKED_SCHEMA, "schema_version": MAGI2_PACKED_SCHEMA_VERSION,
                "layers": layers, "metadata": dict(metadata or {})}
    (target / _MANIFEST).write_text(json.dumps(manifest, indent=2, sort_keys=True), encoding="utf-8")
    return target


def load_magi2_packed_state(path, model, *, expected_metadata: dict | None = None,
                            device=None) -> dict[str, Magi2GroupedExperts]:
    """Restore every layer's payload from ``save_magi2_packed_state`` output,
    rejecting schema, lineage, layer-inventory and buffer mismatches
    (load_magi2_nf4_packed_state, packed_experts.py:81-183). Tensors land on
    ``device`` (default: the current GPU)."""
    import json
    from pathlib import Path

    from safetensors import safe_open

    source = Path(path).expanduser()
    if not source.is_dir():
        raise FileNotFoundError(f"Packed MAGI-2 expert state not found: {source}")
    layers = _magi2_layers(model)
    manifest_path = source / _MANIFEST
    if not manifest_path.is_file():
        raise Magi2PackedExpertStateError("Packed MAGI-2 expert state has no versioned manifest.")
    manifest = json.loads(manifest_path.read_text(encoding="utf-8"))
    if manifest.get("schema") != MAGI2_PACKED_SCHEMA or int(
            manifest.get("schema_version", -1)) != MAGI2_PACKED_SCHEMA_VERSION:
        raise Magi2PackedExpertStateError(
            "Packed MAGI-2 expert state has an unsupported schema or version.")
    lineage = manifest.get("metadata")
    if not isinstance(lineage, dict):
        raise Magi2PackedExpertStateError("Packed MAGI-2 expert state has invalid lineage metadata.")
    for key, value in (expected_metadata or {}).items():
        if str(lineage.get(key, "")) != str(value):
            raise Magi2PackedExpertStateError(f"Packed MAGI-2 expert state has incompatible {key}.")
    specs = manifest.get("layers")
    if not isinstance(specs, dict) or set(specs) != set(layers):
        raise Magi2PackedExpertStateError(
            "Packed MAGI-2 expert layer inventory does not match the model.")
    target = torch.device(device) if device is not None else torch.device("cuda")
    for name, layer in layers.items():
        spec = specs[name]
        shard = str(spec.get("shard", ""))
        if not shard or Path(shard).name != shard:
            raise Magi2PackedExpertStateError(f"Packed MAGI-2 layer '{name}' has an invalid shard path.")
        shard_path = source / shard
        if not shard_path.is_file():
            raise Magi2PackedExpertStateError(f"Packed MAGI-2 layer '{name}' is missing shard '{shard}'.")
        with safe_open(str(shard_path), framework="pt", device="cpu") as handle:
            if set(handle.keys()) != set(spec.get("buffers", [])):
                raise Magi2PackedExpertStateError(
                    f"Packed MAGI-2 layer '{name}' shard inventory is invalid.")
            buffers = {k: handle.get_tensor(k).to(target).contiguous() for k in handle.keys()}
        layer.restore_packed_state(descriptor=spec, buffers=buffers)
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
