"""Frozen quantised grouped experts with fused routed execution on MI355X.

``CompressedGroupedExperts`` keeps the constructor, method names, argument
meaning, error types and autograd contract of the reference class
(mirai/core/models/compressed_weights/execution/experts.py:90-216 and the
methods cited below), so provider code can swap it in. Execution differs by
design: the whole routed layer -- dispatch plan, gathered gate/up grouped GEMM
with in-register NF4/INT8 decode and fused LoRA + SwiGLU, down grouped GEMM
with fused LoRA, deterministic gate-weighted combine -- runs as a handful of
gfx950 HIP kernels on the current stream, with no host synchronisation and no
per-expert-chunk Python loop. ``expert_dequant_chunk_size`` is accepted and
validated as in the reference but does not change the kernels: they never
materialise dequantised weights.
"""

from __future__ import annotations

from typing import Iterable

import torch
import torch.nn as nn

from . import _native as nat
from . import quant
from .lora import ActiveExpertLoRA
from .specs import (
    CANONICAL_PACKED_EXPERT_MLP_SPEC,
    FUSED_GATED_ACTIVATIONS,
    ExpertMLPExecutionSpec,
    as_execution_spec,
    normalize_expert_weight_access_policy,
)

NF4_BLOCKSIZE = quant.NF4_BLOCKSIZE
# Expert chunk used when chunked/fused access leaves the size unset: the
# largest hardware tier of the reference (mirai/config/defaults/hardware_tiers.toml:21),
# which a 288 GB MI355X falls into.
DEFAULT_DEQUANT_CHUNK = 16

# A two-level (bitsandbytes double-quant) absmax kept as stored: buffer suffix
# -> PackedWeight.dq field (the uint8 codes are the _nf4_absmax buffer).
_TWO_LEVEL_BUFFERS = (("_nf4_nabsmax", "nested_absmax"), ("_nf4_offset", "offsets"),
                      ("_nf4_ncode", "code"))

_BUFFER_SUFFIXES = {
    "nf4": ("_nf4", "_nf4_absmax"),
    "int8": ("_int8", "_scale"),
    "bf16": ("_bf16", None),
    "fp32": ("_f32x3", None),
}


class CompressedGroupedExperts(nn.Module):
    """Provider-described grouped experts stored in frozen packed formats."""

    def __init__(self, base: nn.Module, *, group_sizes: str | int | Iterable[int] | None = None,
                 expert_weight_access: str = "full_dequant", expert_dequant_chunk_size: int = 0,
                 quant_format: str = "int8", nf4_blocksize: int = NF4_BLOCKSIZE,
                 execution_spec: ExpertMLPExecutionSpec | None = None):
        super().__init__()
        spec = (execution_spec or getattr(base, "mirai_expert_mlp_spec", None)
                or CANONICAL_PACKED_EXPERT_MLP_SPEC)
        self._init_empty(num_experts=int(getattr(base, "num_experts")), group_sizes=group_sizes,
                         expert_weight_access=expert_weight_access,
                         expert_dequant_chunk_size=expert_dequant_chunk_size,
                         quant_format=quant_format, nf4_blocksize=nf4_blocksize,
                         execution_spec=spec)
        for key in self._spec.tensor_names:
            self.load_dense_weight(key, getattr(base, key))

    @classmethod
    def from_empty(cls, *, num_experts: int, group_sizes=None,
                   expert_weight_access: str = "full_dequant", expert_dequant_chunk_size: int = 0,
                   quant_format: str = "int8", nf4_blocksize: int = NF4_BLOCKSIZE,
                   execution_spec: ExpertMLPExecutionSpec = CANONICAL_PACKED_EXPERT_MLP_SPEC,
                   ) -> "CompressedGroupedExperts":
        module = cls.__new__(cls)
        nn.Module.__init__(module)
        module._init_empty(num_experts=int(num_experts), group_sizes=group_sizes,
                           expert_weight_access=expert_weight_access,
                           expert_dequant_chunk_size=expert_dequant_chunk_size,
                           quant_format=quant_format, nf4_blocksize=nf4_blocksize,
                           execution_spec=execution_spec)
        return module

    # ------------------------------------------------------------------ state
    def _init_empty(self, *, num_experts, group_sizes, expert_weight_access,
                    expert_dequant_chunk_size, quant_format, nf4_blocksize, execution_spec):
        # The provider's spec object may be the reference's own class: it is
        # kept as given (provider code re-reads it and checks its type), and
        # this module works from a validated copy of its fields.
        spec = as_execution_spec(execution_spec)
        if not spec.uses_gated_product or spec.activation not in FUSED_GATED_ACTIVATIONS:
            raise ValueError(
                "The MI355X fused expert kernels implement the gated expert MLP "
                "(activation 'silu' or 'swiglu7', combiner='gated_product')."
            )
        # Activation of the fused gate/up epilogue and of its backward.
        self._kernel_activation = (nat.ACT_SWIGLU7 if spec.activation == "swiglu7"
                                   else nat.ACT_SILU)
        if int(num_experts) <= 0 or int(num_experts) > nat.PLAN_MAX_EXPERTS:
            raise ValueError(f"num_experts must be in [1, {nat.PLAN_MAX_EXPERTS}].")
        if int(nf4_blocksize) != NF4_BLOCKSIZE:
            raise ValueError("The MI355X NF4 format uses blocksize 64.")
        self.num_experts = int(num_experts)
        self.mirai_expert_mlp_spec = execution_spec
        self._spec = spec
        self._group_sizes = group_sizes
        self._quant_format = quant.normalize_quant_format(quant_format)
        self._nf4_blocksize = int(nf4_blocksize)
        self._shapes: dict[str, tuple[int, int, int]] = {}
        self._layouts: dict[str, str] = {}  # key -> "out_in" or "in_out" (PackedWeight.layout)
        # Keys whose NF4 absmax is a bitsandbytes two-level absmax kept as stored.
        self._two_level: set[str] = set()
        self._loaded_dense_keys: set[str] = set()
        self.expert_lora = nn.ModuleDict()
        self.logical_num_experts = int(num_experts)
        self.prototype_logical_ids: tuple[int, ...] = ()
        self.set_expert_weight_access_policy(
            expert_weight_access=expert_weight_access,
            expert_dequant_chunk_size=expert_dequant_chunk_size,
            _allow_default_chunk=True,
        )

    @property
    def expert_mlp_spec(self):
        """The spec object the module was built with (experts.py:282-284)."""
        return self.mirai_expert_mlp_spec

    @property
    def quant_format(self) -> str:
        return self._quant_format

    def projection_for_role(self, role: str) -> str:
        return self._spec.tensor_for_role(role)

    def set_expert_weight_access_policy(self, *, expert_weight_access: str,
                                        expert_dequant_chunk_size: int = 0,
                                        _allow_default_chunk: bool = False) -> None:
        """experts.py:756-769 (validation and normalisation)."""
        access = normalize_expert_weight_access_policy(expert_weight_access)
        if access in {"auto", "disabled"}:
            access = "full_dequant"
        chunk = int(expert_dequant_chunk_size)
        if access in {"chunked_dequant", "fused_kernel"} and chunk <= 0:
            if not _allow_default_chunk:
                raise ValueError(
                    "chunked_dequant/fused_kernel requires expert_dequant_chunk_size > 0.")
            chunk = DEFAULT_DEQUANT_CHUNK
        self.expert_weight_access = access
        self.expert_dequant_chunk_size = max(0, chunk)

    def prefers_for_loop(self) -> bool:
        return self.expert_weight_access in {"active_dequant", "chunked_dequant", "fused_kernel"}

    def is_fully_loaded(self) -> bool:
        return self._loaded_dense_keys.issuperset(self._spec.tensor_names)

    def expert_weight_shape(self, key: str) -> tuple[int, ...]:
        if str(key) in self._shapes:
            return self._shapes[str(key)]
        raise AttributeError(f"Grouped expert weight '{key}' is not loaded.")

    def _set_buffer(self, name: str, value: torch.Tensor) -> None:
        if name in self._buffers:
            self._buffers[name] = value
        else:
            self.register_buffer(name, value)

    def load_dense_weight(self, key: str, source: torch.Tensor, *,
                          rotation: torch.Tensor | None = None) -> None:
        """Quantise a dense [E, out, in] expert tensor into this module's format
        (experts.py:940-996; the MI355X formats of mirai_amd.quant)."""
        if key not in self._spec.tensor_names:
            raise ValueError(f"Unknown compressed_weights grouped expert tensor '{key}'.")
        if source.ndim != 3:
            raise ValueError(
                f"compressed_weights grouped expert tensor {key} must be 3D, got "
                f"{tuple(source.shape)}.")
        if rotation is not None:
            raise ValueError("Learned expert rotations are not part of the MI355X INT8/NF4 formats.")
        if int(source.shape[0]) != self.num_experts:
            raise ValueError(
                f"compressed_weights grouped expert tensor {key} has {int(source.shape[0])} "
                f"experts, expected {self.num_experts}.")
        packed = quant.quantize(source, self._quant_format)
        data_suffix, scale_suffix = _BUFFER_SUFFIXES[packed.fmt]
        self._set_buffer(f"{key}{data_suffix}", packed.data)
        if scale_suffix is not None:
            self._set_buffer(f"{key}{scale_suffix}", packed.scale)
        self._shapes[key] = packed.shape
        self._layouts[key] = packed.layout
        self._loaded_dense_keys.add(key)

    def load_packed_nf4(self, key: str, *, packed: torch.Tensor, absmax: torch.Tensor,
                        nested_absmax: torch.Tensor, offset: torch.Tensor, code: torch.Tensor,
                        nested_code: torch.Tensor, shape: tuple[int, int, int],
                        layout: str = "out_in", two_level: bool = False) -> None:
        """Adopt a bitsandbytes double-quantised NF4 stack as the reference stores it
        (the {key}_nf4* buffers of _store_nf4_grouped, experts.py:998-1031) without
        re-quantising: the GEMMs decode the payload's weights. ``shape`` is the
        logical [E, out, in]; ``layout="in_out"`` takes payloads that quantise
        each expert's [in, out] matrix (MAGI-2 groups). The absmax is decoded to
        fp32 once, or with ``two_level=True`` kept as the payload stores it
        ({key}_nf4_absmax uint8, _nf4_nabsmax, _nf4_offset, _nf4_ncode) and
        decoded by the GEMMs per K step."""
        if self._quant_format != "nf4":
            raise ValueError("packed NF4 payloads load into a module with quant_format='nf4'.")
        if key not in self._spec.tensor_names:
            raise ValueError(f"Unknown compressed_weights grouped expert tensor '{key}'.")
        if int(shape[0]) != self.num_experts:
            raise ValueError(
                f"compressed_weights grouped expert tensor {key} has {int(shape[0])} experts, "
                f"expected {self.num_experts}.")
        packed_w = quant.from_bnb_nf4(packed=packed, absmax=absmax, nested_absmax=nested_absmax,
                                      offset=offset, code=code, nested_code=nested_code,
                                      shape=tuple(int(v) for v in shape), layout=layout,
                                      two_level=two_level)
        data_suffix, scale_suffix = _BUFFER_SUFFIXES["nf4"]
        self._set_buffer(f"{key}{data_suffix}", packed_w.data)
        self._set_buffer(f"{key}{scale_suffix}", packed_w.scale)
        for suffix, field in _TWO_LEVEL_BUFFERS:
            name = f"{key}{suffix}"
            if packed_w.dq is not None:
                self._set_buffer(name, packed_w.dq[field])
            elif name in self._buffers:
                del self._buffers[name]
        if packed_w.dq is not None:
            self._two_level.add(key)
        else:
            self._two_level.discard(key)
        self._shapes[key] = packed_w.shape
        self._layouts[key] = packed_w.layout
        self._loaded_dense_keys.add(key)

    def load_bnb_state_dict(self, state: dict, shapes: dict, *, prefix: str = "",
                            two_level: bool = False) -> None:
        """Load every expert tensor of ``shapes`` ({key: (E, out, in)}) from a
        reference state dict holding its {key}_nf4, _nf4_absmax, _nf4_nabsmax,
        _nf4_offset, _nf4_code and _nf4_ncode buffers (``two_level``: see
        load_packed_nf4)."""
        for key, shape in shapes.items():
            base = f"{prefix}{key}_nf4"
            missing = [n for n in ("", "_absmax", "_nabsmax", "_offset", "_code", "_ncode")
                       if base + n not in state]
            if missing:
                raise RuntimeError(f"packed NF4 state for '{key}' lacks "
                                   + ", ".join(base + n for n in missing) + ".")
            self.load_packed_nf4(key, packed=state[base], absmax=state[base + "_absmax"],
                                 nested_absmax=state[base + "_nabsmax"],
                                 offset=state[base + "_offset"], code=state[base + "_code"],
                                 nested_code=state[base + "_ncode"], shape=shape,
                                 two_level=two_level)

    def packed_buffer_names(self, key: str) -> tuple[str, ...]:
        """Names of the buffers that hold expert tensor ``key`` in this format."""
        data_suffix, scale_suffix = _BUFFER_SUFFIXES[self._quant_format]
        names = (f"{key}{data_suffix}",) + ((f"{key}{scale_suffix}",) if scale_suffix else ())
        if key in self._two_level:
            names += tuple(f"{key}{suffix}" for suffix, _ in _TWO_LEVEL_BUFFERS)
        return names

    def packed_weight(self, key: str) -> quant.PackedWeight:
        if key not in self._loaded_dense_keys:
            raise RuntimeError(f"compressed_weights grouped experts are missing weight '{key}'.")
        data_suffix, scale_suffix = _BUFFER_SUFFIXES[self._quant_format]
        data = getattr(self, f"{key}{data_suffix}")
        scale = getattr(self, f"{key}{scale_suffix}") if scale_suffix else None
        dq = None
        if key in self._two_level:
            dq = {field: getattr(self, f"{key}{suffix}") for suffix, field in _TWO_LEVEL_BUFFERS}
        return quant.PackedWeight(self._quant_format, data, scale, self._shapes[key],
                                  self._layouts.get(key, "out_in"), dq)

    def packed_nbytes(self) -> int:
        return sum(self.packed_weight(k).nbytes() for k in self._loaded_dense_keys)

    # --------------------------------------------------------------- LoRA
    def attach_expert_lora(self, *, tensor_name: str, adapter_name: str, rank: int, alpha: float,
                           init: str = "kaiming", use_rslora: bool = False) -> nn.Module:
        """experts.py:544-571."""
        key = str(tensor_name)
        if key not in self._spec.tensor_names:
            raise ValueError(f"Unknown grouped expert LoRA tensor '{key}'.")
        if key in self.expert_lora:
            raise ValueError(f"Grouped expert LoRA is already attached to '{key}'.")
        shape = self.expert_weight_shape(key)
        adapter = ActiveExpertLoRA(adapter_name=str(adapter_name), num_experts=int(shape[0]),
                                   out_features=int(shape[1]), in_features=int(shape[2]),
                                   rank=int(rank), alpha=float(alpha), init=str(init),
                                   use_rslora=bool(use_rslora))
        data = self.packed_weight(key).data
        if data.device.type == "cuda":
            adapter.to(data.device)
        self.expert_lora[key] = adapter
        return adapter

    # ------------------------------------------------------------ dequant
    def _dequantize(self, key: str, *, dtype: torch.dtype | None = None,
                    device: torch.device | None = None) -> torch.Tensor:
        out = quant.dequantize(self.packed_weight(key), dtype=dtype or torch.bfloat16)
        return out if device is None else out.to(device)

    def _dequantize_expert(self, key: str, expert_idx: int, *, dtype: torch.dtype,
                           device: torch.device) -> torch.Tensor:
        i = int(expert_idx)
        out = quant.dequantize(self.packed_weight(key), dtype=dtype, experts=slice(i, i + 1))
        return out[0].to(device)

    @property
    def w1(self) -> torch.Tensor:
        return self._dequantize("w1")

    @property
    def w2(self) -> torch.Tensor:
        return self._dequantize("w2")

    @property
    def w3(self) -> torch.Tensor:
        return self._dequantize("w3")

    # ----------------------------------------------------------- execution
    def _require_loaded(self) -> None:
        if not self.is_fully_loaded():
            missing = sorted(set(self._spec.tensor_names) - self._loaded_dense_keys)
            raise RuntimeError(
                f"compressed_weights grouped experts are missing weights: {missing}.")

    def _role_keys(self) -> tuple[str, str, str]:
        return (self.projection_for_role("gate"), self.projection_for_role("up"),
                self.projection_for_role("down"))

    def _adapters(self) -> list[ActiveExpertLoRA | None]:
        return [self.expert_lora[k] if k in self.expert_lora else None for k in self._role_keys()]

    def run_direct_routed(self, tokens: torch.Tensor, top_scores: torch.Tensor,
                          top_indices: torch.Tensor) -> torch.Tensor:
        """Gate-weighted routed layer output [T, d] in ``tokens.dtype``
        (experts.py:1749-1912); fp32 accumulation of the k expert outputs."""
        top_scores, top_indices = self.direct_routes(tokens, top_scores, top_indices)
        from .fused import routed_experts
        return routed_experts(self, tokens, top_scores, top_indices)

    def direct_routes(self, tokens: torch.Tensor, top_scores: torch.Tensor,
                      top_indices: torch.Tensor):
        """The checks of run_direct_routed (experts.py:1755-1769) and the physical
        routes it executes: logical aliases coalesced (experts.py:339,
        2361-2367). Token chunking applies this once over all tokens, so each
        chunk runs exactly the routes the unchunked layer would."""
        if not self.prefers_for_loop():
            raise RuntimeError(
                "Direct routed compressed_weights execution requires active_dequant, "
                "chunked_dequant, or fused_kernel expert access.")
        if top_scores.shape != top_indices.shape or top_indices.ndim != 2:
            raise ValueError(
                "Direct routed compressed_weights execution requires matching "
                "[tokens, top_k] score and index tensors.")
        if int(top_indices.shape[0]) != int(tokens.shape[0]):
            raise ValueError("Direct routed expert indices do not match token count.")
        self._require_loaded()
        return self._coalesce_logical_routes(top_scores, top_indices)

    def logical_to_physical_map(self) -> tuple[int, ...]:
        """Logical -> physical expert aliases (empty: identity)."""
        return tuple(getattr(self, "_logical_to_physical", ()))

    def has_logical_expert_aliases(self) -> bool:
        return bool(self.logical_to_physical_map())

    def configure_logical_expert_aliases(self, logical_to_physical, *,
                                         prototype_logical_ids=None) -> None:
        """Attach a validated logical-router -> physical-expert map
        (experts.py:392-431 with validate_logical_to_physical,
        storage/aliases.py:85-107): more logical than physical experts, every
        physical id referenced, one prototype logical id per physical expert."""
        values = tuple(int(v) for v in logical_to_physical)
        if len(values) <= self.num_experts:
            raise ValueError("A consolidated mapping must have more logical than physical experts.")
        invalid = sorted({v for v in values if v < 0 or v >= self.num_experts})
        if invalid:
            raise ValueError(f"Logical-to-physical mapping contains invalid ids: {invalid}.")
        missing = sorted(set(range(self.num_experts)) - set(values))
        if missing:
            raise ValueError(
                f"Logical-to-physical mapping does not reference physical ids: {missing}.")
        if prototype_logical_ids is None:
            prototypes = tuple(values.index(p) for p in range(self.num_experts))
        else:
            prototypes = tuple(int(v) for v in prototype_logical_ids)
        if len(prototypes) != self.num_experts or len(set(prototypes)) != len(prototypes):
            raise ValueError(
                "prototype_logical_ids must contain one unique id per physical expert.")
        if any(v < 0 or v >= len(values) for v in prototypes):
            raise ValueError("prototype_logical_ids contains an out-of-range logical id.")
        if any(values[lid] != pid for pid, lid in enumerate(prototypes)):
            raise ValueError("Each prototype logical id must map to its corresponding physical id.")
        self.set_logical_to_physical_map(values)
        self.logical_num_experts = len(values)
        self.prototype_logical_ids = prototypes

    def set_logical_to_physical_map(self, aliases) -> None:
        aliases = tuple(int(v) for v in aliases)
        if any(v < 0 or v >= self.num_experts for v in aliases):
            raise ValueError("Logical expert alias map contains an invalid physical id.")
        self._logical_to_physical = aliases
        self._alias_device_maps = {}

    def _coalesce_logical_routes(self, top_scores: torch.Tensor, top_indices: torch.Tensor):
        """Token-choice routes over logical experts -> physical routes
        (experts.py:529-542 with coalesce_alias_routes, storage/aliases.py:156-199):
        each slot takes its logical expert's physical id, and the scores of a
        token's slots that land on one physical expert are summed into the
        first such slot. Every slot whose coalesced score is zero (the later
        duplicates, and routes the router scored zero) is then left out of the
        layer, as the reference's dispatch keeps only nonzero scores when
        aliases are active (experts.py:2361-2367): its id becomes
        ROUTE_DROPPED, which the plan and the combine skip. A logical id
        outside the map becomes an invalid physical id, which the dispatch plan
        reports (mirai_amd.check_route_errors) instead of a host sync here."""
        aliases = self.logical_to_physical_map()
        if not aliases:
            return top_scores, top_indices
        device = top_indices.device
        maps = self.__dict__.setdefault("_alias_device_maps", {})
        mapping = maps.get(str(device))
        if mapping is None:
            mapping = maps[str(device)] = torch.tensor(aliases, dtype=torch.long, device=device)
        logical = top_indices.long()
        valid = (logical >= 0) & (logical < len(aliases))
        physical = torch.where(valid, mapping[logical.clamp(0, len(aliases) - 1)],
                               torch.full_like(logical, -1))
        k = int(physical.shape[1])
        if k == 0:
            return top_scores, physical
        current = torch.arange(k, device=device).view(1, k, 1)
        candidate = torch.arange(k, device=device).view(1, 1, k)
        eligible = (physical.unsqueeze(2) == physical.unsqueeze(1)) & (candidate <= current)
        first = torch.where(eligible, candidate.expand_as(eligible),
                            torch.full_like(eligible, k, dtype=torch.long)).amin(dim=2)
        coalesced = torch.zeros_like(top_scores).scatter_add(1, first, top_scores)
        dropped = valid & (coalesced.detach() == 0)
        physical = torch.where(dropped, torch.full_like(physical, nat.ROUTE_DROPPED), physical)
        return coalesced, physical

    def run_expert_choice_routed(self, tokens: torch.Tensor, expert_token_scores: torch.Tensor,
                                 expert_token_indices: torch.Tensor, *,
                                 tokens_per_sample: int) -> torch.Tensor:
        """Expert-choice routes [B, L, C] through the fused kernels
        (experts.py:1954-1974, expert_choice.py:16-152): [B * tokens_per_sample, d]
        in ``tokens.dtype``, each token the fp32 sum of score * expert output
        over the (sample, expert, slot) entries that picked it."""
        if self.expert_weight_access not in {"active_dequant", "chunked_dequant", "fused_kernel"}:
            raise RuntimeError(
                "Expert-Choice compressed dispatch requires active_dequant or "
                "chunked_dequant expert access.")
        if int(tokens.shape[0]) != int(expert_token_indices.shape[0]) * int(tokens_per_sample):
            raise ValueError("Expert-Choice batch/token dimensions do not match tokens.")
        self._require_loaded()
        from .fused import expert_choice_experts
        return expert_choice_experts(self, tokens, expert_token_scores, expert_token_indices,
                                     int(tokens_per_sample), self.logical_to_physical_map())

    def run_for_loop(self, tokens: torch.Tensor, counts: torch.Tensor) -> torch.Tensor:
        """Expert MLP of rows already grouped by expert (experts.py:1656-1747)."""
        self._require_loaded()
        from .fused import sorted_experts
        return sorted_experts(self, tokens, counts)

    def run_batched(self, tokens: torch.Tensor, counts: torch.Tensor) -> torch.Tensor:
        """experts.py:915-938; the grouped kernels need no padding, so this is
        the same computation as run_for_loop."""
        return self.run_for_loop(tokens, counts)

    def grouped_linear(self, key: str, x: torch.Tensor, *, offsets: torch.Tensor) -> torch.Tensor:
        """One projection over expert-sorted rows with inclusive int32 ``offsets``
        (experts.py:803-827); no per-call group-count cap."""
        if self.prefers_for_loop():
            raise RuntimeError(
                "Grouped compressed_weights execution requires resident full_dequant expert weights.")
        from .fused import grouped_projection
        return grouped_projection(self, str(key), x, offsets)

    def extra_repr(self) -> str:
        return (f"num_experts={self.num_experts}, dtype={self._quant_format}, "
                f"expert_weight_access={self.expert_weight_access}")
