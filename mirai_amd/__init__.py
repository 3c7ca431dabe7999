"""MI355X-native sparse-MoE expert layer (gfx950 HIP kernels behind a C ABI).

Drop-in for the routed expert op of seruva19/mirai
(``CompressedGroupedExperts.run_direct_routed`` and friends); see
``mirai_amd.experts``.
"""

from .dispatch import (
    DispatchPlan,
    build_dispatch_plan,
    build_expert_choice_dispatch_plan,
    combine_routed_tokens,
    permute_routed_tokens,
)
from ._native import RouteIndexError, check_route_errors, set_route_check
from .chunking import MoETokenChunkPolicy, fused_chunk_runner
from .experts import CompressedGroupedExperts
from .lora import ActiveExpertLoRA, lora_scale
from .magi2 import (
    Magi2FusedMoEBackend,
    Magi2GroupedExperts,
    Magi2QuantizedExpertError,
    compute_topk_probs_and_indices,
    load_reference_magi2_artifact,
    read_reference_magi2_artifact,
    route_topk_heads,
)
from .router import FusedRouter, fused_router_forward, router_weight_planes
from .routing import route_topk
from .specs import (
    CANONICAL_PACKED_EXPERT_MLP_SPEC,
    ExpertMLPExecutionSpec,
    ExpertProjectionRole,
    as_execution_spec,
)

__all__ = [
    "ActiveExpertLoRA",
    "CANONICAL_PACKED_EXPERT_MLP_SPEC",
    "CompressedGroupedExperts",
    "DispatchPlan",
    "FusedRouter",
    "RouteIndexError",
    "ExpertMLPExecutionSpec",
    "ExpertProjectionRole",
    "Magi2FusedMoEBackend",
    "Magi2GroupedExperts",
    "Magi2QuantizedExpertError",
    "MoETokenChunkPolicy",
    "as_execution_spec",
    "build_dispatch_plan",
    "build_expert_choice_dispatch_plan",
    "check_route_errors",
    "compute_topk_probs_and_indices",
    "combine_routed_tokens",
    "fused_chunk_runner",
    "fused_router_forward",
    "load_reference_magi2_artifact",
    "lora_scale",
    "permute_routed_tokens",
    "read_reference_magi2_artifact",
    "route_topk",
    "route_topk_heads",
    "router_weight_planes",
    "set_route_check",
]
