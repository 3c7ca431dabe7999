"""Expert-MLP layout spec and the MoE runtime policy read by the expert op.

Mirrors the names and validation of mirai/core/moe/runtime/specs.py
(ExpertProjectionRole :111-127, ExpertMLPExecutionSpec :129-213,
CANONICAL_PACKED_EXPERT_MLP_SPEC :222-231, normalize_expert_weight_access_policy
:483-506, MoEOptimizationPolicy :234-267 and the active-policy helpers
:555-600). Only the fields the expert op consumes are interpreted; the rest of
the reference policy surface (storage, streaming, autotune) is out of scope.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass

# "swiglu7" extends the reference set with the MAGI-2 gated activation
# (mirai/core/models/magi2_preview/grouped_moe.py:287-306), which the reference
# runs in its separate MAGI-2 grouped backend rather than through this spec.
EXPERT_MLP_ACTIVATIONS = {"silu", "gelu", "relu", "identity", "swiglu7"}
# Gated activations the fused MI355X kernels implement (with combiner
# "gated_product").
FUSED_GATED_ACTIVATIONS = ("silu", "swiglu7")
EXPERT_MLP_COMBINERS = {"gated_product", "activated"}
EXPERT_WEIGHT_ACCESS_POLICIES = {
    "auto",
    "disabled",
    "full_dequant",
    "active_dequant",
    "chunked_dequant",
    "fused_kernel",
}
MOE_DISPATCH_MODES = ("vectorized", "legacy", "triton", "triton_persistent")
MOE_DISPATCH_PREPROCESS_MODES = ("host", "device", "sonic")
MOE_GEMM_BACKENDS = ("auto", "bmm", "persistent", "torch_grouped", "deepgemm_fp8")

_ACCESS_ALIASES = {
    "": "auto",
    "none": "disabled",
    "off": "disabled",
    "full": "full_dequant",
    "dequant": "full_dequant",
    "active": "active_dequant",
    "selective": "active_dequant",
    "selective_dequant": "active_dequant",
    "chunked": "chunked_dequant",
    "chunk": "chunked_dequant",
    "fused": "fused_kernel",
    "kernel": "fused_kernel",
}


def normalize_expert_weight_access_policy(value: str | None) -> str:
    text = str(value or "auto").strip().lower()
    normalized = _ACCESS_ALIASES.get(text, text)
    if normalized not in EXPERT_WEIGHT_ACCESS_POLICIES:
        raise ValueError(
            "memory.expert_weight_access must be one of: "
            + ", ".join(sorted(EXPERT_WEIGHT_ACCESS_POLICIES))
            + "."
        )
    return normalized


@dataclass(frozen=True)
class ExpertProjectionRole:
    role: str
    tensor_name: str

    def __post_init__(self) -> None:
        role = str(self.role).strip().lower()
        name = str(self.tensor_name).strip()
        if role not in {"input", "gate", "up", "down"}:
            raise ValueError(f"Unsupported expert projection role {role!r}.")
        if not name:
            raise ValueError("Expert projection tensor_name must be non-empty.")
        object.__setattr__(self, "role", role)
        object.__setattr__(self, "tensor_name", name)


@dataclass(frozen=True)
class ExpertMLPExecutionSpec:
    projections: tuple[ExpertProjectionRole, ...]
    activation: str = "silu"
    combiner: str = "gated_product"

    def __post_init__(self) -> None:
        projections = tuple(self.projections)
        roles = [p.role for p in projections]
        names = [p.tensor_name for p in projections]
        if len(roles) != len(set(roles)):
            raise ValueError("Expert MLP projection roles must be unique.")
        if len(names) != len(set(names)):
            raise ValueError("Expert MLP tensor names must be unique.")
        activation = str(self.activation).strip().lower()
        combiner = str(self.combiner).strip().lower()
        if activation not in EXPERT_MLP_ACTIVATIONS:
            raise ValueError(
                "Expert MLP activation must be one of: "
                + ", ".join(sorted(EXPERT_MLP_ACTIVATIONS)) + "."
            )
        if combiner not in EXPERT_MLP_COMBINERS:
            raise ValueError(
                "Expert MLP combiner must be one of: "
                + ", ".join(sorted(EXPERT_MLP_COMBINERS)) + "."
            )
        required = {"gate", "up", "down"} if combiner == "gated_product" else {"input", "down"}
        if set(roles) != required:
            raise ValueError(
                f"Expert MLP combiner {combiner!r} requires roles "
                f"{sorted(required)}, got {sorted(roles)}."
            )
        object.__setattr__(self, "projections", projections)
        object.__setattr__(self, "activation", activation)
        object.__setattr__(self, "combiner", combiner)

    @property
    def tensor_names(self) -> tuple[str, ...]:
        return tuple(p.tensor_name for p in self.projections)

    @property
    def uses_gated_product(self) -> bool:
        return self.combiner == "gated_product"

    def tensor_for_role(self, role: str) -> str:
        normalized = str(role).strip().lower()
        for p in self.projections:
            if p.role == normalized:
                return p.tensor_name
        raise KeyError(f"Expert MLP layout has no {normalized!r} projection.")


CANONICAL_PACKED_EXPERT_MLP_SPEC = ExpertMLPExecutionSpec(
    projections=(
        ExpertProjectionRole("gate", "w1"),
        ExpertProjectionRole("up", "w3"),
        ExpertProjectionRole("down", "w2"),
    ),
    activation="silu",
    combiner="gated_product",
)


# MAGI-2 routed experts (CoreMultiHeadMoE, mirai/vendors/magi2_preview/model/
# magi2_preview.py:2680-2704): gate W_gate, up W_up, down W_down, swiglu7.
MAGI2_EXPERT_MLP_SPEC = ExpertMLPExecutionSpec(
    projections=(
        ExpertProjectionRole("gate", "W_gate"),
        ExpertProjectionRole("up", "W_up"),
        ExpertProjectionRole("down", "W_down"),
    ),
    activation="swiglu7",
    combiner="gated_product",
)


@dataclass(frozen=True)
class MoEOptimizationPolicy:
    """The hot-path subset of the reference MoE runtime policy.

    The dispatch / GEMM-backend fields are accepted for call-site
    compatibility: on this build every setting runs the same fused MI355X
    kernels, so they only have to name a valid reference mode.
    """

    expert_weight_access: str = "auto"
    expert_dequant_chunk_size: int = 0
    moe_dispatch: str = "vectorized"
    moe_dispatch_preprocess: str = "host"
    moe_gemm_backend: str = "auto"
    moe_batched_dequant: bool = True
    moe_pair_dequant: bool = True

    def __post_init__(self) -> None:
        access = normalize_expert_weight_access_policy(self.expert_weight_access)
        dispatch = str(self.moe_dispatch or "vectorized").strip().lower()
        if dispatch not in MOE_DISPATCH_MODES:
            raise ValueError(
                "memory.moe_dispatch must be one of: " + ", ".join(MOE_DISPATCH_MODES) + "."
            )
        preprocess = str(self.moe_dispatch_preprocess or "host").strip().lower()
        if preprocess not in MOE_DISPATCH_PREPROCESS_MODES:
            raise ValueError(
                "memory.moe_dispatch_preprocess must be one of: "
                + ", ".join(MOE_DISPATCH_PREPROCESS_MODES) + "."
            )
        backend = str(self.moe_gemm_backend or "auto").strip().lower()
        if backend not in MOE_GEMM_BACKENDS:
            raise ValueError(
                "memory.moe_gemm_backend must be one of: " + ", ".join(MOE_GEMM_BACKENDS) + "."
            )
        if int(self.expert_dequant_chunk_size) < 0:
            raise ValueError("memory.expert_dequant_chunk_size must be >= 0.")
        object.__setattr__(self, "expert_weight_access", access)
        object.__setattr__(self, "moe_dispatch", dispatch)
        object.__setattr__(self, "moe_dispatch_preprocess", preprocess)
        object.__setattr__(self, "moe_gemm_backend", backend)


_ACTIVE_POLICY: MoEOptimizationPolicy | None = None


def set_active_moe_optimization_policy(policy: MoEOptimizationPolicy | None) -> None:
    global _ACTIVE_POLICY
    _ACTIVE_POLICY = policy


@contextmanager
def active_moe_optimization_policy(policy: MoEOptimizationPolicy):
    previous = _ACTIVE_POLICY
    set_active_moe_optimization_policy(policy)
    try:
        yield policy
    finally:
        set_active_moe_optimization_policy(previous)


def get_active_moe_optimization_policy() -> MoEOptimizationPolicy:
    return _ACTIVE_POLICY or MoEOptimizationPolicy()
