"""Expert-MLP layout spec read by the expert op.

Mirrors the names and validation of mirai/core/moe/runtime/specs.py
(ExpertProjectionRole :111-127, ExpertMLPExecutionSpec :129-213,
CANONICAL_PACKED_EXPERT_MLP_SPEC :222-231, normalize_expert_weight_access_policy
:483-506). Provider code hands the expert module its own spec objects
(prepare.py:46-48, lingbot_video/pipeline.py:1678), so ``as_execution_spec``
accepts any object with the same fields and converts it.
"""

from __future__ import annotations

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


def as_execution_spec(spec) -> ExpertMLPExecutionSpec:
    """This package's spec for ``spec``: the object itself, or a validated copy
    of any spec object exposing ``projections`` (items with ``role`` and
    ``tensor_name``), ``activation`` and ``combiner`` -- the reference's own
    ExpertMLPExecutionSpec included. Anything else raises TypeError, as the
    reference's isinstance check does (experts.py:164-165)."""
    if isinstance(spec, ExpertMLPExecutionSpec):
        return spec
    try:
        projections = tuple(spec.projections)
        roles = tuple(ExpertProjectionRole(str(p.role), str(p.tensor_name)) for p in projections)
        activation = str(spec.activation)
        combiner = str(spec.combiner)
    except (AttributeError, TypeError) as exc:
        raise TypeError("execution_spec must use ExpertMLPExecutionSpec.") from exc
    return ExpertMLPExecutionSpec(projections=roles, activation=activation, combiner=combiner)
