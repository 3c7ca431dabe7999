"""Seeded synthetic workloads of the benchmark configurations.

C1-C5 are the five configurations of the benchmark definition; ``target`` is
the C2 geometry at 32768 tokens on which the throughput goal is stated.
Seeds: 1000 + config index for logits, +1 weights, +2 LoRA, +3 tokens, +4 dY.
Inputs: tokens ~ N(0, 1) in the activation dtype, frozen weights ~ N(0, 0.02)
(fp32 for C1's unquantised fp32 layer, else rounded to bf16 before any
quantisation), LoRA A, B ~ N(0, 0.02), router logits ~ N(0, 1) (plus a
per-expert Zipf(1.2) bias for C3), upstream gradient ~ N(0, 1).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, replace

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    index: int
    tokens: int
    hidden: int
    ffn: int
    experts: int
    top_k: int
    rank: int
    alpha: float
    fmt: str                  # "fp32" | "bf16" | "nf4" | "int8"
    dtype: torch.dtype
    zipf: float = 0.0         # Zipf exponent of the per-expert logit bias (0: none)
    backward: bool = False

    @property
    def routed_rows(self) -> int:
        return self.tokens * self.top_k

    def flops(self) -> int:
        """Algorithmic forward FLOPs: base 2*R*3*d*f plus LoRA 2*R*r*3*(d+f)."""
        R, d, f, r = self.routed_rows, self.hidden, self.ffn, self.rank
        return 2 * R * 3 * d * f + 2 * R * r * 3 * (d + f)

    def with_tokens(self, tokens: int) -> "Workload":
        return replace(self, tokens=int(tokens))


WORKLOADS = {
    "c1": Workload("c1_fp32_plumbing", 0, 512, 512, 1024, 8, 2, 8, 16.0, "fp32", torch.float32),
    "c2": Workload("c2_nf4_balanced", 1, 4096, 2048, 1408, 64, 4, 16, 16.0, "nf4", torch.bfloat16),
    "c3": Workload("c3_nf4_zipf", 2, 8192, 2048, 768, 128, 8, 8, 16.0, "nf4", torch.bfloat16,
                   zipf=1.2),
    "c4": Workload("c4_int8_cfg", 3, 32760, 3072, 2048, 64, 4, 32, 32.0, "int8", torch.bfloat16),
    "c5": Workload("c5_nf4_train", 4, 8192, 2048, 1408, 64, 4, 16, 16.0, "nf4", torch.bfloat16,
                   backward=True),
    "target": Workload("c2_nf4_T32768", 1, 32768, 2048, 1408, 64, 4, 16, 16.0, "nf4",
                       torch.bfloat16),
}

ZIPF_BETA_LADDER = (0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, 8.0)


def _gen(seed: int, device) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(int(seed))


def zipf_bias(w: Workload, logits: torch.Tensor) -> torch.Tensor:
    """Per-expert bias beta * log(p_e), p_e ~ (pi(e)+1)^-s with a seeded
    permutation pi; beta is the first ladder value leaving >= 5 experts empty."""
    g = _gen(1000 + w.index + 5, "cpu")
    perm = torch.randperm(w.experts, generator=g)
    logp = -w.zipf * torch.log(perm.double() + 1.0)
    logp = logp - torch.logsumexp(logp, dim=0)
    for beta in ZIPF_BETA_LADDER:
        bias = (beta * logp).float().to(logits.device)
        top = torch.topk(logits + bias, w.top_k, dim=1).indices
        used = torch.bincount(top.reshape(-1), minlength=w.experts)
        if int((used == 0).sum()) >= 5:
            return bias
    raise RuntimeError("no Zipf bias in the ladder leaves 5 experts without tokens")


def router_logits(w: Workload, device="cpu") -> torch.Tensor:
    logits = torch.randn(w.tokens, w.experts, generator=_gen(1000 + w.index, device),
                         device=device, dtype=torch.float32)
    if w.zipf:
        logits = logits + zipf_bias(w, logits)
    return logits


def tokens(w: Workload, device="cpu") -> torch.Tensor:
    return torch.randn(w.tokens, w.hidden, generator=_gen(1000 + w.index + 3, device),
                       device=device, dtype=torch.float32).to(w.dtype)


def upstream_grad(w: Workload, device="cpu") -> torch.Tensor:
    return torch.randn(w.tokens, w.hidden, generator=_gen(1000 + w.index + 4, device),
                       device=device, dtype=torch.float32).to(w.dtype)


def dense_weights(w: Workload, device="cpu", experts: int | None = None) -> dict[str, torch.Tensor]:
    """Frozen weights {w1, w3: [E, f, d], w2: [E, d, f]}, ~N(0, 0.02): fp32 for
    the fp32 format, else bf16."""
    E = w.experts if experts is None else int(experts)
    g = _gen(1000 + w.index + 1, device)
    dtype = torch.float32 if w.fmt == "fp32" else torch.bfloat16
    out = {}
    for key, shape in (("w1", (E, w.ffn, w.hidden)), ("w3", (E, w.ffn, w.hidden)),
                       ("w2", (E, w.hidden, w.ffn))):
        t = torch.empty(shape, dtype=dtype, device=device)
        for e in range(E):  # per expert keeps the fp32 temporary small
            t[e] = (torch.randn(shape[1:], generator=g, device=device) * 0.02).to(dtype)
        out[key] = t
    return out


def lora_factors(w: Workload, device="cpu") -> dict[str, tuple[torch.Tensor, torch.Tensor]]:
    """fp32 LoRA factors {key: (A [E, r, in], B [E, out, r])}, ~N(0, 0.02)."""
    g = _gen(1000 + w.index + 2, device)
    E, d, f, r = w.experts, w.hidden, w.ffn, w.rank
    out = {}
    for key, (o, i) in (("w1", (f, d)), ("w3", (f, d)), ("w2", (d, f))):
        a = torch.randn(E, r, i, generator=g, device=device) * 0.02
        b = torch.randn(E, o, r, generator=g, device=device) * 0.02
        out[key] = (a, b)
    return out


def lora_scale(w: Workload) -> float:
    return float(w.alpha) / float(w.rank)


def active_weight_bytes(w: Workload, counts) -> int:
    """Packed bytes of the experts that receive at least one row (3 projections)."""
    d, f, r = w.hidden, w.ffn, w.rank
    per = {"nf4": 3 * d * f // 2 + 3 * d * f // 64 * 2, "int8": 3 * d * f + (2 * f + d) * 2,
           "bf16": 3 * d * f * 2, "fp32": 3 * d * f * 4}[w.fmt]
    per += 3 * r * (d + f) * 2
    active = int((torch.as_tensor(counts) > 0).sum())
    return active * per


def algorithmic_bytes(w: Workload, counts) -> int:
    """HBM bytes a perfect fused layer must move: active packed weights + LoRA
    factors, tokens in, output out, routing metadata."""
    act = 2 if w.dtype == torch.bfloat16 else 4
    return (active_weight_bytes(w, counts) + 2 * w.tokens * w.hidden * act
            + w.routed_rows * (8 + 4))


def describe(w: Workload) -> dict:
    return {"workload": w.name, "tokens": w.tokens, "hidden": w.hidden, "ffn": w.ffn,
            "experts": w.experts, "top_k": w.top_k, "lora_rank": w.rank, "weights": w.fmt,
            "routed_rows": w.routed_rows}


def gflop(w: Workload) -> float:
    return w.flops() / 1e9


__all__ = ["Workload", "WORKLOADS", "router_logits", "tokens", "dense_weights", "lora_factors",
           "lora_scale", "algorithmic_bytes", "describe", "gflop", "upstream_grad", "math"]
