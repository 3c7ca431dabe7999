"""Per-expert LoRA factors (the state of the reference's ActiveExpertLoRA).

Parameter names, shapes and scaling follow
mirai/core/models/compressed_weights/execution/active_expert_lora.py:43-116:
``lora_a`` [E, r, in] (kaiming-uniform, a=sqrt(5), as
mirai/core/models/adapters/lora_initialization.py:208-212), ``lora_b``
[E, out, r] (zeros), ``lora_alpha`` buffer, scale
``lora_scale(alpha, r, use_rslora) * _lora_scale * _rank_schedule_scale``
(mirai/core/models/adapters/lora_allocation.py:163-168). The delta itself is
computed inside the fused grouped GEMMs of the expert op.
"""

from __future__ import annotations

import math

import torch
import torch.nn as nn

# Largest rank the fused kernels take: ranks up to 32 run as one LDS-staged
# K chunk of the GEMM epilogues, larger ones add 32-wide chunks.
MAX_FUSED_RANK = 256


def lora_scale(alpha: float, rank: int, *, use_rslora: bool) -> float:
    resolved = int(rank)
    if resolved <= 0:
        raise ValueError("LoRA rank must be positive when computing scale.")
    denominator = math.sqrt(resolved) if bool(use_rslora) else float(resolved)
    return float(alpha) / denominator


_INITIALIZERS = ("kaiming", "gaussian", "zeros")


class ActiveExpertLoRA(nn.Module):
    _mirai_expert_lora_adapter = True

    def __init__(self, *, adapter_name: str, num_experts: int, in_features: int,
                 out_features: int, rank: int, alpha: float, init: str = "kaiming",
                 use_rslora: bool = False) -> None:
        super().__init__()
        if int(rank) <= 0:
            raise ValueError("Expert LoRA rank must be > 0.")
        if int(rank) > MAX_FUSED_RANK:
            raise ValueError(
                f"Expert LoRA rank {rank} exceeds the fused-kernel limit of {MAX_FUSED_RANK}."
            )
        init_name = str(init).strip().lower()
        if init_name not in _INITIALIZERS:
            raise ValueError(f"Unknown LoRA initializer {init!r}; supported: {_INITIALIZERS}.")
        self.adapter_name = str(adapter_name)
        self.rank = int(rank)
        self.use_rslora = bool(use_rslora)
        self.in_features = int(in_features)
        self.out_features = int(out_features)
        self.lora_a = nn.Parameter(torch.empty(int(num_experts), self.rank, self.in_features))
        self.lora_b = nn.Parameter(torch.zeros(int(num_experts), self.out_features, self.rank))
        self.register_buffer("lora_alpha", torch.tensor(float(alpha), dtype=torch.float32),
                             persistent=True)
        self._lora_scale = 1.0
        self._rank_schedule_scale = 1.0
        with torch.no_grad():
            if init_name == "kaiming":
                nn.init.kaiming_uniform_(self.lora_a, a=math.sqrt(5))
            elif init_name == "gaussian":
                nn.init.normal_(self.lora_a, std=1.0 / self.rank)
            else:
                self.lora_a.zero_()

    def _alpha(self) -> float:
        """lora_alpha as a Python float, read from the (device) buffer only when
        the buffer changes: a read per call would synchronise the host with the
        GPU on every forward, and cannot happen under HIP graph capture."""
        buf = self.lora_alpha
        key = (buf.data_ptr(), buf._version, str(buf.device))
        cached = self.__dict__.get("_alpha_cache")
        if cached is None or cached[0] != key:
            cached = (key, float(buf))
            self.__dict__["_alpha_cache"] = cached
        return cached[1]

    def scale(self) -> float:
        return (
            lora_scale(self._alpha(), self.rank, use_rslora=self.use_rslora)
            * self._lora_scale
            * self._rank_schedule_scale
        )

    def padded_rank(self) -> int:
        """Rank rounded up to the kernel's multiple of 8 (zero-padded factors)."""
        return (self.rank + 7) // 8 * 8

    def kernel_factors(self, device: torch.device, *,
                       split: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """bf16 copies of A [E, r8, in] and B [E, out, r8] for the fused kernels.

        Padding rows of A and columns of B are zero, which leaves the product
        unchanged. ``split`` (the fp32 layer) returns the fp32 factors as bf16
        planes [hi | lo | hi] instead: A [E, r8, 3*in], B [E, out, 3*r8].
        """
        # The packed copies are kept while the parameters are unchanged (same
        # storage, same in-place version), so inference packs them once.
        key = (str(device), bool(split), self.lora_a.data_ptr(), self.lora_a._version,
               self.lora_b.data_ptr(), self.lora_b._version)
        cached = self.__dict__.get("_kernel_cache")
        if cached is not None and cached[0] == key:
            return cached[1]
        factors = self._pack_factors(device, split)
        self.__dict__["_kernel_cache"] = (key, factors)
        return factors

    def _pack_factors(self, device, split):
        dtype = torch.float32 if split else torch.bfloat16
        a = self.lora_a.detach().to(device=device, dtype=dtype)
        b = self.lora_b.detach().to(device=device, dtype=dtype)
        pad = self.padded_rank() - self.rank
        if pad:
            a = torch.cat([a, a.new_zeros(a.shape[0], pad, a.shape[2])], dim=1)
            b = torch.cat([b, b.new_zeros(b.shape[0], b.shape[1], pad)], dim=2)
        if split:
            from .quant import split_planes
            from ._native import SPLIT_WEIGHT
            return split_planes(a, SPLIT_WEIGHT), split_planes(b, SPLIT_WEIGHT)
        return a.contiguous(), b.contiguous()

    def extra_repr(self) -> str:
        return (f"adapter={self.adapter_name}, experts={self.lora_a.shape[0]}, "
                f"in={self.in_features}, out={self.out_features}, rank={self.rank}")
