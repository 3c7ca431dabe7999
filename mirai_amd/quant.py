"""Frozen-weight storage formats, quantised and decoded on the GPU.

* ``nf4``  : codes uint8 [E, out, in/2] (per group of 8 elements, byte i holds
  element i in the low nibble and element i + 4 in the high nibble) and
             bf16 absmax [E, out, in/64]; blocksize 64, no double quantisation.
             A bitsandbytes double-quantised payload ingested with
             ``from_bnb_nf4`` keeps the same codes with an fp32 absmax
             (kernel format MX_FMT_NF4_F32).
* ``int8`` : int8 [E, out, in] and bf16 per-output-row scale [E, out].
* ``bf16`` : unquantised bf16 [E, out, in].
* ``fp32`` : unquantised fp32 as bf16 planes [E, out, 3*in] = [hi | lo | hi]
             (hi = bf16(w), lo = bf16(w - hi)); with fp32 tokens split as
             [hi | hi | lo] the bf16 MFMA products reach fp32 accuracy.

Replaces the storage side of mirai/core/models/compressed_weights/quantization/quant.py
(_quantize_weight :189-235, _dequantize_weight :238-260, _nf4_quantize_2d
:315-358, nf4_dequantize_stack / _nf4_dequantize :380-472) in the BASELINE
formats; the per-element rules are documented in include/mirai_moe.h.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _native as nat

NF4_BLOCKSIZE = 64
QUANT_FORMATS = ("nf4", "int8", "bf16", "fp32")
_FORMAT_CODES = {"bf16": nat.FMT_BF16, "nf4": nat.FMT_NF4, "int8": nat.FMT_INT8,
                 "fp32": nat.FMT_F32X3}


def normalize_quant_format(value: str | None) -> str:
    text = str(value or "int8").strip().lower()
    text = {"": "int8", "auto": "int8", "bfloat16": "bf16", "none": "bf16", "float32": "fp32",
            "f32": "fp32"}.get(text, text)
    if text not in QUANT_FORMATS:
        raise ValueError(
            "compressed_weights quant_format must be one of: " + ", ".join(QUANT_FORMATS) + "."
        )
    return text


@dataclass
class PackedWeight:
    """One stored projection [E, out, in] in a GPU-resident format."""

    fmt: str
    data: torch.Tensor
    scale: torch.Tensor | None
    shape: tuple[int, int, int]
    # "out_in": data [E, out, ...] (the quantiser's layout); "in_out": data
    # [E, in, ...] with the NF4 blocks along out (an ingested MAGI-2 group
    # payload, x @ W[g]).
    layout: str = "out_in"
    # A bitsandbytes two-level absmax kept as stored (MX_FMT_NF4_DQ): ``scale``
    # holds the uint8 absmax codes [E, rows, cols / 64], this dict the nested
    # scales ``nested_absmax`` [E, n] fp32, the ``offsets`` [E] fp32 and the
    # 256-entry ``code`` table (fp32).
    dq: dict | None = None
    _dq_struct: object = field(default=None, repr=False, compare=False)

    def format_code(self) -> int:
        if self.fmt == "nf4" and self.dq is not None:
            return nat.FMT_NF4_DQ_KN if self.layout == "in_out" else nat.FMT_NF4_DQ
        if self.fmt == "nf4" and self.scale is not None and self.scale.dtype == torch.float32:
            return nat.FMT_NF4_F32_KN if self.layout == "in_out" else nat.FMT_NF4_F32
        if self.layout != "out_in":
            raise ValueError(f"the {self.fmt} format has no [E, in, out] kernel layout")
        return _FORMAT_CODES[self.fmt]

    def dq_struct(self, experts: slice | None = None) -> nat.MxNf4Dq:
        """The mx_nf4_dq of a two-level absmax (of an expert slice). The whole
        weight's struct is kept with the weight, which must outlive the calls
        that use its descriptor."""
        if experts is None and self._dq_struct is not None:
            return self._dq_struct
        sel = experts if experts is not None else slice(None)
        q = self.scale[sel]
        nested = self.dq["nested_absmax"][sel]
        offsets = self.dq["offsets"][sel]
        st = nat.MxNf4Dq(q.data_ptr(), nested.data_ptr(), offsets.data_ptr(),
                         self.dq["code"].data_ptr(), int(nested.shape[-1]))
        if experts is None:
            self._dq_struct = st
        return st

    def descriptor(self) -> nat.MxWeight:
        _, out_f, in_f = self.shape
        if self.dq is not None:
            scale = ctypes.addressof(self.dq_struct())
        else:
            scale = self.scale.data_ptr() if self.scale is not None else None
        return nat.MxWeight(self.format_code(), self.data.data_ptr(), scale, out_f, in_f)

    def nbytes(self) -> int:
        extra = sum(t.numel() * t.element_size() for t in (self.dq or {}).values())
        return self.data.numel() * self.data.element_size() + extra + (
            0 if self.scale is None else self.scale.numel() * self.scale.element_size()
        )


def quantize(source: torch.Tensor, fmt: str) -> PackedWeight:
    """Quantise a dense [E, out, in] tensor on the GPU into ``fmt``."""
    fmt = normalize_quant_format(fmt)
    if source.ndim != 3:
        raise ValueError(f"grouped expert tensor must be 3D, got {tuple(source.shape)}.")
    E, out_f, in_f = (int(v) for v in source.shape)
    if in_f % 64:
        raise ValueError(f"in_features must be a multiple of 64 for the MI355X kernels, got {in_f}.")
    device = source.device if source.device.type == "cuda" else torch.device("cuda")
    if not torch.cuda.is_available():
        raise nat.NativeLibraryError("quantisation runs on the GPU; no ROCm device is available.")
    w = source.detach().to(device=device)
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.float()
    w = w.contiguous()
    nat.require_gpu(w)
    rows = E * out_f
    s = nat.stream(device)
    if fmt == "bf16":
        return PackedWeight("bf16", w.to(torch.bfloat16).contiguous(), None, (E, out_f, in_f))
    if fmt == "fp32":
        return PackedWeight("fp32", split_planes(w.float(), nat.SPLIT_WEIGHT), None,
                            (E, out_f, in_f))
    if fmt == "nf4":
        codes = torch.empty((E, out_f, in_f // 2), dtype=torch.uint8, device=device)
        absmax = torch.empty((E, out_f, in_f // NF4_BLOCKSIZE), dtype=torch.bfloat16, device=device)
        nat.call("mx_nf4_quantize", w.data_ptr(), nat.dtype_code(w.dtype), rows, in_f,
                 codes.data_ptr(), absmax.data_ptr(), s)
        return PackedWeight("nf4", codes, absmax, (E, out_f, in_f))
    q = torch.empty((E, out_f, in_f), dtype=torch.int8, device=device)
    scale = torch.empty((E, out_f), dtype=torch.bfloat16, device=device)
    nat.call("mx_int8_quantize", w.data_ptr(), nat.dtype_code(w.dtype), rows, in_f,
             q.data_ptr(), scale.data_ptr(), s)
    return PackedWeight("int8", q, scale, (E, out_f, in_f))


def dequantize(packed: PackedWeight, *, dtype: torch.dtype = torch.bfloat16,
               experts: slice | None = None) -> torch.Tensor:
    """Dense weights (bit-exact codec output) of all or a slice of experts."""
    sel = experts if experts is not None else slice(None)
    data = packed.data[sel]
    E = int(data.shape[0])
    _, out_f, in_f = packed.shape
    device = data.device
    if packed.fmt == "bf16":
        return data.to(dtype)
    if packed.fmt == "fp32":  # hi + lo planes
        return (data[..., :in_f].float() + data[..., in_f:2 * in_f].float()).to(dtype)
    nat.require_gpu(data)
    scale_all = packed.scale
    if packed.dq is not None:
        # The two-level absmax as the GEMMs decode it, then the fp32-absmax path.
        scale_all = torch.empty((E, *packed.scale.shape[1:]), dtype=torch.float32, device=device)
        st = packed.dq_struct(sel)
        nat.call("mx_nf4_dq_absmax", ctypes.byref(st), E, int(packed.scale[0].numel()),
                 scale_all.data_ptr(), nat.stream(device))
        sel = slice(None)
    if packed.layout == "in_out":
        # Rows of the stored [E, in, out] payload, then the [E, out, in] view.
        flat = torch.empty((E, in_f, out_f), dtype=dtype, device=device)
        nat.call("mx_nf4_dequantize_ex", data.contiguous().data_ptr(),
                 scale_all[sel].contiguous().data_ptr(),
                 nat.dtype_code(scale_all.dtype), E * in_f, out_f, flat.data_ptr(),
                 nat.dtype_code(dtype), nat.stream(device))
        return flat.transpose(1, 2).contiguous()
    out = torch.empty((E, out_f, in_f), dtype=dtype, device=device)
    rows = E * out_f
    s = nat.stream(device)
    scale = scale_all[sel].contiguous()
    data = data.contiguous()
    if packed.fmt == "nf4":
        nat.call("mx_nf4_dequantize_ex", data.data_ptr(), scale.data_ptr(),
                 nat.dtype_code(scale.dtype), rows, in_f, out.data_ptr(), nat.dtype_code(dtype), s)
    else:
        nat.call("mx_int8_dequantize", data.data_ptr(), scale.data_ptr(), rows, in_f,
                 out.data_ptr(), nat.dtype_code(dtype), s)
    return out


def from_bnb_nf4(*, packed: torch.Tensor, absmax: torch.Tensor, nested_absmax: torch.Tensor,
                 offset: torch.Tensor, code: torch.Tensor, nested_code: torch.Tensor,
                 shape: tuple[int, int, int], blocksize: int = NF4_BLOCKSIZE,
                 nested_blocksize: int = 256, layout: str = "out_in",
                 two_level: bool = False) -> PackedWeight:
    """Ingest a bitsandbytes double-quantised NF4 expert stack without
    re-quantising (mx_nf4_from_bnb).

    The arguments are the reference's per-key buffers
    (CompressedGroupedExperts._store_nf4_grouped, experts.py:998-1031):
    ``{key}_nf4`` packed codes [E, out*in/2(, 1)] uint8, ``{key}_nf4_absmax``
    quantised absmax [E, out*in/64] uint8, ``{key}_nf4_nabsmax`` [E, n2] fp32,
    ``{key}_nf4_offset`` [E] fp32, ``{key}_nf4_code`` (the 16 NF4 levels) and
    ``{key}_nf4_ncode`` (256 fp32). Returns the codes in this library's layout
    with the decoded fp32 absmax. ``shape`` is the logical [E, out, in]; with
    ``layout="in_out"`` each expert's payload quantises the [in, out] matrix
    (the MAGI-2 store's [G, in, out] groups, quantized_experts.py:275-347, whose
    64-blocks run along out) and is kept in that orientation. With
    ``two_level=True`` the absmax stays as the payload stores it (uint8 codes,
    nested scales, offsets, code table) and the GEMMs decode it per K step
    (MX_FMT_NF4_DQ); otherwise it is decoded once to fp32 here.
    """
    E, out_f, in_f = (int(v) for v in shape)
    if layout not in ("out_in", "in_out"):
        raise ValueError(f"unknown layout {layout!r}")
    rows_f, cols_f = (out_f, in_f) if layout == "out_in" else (in_f, out_f)
    if int(blocksize) != NF4_BLOCKSIZE or int(nested_blocksize) != 256:
        raise ValueError("bitsandbytes NF4 payloads are ingested with blocksize 64 and "
                         "nested blocksize 256.")
    if cols_f % NF4_BLOCKSIZE:
        raise ValueError(f"the payload's row length must be a multiple of 64, got {cols_f}.")
    device = packed.device
    nat.require_gpu(packed)
    levels = code.detach().to(device="cpu", dtype=torch.float32).reshape(-1)
    if levels.numel() != 16 or not torch.equal(levels, nf4_levels()):
        raise ValueError("the payload's 4-bit code table is not the NF4 table (quant_type='nf4').")
    n = out_f * in_f
    n2 = -(-(n // NF4_BLOCKSIZE) // 256)
    want = {"packed": (packed, E * n // 2, torch.uint8), "absmax": (absmax, E * n // 64, torch.uint8),
            "nested_absmax": (nested_absmax, E * n2, torch.float32),
            "offset": (offset, E, torch.float32), "nested_code": (nested_code, 256, torch.float32)}
    flat = {}
    for name, (t, numel, dtype) in want.items():
        if int(t.numel()) != numel or t.dtype != dtype:
            raise ValueError(f"bitsandbytes field {name} must hold {numel} {dtype} values, got "
                             f"{int(t.numel())} {t.dtype}.")
        flat[name] = t.detach().to(device).reshape(-1).contiguous()
    codes = torch.empty((E, rows_f, cols_f // 2), dtype=torch.uint8, device=device)
    if two_level:
        if cols_f > 16384:
            raise ValueError("two-level absmax rows hold at most 16384 elements; ingest with "
                             "two_level=False (fp32 absmax).")
        nat.call("mx_nf4_from_bnb", flat["packed"].data_ptr(), None, None, None, None, E, rows_f,
                 cols_f, codes.data_ptr(), None, nat.stream(device))
        dq = {"nested_absmax": flat["nested_absmax"].reshape(E, n2),
              "offsets": flat["offset"], "code": flat["nested_code"]}
        q = flat["absmax"].reshape(E, rows_f, cols_f // NF4_BLOCKSIZE)
        return PackedWeight("nf4", codes, q, (E, out_f, in_f), layout, dq)
    amax = torch.empty((E, rows_f, cols_f // NF4_BLOCKSIZE), dtype=torch.float32, device=device)
    nat.call("mx_nf4_from_bnb", flat["packed"].data_ptr(), flat["absmax"].data_ptr(),
             flat["nested_absmax"].data_ptr(), flat["offset"].data_ptr(),
             flat["nested_code"].data_ptr(), E, rows_f, cols_f, codes.data_ptr(),
             amax.data_ptr(), nat.stream(device))
    return PackedWeight("nf4", codes, amax, (E, out_f, in_f), layout)


def nf4_levels() -> torch.Tensor:
    """The 16 NF4 levels as fp32 (mirai/core/models/quantization.py:100-117)."""
    return torch.tensor([
        -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
        -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
        0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
        0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=torch.float32)


def split_planes(x: torch.Tensor, pattern: int) -> torch.Tensor:
    """fp32 [..., n] -> bf16 [..., 3n] planes on the GPU (mx_split_f32):
    [hi | hi | lo] for ``SPLIT_ACT``, [hi | lo | hi] for ``SPLIT_WEIGHT``."""
    if x.dtype != torch.float32:
        raise ValueError(f"split_planes takes fp32, got {x.dtype}")
    x = x.contiguous()
    device = nat.require_gpu(x)
    cols = int(x.shape[-1])
    rows = x.numel() // max(cols, 1)
    out = torch.empty((*x.shape[:-1], 3 * cols), dtype=torch.bfloat16, device=device)
    nat.call("mx_split_f32", x.data_ptr(), rows, cols, pattern, out.data_ptr(), nat.stream(device))
    return out
