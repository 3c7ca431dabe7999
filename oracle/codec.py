"""NF4 / INT8 frozen-weight codecs and bf16 rounding, restated in numpy.

Formats (the BASELINE storage formats of this build):
* NF4: blocks of 64 consecutive ``in`` elements, absmax stored as bf16, no
  double quantisation. Codebook and nearest-level rule from
  mirai/core/models/quantization.py:100-117 and :158-168 (argmin, first index
  on ties). Packing: in each group of 8 consecutive elements, byte i holds
  element i in its low nibble and element i + 4 in its high nibble (the build's
  own layout; NF4Linear, quantization.py:171-175, packs element 2i / 2i+1
  instead, and the bitsandbytes layout is not available here).
  Dequantisation is ``bf16(fp32(level) * fp32(absmax))``, the fp32-product-
  then-cast convention of the bitsandbytes call sites in
  mirai/core/models/compressed_weights/quantization/quant.py:413-431.
* INT8: per output row, scale = bf16(max(absmax_row / 127, 1e-30)),
  q = clamp(round_half_even(w / scale), -127, 127); dequant bf16(q * scale).
  Rule of _quantize_weight / _dequantize_weight with group_size=0
  (quant.py:189-260), scale stored in bf16.
Inputs are taken as bf16 values, as the reference casts frozen weights to bf16
before quantize_4bit (quant.py:328).
"""

from __future__ import annotations

import numpy as np

NF4_BLOCKSIZE = 64

# mirai/core/models/quantization.py:100-117, converted to float32 exactly as
# torch.tensor(_NF4_LEVELS, dtype=torch.float32) does.
NF4_LEVELS = np.array(
    [
        -1.0,
        -0.6961928009986877,
        -0.5250730514526367,
        -0.39491748809814453,
        -0.28444138169288635,
        -0.18477343022823334,
        -0.09105003625154495,
        0.0,
        0.07958029955625534,
        0.16093020141124725,
        0.24611230194568634,
        0.33791524171829224,
        0.44070982933044434,
        0.5626170039176941,
        0.7229568362236023,
        1.0,
    ],
    dtype=np.float64,
).astype(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bf16 (round to nearest even); returns uint16 bits."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    rounded = np.where(np.isnan(x), np.uint16(0x7FC0), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns (uint16) to float32 exactly."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bf16 value, as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def _as_bf16_values(w) -> np.ndarray:
    """Accept uint16 bf16 bits or float arrays; return the bf16 values as float32."""
    w = np.asarray(w)
    if w.dtype == np.uint16:
        return bf16_bits_to_f32(w)
    return round_bf16(w.astype(np.float32))


def nf4_quantize(w) -> tuple[np.ndarray, np.ndarray]:
    """NF4-quantise ``w`` [rows, cols] (cols % 64 == 0).

    Returns ``codes`` uint8 [rows, cols/2] and ``absmax`` bf16 bits uint16
    [rows, cols/64]. Follows NF4Linear.__init__ (quantization.py:158-175) per
    64-element block with the bf16-absmax storage of the BASELINE format; a
    block whose absmax is zero maps every element to the 0.0 code (7).
    """
    values = _as_bf16_values(w)
    rows, cols = values.shape
    if cols % NF4_BLOCKSIZE:
        raise ValueError("NF4 needs cols to be a multiple of 64")
    blocks = values.reshape(rows, cols // NF4_BLOCKSIZE, NF4_BLOCKSIZE)
    absmax = np.abs(blocks).max(axis=-1)  # a bf16 input value, so exact in bf16
    with np.errstate(divide="ignore", invalid="ignore"):
        scaled = np.where(
            absmax[..., None] > 0,
            blocks / absmax[..., None],
            np.float32(0.0),
        ).astype(np.float32)
    dist = np.abs(scaled[..., None] - NF4_LEVELS)  # float32
    codes = dist.argmin(axis=-1).astype(np.uint8).reshape(rows, cols)
    return nf4_pack(codes), f32_to_bf16_bits(absmax.astype(np.float32))


def nf4_pack(codes: np.ndarray) -> np.ndarray:
    """Code indices uint8 [rows, cols] -> packed uint8 [rows, cols/2]: per group of
    8 elements, byte i = element i | element (i + 4) << 4."""
    codes = np.asarray(codes, dtype=np.uint8)
    rows, cols = codes.shape
    g = codes.reshape(rows, cols // 8, 8)
    return (g[..., :4] | (g[..., 4:] << 4)).astype(np.uint8).reshape(rows, cols // 2)


def nf4_unpack(packed: np.ndarray) -> np.ndarray:
    """uint8 [rows, cols/2] -> code indices uint8 [rows, cols] (inverse of nf4_pack)."""
    packed = np.asarray(packed, dtype=np.uint8)
    rows, half = packed.shape
    p = packed.reshape(rows, half // 4, 4)
    out = np.empty((rows, half // 4, 8), dtype=np.uint8)
    out[..., :4] = p & 0x0F
    out[..., 4:] = p >> 4
    return out.reshape(rows, half * 2)


def nf4_dequantize(packed: np.ndarray, absmax_bits: np.ndarray) -> np.ndarray:
    """Dequantised bf16 bits [rows, cols]: bf16(fp32(level[q]) * fp32(absmax))."""
    codes = nf4_unpack(packed)
    rows, cols = codes.shape
    a = bf16_bits_to_f32(absmax_bits).reshape(rows, cols // NF4_BLOCKSIZE, 1)
    levels = NF4_LEVELS[codes].reshape(rows, cols // NF4_BLOCKSIZE, NF4_BLOCKSIZE)
    prod = (levels * a).astype(np.float32)
    return f32_to_bf16_bits(prod.reshape(rows, cols))


INT8_SCALE_FLOOR = np.float32(1e-30)


def int8_quantize(w) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric INT8; returns q int8 [rows, cols] and bf16 scale bits [rows]."""
    values = _as_bf16_values(w)
    amax = np.abs(values).max(axis=1)
    scale32 = np.maximum((amax / np.float32(127.0)).astype(np.float32), INT8_SCALE_FLOOR)
    scale_bits = f32_to_bf16_bits(scale32)
    scale = bf16_bits_to_f32(scale_bits)
    ratio = (values / scale[:, None]).astype(np.float32)
    q = np.clip(np.rint(ratio), -127, 127).astype(np.int8)
    return q, scale_bits


def int8_dequantize(q: np.ndarray, scale_bits: np.ndarray) -> np.ndarray:
    """Dequantised bf16 bits: bf16(fp32(q) * fp32(scale)) (the product is exact)."""
    s = bf16_bits_to_f32(scale_bits)[:, None]
    return f32_to_bf16_bits((np.asarray(q, dtype=np.float32) * s).astype(np.float32))


# --------------------------------------------------------------------------
# bitsandbytes double-quantised NF4 (the reference's NF4 storage, quant.py:
# 315-358 / 407-431, through bitsandbytes==0.49.2, which is not installed
# here: parity with bitsandbytes itself is unpinned). Restated from its
# published format: per 64-element block an absmax, stored as a uint8 code
# of a 256-entry table with an fp32 absmax per 256 blocks and a per-tensor
# fp32 offset; 4-bit codes packed two per byte with element 2j in the HIGH
# nibble of byte j.

def bnb_nf4_absmax(absmax_q: np.ndarray, nested_absmax: np.ndarray, offset, nested_code):
    """Decoded fp32 block absmax: fp32(fp32(code2[q] * nested[b // 256]) + offset)."""
    q = np.asarray(absmax_q, dtype=np.uint8).reshape(-1)
    nested = np.asarray(nested_absmax, dtype=np.float32).reshape(-1)
    code2 = np.asarray(nested_code, dtype=np.float32).reshape(-1)
    scaled = (code2[q] * nested[np.arange(q.size) // 256]).astype(np.float32)
    return (scaled + np.float32(offset)).astype(np.float32)


def bnb_nf4_unpack(packed: np.ndarray) -> np.ndarray:
    """uint8 [n/2] -> codes [n], element 2j in the high nibble of byte j."""
    p = np.asarray(packed, dtype=np.uint8).reshape(-1)
    out = np.empty(p.size * 2, dtype=np.uint8)
    out[0::2] = p >> 4
    out[1::2] = p & 0x0F
    return out


def bnb_nf4_dequantize(packed, absmax_q, nested_absmax, offset, nested_code, rows, cols):
    """One expert's weights as bf16 bits [rows, cols]: bf16(fp32(NF4[c] * absmax))."""
    codes = bnb_nf4_unpack(packed).reshape(-1, NF4_BLOCKSIZE)
    a = bnb_nf4_absmax(absmax_q, nested_absmax, offset, nested_code)
    prod = (NF4_LEVELS[codes] * a[:, None]).astype(np.float32)
    return f32_to_bf16_bits(prod.reshape(rows, cols))


def bnb_nf4_quantize(w, nested_code) -> dict:
    """A double-quantised payload of one expert [rows, cols] for fixtures:
    fp32 absmax per 64 block, nearest NF4 level (first index on ties), offset =
    mean absmax, nested absmax per 256 blocks, nearest code of the table."""
    values = _as_bf16_values(w).astype(np.float32)
    rows, cols = values.shape
    blocks = values.reshape(-1, NF4_BLOCKSIZE)
    absmax = np.abs(blocks).max(axis=1).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        scaled = np.where(absmax[:, None] > 0, blocks / absmax[:, None], 0.0).astype(np.float32)
    codes = np.abs(scaled[..., None] - NF4_LEVELS).argmin(axis=-1).astype(np.uint8).reshape(-1)
    packed = ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)
    offset = np.float32(absmax.mean(dtype=np.float64))
    centered = (absmax - offset).astype(np.float32)
    n2 = -(-centered.size // 256)
    pad = np.zeros(n2 * 256, dtype=np.float32)
    pad[:centered.size] = centered
    nested = np.abs(pad.reshape(n2, 256)).max(axis=1).astype(np.float32)
    nested = np.where(nested > 0, nested, np.float32(1.0)).astype(np.float32)
    norm = (centered / nested[np.arange(centered.size) // 256]).astype(np.float32)
    code2 = np.asarray(nested_code, dtype=np.float32)
    absmax_q = np.abs(norm[:, None] - code2[None, :]).argmin(axis=1).astype(np.uint8)
    return {"packed": packed, "absmax": absmax_q, "nested_absmax": nested, "offset": offset,
            "code": NF4_LEVELS.copy(), "nested_code": code2}
