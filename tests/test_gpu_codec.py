"""GPU codec parity: NF4 / INT8 quantise + dequantise are bit-exact vs the oracle."""

import numpy as np
import pytest
import torch

from mirai_amd import quant
from oracle import codec

pytestmark = pytest.mark.gpu


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _weights(shape, seed, *, special=True) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(shape, generator=g) * 0.02).to(torch.bfloat16)
    if special:
        flat = w.view(-1, 64)
        flat[0] = 0                       # all-zero block -> absmax 0
        flat[1, :] = 0.0
        flat[1, 5] = -0.5                 # one non-zero element
        levels = torch.tensor(codec.NF4_LEVELS) * 0.25
        flat[2, :16] = levels.to(torch.bfloat16)   # values exactly on the codebook
        flat[3, :] = 1e-3
    return w


@pytest.mark.parametrize("shape", [(2, 64, 128), (3, 96, 2048), (1, 8, 1408)])
def test_nf4_quantize_and_dequantize_bit_exact(shape):
    w = _weights(shape, seed=11)
    packed = quant.quantize(w.cuda(), "nf4")
    E, o, i = shape
    codes_ref, absmax_ref = codec.nf4_quantize(_bf16_bits(w).reshape(E * o, i))
    np.testing.assert_array_equal(packed.data.cpu().numpy().reshape(E * o, i // 2), codes_ref)
    np.testing.assert_array_equal(_bf16_bits(packed.scale).reshape(E * o, i // 64), absmax_ref)
    deq = quant.dequantize(packed)
    np.testing.assert_array_equal(_bf16_bits(deq).reshape(E * o, i),
                                  codec.nf4_dequantize(codes_ref, absmax_ref))


@pytest.mark.parametrize("shape", [(2, 64, 128), (3, 96, 3072)])
def test_int8_quantize_and_dequantize_bit_exact(shape):
    w = _weights(shape, seed=12)
    packed = quant.quantize(w.cuda(), "int8")
    E, o, i = shape
    q_ref, s_ref = codec.int8_quantize(_bf16_bits(w).reshape(E * o, i))
    np.testing.assert_array_equal(packed.data.cpu().numpy().reshape(E * o, i), q_ref)
    np.testing.assert_array_equal(_bf16_bits(packed.scale).reshape(E * o), s_ref)
    deq = quant.dequantize(packed)
    np.testing.assert_array_equal(_bf16_bits(deq).reshape(E * o, i),
                                  codec.int8_dequantize(q_ref, s_ref))


def test_fp32_input_is_rounded_to_bf16_first():
    g = torch.Generator().manual_seed(3)
    w32 = torch.randn(2, 32, 256, generator=g) * 0.02
    a = quant.quantize(w32.cuda(), "nf4")
    b = quant.quantize(w32.to(torch.bfloat16).cuda(), "nf4")
    assert torch.equal(a.data, b.data) and torch.equal(a.scale, b.scale)


def test_nf4_full_expert_stack_round_trip_bound():
    """C2-sized w1 stack: |w - deq(q(w))| <= absmax * max half-gap of the codebook."""
    g = torch.Generator(device="cuda").manual_seed(1001)
    w = (torch.randn(64, 1408, 2048, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    packed = quant.quantize(w, "nf4")
    deq = quant.dequantize(packed).float()
    err = (deq - w.float()).abs().view(64, 1408, 32, 64)
    amax = packed.scale.float().view(64, 1408, 32, 1)
    half_gap = float(np.max(np.diff(codec.NF4_LEVELS.astype(np.float64))) / 2)
    # bf16 rounding of the product adds at most 2^-9 relative to |w| <= absmax.
    assert bool((err <= amax * (half_gap + 2.0**-8) + 1e-12).all())
