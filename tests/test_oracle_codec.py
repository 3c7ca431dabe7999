"""Pins the oracle's NF4 / INT8 codecs and bf16 rounding (CPU only).

Each check is independent of the oracle's own formulas: the NF4 table is
rebuilt from the published QLoRA construction (normal quantiles), rounding is
compared with torch's bf16 cast, quantisation with a brute-force scalar search,
dequantisation with an exact fp64 product, packing with a hand-made block, and
INT8 with torch's half-to-even rounding and the codec's error bound.
"""

import numpy as np
import pytest
import torch
from scipy.stats import norm

from oracle import codec, fastcodec


def _bf16_bits_torch(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def test_nf4_levels_match_the_normal_quantile_construction():
    # QLoRA (Dettmers et al. 2023), NF4 data type: 8 positive quantiles of
    # N(0,1) between 0.5 and offset, 7 negative ones, and an exact zero,
    # normalised to [-1, 1]; offset = 0.9677083.
    offset = 0.9677083
    pos = norm.ppf(np.linspace(offset, 0.5, 9)[:-1])
    neg = -norm.ppf(np.linspace(offset, 0.5, 8)[:-1])
    values = np.sort(np.concatenate([pos, [0.0], neg]))
    values /= np.abs(values).max()
    assert codec.NF4_LEVELS.dtype == np.float32 and codec.NF4_LEVELS.shape == (16,)
    np.testing.assert_allclose(codec.NF4_LEVELS, values, rtol=0, atol=2e-7)
    assert codec.NF4_LEVELS[7] == 0.0 and codec.NF4_LEVELS[0] == -1.0 and codec.NF4_LEVELS[15] == 1.0
    assert np.all(np.diff(codec.NF4_LEVELS) > 0)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 100000),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, 1.0 + 2.0 ** -8,
                  1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -20], dtype=np.float32),
        # exact ties between two bf16 neighbours, both parities
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ]).astype(np.float32)
    np.testing.assert_array_equal(codec.f32_to_bf16_bits(x), _bf16_bits_torch(x))
    nan = codec.f32_to_bf16_bits(np.array([np.nan], dtype=np.float32))
    assert (nan[0] & 0x7F80) == 0x7F80 and (nan[0] & 0x007F) != 0


def _nearest_level_scalar(v: np.float32) -> int:
    # Linear scan with a strict comparison: the first minimum wins.
    best, best_d = 0, None
    for j in range(16):
        d = np.float32(abs(np.float32(v) - codec.NF4_LEVELS[j]))
        if best_d is None or d < best_d:
            best, best_d = j, d
    return best


def test_nf4_quantize_matches_brute_force_search():
    rng = np.random.default_rng(1)
    rows = 6
    w = (rng.standard_normal((rows, 128)) * 0.02).astype(np.float32)
    w[2, :64] = 0.0                       # all-zero block
    w[3, 64:] = np.float32(0.5)           # constant block
    bits = codec.f32_to_bf16_bits(w)
    packed, absmax = codec.nf4_quantize(bits)
    vals = codec.bf16_bits_to_f32(bits)
    codes = codec.nf4_unpack(packed)
    for r in range(rows):
        for b in range(2):
            blk = vals[r, 64 * b:64 * (b + 1)]
            amax = np.float32(np.abs(blk).max())
            assert codec.bf16_bits_to_f32(absmax[r, b]) == amax
            for i in range(64):
                want = 7 if amax == 0 else _nearest_level_scalar(np.float32(blk[i] / amax))
                assert codes[r, 64 * b + i] == want, (r, b, i)


def test_nf4_pack_order_and_exact_levels():
    # A block holding the 16 levels themselves (times absmax 1): each maps to
    # its own code; in each group of 8 elements, byte i holds element i in the
    # low nibble and element i + 4 in the high nibble.
    order = np.array([0, 15, 3, 12, 7, 8, 1, 14, 5, 10, 2, 13, 4, 11, 6, 9] * 4)
    w = codec.NF4_LEVELS[order].reshape(1, 64)
    packed, absmax = codec.nf4_quantize(w)
    assert codec.bf16_bits_to_f32(absmax)[0, 0] == 1.0
    # group 0 = codes 0 15 3 12 | 7 8 1 14 -> bytes 0x70 0x8F 0x13 0xEC
    assert list(packed[0, :4]) == [0x70, 0x8F, 0x13, 0xEC]
    # group 1 = codes 5 10 2 13 | 4 11 6 9 -> bytes 0x45 0xBA 0x62 0x9D
    assert list(packed[0, 4:8]) == [0x45, 0xBA, 0x62, 0x9D]
    np.testing.assert_array_equal(codec.nf4_unpack(packed)[0], order)
    np.testing.assert_array_equal(codec.nf4_pack(order.reshape(1, 64).astype(np.uint8)), packed)


def test_nf4_dequantize_is_one_rounding_of_the_exact_product():
    rng = np.random.default_rng(2)
    codes = rng.integers(0, 16, (8, 64)).astype(np.uint8)
    g = codes.reshape(8, 8, 8)
    packed = (g[..., :4] | (g[..., 4:] << 4)).astype(np.uint8).reshape(8, 32)
    amax = np.abs(rng.standard_normal(8)).astype(np.float32) * np.float32(0.05)
    amax_bits = codec.f32_to_bf16_bits(amax).reshape(8, 1)
    got = codec.nf4_dequantize(packed, amax_bits)
    # level (24-bit) x bf16 absmax (8-bit) is exact in fp64; fp64 -> fp32 is
    # then the one fp32 rounding, fp32 -> bf16 (torch) the second.
    exact = codec.NF4_LEVELS.astype(np.float64)[codes] * codec.bf16_bits_to_f32(amax_bits).astype(np.float64)
    want = _bf16_bits_torch(exact.astype(np.float32))
    np.testing.assert_array_equal(got, want)


def test_nf4_round_trip_error_bound():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    bits = codec.f32_to_bf16_bits(w)
    packed, absmax = codec.nf4_quantize(bits)
    deq = codec.bf16_bits_to_f32(codec.nf4_dequantize(packed, absmax))
    vals = codec.bf16_bits_to_f32(bits)
    amax = np.repeat(codec.bf16_bits_to_f32(absmax), 64, axis=1)
    half_gap = np.diff(codec.NF4_LEVELS).max() / 2
    assert np.all(np.abs(deq - vals) <= amax * (half_gap * 1.01) + np.abs(vals) * 2.0 ** -8)
    # The block maximum is a level endpoint: it round-trips exactly.
    for r in range(16):
        for b in range(4):
            blk = vals[r, 64 * b:64 * (b + 1)]
            i = int(np.abs(blk).argmax())
            assert deq[r, 64 * b + i] == blk[i]


def test_int8_matches_torch_half_even_and_error_bound():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((32, 192)) * 0.02).astype(np.float32)
    w[5] = 0.0
    bits = codec.f32_to_bf16_bits(w)
    q, s_bits = codec.int8_quantize(bits)
    vals = torch.from_numpy(codec.bf16_bits_to_f32(bits))
    amax = vals.abs().amax(dim=1)
    s = (amax / 127.0).clamp_min(1e-30).to(torch.bfloat16).float()
    np.testing.assert_array_equal(s_bits, s.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    q_ref = torch.round(vals / s[:, None]).clamp(-127, 127).to(torch.int8)
    np.testing.assert_array_equal(q, q_ref.numpy())
    deq = codec.bf16_bits_to_f32(codec.int8_dequantize(q, s_bits))
    assert np.all(np.abs(deq - vals.numpy()) <= s.numpy()[:, None] * 0.5 + np.abs(vals.numpy()) * 2.0 ** -8)
    assert np.all(np.abs(q[np.arange(32) != 5]).max(axis=1) >= 126)
    assert np.all(q[5] == 0)
    # Symmetric: quantise(-w) == -quantise(w).
    qn, sn = codec.int8_quantize(codec.f32_to_bf16_bits(-codec.bf16_bits_to_f32(bits)))
    np.testing.assert_array_equal(qn, -q)
    np.testing.assert_array_equal(sn, s_bits)


def test_c_oracle_equals_numpy_oracle():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    w[3, :64] = 0
    bits = codec.f32_to_bf16_bits(w)
    c_codes, c_abs = fastcodec.nf4_quantize(bits)
    n_codes, n_abs = codec.nf4_quantize(bits)
    np.testing.assert_array_equal(c_codes, n_codes)
    np.testing.assert_array_equal(c_abs, n_abs)
    np.testing.assert_array_equal(fastcodec.nf4_dequantize(c_codes, c_abs),
                                  codec.nf4_dequantize(n_codes, n_abs))
    c_q, c_s = fastcodec.int8_quantize(bits)
    n_q, n_s = codec.int8_quantize(bits)
    np.testing.assert_array_equal(c_q, n_q)
    np.testing.assert_array_equal(c_s, n_s)
    np.testing.assert_array_equal(fastcodec.int8_dequantize(c_q, c_s), codec.int8_dequantize(n_q, n_s))


@pytest.mark.parametrize("mistake", ["bf16_level_first", "high_nibble_first", "pairwise_packing"])
def test_planted_mistakes_are_caught(mistake):
    """A plausible codec slip must change the output the checks above compare."""
    rng = np.random.default_rng(6)
    codes = rng.integers(0, 16, (4, 64)).astype(np.uint8)
    amax_bits = codec.f32_to_bf16_bits(np.abs(rng.standard_normal((4, 1))).astype(np.float32) * 0.05)
    a = codec.bf16_bits_to_f32(amax_bits)
    right = codec.f32_to_bf16_bits((codec.NF4_LEVELS[codes] * a).astype(np.float32))
    if mistake == "bf16_level_first":
        # NF4Linear's in-tree rule rounds the level to bf16 before the product.
        lv = codec.round_bf16(codec.NF4_LEVELS)
        wrong = codec.f32_to_bf16_bits((lv[codes] * a).astype(np.float32))
    elif mistake == "high_nibble_first":
        g = codes.reshape(4, 8, 8)
        swapped = np.concatenate([g[..., 4:], g[..., :4]], axis=-1).reshape(4, 64)
        wrong = codec.f32_to_bf16_bits((codec.NF4_LEVELS[swapped] * a).astype(np.float32))
    else:
        # Reading the bytes as element pairs (2i, 2i + 1), NF4Linear's packing.
        packed = codec.nf4_pack(codes)
        pairwise = np.empty_like(codes)
        pairwise[:, 0::2], pairwise[:, 1::2] = packed & 0x0F, packed >> 4
        wrong = codec.f32_to_bf16_bits((codec.NF4_LEVELS[pairwise] * a).astype(np.float32))
    assert not np.array_equal(right, wrong)


def test_bnb_nf4_dequantize_known_answer_and_nibble_order():
    # One block of 64: byte 0 = 0xF0 holds element 0 = code 15 (high nibble)
    # and element 1 = code 0 (low nibble); absmax code 5 with table value 0.5,
    # nested absmax 0.5 and offset 0.25 gives absmax 0.5 * 0.5 + 0.25 = 0.5.
    packed = np.full(32, 0x77, dtype=np.uint8)  # codes 7 (level 0.0) elsewhere
    packed[0] = 0xF0
    table = np.linspace(-1.0, 1.0, 256).astype(np.float32)
    table[5] = 0.5
    out = codec.bnb_nf4_dequantize(packed, np.array([5], np.uint8), np.array([0.5], np.float32),
                                   np.float32(0.25), table, 1, 64)
    vals = codec.bf16_bits_to_f32(out)[0]
    assert vals[0] == 0.5 and vals[1] == -0.5 and np.all(vals[2:] == 0.0)
    assert list(codec.bnb_nf4_unpack(packed)[:2]) == [15, 0]
    # A plausible slip (reading the pair low nibble first) swaps the two.
    low_first = np.empty(64, dtype=np.uint8)
    low_first[0::2], low_first[1::2] = packed & 0x0F, packed >> 4
    assert list(low_first[:2]) == [0, 15]


def test_bnb_nf4_absmax_rounds_product_then_sum():
    # fp32(fp32(a * b) + c) differs from one fused rounding for these values.
    a, b, c = np.float32(1.0000001), np.float32(3.0000002), np.float32(-3.0000005)
    got = codec.bnb_nf4_absmax(np.array([0], np.uint8), np.array([b], np.float32), c,
                               np.array([a], np.float32))
    prod = np.float32(a * b)
    assert got[0] == np.float32(prod + c)
    assert got[0] != np.float32(np.float64(a) * np.float64(b) + np.float64(c))


def test_bnb_nf4_quantize_round_trip_error_bound():
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((6, 4096)) * 0.02).astype(np.float32)
    table = np.sort(np.concatenate([np.linspace(-1, 1, 255), [0.0]])).astype(np.float32)
    p = codec.bnb_nf4_quantize(w, table)
    got = codec.bf16_bits_to_f32(codec.bnb_nf4_dequantize(
        p["packed"], p["absmax"], p["nested_absmax"], p["offset"], p["nested_code"], 6, 4096))
    err = np.abs(got - codec.round_bf16(w)).reshape(-1, 64).max(axis=1)
    amax = np.abs(codec.round_bf16(w)).reshape(-1, 64).max(axis=1)
    # NF4 half-gap (0.16) plus the absmax code error (table step 1/127 of the
    # nested absmax) bounds the per-block error.
    assert np.all(err <= 0.16 * amax + 0.02 * amax + 1e-3)
