"""GPU codec parity: NF4 / INT8 quantise + dequantise are bit-exact vs the oracle."""

import numpy as np
import pytest
import torch

from mirai_amd import _native as nat
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


def _bnb_payload(E, rows, cols, seed):
    rng = np.random.default_rng(seed)
    table = np.sort(np.concatenate([np.linspace(-1, 1, 255), [0.0]])).astype(np.float32)
    w = (rng.standard_normal((E, rows, cols)) * 0.02).astype(np.float32)
    parts = [codec.bnb_nf4_quantize(w[e], table) for e in range(E)]
    stacked = {
        "packed": np.stack([p["packed"] for p in parts]),
        "absmax": np.stack([p["absmax"] for p in parts]),
        "nested_absmax": np.stack([p["nested_absmax"] for p in parts]),
        "offset": np.array([p["offset"] for p in parts], dtype=np.float32),
        "code": parts[0]["code"],
        "nested_code": table,
    }
    return stacked, parts, table


def test_bnb_nf4_ingest_is_bit_exact():
    # 96 x 384 per expert = 576 absmax blocks: the last nested block is partial.
    E, rows, cols = 3, 96, 384
    stacked, parts, table = _bnb_payload(E, rows, cols, 21)
    t = {k: torch.from_numpy(np.asarray(v)).cuda() for k, v in stacked.items()}
    pw = quant.from_bnb_nf4(packed=t["packed"], absmax=t["absmax"],
                            nested_absmax=t["nested_absmax"], offset=t["offset"], code=t["code"],
                            nested_code=t["nested_code"], shape=(E, rows, cols))
    assert pw.format_code() == nat.FMT_NF4_F32
    for e, p in enumerate(parts):
        want_codes = codec.nf4_pack(codec.bnb_nf4_unpack(p["packed"]).reshape(rows, cols))
        np.testing.assert_array_equal(pw.data[e].cpu().numpy(), want_codes)
        want_abs = codec.bnb_nf4_absmax(p["absmax"], p["nested_absmax"], p["offset"], table)
        np.testing.assert_array_equal(pw.scale[e].cpu().numpy().reshape(-1), want_abs)
    deq = quant.dequantize(pw).view(torch.int16).cpu().numpy().view(np.uint16)
    for e, p in enumerate(parts):
        want = codec.bnb_nf4_dequantize(p["packed"], p["absmax"], p["nested_absmax"], p["offset"],
                                        table, rows, cols)
        np.testing.assert_array_equal(deq[e], want)


def test_bnb_nf4_ingest_rejects_a_non_nf4_code_table():
    stacked, _, _ = _bnb_payload(1, 64, 64, 3)
    t = {k: torch.from_numpy(np.asarray(v)).cuda() for k, v in stacked.items()}
    with pytest.raises(ValueError, match="NF4 table"):
        quant.from_bnb_nf4(packed=t["packed"], absmax=t["absmax"],
                           nested_absmax=t["nested_absmax"], offset=t["offset"],
                           code=torch.linspace(-1, 1, 16).cuda(), nested_code=t["nested_code"],
                           shape=(1, 64, 64))


def test_layer_runs_on_ingested_bnb_nf4_weights():
    from mirai_amd import CompressedGroupedExperts, route_topk
    from oracle import layer as olayer
    from helpers import assert_layer_close

    E, d, f, T, k = 8, 256, 192, 200, 2
    shapes = {"w1": (E, f, d), "w3": (E, f, d), "w2": (E, d, f)}
    state, dense = {}, {}
    for i, (key, (e_, o, n)) in enumerate(shapes.items()):
        stacked, parts, table = _bnb_payload(e_, o, n, 40 + i)
        for name, suffix in (("packed", ""), ("absmax", "_absmax"), ("nested_absmax", "_nabsmax"),
                             ("offset", "_offset"), ("code", "_code"),
                             ("nested_code", "_ncode")):
            state[f"{key}_nf4{suffix}"] = torch.from_numpy(np.asarray(stacked[name])).cuda()
        bits = np.stack([codec.bnb_nf4_dequantize(p["packed"], p["absmax"], p["nested_absmax"],
                                                  p["offset"], table, o, n) for p in parts])
        dense[key] = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    m = CompressedGroupedExperts.from_empty(num_experts=E, quant_format="nf4",
                                            expert_weight_access="fused_kernel",
                                            expert_dequant_chunk_size=8)
    m.load_bnb_state_dict(state, shapes)
    assert m.is_fully_loaded()
    g = torch.Generator().manual_seed(5)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    idx, scores = route_topk(torch.randn(T, E, generator=g).cuda(), k)
    with torch.no_grad():
        out = m.run_direct_routed(x.cuda(), scores, idx)
    ref = olayer.layer_forward(x, scores.cpu(), idx.cpu(), dense, {}, E)
    print(f"ingested bnb nf4 layer: {assert_layer_close(out.cpu(), ref)}")


def _bnb_state(E, d, f, seed):
    table = None
    shapes = {"w1": (E, f, d), "w3": (E, f, d), "w2": (E, d, f)}
    state, dense = {}, {}
    for i, (key, (e_, o, n)) in enumerate(shapes.items()):
        stacked, parts, table = _bnb_payload(e_, o, n, seed + i)
        for name, suffix in (("packed", ""), ("absmax", "_absmax"), ("nested_absmax", "_nabsmax"),
                             ("offset", "_offset"), ("code", "_code"),
                             ("nested_code", "_ncode")):
            state[f"{key}_nf4{suffix}"] = torch.from_numpy(np.asarray(stacked[name])).cuda()
        bits = np.stack([codec.bnb_nf4_dequantize(p["packed"], p["absmax"], p["nested_absmax"],
                                                  p["offset"], table, o, n) for p in parts])
        dense[key] = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    return state, dense, shapes


def test_two_level_absmax_decodes_like_the_load_time_absmax():
    # mx_nf4_dq_absmax (the GEMMs' per-step arithmetic) against mx_nf4_from_bnb's
    # fp32 absmax, and the dequantised weights of both ingestions against the
    # bitsandbytes restatement, bit for bit (nested blocks of 256 cross rows
    # here: 6 blocks per row).
    from mirai_amd import CompressedGroupedExperts, quant

    E, d, f = 3, 384, 320
    state, dense, shapes = _bnb_state(E, d, f, 70)
    mods = {}
    for two in (False, True):
        m = CompressedGroupedExperts.from_empty(num_experts=E, quant_format="nf4",
                                                expert_weight_access="fused_kernel")
        m.load_bnb_state_dict(state, shapes, two_level=two)
        mods[two] = m
    for key in shapes:
        pf, pq = mods[False].packed_weight(key), mods[True].packed_weight(key)
        assert pf.format_code() == nat.FMT_NF4_F32 and pq.format_code() == nat.FMT_NF4_DQ
        assert pq.nbytes() < pf.nbytes()
        assert torch.equal(pf.data, pq.data)
        amax = torch.empty_like(pf.scale)
        st = pq.dq_struct()
        import ctypes
        nat.call("mx_nf4_dq_absmax", ctypes.byref(st), E, int(pq.scale[0].numel()),
                 amax.data_ptr(), nat.stream(amax.device))
        assert torch.equal(amax, pf.scale)
        for sel in (None, slice(1, 2)):
            a = quant.dequantize(pq, experts=sel)
            b = quant.dequantize(pf, experts=sel)
            assert torch.equal(a, b)
        assert torch.equal(quant.dequantize(pq).cpu(), dense[key])


def test_two_level_absmax_layer_equals_the_fp32_absmax_layer():
    # The same payload ingested with its absmax decoded at load (NF4_F32) and
    # kept two-level (NF4_DQ, decoded in the GEMMs): the same absmax arithmetic,
    # so forward (256-row, remainder and light tiles) and backward (LoRA) agree
    # bit for bit; and both match the oracle on the bitsandbytes weights.
    from mirai_amd import CompressedGroupedExperts
    from oracle import layer as olayer
    from helpers import assert_layer_close
    from test_gpu_light_tiles import LIGHT_COUNTS, skewed_routes

    E, d, f, T, k, r = 9, 256, 384, 1400, 2, 16
    state, dense, shapes = _bnb_state(E, d, f, 80)
    g = torch.Generator().manual_seed(81)
    lora = {key: (torch.randn(E, r, n, generator=g) * 0.02, torch.randn(E, o, r, generator=g) * 0.02)
            for key, (_, o, n) in shapes.items()}
    mods = {}
    for two in (False, True):
        m = CompressedGroupedExperts.from_empty(num_experts=E, quant_format="nf4",
                                                expert_weight_access="fused_kernel")
        m.load_bnb_state_dict(state, shapes, two_level=two)
        for key, (a, b) in lora.items():
            ad = m.attach_expert_lora(tensor_name=key, adapter_name="t", rank=r, alpha=16.0)
            with torch.no_grad():
                ad.lora_a.copy_(a.cuda())
                ad.lora_b.copy_(b.cuda())
        mods[two] = m
    idx, scores = skewed_routes(T, E, k, LIGHT_COUNTS, seed=82)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16).cuda()
    dy = torch.randn(T, d, generator=g).to(torch.bfloat16).cuda()
    outs, grads = {}, {}
    for two, m in mods.items():
        with torch.no_grad():
            outs[two] = m.run_direct_routed(x, scores.cuda(), idx.cuda())
        xg = x.clone().requires_grad_(True)
        sg = scores.cuda().requires_grad_(True)
        y = m.run_direct_routed(xg, sg, idx.cuda())
        y.backward(dy)
        grads[two] = [xg.grad, sg.grad] + [p.grad for ad in m.expert_lora.values()
                                           for p in (ad.lora_a, ad.lora_b)]
        assert torch.equal(y.detach(), outs[two])
    assert torch.equal(outs[True], outs[False])
    for a, b in zip(grads[True], grads[False]):
        assert torch.equal(a, b)
    ref = olayer.layer_forward(x.cpu(), scores, idx, dense,
                               {k_: (a, b, 16.0 / r) for k_, (a, b) in lora.items()}, E)
    print(f"two-level absmax layer: {assert_layer_close(outs[True].cpu(), ref)}")
