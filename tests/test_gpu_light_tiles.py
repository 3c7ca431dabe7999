"""GPU parity of the light tiles against the reference-order oracle.

An expert with at most 32 rows in a launch runs a tile body of its own: its
token rows are staged in LDS once and each wave decodes its NF4 weight rows
straight into MFMA operands (no per-step B stage). The cases below route
exact row counts to chosen experts (0, 1, 5, 16, 31, 32 and 33 rows: both
sides of the threshold), next to heavy experts that keep the 256-row tiles
running in the same launch, or with few rows overall (128-row tile launch).
Both GEMMs take the light body when their K is a multiple of 128 (d = 256,
f = 384 here). Bounds: the layer bound of test_gpu_layer.py forward, the
per-gradient bounds of test_gpu_backward.py for training.
"""

import numpy as np
import pytest
import torch

from mirai_amd import workloads as wl
from oracle import codec
from oracle import layer as olayer

from helpers import (assert_layer_close, build_module, mixed_rank_factors, oracle_loras,
                     oracle_weights)

pytestmark = pytest.mark.gpu

LIGHT_COUNTS = (0, 1, 5, 16, 31, 32, 33)


def skewed_routes(T, E, k, light_counts, seed):
    """Routes [T, k] where expert H + i (H = E - len(light_counts)) gets exactly
    light_counts[i] rows and experts 0 .. H - 1 take every other slot. Scores
    are positive and sum to 1 per token."""
    rng = np.random.default_rng(seed)
    H = E - len(light_counts)
    assert H >= k and sum(light_counts) <= T
    idx = np.full((T, k), -1, np.int64)
    fill = np.zeros(T, np.int64)
    for i, c in enumerate(light_counts):
        free = np.nonzero(fill < k - 1)[0]  # one slot per token stays for a heavy expert
        toks = rng.choice(free, size=c, replace=False)
        idx[toks, fill[toks]] = H + i
        fill[toks] += 1
    for t in range(T):
        heavy = [int(e) for e in rng.permutation(H)]
        for j in range(fill[t], k):
            idx[t, j] = heavy.pop()
    scores = rng.random((T, k)).astype(np.float32) + 0.1
    scores /= scores.sum(axis=1, keepdims=True)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    assert tuple(counts[H:]) == tuple(light_counts)
    return torch.from_numpy(idx), torch.from_numpy(scores)


def _workload(fmt, *, T, E, k=2, d=256, f=384, r=16):
    return wl.Workload(f"light_{fmt}", 11, T, d, f, E, k, r, 16.0, fmt, torch.bfloat16)


def _forward_case(w, idx, scores, lora):
    dense = wl.dense_weights(w)
    x = wl.tokens(w)
    m = build_module(w, dense, lora)
    with torch.no_grad():
        out = m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda())
    ref = olayer.layer_forward(x, scores, idx, oracle_weights(w, dense, dtype=w.dtype),
                               oracle_loras(w, lora), w.experts)
    stats = assert_layer_close(out.cpu(), ref)
    print(f"light tiles {w.name} T={w.tokens} E={w.experts}: {stats}")


@pytest.mark.parametrize("lora_case", ["none", "r16", "r64", "mixed"])
def test_light_tiles_beside_tall_tiles(lora_case):
    # 2800 routed rows over 9 experts: the 256-row tile launch (rows >= 256 E),
    # with the light experts' tiles among its remainder tiles.
    w = _workload("nf4", T=1400, E=9, r=64 if lora_case == "r64" else 16)
    idx, scores = skewed_routes(w.tokens, w.experts, w.top_k, LIGHT_COUNTS, seed=3)
    lora = {"none": None, "r16": wl.lora_factors(w), "r64": wl.lora_factors(w),
            "mixed": mixed_rank_factors(w, {"w1": 8, "w3": 40, "w2": 24})}[lora_case]
    _forward_case(w, idx, scores, lora)


def test_light_tiles_in_the_128_row_launch():
    # 600 rows over 16 experts: 128-row tiles only, most experts light.
    counts = (0, 1, 2, 3, 5, 8, 13, 21, 31, 32, 33, 40, 64)
    w = _workload("nf4", T=300, E=16)
    idx, scores = skewed_routes(w.tokens, w.experts, w.top_k, counts, seed=4)
    _forward_case(w, idx, scores, wl.lora_factors(w))


def test_light_tiles_top4_and_odd_column_tiles():
    # top-4, f = 640: the gate/up column tiles cover 128 ffn columns, the last
    # one and the down projection's last 256-column tile partly past N.
    w = _workload("nf4", T=700, E=12, k=4, d=384, f=640)
    idx, scores = skewed_routes(w.tokens, w.experts, w.top_k, LIGHT_COUNTS, seed=5)
    _forward_case(w, idx, scores, wl.lora_factors(w))


def test_light_tiles_on_fp32_absmax_weights():
    # MX_FMT_NF4_F32 (bitsandbytes double-quant payloads decoded at load).
    from mirai_amd import CompressedGroupedExperts

    E, d, f, T, k = 9, 256, 384, 1400, 2
    rng = np.random.default_rng(21)
    table = np.sort(np.concatenate([np.linspace(-1, 1, 255), [0.0]])).astype(np.float32)
    shapes = {"w1": (E, f, d), "w3": (E, f, d), "w2": (E, d, f)}
    state, dense = {}, {}
    for key, (e_, o, n) in shapes.items():
        wts = (rng.standard_normal((e_, o, n)) * 0.02).astype(np.float32)
        parts = [codec.bnb_nf4_quantize(wts[e], table) for e in range(e_)]
        stacked = {"": np.stack([p["packed"] for p in parts]),
                   "_absmax": np.stack([p["absmax"] for p in parts]),
                   "_nabsmax": np.stack([p["nested_absmax"] for p in parts]),
                   "_offset": np.array([p["offset"] for p in parts], dtype=np.float32),
                   "_code": parts[0]["code"], "_ncode": table}
        for suffix, v in stacked.items():
            state[f"{key}_nf4{suffix}"] = torch.from_numpy(np.asarray(v)).cuda()
        bits = np.stack([codec.bnb_nf4_dequantize(p["packed"], p["absmax"], p["nested_absmax"],
                                                  p["offset"], table, o, n) for p in parts])
        dense[key] = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    m = CompressedGroupedExperts.from_empty(num_experts=E, quant_format="nf4",
                                            expert_weight_access="fused_kernel",
                                            expert_dequant_chunk_size=8)
    m.load_bnb_state_dict(state, shapes)
    idx, scores = skewed_routes(T, E, k, LIGHT_COUNTS, seed=6)
    x = (torch.randn(T, d, generator=torch.Generator().manual_seed(7))).to(torch.bfloat16)
    with torch.no_grad():
        out = m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda())
    ref = olayer.layer_forward(x, scores, idx, dense, {}, E)
    print(f"light tiles on fp32-absmax weights: {assert_layer_close(out.cpu(), ref)}")


@pytest.mark.parametrize("T,E", [(1400, 9), (300, 16)])
def test_light_tiles_backward(T, E):
    # The training forward's gate / up saves come from the light tiles too.
    from test_gpu_backward import _close, _gpu_grads, _oracle_grads

    w = _workload("nf4", T=T, E=E)
    counts = LIGHT_COUNTS if E == 9 else (0, 1, 2, 3, 5, 8, 13, 21, 31, 32, 33, 40, 64)
    idx, scores = skewed_routes(w.tokens, w.experts, w.top_k, counts, seed=8)
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    x = wl.tokens(w)
    dy = wl.upstream_grad(w)
    m = build_module(w, dense, lora)
    _, g = _gpu_grads(m, x, scores, idx, dy)
    _, ref = _oracle_grads(w, dense, lora, x, scores, idx, dy, torch.arange(T))
    for name, e in ref.items():
        _close(name, g[name], e)
