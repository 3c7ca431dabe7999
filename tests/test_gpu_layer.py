"""GPU layer parity: the fused routed expert op vs the reference-order oracle.

Tolerance (benchmark definition): max-abs 2e-2 and mean-relative 5e-3 on the
bf16 layer output versus the oracle's fp32-accumulated reference path.
"""

import numpy as np
import pytest
import torch

from mirai_amd import route_topk
from mirai_amd import workloads as wl
from oracle import layer as olayer
from oracle import routing as oroute

from helpers import (assert_layer_close, build_module, mixed_rank_factors, oracle_loras,
                     oracle_weights)

pytestmark = pytest.mark.gpu


def small(fmt, *, T=256, d=256, f=192, E=8, k=2, r=16, alpha=16.0, dtype=torch.bfloat16):
    return wl.Workload(f"small_{fmt}", 7, T, d, f, E, k, r, alpha, fmt, dtype)


def _run_case(w: wl.Workload, *, with_lora=True, token_subset=None, lora=None):
    dense = wl.dense_weights(w)
    if lora is None:
        lora = wl.lora_factors(w) if with_lora else None
    x = wl.tokens(w)
    logits = wl.router_logits(w)
    idx_np, scores_np = oroute.route_topk(logits.numpy(), w.top_k)
    idx, scores = torch.from_numpy(idx_np), torch.from_numpy(scores_np)
    m = build_module(w, dense, lora)
    with torch.no_grad():
        out = m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda())
    assert out.dtype == x.dtype and tuple(out.shape) == tuple(x.shape)
    rows = torch.arange(w.tokens) if token_subset is None else token_subset
    ref = olayer.layer_forward(x[rows], scores[rows], idx[rows],
                               oracle_weights(w, dense, dtype=w.dtype), oracle_loras(w, lora),
                               w.experts)
    stats = assert_layer_close(out.cpu()[rows], ref)
    print(f"parity {w.name}: {stats}")
    return stats


@pytest.mark.parametrize("fmt", ["bf16", "nf4", "int8"])
@pytest.mark.parametrize("with_lora", [False, True])
def test_small_layer_matches_oracle(fmt, with_lora):
    _run_case(small(fmt), with_lora=with_lora)


@pytest.mark.parametrize("r", [8, 24, 32, 48, 64, 104, 128])
def test_lora_ranks(r):
    # Ranks above 32 add 32-wide K chunks to the epilogue's LoRA product (104:
    # a partial last chunk) and split the down-projection into 32-row slices.
    _run_case(small("nf4", r=r, alpha=2.0 * r, E=5, k=3, T=300, f=320, d=192))


@pytest.mark.parametrize("fmt,r", [("nf4", 64), ("int8", 256)])
def test_wide_lora_on_tall_tiles(fmt, r):
    # ~1024 rows per expert: 256-row tiles and 128-row remainders.
    _run_case(small(fmt, r=r, alpha=float(r), E=4, k=2, T=2000, f=384, d=256))


def test_mixed_lora_ranks():
    # Each projection its own rank; the low-rank planes take the widest (128).
    w = small("int8", E=6, k=2, T=400, f=256, d=192, alpha=32.0)
    _run_case(w, lora=mixed_rank_factors(w, {"w1": 64, "w3": 8, "w2": 128}))


def test_ragged_and_empty_experts():
    # Few tokens over many experts: most experts get 0-2 rows, many tiles are partial.
    _run_case(small("int8", T=37, E=64, k=4, d=128, f=128))


def test_fp32_tokens_c1_plumbing():
    # fp32 tokens, fp32 weights (split bf16 planes on MFMA), fp32 LoRA and output.
    stats = _run_case(wl.WORKLOADS["c1"])
    # fp32 precision end to end (split bf16 planes on MFMA): far inside the bound.
    assert stats["mean_rel"] < 1e-4, stats


@pytest.mark.parametrize("with_lora", [False, True])
def test_fp32_layer_small(with_lora):
    w = small("fp32", dtype=torch.float32, r=8, alpha=16.0, T=300, E=6, k=2, d=192, f=320)
    stats = _run_case(w, with_lora=with_lora)
    assert stats["mean_rel"] < 1e-4, stats


@pytest.mark.parametrize("d,f", [(192, 640), (320, 1024), (384, 640), (512, 1024)])
def test_fp32_layer_in_k_parts(d, f):
    # 600 routed rows, so few tiles: the down projection splits each tile's K
    # (3 f) over 3 (f = 640: 30 K steps) or 6 (f = 1024: 48) workgroups, each
    # writing its own [hi | lo] planes (part 0 with the LoRA delta) that the
    # combine adds; d = 192 and 320 leave a partial column tile. The LoRA
    # down-projections run in K parts where K allows (3 d = 1152 and 1536: 2
    # and 3 parts; 3 f = 1920 and 3072: 3 and 6), summed by their finishing
    # pass.
    w = small("fp32", dtype=torch.float32, r=8, alpha=16.0, T=300, E=6, k=2, d=d, f=f)
    stats = _run_case(w, with_lora=True)
    assert stats["mean_rel"] < 1e-4, stats


@pytest.mark.parametrize("chunk", [0, 128])
def test_fp32_layer_trains_like_fp64_autograd(chunk):
    # fp32 weights under autograd: the split-precision kernels run the forward,
    # the backward differentiates the fp32 layer over the stored weights (hi + lo,
    # within 2^-16 of the fp32 weights). Gradients to tokens, scores and every
    # LoRA factor against fp64 autograd of the oracle on the fp32 weights: mean
    # relative error <= 1e-4 (measured about 1e-6). With token chunks of 128
    # each chunk's backward recomputes its own rows: the same gradients.
    from mirai_amd import MoETokenChunkPolicy, fused_chunk_runner

    w = small("fp32", dtype=torch.float32, r=8, alpha=16.0, T=300, E=6, k=2, d=192, f=320)
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    m = build_module(w, dense, lora)
    idx_np, scores_np = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    idx, scores = torch.from_numpy(idx_np), torch.from_numpy(scores_np)
    x = wl.tokens(w)
    dy = wl.upstream_grad(w).float()
    xg = x.cuda().requires_grad_(True)
    sg = scores.cuda().requires_grad_(True)
    if chunk:
        out = MoETokenChunkPolicy(token_chunk_size=chunk).execute(
            xg, sg, idx.cuda(), runner=fused_chunk_runner(m), training=True)
    else:
        out = m.run_direct_routed(xg, sg, idx.cuda())
    assert out.dtype == torch.float32
    out.backward(dy.cuda())
    got = {"tokens": xg.grad, "scores": sg.grad}
    for key, ad in m.expert_lora.items():
        got[f"{key}.a"], got[f"{key}.b"] = ad.lora_a.grad, ad.lora_b.grad

    xo = x.double().requires_grad_(True)
    so = scores.double().requires_grad_(True)
    leaves = {k_: (a.double().requires_grad_(True), b.double().requires_grad_(True))
              for k_, (a, b) in lora.items()}
    weights = {k_: v.double() for k_, v in dense.items()}
    ref = olayer.layer_forward(xo, so, idx, weights,
                               {k_: (a, b, float(w.alpha) / int(a.shape[1]))
                                for k_, (a, b) in leaves.items()}, w.experts)
    ref.backward(dy.double())
    want = {"tokens": xo.grad, "scores": so.grad}
    for k_, (a, b) in leaves.items():
        want[f"{k_}.a"], want[f"{k_}.b"] = a.grad, b.grad
    assert_layer_close(out.detach().cpu(), ref.detach().float())
    for name, e in want.items():
        a = got[name].detach().double().cpu()
        rel = float((a - e).abs().sum() / e.abs().sum().clamp_min(1e-30))
        print(f"fp32 training {name}: mean_rel={rel:.2e}")
        assert rel <= 1e-4, (name, rel)


def test_fp32_run_for_loop_matches_oracle():
    # run_for_loop of the fp32 layer (experts.py:1656-1747 is dtype-agnostic):
    # rows grouped by expert, fp32 in and out, against the oracle's fp32 loop.
    w = small("fp32", dtype=torch.float32, r=8, alpha=16.0, T=300, E=6, k=1, d=192, f=320)
    dense, lora = wl.dense_weights(w), wl.lora_factors(w)
    m = build_module(w, dense, lora)
    counts = torch.tensor([60, 0, 90, 1, 149, 0])
    x = wl.tokens(w)
    with torch.no_grad():
        out = m.run_for_loop(x.cuda(), counts.cuda())
    assert out.dtype == torch.float32
    ref = olayer.for_loop_forward(x, counts, oracle_weights(w, dense, dtype=w.dtype),
                                  oracle_loras(w, lora))
    stats = assert_layer_close(out.cpu(), ref)
    assert stats["mean_rel"] < 1e-4, stats


def test_c2_full_size_on_token_subset():
    w = wl.WORKLOADS["c2"]
    subset = torch.arange(0, w.tokens, 16)
    _run_case(w, token_subset=subset)


def test_target_shape_full_size_on_token_subset():
    # The headline shape (C2 geometry at T = 32768, R = 131072): 256-row tiles
    # and remainder tiles, as in the benchmark; compared on every 128th token.
    w = wl.WORKLOADS["target"]
    _run_case(w, token_subset=torch.arange(0, w.tokens, 128))


def test_c3_zipf_full_size_on_token_subset():
    # E=128, top-8, Zipf-biased logits: at least 5 experts receive no token.
    w = wl.WORKLOADS["c3"]
    logits = wl.router_logits(w)
    idx_np, _ = oroute.route_topk(logits.numpy(), w.top_k)
    assert (np.bincount(idx_np.reshape(-1), minlength=w.experts) == 0).sum() >= 5
    _run_case(w, token_subset=torch.arange(0, w.tokens, 32))


def test_c4_int8_rank32_full_size_on_token_subset():
    w = wl.WORKLOADS["c4"]
    _run_case(w, token_subset=torch.arange(0, w.tokens, 128))


@pytest.mark.parametrize("r", [16, 72])
def test_run_for_loop_matches_oracle(r):
    w = small("nf4", T=200, E=6, k=1, r=r, alpha=float(r))
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    m = build_module(w, dense, lora)
    counts = torch.tensor([50, 0, 70, 1, 79, 0])
    x = wl.tokens(w)
    with torch.no_grad():
        out = m.run_for_loop(x.cuda(), counts.cuda())
    ref = olayer.for_loop_forward(x, counts, oracle_weights(w, dense), oracle_loras(w, lora))
    assert_layer_close(out.cpu(), ref)


@pytest.mark.parametrize("r", [16, 160])
def test_grouped_linear_matches_oracle(r):
    w = small("int8", T=150, E=4, k=1, d=256, f=320, r=r, alpha=float(r))
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    m = build_module(w, dense, lora, access="full_dequant")
    counts = torch.tensor([40, 60, 0, 50])
    offsets = counts.cumsum(0).to(torch.int32)
    x = wl.tokens(w)
    with torch.no_grad():
        out = m.grouped_linear("w1", x.cuda(), offsets=offsets.cuda())
    ref = olayer.grouped_linear(x, counts, oracle_weights(w, dense)["w1"],
                                oracle_loras(w, lora)["w1"])
    assert_layer_close(out.cpu(), ref)


def test_routed_layer_is_deterministic():
    w = small("nf4", T=512, E=16, k=4)
    dense = wl.dense_weights(w)
    m = build_module(w, dense, wl.lora_factors(w))
    x = wl.tokens(w).cuda()
    idx, scores = route_topk(wl.router_logits(w).cuda(), w.top_k)
    with torch.no_grad():
        a = m.run_direct_routed(x, scores, idx)
        b = m.run_direct_routed(x, scores, idx)
    assert torch.equal(a, b)
    np.testing.assert_array_equal(a.float().cpu().numpy(), b.float().cpu().numpy())


def test_module_built_from_a_provider_base_with_a_foreign_spec():
    """CompressedGroupedExperts(base) where the base carries its own spec class
    and tensor names (as LingBot providers set mirai_expert_mlp_spec,
    lingbot_video/pipeline.py:1678); the layer then matches the oracle."""
    from dataclasses import dataclass

    from mirai_amd import CompressedGroupedExperts

    @dataclass(frozen=True)
    class Role:
        role: str
        tensor_name: str

    @dataclass(frozen=True)
    class Spec:
        projections: tuple
        activation: str = "silu"
        combiner: str = "gated_product"

    w = small("nf4", T=200, E=6, k=2)
    dense = wl.dense_weights(w)
    spec = Spec((Role("gate", "gate_proj"), Role("up", "up_proj"), Role("down", "down_proj")))

    class Base(torch.nn.Module):
        num_experts = w.experts
        mirai_expert_mlp_spec = spec

        def __init__(self):
            super().__init__()
            self.gate_proj = dense["w1"].cuda()
            self.up_proj = dense["w3"].cuda()
            self.down_proj = dense["w2"].cuda()

    m = CompressedGroupedExperts(Base(), quant_format="nf4", expert_weight_access="chunked_dequant",
                                 expert_dequant_chunk_size=8)
    assert m.expert_mlp_spec is spec and m.is_fully_loaded()
    x = wl.tokens(w)
    idx_np, scores_np = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    idx, scores = torch.from_numpy(idx_np), torch.from_numpy(scores_np)
    with torch.no_grad():
        out = m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda())
    ref = olayer.layer_forward(x, scores, idx, oracle_weights(w, dense), {}, w.experts)
    assert_layer_close(out.cpu(), ref)


def test_logical_aliases_coalesce_token_choice_routes():
    """Routes over 10 logical experts aliased onto 6 physical ones
    (experts.py:1767-1770): same output as the oracle on the coalesced
    physical routes (duplicate physical slots summed into the first)."""
    w = small("nf4", T=240, E=6, k=3)
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    m = build_module(w, dense, lora)
    aliases = (0, 1, 2, 3, 4, 5, 2, 0, 5, 1)
    m.configure_logical_expert_aliases(aliases)
    g = torch.Generator().manual_seed(8)
    idx = torch.stack([torch.randperm(10, generator=g)[:3] for _ in range(w.tokens)])
    scores = torch.rand(w.tokens, 3, generator=g)
    x = wl.tokens(w)
    with torch.no_grad():
        out = m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda())
    phys = torch.tensor(aliases)[idx]
    coalesced = torch.zeros_like(scores)
    for t in range(w.tokens):
        for j in range(3):
            first = min(i for i in range(3) if phys[t, i] == phys[t, j])
            coalesced[t, first] += scores[t, j]
    assert bool((coalesced == 0).any())
    ref = olayer.layer_forward(x, coalesced, phys, oracle_weights(w, dense),
                               oracle_loras(w, lora), w.experts)
    assert_layer_close(out.cpu(), ref)


def test_out_of_range_route_ids_are_reported():
    """Expert ids outside [0, E) are left out of the computation and reported
    as RouteIndexError (a ValueError, as the reference's bincount refuses
    negative ids, dispatch_preprocess.py:155-157): after the fact by default,
    at the call in "sync" mode."""
    import mirai_amd
    from mirai_amd import _native as nat

    w = small("bf16", T=64, E=8, k=2)
    dense = wl.dense_weights(w)
    m = build_module(w, dense, None)
    x = wl.tokens(w)
    idx_np, scores_np = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    idx, scores = torch.from_numpy(idx_np), torch.from_numpy(scores_np)
    bad = idx.clone()
    bad[3, 1] = 8
    bad[10, 0] = -1
    mirai_amd.check_route_errors()
    with torch.no_grad():
        out = m.run_direct_routed(x.cuda(), scores.cuda(), bad.cuda())
    with pytest.raises(mirai_amd.RouteIndexError, match="2 route slot"):
        mirai_amd.check_route_errors()
    # The valid slots are computed as usual.
    kept = scores.clone()
    kept[3, 1] = 0.0
    kept[10, 0] = 0.0
    ref = olayer.layer_forward(x, kept, bad.clamp(0, w.experts - 1), oracle_weights(w, dense),
                               {}, w.experts)
    assert_layer_close(out.cpu(), ref)
    # Valid routes leave nothing behind.
    with torch.no_grad():
        m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda())
    mirai_amd.check_route_errors()
    previous = nat.route_check_mode()
    mirai_amd.set_route_check("sync")
    try:
        with pytest.raises(ValueError, match="expert id outside"), torch.no_grad():
            m.run_direct_routed(x.cuda(), scores.cuda(), bad.cuda())
    finally:
        mirai_amd.set_route_check(previous)


def test_empty_inputs_through_every_inference_entry_point():
    """No rows: each call returns an empty result and leaves no deferred route
    error behind (the next call with rows checks the plan it builds)."""
    w = small("nf4", T=64, E=4, k=2, d=128, f=128)
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    m = build_module(w, dense, lora)
    d = w.hidden
    empty = torch.empty(0, d, dtype=torch.bfloat16, device="cuda")
    with torch.no_grad():
        assert tuple(m.run_direct_routed(empty, torch.empty(0, 2, device="cuda"),
                                         torch.empty(0, 2, dtype=torch.int64, device="cuda")).shape) == (0, d)
        assert tuple(m.run_for_loop(empty, torch.zeros(w.experts, dtype=torch.int64,
                                                        device="cuda")).shape) == (0, d)
        ec = m.run_expert_choice_routed(empty, torch.empty(0, w.experts, 4, device="cuda"),
                                        torch.empty(0, w.experts, 4, dtype=torch.int64,
                                                    device="cuda"), tokens_per_sample=16)
        assert tuple(ec.shape) == (0, d)
    fl = build_module(w, dense, lora, access="full_dequant")
    with torch.no_grad():
        out = fl.grouped_linear("w1", empty, offsets=torch.zeros(w.experts, dtype=torch.int32,
                                                                 device="cuda"))
    assert tuple(out.shape) == (0, w.ffn)
    # A call with rows afterwards still matches the oracle (and raises nothing).
    _run_case(w)


@pytest.mark.parametrize("keys", [("w2",), ("w1",), ("w3", "w2")])
def test_inference_with_a_subset_of_adapters(keys):
    w = small("nf4", T=1100, E=4, k=2, d=192, f=256)
    lora = {k: v for k, v in wl.lora_factors(w).items() if k in keys}
    _run_case(w, lora=lora)


@pytest.mark.parametrize("k", [1, 3, 5, 7])
def test_routed_layer_top_k(k):
    """top-1 and the odd top-k values (the combine's unrolled and generic paths)."""
    _run_case(small("nf4", T=300, E=8, k=k, d=128, f=192))


@pytest.mark.parametrize("r", [4, 12, 36])
def test_lora_ranks_off_the_multiple_of_eight(r):
    _run_case(small("nf4", r=r, alpha=2.0 * r, E=5, k=3, T=300, f=320, d=192))


@pytest.mark.parametrize("fmt,r,T,E,k", [("nf4", 16, 1400, 9, 2), ("int8", 32, 600, 8, 2),
                                         ("bf16", 8, 300, 16, 2), ("nf4", 64, 700, 6, 2),
                                         ("nf4", 24, 500, 12, 4)])
def test_inference_forward_equals_training_forward(fmt, r, T, E, k):
    # The training forward (saved activations, LoRA rows kept) and the
    # inference forward run the same kernels on the same rows: the outputs
    # agree bit for bit. Skewed routes put light experts (at most 32 rows)
    # next to tall tiles.
    from test_gpu_light_tiles import LIGHT_COUNTS, skewed_routes

    w = wl.Workload(f"inf_train_{fmt}", 12, T, 256, 384, E, k, r, 16.0, fmt, torch.bfloat16)
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    m = build_module(w, dense, lora)
    counts = LIGHT_COUNTS[: E - k]
    idx, scores = skewed_routes(T, E, k, counts, seed=9)
    x = wl.tokens(w).cuda()
    with torch.no_grad():
        out_inf = m.run_direct_routed(x, scores.cuda(), idx.cuda())
    xg = x.clone().requires_grad_(True)
    out_train = m.run_direct_routed(xg, scores.cuda(), idx.cuda())
    assert torch.equal(out_inf, out_train.detach())
    ref = olayer.layer_forward(x.cpu(), scores, idx, oracle_weights(w, dense, dtype=w.dtype),
                               oracle_loras(w, lora), w.experts)
    assert_layer_close(out_inf.cpu(), ref)
