"""GPU parity of expert-choice routing: the plan bit-exact against the
oracle restatement of build_expert_choice_dispatch_plan, and the routed layer
against the oracle's per-expert index_add composition (layer tolerance)."""

import numpy as np
import pytest
import torch

from mirai_amd import build_expert_choice_dispatch_plan
from mirai_amd import workloads as wl
from oracle import expert_choice as oec

from helpers import assert_layer_close, build_module, oracle_loras, oracle_weights

pytestmark = pytest.mark.gpu


def _routes(B, L, C, tps, seed, score_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(tps, generator=g)[:C] for _ in range(B * L)]).view(B, L, C)
    scores = torch.rand(B, L, C, generator=g).to(score_dtype)
    return idx, scores


@pytest.mark.parametrize("B,L,C,tps,alias", [
    (1, 4, 1, 3, ()),
    (2, 8, 16, 64, ()),
    (3, 6, 5, 20, (2, 0, 2, 1, 0, 2)),
    (1, 64, 2048, 32768, ()),
    (2, 128, 96, 3000, tuple((7 * l) % 40 for l in range(128))),
])
@pytest.mark.parametrize("score_dtype", [torch.float32, torch.bfloat16])
def test_plan_matches_oracle(B, L, C, tps, alias, score_dtype):
    idx, scores = _routes(B, L, C, tps, B * L + C, score_dtype)
    E = max(alias) + 1 if alias else L
    plan = build_expert_choice_dispatch_plan(idx.cuda(), scores.cuda(), tokens_per_sample=tps,
                                             num_physical_experts=E, logical_to_physical=alias)
    ref = oec.build_expert_choice_plan(idx.numpy(), scores.float().numpy(), tps, E, alias)
    for key in ("counts", "starts", "offsets", "sort_positions", "sorted_token_indices",
                "inverse_order"):
        np.testing.assert_array_equal(getattr(plan, key).cpu().numpy(), ref[key], err_msg=key)
    np.testing.assert_array_equal(plan.sorted_scores.float().cpu().numpy(), ref["sorted_scores"])
    assert plan.top_k == 0 and plan.total_slots == B * L * C


def _layer_case(fmt, B, L, C, tps, *, alias=(), lora=True, d=128, f=192, seed=0,
                token_dtype=torch.bfloat16):
    E = max(alias) + 1 if alias else L
    w = wl.Workload(f"ec_{fmt}", 11 + seed, B * tps, d, f, E, 1, 16, 16.0, fmt, torch.bfloat16)
    dense = wl.dense_weights(w)
    factors = wl.lora_factors(w) if lora else None
    m = build_module(w, dense, factors, access="active_dequant")
    if alias:
        m.set_logical_to_physical_map(alias)
    idx, scores = _routes(B, L, C, tps, seed + 5)
    x = wl.tokens(w).to(token_dtype)
    with torch.no_grad():
        out = m.run_expert_choice_routed(x.cuda(), scores.cuda(), idx.cuda(),
                                         tokens_per_sample=tps)
    assert out.dtype == x.dtype and out.shape == x.shape
    ref = oec.expert_choice_forward(x.to(torch.bfloat16), scores, idx, tps,
                                    oracle_weights(w, dense), oracle_loras(w, factors), E, alias)
    return out.cpu(), ref, idx


@pytest.mark.parametrize("fmt", ["nf4", "int8", "bf16"])
def test_layer_matches_oracle(fmt):
    out, ref, idx = _layer_case(fmt, 2, 8, 24, 96)
    print(f"expert choice {fmt}: {assert_layer_close(out, ref)}")
    picked = torch.zeros(2 * 96, dtype=torch.bool)
    picked[(idx + (torch.arange(2) * 96).view(2, 1, 1)).reshape(-1)] = True
    assert torch.count_nonzero(out[~picked]) == 0  # tokens no expert picked stay zero


def test_layer_with_aliases_and_fp32_tokens():
    alias = (3, 0, 3, 1, 2, 0)
    out, ref, _ = _layer_case("nf4", 2, 6, 10, 40, alias=alias, seed=3,
                              token_dtype=torch.float32)
    assert out.dtype == torch.float32
    print(f"expert choice aliases: {assert_layer_close(out, ref.float())}")


def test_layer_at_scale_on_a_token_subset():
    # capacity = T * k / E for T = 8192, k = 4, E = 64
    out, ref, _ = _layer_case("nf4", 1, 64, 512, 8192, lora=True, d=256, f=128, seed=7)
    print(f"expert choice at scale: {assert_layer_close(out, ref)}")


def test_reference_contract_routes():
    # expert 0 and 3 both pick token 0 (artifact_transforms.py:1855-1858)
    w = wl.Workload("ec_contract", 31, 3, 64, 64, 4, 1, 8, 8.0, "bf16", torch.bfloat16)
    dense = wl.dense_weights(w)
    m = build_module(w, dense, None, access="chunked_dequant")
    idx = torch.tensor([[[0], [1], [2], [0]]])
    scores = torch.tensor([[[0.8], [0.7], [0.6], [0.5]]])
    x = wl.tokens(w)
    with torch.no_grad():
        out = m.run_expert_choice_routed(x.cuda(), scores.cuda(), idx.cuda(), tokens_per_sample=3)
    ref = oec.expert_choice_forward(x, scores, idx, 3, oracle_weights(w, dense), {}, 4)
    assert_layer_close(out.cpu(), ref)
    with pytest.raises(ValueError):
        m.run_expert_choice_routed(x.cuda(), scores.cuda(), idx.cuda(), tokens_per_sample=2)


def _close_grad(name, actual, expected, mean_rel=5e-3, max_rel=3e-2):
    a, e = actual.detach().float().cpu(), expected.detach().float().cpu()
    diff = (a - e).abs()
    stats = {"mean_rel": float(diff.sum() / e.abs().sum().clamp_min(1e-30)),
             "max_rel": float(diff.max()) / float(e.abs().max().clamp_min(1e-30))}
    assert stats["mean_rel"] <= mean_rel and stats["max_rel"] <= max_rel, (name, stats)
    return stats


@pytest.mark.parametrize("fmt,alias,rank", [("nf4", (), 16), ("int8", (), 16),
                                            ("nf4", (3, 0, 3, 1, 2, 0, 1, 2), 16),
                                            ("int8", (), 64)])
def test_backward_matches_oracle_autograd(fmt, alias, rank):
    # Gradients to tokens, [B, L, C] scores and every LoRA factor against torch
    # autograd through the oracle's gather / per-expert MLP / index_add
    # composition (bounds as the token-choice backward: mean-rel 5e-3, max
    # 3e-2 of the oracle's max). Tokens picked by several experts sum their
    # slots' dx rows; tokens no expert picked get zero.
    B, L, C, tps = 2, 8, 24, 96
    E = max(alias) + 1 if alias else L
    w = wl.Workload(f"ec_bwd_{fmt}", 21, B * tps, 256, 192, E, 1, rank, float(rank), fmt,
                    torch.bfloat16)
    dense, lora = wl.dense_weights(w), wl.lora_factors(w)
    m = build_module(w, dense, lora, access="active_dequant")
    if alias:
        m.set_logical_to_physical_map(alias)
    idx, scores = _routes(B, L, C, tps, 9)
    x = wl.tokens(w)
    dy = wl.upstream_grad(w)
    xg = x.cuda().requires_grad_(True)
    sg = scores.cuda().requires_grad_(True)
    out = m.run_expert_choice_routed(xg, sg, idx.cuda(), tokens_per_sample=tps)
    out.backward(dy.cuda())
    xo = x.clone().requires_grad_(True)
    so = scores.clone().requires_grad_(True)
    leaves = {k: (a.clone().float().requires_grad_(True), b.clone().float().requires_grad_(True))
              for k, (a, b) in lora.items()}
    ref = oec.expert_choice_forward(xo, so, idx, tps, oracle_weights(w, dense),
                                    {k: (a, b, wl.lora_scale(w)) for k, (a, b) in leaves.items()},
                                    E, alias)
    ref.backward(dy)
    assert_layer_close(out.detach().cpu(), ref)
    report = {"tokens": _close_grad("tokens", xg.grad, xo.grad),
              "scores": _close_grad("scores", sg.grad, so.grad)}
    for k, (a, b) in leaves.items():
        report[f"{k}.a"] = _close_grad(f"{k}.a", m.expert_lora[k].lora_a.grad, a.grad)
        report[f"{k}.b"] = _close_grad(f"{k}.b", m.expert_lora[k].lora_b.grad, b.grad)
    picked = torch.zeros(B * tps, dtype=torch.bool)
    picked[(idx + (torch.arange(B) * tps).view(B, 1, 1)).reshape(-1)] = True
    assert torch.count_nonzero(xg.grad[~picked.cuda()]) == 0
    print(f"expert choice backward {fmt} {alias}: {report}")
