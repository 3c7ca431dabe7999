"""GPU dispatch plan parity: every field bit-exact vs the oracle."""

import numpy as np
import pytest
import torch

from mirai_amd import build_dispatch_plan, combine_routed_tokens, permute_routed_tokens
from mirai_amd import workloads as wl
from oracle import plan as oplan
from oracle import routing as oroute

pytestmark = pytest.mark.gpu


def _check(top_idx: np.ndarray, top_scores: np.ndarray, E: int):
    plan = build_dispatch_plan(torch.from_numpy(top_idx).cuda(),
                               torch.from_numpy(top_scores).cuda(), E)
    ref = oplan.build_dispatch_plan(top_idx, top_scores, E)
    np.testing.assert_array_equal(plan.counts.cpu().numpy(), ref.counts)
    np.testing.assert_array_equal(plan.starts.cpu().numpy(), ref.starts)
    np.testing.assert_array_equal(plan.offsets.cpu().numpy(), ref.offsets)
    S = ref.sort_positions.shape[0]
    np.testing.assert_array_equal(plan.sort_positions.cpu().numpy()[:S], ref.sort_positions)
    np.testing.assert_array_equal(plan.sorted_token_indices.cpu().numpy()[:S],
                                  ref.sorted_token_indices)
    np.testing.assert_array_equal(plan.sorted_scores.cpu().numpy()[:S], ref.sorted_scores)
    np.testing.assert_array_equal(plan.inverse_order.cpu().numpy(), ref.inverse_order)
    return plan


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "target"])
def test_plan_on_benchmark_routes(name):
    w = wl.WORKLOADS[name]
    idx, scores = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    plan = _check(idx, scores, w.experts)
    if name == "c3":
        assert int((plan.counts == 0).sum()) >= 5  # the skewed config leaves experts empty


def test_plan_known_answer():
    # Routes of tests/test_moe_expert_optimizations.py:447-449 style: [T=3, k=2].
    idx = np.array([[2, 0], [2, 1], [0, 3]], dtype=np.int64)
    scores = np.arange(6, dtype=np.float32).reshape(3, 2)
    plan = _check(idx, scores, 4)
    assert plan.sort_positions.cpu().tolist() == [1, 4, 3, 0, 2, 5]
    assert plan.counts.cpu().tolist() == [2, 1, 2, 1]
    assert plan.offsets.cpu().tolist() == [2, 3, 5, 6]


@pytest.mark.parametrize("T,k,E", [(1, 1, 1), (7, 3, 5), (4097, 2, 1024), (20000, 8, 3),
                                   (3000, 4, 700), (3000, 2, 1025), (9000, 3, 3072),
                                   (500, 4, 8192)])
def test_plan_random_with_duplicates_and_invalid_ids(T, k, E):
    rng = np.random.default_rng(T + k + E)
    idx = rng.integers(0, E, size=(T, k)).astype(np.int64)
    idx[::13, 0] = idx[::13, -1]            # duplicate expert within a token
    idx[5::97, -1] = E + 3                  # out-of-range ids are dropped
    idx[9::101, 0] = -1
    scores = rng.standard_normal((T, k)).astype(np.float32)
    _check(idx, scores, E)


def test_plan_bf16_scores_and_zero_tokens():
    idx = np.zeros((0, 4), dtype=np.int64)
    plan = build_dispatch_plan(torch.from_numpy(idx).cuda(), torch.zeros((0, 4)).cuda(), 8)
    assert plan.counts.cpu().tolist() == [0] * 8
    rng = np.random.default_rng(0)
    idx = rng.integers(0, 16, size=(100, 2)).astype(np.int64)
    s = torch.randn(100, 2).to(torch.bfloat16)
    plan = build_dispatch_plan(torch.from_numpy(idx).cuda(), s.cuda(), 16)
    ref = oplan.build_dispatch_plan(idx, s.float().numpy(), 16)
    np.testing.assert_array_equal(plan.sorted_scores.float().cpu().numpy(), ref.sorted_scores)


def test_permute_and_combine_match_index_add_with_duplicates():
    """tests/test_moe_expert_optimizations.py:443-470 on the GPU kernels."""
    torch.manual_seed(7)
    tokens = torch.randn(3, 8, requires_grad=True)
    indices = torch.tensor([2, 0, 2, 1, 0])
    scores = torch.randn(5, requires_grad=True)
    tg = tokens.detach().cuda().requires_grad_(True)
    sg = scores.detach().cuda().requires_grad_(True)
    sorted_tokens = permute_routed_tokens(tg, indices.cuda())
    expert_output = sorted_tokens.square()
    actual = combine_routed_tokens(expert_output, sg, indices.cuda(), output_rows=3,
                                   output_dtype=torch.float32)
    reference = torch.zeros(3, 8).index_add(0, indices, tokens.index_select(0, indices).square()
                                            * scores.unsqueeze(1))
    torch.testing.assert_close(actual.cpu(), reference)
    grad = torch.randn(3, 8)
    actual.backward(grad.cuda())
    reference.backward(grad)
    torch.testing.assert_close(tg.grad.cpu(), tokens.grad)
    torch.testing.assert_close(sg.grad.cpu(), scores.grad)


def test_empty_routes_plan_permute_and_combine():
    """No routed slots: an all-zero plan, empty permutation arrays, and
    permute / combine (forward and backward) over empty rows."""
    idx = torch.empty(0, 2, dtype=torch.int64, device="cuda")
    scores = torch.empty(0, 2, device="cuda")
    plan = build_dispatch_plan(idx, scores, 5)
    assert plan.counts.tolist() == [0] * 5 and plan.starts.tolist() == [0] * 5
    assert plan.offsets.tolist() == [0] * 5 and plan.total_slots == 0
    assert plan.sort_positions.numel() == 0 and plan.inverse_order.numel() == 0
    tokens = torch.randn(3, 8, device="cuda").requires_grad_(True)
    none = torch.empty(0, dtype=torch.int64, device="cuda")
    rows = permute_routed_tokens(tokens, none)
    assert tuple(rows.shape) == (0, 8)
    sc = torch.empty(0, device="cuda").requires_grad_(True)
    out = combine_routed_tokens(rows, sc, none, output_rows=3, output_dtype=torch.float32)
    assert torch.equal(out, torch.zeros(3, 8, device="cuda"))
    out.sum().backward()
    assert torch.equal(tokens.grad, torch.zeros_like(tokens))
    assert tuple(sc.grad.shape) == (0,)


def test_empty_expert_choice_plan():
    from mirai_amd import build_expert_choice_dispatch_plan

    idx = torch.empty(0, 4, 3, dtype=torch.int64, device="cuda")
    plan = build_expert_choice_dispatch_plan(idx, torch.empty(0, 4, 3, device="cuda"),
                                             tokens_per_sample=8, num_physical_experts=4)
    assert plan.counts.tolist() == [0] * 4 and plan.total_slots == 0
    assert plan.sorted_token_indices.numel() == 0
