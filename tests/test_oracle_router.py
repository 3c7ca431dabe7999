"""CPU checks of the LingBot router oracle (oracle/router.py) against brute
force, known answers and properties that fix the selection rule."""

import itertools

import numpy as np
import pytest
import torch

from oracle import router as orr


def _case(T=24, E=12, d=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g).to(torch.bfloat16)
    w = torch.randn(E, d, generator=g) * 0.05
    bias = torch.randn(E, generator=g) * 0.02
    return x, w, bias


@pytest.mark.parametrize("score_func", ["softmax", "sigmoid"])
def test_selection_is_the_k_largest_keys_with_low_index_ties(score_func):
    x, w, bias = _case()
    idx, top, logits, scores, choice = orr.router_forward(
        x, w, 4, score_func=score_func, expert_bias=bias, norm_topk_prob=False)
    for t in range(x.shape[0]):
        picked = idx[t].tolist()
        assert len(set(picked)) == 4
        keys = choice[t].tolist()
        # every pick beats every non-pick (ties: lower id first), picks in order
        for e in picked:
            for f in range(len(keys)):
                if f not in picked:
                    assert keys[e] > keys[f] or (keys[e] == keys[f] and e < f)
        for a, b in zip(picked, picked[1:]):
            assert keys[a] > keys[b] or (keys[a] == keys[b] and a < b)
        # the gating weights are the bias-free scores
        torch.testing.assert_close(top[t].float(), scores[t, picked].to(x.dtype).float())


def test_exact_ties_go_to_the_lower_expert():
    logits = torch.tensor([[0.5, 1.0, 1.0, 0.2, 1.0]])
    idx, _, _, _ = orr.route_from_logits(logits, 2, score_func="sigmoid")
    assert idx.tolist() == [[1, 2]]
    idx, _, _, _ = orr.route_from_logits(logits, 3, score_func="softmax")
    assert idx.tolist() == [[1, 2, 4]]


def test_bias_steers_selection_only():
    logits = torch.tensor([[2.0, 1.0, 0.0, -1.0]])
    bias = torch.tensor([0.0, 0.0, 0.0, 5.0])
    idx, top, scores, _ = orr.route_from_logits(logits, 2, score_func="sigmoid", expert_bias=bias,
                                                norm_topk_prob=False)
    assert idx.tolist() == [[3, 0]]
    s = torch.sigmoid(torch.tensor([-1.0, 2.0]))
    torch.testing.assert_close(top[0], s)


def test_renorm_adds_1e20_instead_of_clamping():
    # sigmoid(-50) = 1.93e-22: the picks' sum 3.9e-22 is far below 1e-20, so
    # p / (sum + 1e-20) is 0.0186 each; a clamp at 1e-20 would give 0.0193
    # (4 % more) and a plain p / sum 0.5.
    logits = torch.full((1, 6), -60.0)
    logits[0, 1] = -50.0
    logits[0, 4] = -50.0
    idx, top, _, _ = orr.route_from_logits(logits, 2, score_func="sigmoid", route_scale=2.0)
    assert idx.tolist() == [[1, 4]]
    p = 1.0 / (1.0 + np.exp(50.0))
    s32 = np.float32(p)
    want = np.float32(s32 / np.float32(np.float32(s32 + s32) + np.float32(1e-20))) * np.float32(2.0)
    np.testing.assert_allclose(top[0].numpy(), [want, want], rtol=1e-6)
    assert abs(float(top[0, 0]) - 2.0 * 0.5) > 0.5


def test_top1_is_never_renormalised():
    logits = torch.tensor([[0.3, -0.2, 1.1]])
    _, top, _, _ = orr.route_from_logits(logits, 1, score_func="sigmoid", route_scale=1.5)
    np.testing.assert_allclose(float(top[0, 0]), 1.5 / (1 + np.exp(-1.1)), rtol=1e-6)
    _, top, _, _ = orr.route_from_logits(logits, 2, score_func="sigmoid", route_scale=1.5)
    np.testing.assert_allclose(float(top[0].sum()), 1.5, rtol=1e-6)


def _brute_group_limited(keys, k, n_group, topk_group):
    """Plain-loop restatement: group scores, best groups, then best experts."""
    E = len(keys)
    epg = E // n_group
    gsc = []
    for g in range(n_group):
        vals = sorted(keys[g * epg:(g + 1) * epg], reverse=True)
        gsc.append(vals[0] + vals[1])
    best = None
    for combo in itertools.combinations(range(n_group), topk_group):
        score = sorted((gsc[g] for g in combo), reverse=True)
        key = (score, [-g for g in combo])
        if best is None or key > best[0]:
            best = (key, combo)
    allowed = [e for e in range(E) if e // epg in best[1]]
    ranked = sorted(allowed, key=lambda e: (-keys[e], e))
    return ranked[:k]


@pytest.mark.parametrize("n_group,topk_group,k", [(4, 2, 3), (6, 3, 4), (3, 1, 2)])
def test_group_limited_choice_matches_brute_force(n_group, topk_group, k):
    g = torch.Generator().manual_seed(n_group * 10 + topk_group)
    logits = torch.randn(40, 24, generator=g)
    bias = torch.randn(24, generator=g) * 0.1
    idx, _, _, choice = orr.route_from_logits(logits, k, score_func="sigmoid", expert_bias=bias,
                                              n_group=n_group, topk_group=topk_group)
    for t in range(logits.shape[0]):
        want = _brute_group_limited([float(v) for v in choice[t]], k, n_group, topk_group)
        assert idx[t].tolist() == want


def test_group_limited_changes_the_choice_somewhere():
    # Planted-mistake guard: ignoring the group limit gives different picks.
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(64, 16, generator=g)
    a, _, _, _ = orr.route_from_logits(logits, 4, n_group=4, topk_group=1)
    b, _, _, _ = orr.route_from_logits(logits, 4)
    assert not torch.equal(a, b)


def test_softmax_without_bias_picks_the_largest_logits():
    x, w, _ = _case(T=50, E=32, seed=3)
    idx, _, logits, _, _ = orr.router_forward(x, w, 6, score_func="softmax")
    want = np.argsort(-logits.numpy(), axis=1, kind="stable")[:, :6]
    np.testing.assert_array_equal(idx.numpy(), want)


def test_logits_are_fp32_linear_within_the_stated_bound():
    x, w, _ = _case(T=16, E=8, d=512, seed=2)
    logits = orr.router_logits(x, w)
    exact = x.double() @ w.double().t()
    err = (logits.double() - exact).abs().max(dim=1).values
    assert bool((err <= orr.logits_error_bound(x, w)).all())
    assert logits.dtype == torch.float32


def test_scores_come_back_in_the_token_dtype():
    x, w, bias = _case()
    _, top, _, _, _ = orr.router_forward(x, w, 2, expert_bias=bias)
    assert top.dtype == torch.bfloat16
    _, top32, _, _, _ = orr.router_forward(x.float(), w, 2, expert_bias=bias)
    assert top32.dtype == torch.float32
