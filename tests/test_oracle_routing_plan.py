"""Pins the oracle's routing and dispatch plan (CPU only) against torch's
library routines, the reference tests' known answers, closed forms and
finite differences."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import plan as oplan
from oracle import routing as oroute

GOLDEN = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


# ------------------------------------------------------------------ routing
def test_route_index_sets_match_torch_topk():
    rng = np.random.default_rng(10)
    logits = rng.standard_normal((512, 64)).astype(np.float32)
    idx, scores = oroute.route_topk(logits, 4, renorm=oroute.RENORM_NONE)
    probs = torch.softmax(torch.from_numpy(logits), dim=-1)
    tv, ti = torch.topk(probs, 4, dim=-1, sorted=True)
    # No ties in continuous random data: the sets, and the descending order, agree.
    np.testing.assert_array_equal(idx, ti.numpy())
    np.testing.assert_allclose(scores, tv.numpy(), rtol=2e-6, atol=1e-9)


@pytest.mark.parametrize("case", GOLDEN["route_ties"]["cases"])
def test_route_tie_rule_known_answers(case):
    idx, _ = oroute.route_topk(np.array([case["logits"]], dtype=np.float32), case["k"])
    assert idx[0].tolist() == case["top_idx"]


def test_route_renormalisation_modes():
    rng = np.random.default_rng(11)
    logits = rng.standard_normal((64, 16)).astype(np.float32)
    _, clamp = oroute.route_topk(logits, 3, renorm=oroute.RENORM_CLAMP, route_scale=2.5)
    np.testing.assert_allclose(clamp.astype(np.float64).sum(axis=1), 2.5, rtol=1e-6)
    idx, none = oroute.route_topk(logits, 3, renorm=oroute.RENORM_NONE)
    _, eps = oroute.route_topk(logits, 3, renorm=oroute.RENORM_EPS)
    np.testing.assert_allclose(eps, none / none.sum(axis=1, keepdims=True), rtol=1e-6)
    # Scores are the selected softmax probabilities, in slot order.
    probs = torch.softmax(torch.from_numpy(logits).double(), dim=-1).numpy()
    np.testing.assert_allclose(none, np.take_along_axis(probs, idx, axis=1), rtol=1e-6)


@pytest.mark.parametrize("renorm", [oroute.RENORM_NONE, oroute.RENORM_CLAMP, oroute.RENORM_EPS])
def test_route_backward_matches_finite_differences(renorm):
    rng = np.random.default_rng(12)
    logits = rng.standard_normal((3, 6)).astype(np.float64)
    idx, _ = oroute.route_topk(logits.astype(np.float32), 2, renorm=renorm, route_scale=1.7)
    g = rng.standard_normal((3, 2))
    grad = oroute.route_topk_backward(logits, idx, g, renorm=renorm, route_scale=1.7)

    def f(lg):
        p = np.exp(lg - lg.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        s = np.take_along_axis(p, idx, axis=1)
        tot = s.sum(axis=1, keepdims=True)
        if renorm == oroute.RENORM_CLAMP:
            s = s / np.maximum(tot, 1e-20)
        elif renorm == oroute.RENORM_EPS:
            s = s / (tot + 1e-20)
        return float((s * 1.7 * g).sum())

    h = 1e-6
    num = np.zeros_like(logits)
    for i in range(logits.shape[0]):
        for j in range(logits.shape[1]):
            lp, lm = logits.copy(), logits.copy()
            lp[i, j] += h
            lm[i, j] -= h
            num[i, j] = (f(lp) - f(lm)) / (2 * h)
    np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-8)


# --------------------------------------------------------------------- plan
@pytest.mark.parametrize("key", ["plan_specialization", "plan_six_slots"])
def test_plan_known_answers(key):
    case = GOLDEN[key]
    p = oplan.build_dispatch_plan(np.array(case["top_idx"]), None, case["num_experts"])
    for field in ("counts", "starts", "offsets", "sort_positions", "sorted_token_indices",
                  "inverse_order"):
        assert getattr(p, field).tolist() == case[field], field
    assert p.offsets.dtype == np.int32 and p.counts.dtype == np.int64


def test_plan_matches_torch_stable_argsort_bincount_cumsum():
    g = torch.Generator().manual_seed(11)
    idx = torch.randint(0, 23, (257, 4), generator=g)  # shapes of the reference's plan test
    scores = torch.randn(257, 4, generator=g)
    p = oplan.build_dispatch_plan(idx.numpy(), scores.numpy(), 23)
    flat = idx.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=23)
    np.testing.assert_array_equal(p.sort_positions, order.numpy())
    np.testing.assert_array_equal(p.sorted_token_indices, (order // 4).numpy())
    np.testing.assert_array_equal(p.counts, counts.numpy())
    np.testing.assert_array_equal(p.offsets, torch.cumsum(counts, 0).to(torch.int32).numpy())
    np.testing.assert_array_equal(p.starts, (torch.cumsum(counts, 0) - counts).numpy())
    np.testing.assert_array_equal(p.sorted_scores, scores.reshape(-1)[order].numpy())
    inv = torch.empty_like(order)
    inv[order] = torch.arange(order.numel())
    np.testing.assert_array_equal(p.inverse_order, inv.numpy())


def test_plan_invariants_and_dropped_ids():
    rng = np.random.default_rng(13)
    idx = rng.integers(-2, 10, (300, 3))
    p = oplan.build_dispatch_plan(idx, None, 8)
    valid = (idx >= 0) & (idx < 8)
    assert p.offsets[-1] == valid.sum() == p.sort_positions.size
    np.testing.assert_array_equal(p.inverse_order[p.sort_positions], np.arange(p.sort_positions.size))
    assert np.all(p.inverse_order[~valid.reshape(-1)] == -1)
    for e in range(8):
        seg = p.sorted_token_indices[p.starts[e]:p.offsets[e]]
        assert np.all(np.diff(seg) >= 0)  # stable: ascending (token, slot) order
        assert np.all(idx.reshape(-1)[p.sort_positions[p.starts[e]:p.offsets[e]]] == e)
