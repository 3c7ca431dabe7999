"""CPU checks of the MAGI-2 oracle (routing, swiglu7, layer) against closed
forms, brute force, finite differences and an independent fp64 formulation."""

import itertools

import numpy as np
import pytest
import torch

from oracle import magi2 as om
from oracle import routing as oroute


@pytest.mark.parametrize("score_func", ["softmax", "sigmoid"])
def test_route_without_bias_is_topk_by_logit(score_func):
    # softmax and sigmoid are strictly increasing: with no bias the picks are
    # the largest logits (ties to the lower id), whatever the score function.
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(3, 40, 24, generator=g)
    probs, idx = om.route_topk_heads(logits, 5, score_func=score_func, route_norm=False)
    want, _ = oroute.route_topk(logits.reshape(-1, 24).numpy(), 5, renorm=oroute.RENORM_NONE)
    np.testing.assert_array_equal(idx.reshape(-1, 5).numpy(), want)
    scores = torch.sigmoid(logits) if score_func == "sigmoid" else torch.softmax(logits, -1)
    torch.testing.assert_close(probs, scores.gather(-1, idx))


def test_route_with_bias_matches_brute_force():
    g = torch.Generator().manual_seed(11)
    H, S, E, k = 2, 7, 6, 3
    logits = torch.randn(H, S, E, generator=g)
    bias = torch.randn(H, E, generator=g) * 0.3
    probs, idx = om.route_topk_heads(logits, k, score_func="sigmoid", expert_bias=bias,
                                     route_norm=True, route_scale=2.5)
    scores = 1.0 / (1.0 + np.exp(-logits.double().numpy()))
    for h, s in itertools.product(range(H), range(S)):
        keys = [(-(scores[h, s, e] + float(bias[h, e])), e) for e in range(E)]
        pick = [e for _, e in sorted(keys)[:k]]
        assert idx[h, s].tolist() == pick
        sel = scores[h, s, pick]
        np.testing.assert_allclose(probs[h, s].numpy(), 2.5 * sel / sel.sum(), rtol=1e-6)


@pytest.mark.parametrize("E,nvg,tvg,k", [(12, 4, 2, 3), (8, 8, 3, 2), (9, 3, 1, 3)])
def test_virtual_group_route_matches_brute_force(E, nvg, tvg, k):
    # route.py:62-105 restated one token at a time: group score = sum of the
    # two largest biased scores of the group (the largest for a one-expert
    # group), keep the tvg best groups (ties to the lower id), keys of the
    # other experts become 0.0, then the k largest keys (ties to the lower id).
    g = torch.Generator().manual_seed(E * 7 + nvg)
    H, S = 2, 25
    logits = torch.randn(H, S, E, generator=g) * 2
    bias = torch.randn(H, E, generator=g) * 0.2  # negative keys occur: 0.0 can win
    probs, idx = om.route_topk_heads(logits, k, score_func="sigmoid", expert_bias=bias,
                                     route_norm=False, num_virtual_group=nvg,
                                     topk_virtual_group=tvg)
    scores = torch.sigmoid(logits)
    keys = (scores + bias.view(H, 1, E)).tolist()
    epg = E // nvg
    saw_zero_pick = False
    for h, s in itertools.product(range(H), range(S)):
        kv = keys[h][s]
        gs = []
        for grp in range(nvg):
            vals = sorted(kv[grp * epg:(grp + 1) * epg], reverse=True)
            gs.append(np.float32(vals[0]) + (np.float32(vals[1]) if epg >= 2 else np.float32(0)))
        kept = [grp for _, grp in sorted((-float(v), grp) for grp, v in enumerate(gs))[:tvg]]
        masked = [kv[e] if e // epg in kept else 0.0 for e in range(E)]
        pick = [e for _, e in sorted((-masked[e], e) for e in range(E))[:k]]
        assert idx[h, s].tolist() == pick, (h, s)
        saw_zero_pick |= any(e // epg not in kept for e in pick)
        torch.testing.assert_close(probs[h, s], scores[h, s, pick])
    if nvg == 3:
        assert saw_zero_pick  # a masked expert outranked negative kept keys somewhere


def test_virtual_groups_reduce_to_plain_selection():
    # Every group kept: the plain selection. One expert per group and
    # topk_virtual_group = k with positive keys: the plain top-k as well.
    g = torch.Generator().manual_seed(2)
    logits = torch.randn(2, 30, 16, generator=g)
    plain = om.route_topk_heads(logits, 4, score_func="softmax")
    allg = om.route_topk_heads(logits, 4, score_func="softmax", num_virtual_group=4,
                               topk_virtual_group=4)
    single = om.route_topk_heads(logits, 4, score_func="softmax", num_virtual_group=16,
                                 topk_virtual_group=4)
    for got in (allg, single):
        assert torch.equal(got[1], plain[1])
        torch.testing.assert_close(got[0], plain[0])


def test_route_probs_for_picks_is_the_forward_and_its_gradient():
    g = torch.Generator().manual_seed(6)
    logits = torch.randn(2, 10, 8, generator=g, dtype=torch.float64)
    probs, idx = om.route_topk_heads(logits.float(), 3, score_func="softmax", route_scale=1.5)
    again = om.route_probs_for_picks(logits.float(), idx, score_func="softmax", route_scale=1.5)
    torch.testing.assert_close(again, probs)
    # Its autograd against central differences of the same function in fp64.
    lg = logits.clone().requires_grad_(True)
    w = torch.randn(2, 10, 3, generator=g, dtype=torch.float64)
    f = lambda z: (om.route_probs_for_picks(z, idx, score_func="softmax", route_scale=1.5)
                   .double() * w).sum()
    assert torch.autograd.gradcheck(f, (lg,), eps=1e-6, atol=1e-7)


def test_route_norm_floor_known_answer():
    # Sigmoid scores of -110 are ~1.7e-48 (zero in fp32): the sum stays below
    # the 1e-12 floor, so F.normalize divides by the floor, not by the sum.
    logits = torch.full((1, 1, 4), -110.0)
    logits[0, 0, 2] = -30.0  # sigmoid = 9.4e-14
    probs, idx = om.route_topk_heads(logits, 2, score_func="sigmoid", route_norm=True)
    assert idx[0, 0].tolist() == [2, 0]
    np.testing.assert_allclose(float(probs[0, 0, 0]),
                               float(torch.sigmoid(torch.tensor(-30.0))) / 1e-12, rtol=1e-6)
    probs, _ = om.route_topk_heads(logits, 2, score_func="sigmoid", route_norm=True, norm_eps=1e-30)
    np.testing.assert_allclose(float(probs[0, 0].sum()), 1.0, rtol=1e-6)


def test_heads_to_rows_known_answer():
    idx = torch.tensor([[[1, 0], [2, 3]], [[0, 1], [3, 3]]])  # [H=2, S=2, k=2]
    probs = torch.arange(8, dtype=torch.float32).view(2, 2, 2)
    p, g = om.heads_to_rows(probs, idx, 4)
    # row s*H+h: (s0,h0), (s0,h1), (s1,h0), (s1,h1); group h*E+e
    assert g.tolist() == [[1, 0], [4, 5], [2, 3], [7, 7]]
    assert p.tolist() == [[0, 1], [4, 5], [2, 3], [6, 7]]


def test_swiglu7_known_answers_and_clamps():
    g = torch.tensor([0.0, 1.5, -2.0, 7.0, 10.0, 3.0, 3.0, 3.0])
    u = torch.tensor([5.0, -1.0, 0.5, 2.0, 2.0, 9.0, -9.0, 6.0])
    h = om.swiglu7(g, u, torch.float32)
    assert h[0] == 0.0 and h[1] == 0.0          # gate 0, or up + 1 = 0
    assert h[3] == h[4]                          # gate clamps at 7
    s3 = float(torch.sigmoid(torch.tensor(1.702 * 3.0)))
    np.testing.assert_allclose(float(h[5]), 3.0 * s3 * 8.0, rtol=1e-6)    # up clamps at 7
    np.testing.assert_allclose(float(h[6]), 3.0 * s3 * -6.0, rtol=1e-6)   # and at -7
    np.testing.assert_allclose(float(h[2]), -2.0 / (1 + np.exp(3.404)) * 1.5, rtol=1e-6)


def test_swiglu7_backward_matches_finite_differences_and_masks():
    g = torch.tensor([-3.0, -0.4, 0.7, 2.9, 6.2, 7.5, 1.0, 1.0], dtype=torch.float64)
    u = torch.tensor([0.3, -2.5, 4.0, -6.0, 1.0, 1.0, 7.5, -8.0], dtype=torch.float64)
    dh = torch.tensor([1.0, -0.5, 2.0, 0.25, -1.5, 1.0, 1.0, 1.0], dtype=torch.float64)
    dg, du = om.swiglu7_backward(g, u, dh)

    def f(gg, uu):
        gc, uc = np.minimum(gg, 7.0), np.clip(uu, -7.0, 7.0)
        return gc / (1 + np.exp(-1.702 * gc)) * (uc + 1.0)

    eps = 1e-6
    gn, un, dn = g.numpy(), u.numpy(), dh.numpy()
    fd_g = dn * (f(gn + eps, un) - f(gn - eps, un)) / (2 * eps)
    fd_u = dn * (f(gn, un + eps) - f(gn, un - eps)) / (2 * eps)
    np.testing.assert_allclose(dg.numpy(), fd_g, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(du.numpy(), fd_u, rtol=1e-6, atol=1e-9)
    assert dg[5] == 0.0                          # gate past the clamp
    assert du[6] == 0.0 and du[7] == 0.0         # up past either clamp


def _fp32_case(H=2, E=4, d=64, f=64, S=12, k=2, seed=5):
    g = torch.Generator().manual_seed(seed)
    G = H * E
    w = {
        "W_gate": torch.randn(G, d, f, generator=g) * 0.1,
        "W_up": torch.randn(G, d, f, generator=g) * 0.1,
        "W_down": torch.randn(G, f, d, generator=g) * 0.1,
    }
    x = torch.randn(S, H, d, generator=g)
    logits = torch.randn(H, S, E, generator=g)
    probs, idx = om.route_topk_heads(logits, k, score_func="sigmoid", route_norm=True,
                                     route_scale=4.9)
    return x, probs, idx, w, E


def test_layer_oracle_matches_fp64_per_token_formulation():
    x, probs, idx, w, E = _fp32_case()
    got = om.layer_forward(x, probs, idx, w, E)
    want = om.layer_forward_fp64(x, probs, idx, w, E)
    torch.testing.assert_close(got.double(), want, rtol=1e-4, atol=1e-5)


def test_layer_oracle_gradients_match_fp64_autograd():
    x, probs, idx, w, E = _fp32_case(S=6)
    xg = x.clone().requires_grad_(True)
    pg = probs.clone().requires_grad_(True)
    om.layer_forward(xg, pg, idx, w, E).square().sum().backward()
    xd = x.double().requires_grad_(True)
    pd = probs.double().requires_grad_(True)
    wd = {k: v.double() for k, v in w.items()}
    # fp64 reference through plain autograd (the custom swiglu7 backward is
    # the thing checked).
    S, H, _ = x.shape
    out = []
    for s in range(S):
        row = []
        for h in range(H):
            acc = 0
            for j in range(idx.shape[2]):
                gid = h * E + int(idx[h, s, j])
                gate = (xd[s, h] @ wd["W_gate"][gid]).clamp(max=7.0)
                up = (xd[s, h] @ wd["W_up"][gid]).clamp(min=-7.0, max=7.0)
                hid = gate * torch.sigmoid(1.702 * gate) * (up + 1.0)
                acc = acc + pd[h, s, j] * (hid @ wd["W_down"][gid])
            row.append(acc)
        out.append(torch.stack(row))
    torch.stack(out).square().sum().backward()
    torch.testing.assert_close(xg.grad.double(), xd.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(pg.grad.double(), pd.grad, rtol=1e-4, atol=1e-5)
