"""Pins the oracle's expert-layer composition (CPU only).

The per-expert reference loop (gather -> projections + LoRA -> SwiGLU -> down
-> fp32 index_add) is compared with an independent per-token formulation in
fp32, where both are exact up to fp32 summation order; a mistake in the gather,
the slot/score pairing, the LoRA scale or the activation breaks the match.
"""

import json
import math
from pathlib import Path

import pytest
import torch

from oracle import layer as olayer

GOLDEN = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


def _problem(T=40, d=16, f=24, E=5, k=2, r=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g)
    w = {
        "w1": torch.randn(E, f, d, generator=g) * 0.2,
        "w3": torch.randn(E, f, d, generator=g) * 0.2,
        "w2": torch.randn(E, d, f, generator=g) * 0.2,
    }
    loras = {
        "w1": (torch.randn(E, r, d, generator=g) * 0.2, torch.randn(E, f, r, generator=g) * 0.2, 0.75),
        "w3": (torch.randn(E, r, d, generator=g) * 0.2, torch.randn(E, f, r, generator=g) * 0.2, 0.75),
        "w2": (torch.randn(E, r, f, generator=g) * 0.2, torch.randn(E, d, r, generator=g) * 0.2, 0.75),
    }
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)])
    scores = torch.rand(T, k, generator=g)
    return x, w, loras, idx, scores


def _per_token(x, w, loras, idx, scores):
    out = torch.zeros_like(x, dtype=torch.float64)
    xd = x.double()

    def proj(v, key, e):
        a, b, s = loras[key]
        return v @ w[key][e].double().T + (v @ a[e].double().T) @ b[e].double().T * s

    for t in range(x.shape[0]):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            gt = proj(xd[t], "w1", e)
            up = proj(xd[t], "w3", e)
            h = gt / (1.0 + torch.exp(-gt)) * up
            out[t] += float(scores[t, j]) * proj(h, "w2", e)
    return out


def test_expert_loop_matches_per_token_formulation():
    x, w, loras, idx, scores = _problem()
    got = olayer.layer_forward(x, scores, idx, w, loras, 5)
    torch.testing.assert_close(got.double(), _per_token(x, w, loras, idx, scores), rtol=1e-5, atol=1e-5)


def test_unrouted_experts_and_duplicate_free_slots():
    x, w, loras, idx, scores = _problem(E=9, k=3, seed=1)
    idx[:, :] = torch.tensor([0, 4, 8])  # experts 1-3, 5-7 receive nothing
    got = olayer.layer_forward(x, scores, idx, w, loras, 9)
    torch.testing.assert_close(got.double(), _per_token(x, w, loras, idx, scores), rtol=1e-5, atol=1e-5)


def test_zero_lora_b_equals_no_lora():
    x, w, loras, idx, scores = _problem(seed=2)
    zero = {k: (a, torch.zeros_like(b), s) for k, (a, b, s) in loras.items()}
    torch.testing.assert_close(olayer.layer_forward(x, scores, idx, w, zero, 5),
                               olayer.layer_forward(x, scores, idx, w, {}, 5), rtol=0, atol=0)


def test_for_loop_is_the_top1_unit_score_layer():
    x, w, loras, _, _ = _problem(seed=3)
    counts = torch.tensor([7, 0, 13, 20, 0])
    idx = torch.repeat_interleave(torch.arange(5), counts).view(-1, 1)
    got = olayer.for_loop_forward(x, counts, w, loras)
    ref = olayer.layer_forward(x, torch.ones(40, 1), idx, w, loras, 5)
    torch.testing.assert_close(got, ref, rtol=0, atol=0)


def test_grouped_linear_is_the_per_row_expert_product():
    x, w, loras, _, _ = _problem(seed=4)
    counts = torch.tensor([10, 0, 5, 25, 0])
    got = olayer.grouped_linear(x, counts, w["w1"], loras["w1"])
    experts = torch.repeat_interleave(torch.arange(5), counts)
    a, b, s = loras["w1"]
    ref = torch.stack([x[i] @ w["w1"][e].T + (x[i] @ a[e].T) @ b[e].T * s
                       for i, e in enumerate(experts.tolist())])
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("case", GOLDEN["lora_scale"]["cases"])
def test_lora_scale_known_answers(case):
    assert math.isclose(olayer.lora_scale(case["alpha"], case["rank"], use_rslora=case["rslora"]),
                        case["scale"], rel_tol=0, abs_tol=0)


def test_lora_scale_rejects_nonpositive_rank():
    with pytest.raises(ValueError):
        olayer.lora_scale(16.0, 0)


def test_layer_backward_is_torch_autograd_of_the_composition():
    # The backward oracle is autograd through these ops; check it against the
    # per-token double-precision formulation's autograd on the LoRA factors.
    x, w, loras, idx, scores = _problem(T=12, seed=5)
    leaves = {k: (a.clone().requires_grad_(True), b.clone().requires_grad_(True), s)
              for k, (a, b, s) in loras.items()}
    xs = x.clone().requires_grad_(True)
    ss = scores.clone().requires_grad_(True)
    out = olayer.layer_forward(xs, ss, idx, w, leaves, 5)
    gy = torch.randn(out.shape, generator=torch.Generator().manual_seed(9))
    out.backward(gy)
    leaves_d = {k: (a.detach().double().requires_grad_(True), b.detach().double().requires_grad_(True), s)
                for k, (a, b, s) in leaves.items()}
    xd = x.double().requires_grad_(True)
    sd = scores.double().requires_grad_(True)
    out_d = torch.zeros(x.shape, dtype=torch.float64)
    for t in range(x.shape[0]):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])

            def proj(v, key):
                a, b, s = leaves_d[key]
                return v @ w[key][e].double().T + (v @ a[e].T) @ b[e].T * s

            gt, up = proj(xd[t], "w1"), proj(xd[t], "w3")
            out_d = out_d.index_add(0, torch.tensor([t]),
                                    (sd[t, j] * proj(gt * torch.sigmoid(gt) * up, "w2")).unsqueeze(0))
    out_d.backward(gy.double())
    torch.testing.assert_close(xs.grad.double(), xd.grad, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(ss.grad.double(), sd.grad, rtol=1e-4, atol=1e-5)
    for k in leaves:
        torch.testing.assert_close(leaves[k][0].grad.double(), leaves_d[k][0].grad, rtol=1e-4, atol=1e-5)
        torch.testing.assert_close(leaves[k][1].grad.double(), leaves_d[k][1].grad, rtol=1e-4, atol=1e-5)
