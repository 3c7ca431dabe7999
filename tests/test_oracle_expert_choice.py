"""CPU checks of the expert-choice oracle: the plan against plain loops and
invariants, the layer against the per-slot reference formula of the
reference's own contract (artifact_transforms.py:1819-1893: every (expert,
slot) adds score * mlp(token) to its token)."""

import numpy as np
import torch

from oracle import expert_choice as oec
from oracle import layer as olayer


def test_plan_matches_plain_loops_with_aliases():
    rng = np.random.default_rng(0)
    B, L, C, tps = 3, 6, 4, 10
    idx = rng.integers(0, tps, size=(B, L, C))
    scores = rng.random((B, L, C)).astype(np.float32)
    alias = (2, 0, 2, 1, 0, 2)
    p = oec.build_expert_choice_plan(idx, scores, tps, 3, alias)
    # expected order: physical expert ascending, then flat slot order
    slots = [(alias[l], b * L * C + l * C + c, b, l, c)
             for b in range(B) for l in range(L) for c in range(C)]
    slots.sort(key=lambda v: (v[0], v[1]))
    assert p["sort_positions"].tolist() == [s[1] for s in slots]
    assert p["sorted_token_indices"].tolist() == [idx[b, l, c] + b * tps for _, _, b, l, c in slots]
    assert p["counts"].tolist() == [sum(1 for s in slots if s[0] == e) for e in range(3)]
    assert p["offsets"].tolist() == np.cumsum(p["counts"]).tolist()
    assert (p["sort_positions"][p["inverse_order"]] == np.arange(B * L * C)).all()
    np.testing.assert_array_equal(p["sorted_scores"], scores.reshape(-1)[p["sort_positions"]])


def test_layer_matches_the_per_slot_reference_formula():
    # The reference contract's routes: 4 experts, capacity 1, token 0 picked twice.
    g = torch.Generator().manual_seed(1)
    idx = torch.tensor([[[0], [1], [2], [0]]])
    scores = torch.tensor([[[0.8], [0.7], [0.6], [0.5]]])
    x = torch.randn(3, 16, generator=g, dtype=torch.float64)
    w = {"w1": torch.randn(4, 8, 16, generator=g, dtype=torch.float64),
         "w3": torch.randn(4, 8, 16, generator=g, dtype=torch.float64),
         "w2": torch.randn(4, 16, 8, generator=g, dtype=torch.float64)}
    out = oec.expert_choice_forward(x, scores, idx, 3, w, {}, 4)
    ref = torch.zeros_like(x)
    for e in range(4):
        t = int(idx[0, e, 0])
        h = torch.nn.functional.silu(x[t] @ w["w1"][e].T) * (x[t] @ w["w3"][e].T)
        ref[t] = ref[t] + h @ w["w2"][e].T * float(scores[0, e, 0])
    torch.testing.assert_close(out, ref, rtol=1e-6, atol=1e-6)


def test_layer_with_aliases_sums_in_physical_order():
    g = torch.Generator().manual_seed(2)
    B, L, C, tps = 2, 4, 3, 5
    idx = torch.stack([torch.randperm(tps, generator=g)[:C] for _ in range(B * L)]).view(B, L, C)
    scores = torch.rand(B, L, C, generator=g)
    x = torch.randn(B * tps, 32, generator=g)
    w = {"w1": torch.randn(2, 16, 32, generator=g), "w3": torch.randn(2, 16, 32, generator=g),
         "w2": torch.randn(2, 32, 16, generator=g)}
    alias = (1, 0, 1, 0)
    out = oec.expert_choice_forward(x, scores, idx, tps, w, {}, 2, alias)
    ref = torch.zeros(B * tps, 32, dtype=torch.float64)
    for b in range(B):
        for l in range(L):
            for c in range(C):
                t = int(idx[b, l, c]) + b * tps
                y = olayer.expert_mlp(x[t:t + 1], alias[l], w, {})
                ref[t] += (y.double() * float(scores[b, l, c]))[0]
    torch.testing.assert_close(out.double(), ref, rtol=1e-4, atol=1e-4)  # fp32 oracle vs fp64 loop
    assert torch.count_nonzero(out.abs().sum(1)) <= B * tps


def test_backward_matches_autograd_of_the_per_slot_formula():
    # Gradients of the oracle composition (plan, sorted gather, per-expert MLP
    # with LoRA, index_add) against fp64 autograd of the per-slot formula
    # written out independently: out[t] += s * (silu(g) * u) W2^T + LoRA terms,
    # over every (b, l, c) slot, with an alias map.
    g = torch.Generator().manual_seed(3)
    B, L, C, tps, d, f, r = 2, 4, 3, 6, 16, 8, 4
    alias = (1, 0, 1, 2)
    E = 3
    idx = torch.stack([torch.randperm(tps, generator=g)[:C] for _ in range(B * L)]).view(B, L, C)
    leaf = lambda *shape: torch.randn(*shape, generator=g, dtype=torch.float64).requires_grad_(True)
    x, scores = leaf(B * tps, d), leaf(B, L, C)
    w = {"w1": torch.randn(E, f, d, generator=g, dtype=torch.float64),
         "w3": torch.randn(E, f, d, generator=g, dtype=torch.float64),
         "w2": torch.randn(E, d, f, generator=g, dtype=torch.float64)}
    fac = {"w1": (leaf(E, r, d), leaf(E, f, r)), "w3": (leaf(E, r, d), leaf(E, f, r)),
           "w2": (leaf(E, r, f), leaf(E, d, r))}
    s = 0.75
    dy = torch.randn(B * tps, d, generator=g, dtype=torch.float64)

    out = oec.expert_choice_forward(x, scores, idx, tps, w, {k: (a, b, s) for k, (a, b) in fac.items()},
                                    E, alias)
    got = torch.autograd.grad((out.double() * dy).sum(), [x, scores] + [t for p in fac.values() for t in p])

    def proj(v, key, e):
        a, b = fac[key]
        return v @ w[key][e].T + ((v @ a[e].T) @ b[e].T) * s

    ref = torch.zeros(B * tps, d, dtype=torch.float64)
    for b_ in range(B):
        for l in range(L):
            for c in range(C):
                t = int(idx[b_, l, c]) + b_ * tps
                e = alias[l]
                gate, up = proj(x[t], "w1", e), proj(x[t], "w3", e)
                h = gate * torch.sigmoid(gate) * up
                ref = ref.index_add(0, torch.tensor([t]), (proj(h, "w2", e) * scores[b_, l, c])[None])
    want = torch.autograd.grad((ref * dy).sum(), [x, scores] + [t for p in fac.values() for t in p])
    names = ["tokens", "scores"] + [f"{k}.{n}" for k in fac for n in ("a", "b")]
    for name, a, b in zip(names, got, want):
        torch.testing.assert_close(a, b, rtol=2e-5, atol=2e-5, msg=name)
    assert float(want[1].abs().sum()) > 0  # the score gradient is not trivially zero
