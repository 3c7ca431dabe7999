"""GPU parity of the layer backward (adapter training, frozen base) against
torch autograd through the reference-order oracle on the CPU.

Gradients compared: d tokens (bf16), d top_scores (fp32) and the fp32 LoRA
factor gradients dA / dB of gate, up and down. The GPU path keeps every
reduction in fp32 and rounds intermediates (dy, dh, dG, dU, dz) to bf16 where
the bf16 reference composition does, but the reference's autograd also sums
the k routes of a token and the base/LoRA parts of each gradient in bf16, in
an order torch does not fix. Bounds (stated per gradient, relative to the
oracle): mean-relative error <= 5e-3 and max-abs error <= 3e-2 * max|oracle|.
Production tile shapes: experts averaging >= 256 rows run 256-row tiles plus
one 128-row remainder tile per expert whose last rows number 1..128 (an
expert whose last rows number 129..255 gets a partial 256-row tile). The
tall-tile cases below meet that threshold and assert which tiles they cover;
full C5 runs on every token (so on the production tiles) and is compared with
the oracle on a token subset for d tokens / d scores, and per expert for the
LoRA gradients (an expert's LoRA gradients sum only its own rows, so the
oracle reproduces them from that expert's routes alone). Size-independent
checks at full C5 size: linearity in the upstream gradient (scaling dY by 2
scales every gradient by exactly 2) and run-to-run determinism.
"""

import pytest
import torch

from mirai_amd import workloads as wl
from oracle import layer as olayer
from oracle import routing as oroute

from helpers import build_module, mixed_rank_factors, oracle_weights

pytestmark = pytest.mark.gpu

MEAN_REL = 5e-3
MAX_REL = 3e-2


def small(fmt, *, T=256, d=256, f=192, E=8, k=2, r=16, alpha=16.0):
    return wl.Workload(f"bwd_{fmt}", 9, T, d, f, E, k, r, alpha, fmt, torch.bfloat16)


def _close(name, actual, expected):
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    diff = (a - e).abs()
    scale = float(e.abs().max().clamp_min(1e-30))
    stats = {
        "max_abs": float(diff.max()),
        "max_rel": float(diff.max()) / scale,
        "mean_rel": float(diff.sum() / e.abs().sum().clamp_min(1e-30)),
    }
    assert stats["mean_rel"] <= MEAN_REL and stats["max_rel"] <= MAX_REL, (name, stats)
    return stats


def _gpu_grads(m, x, scores, idx, dy):
    xg = x.cuda().requires_grad_(True)
    sg = scores.cuda().requires_grad_(True)
    for ad in m.expert_lora.values():
        ad.lora_a.grad = None
        ad.lora_b.grad = None
    out = m.run_direct_routed(xg, sg, idx.cuda())
    out.backward(dy.cuda())
    grads = {"tokens": xg.grad, "scores": sg.grad}
    for key, ad in m.expert_lora.items():
        grads[f"{key}.a"] = ad.lora_a.grad
        grads[f"{key}.b"] = ad.lora_b.grad
    return out, {k: v.detach().clone() for k, v in grads.items()}


def _oracle_grads(w, dense, lora, x, scores, idx, dy, rows, weights=None):
    xo = x[rows].clone().requires_grad_(True)
    so = scores[rows].clone().requires_grad_(True)
    loras = {}
    leaves = {}
    for key, (a, b) in lora.items():
        a = a.clone().float().requires_grad_(True)
        b = b.clone().float().requires_grad_(True)
        leaves[key] = (a, b)
        loras[key] = (a, b, float(w.alpha) / int(a.shape[1]))
    if weights is None:
        weights = oracle_weights(w, dense, dtype=torch.bfloat16)
    out = olayer.layer_forward(xo, so, idx[rows], weights, loras, w.experts)
    out.backward(dy[rows])
    grads = {"tokens": xo.grad, "scores": so.grad}
    for key, (a, b) in leaves.items():
        grads[f"{key}.a"] = a.grad
        grads[f"{key}.b"] = b.grad
    return out, grads


def _case(w, rows=None, lora=None):
    dense = wl.dense_weights(w)
    if lora is None:
        lora = wl.lora_factors(w)
    x = wl.tokens(w)
    idx_np, scores_np = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    idx, scores = torch.from_numpy(idx_np), torch.from_numpy(scores_np)
    dy = wl.upstream_grad(w)
    m = build_module(w, dense, lora)
    if rows is None:
        rows = torch.arange(w.tokens)
    # The GPU runs only the token subset too, so LoRA gradients sum the same rows.
    _, g = _gpu_grads(m, x[rows], scores[rows], idx[rows], dy[rows])
    _, ref = _oracle_grads(w, dense, lora, x, scores, idx, dy, rows)
    report = {}
    for name, e in ref.items():
        report[name] = _close(name, g[name], e)
    print(f"backward parity {w.name}: " + ", ".join(
        f"{k}: mean_rel {v['mean_rel']:.2e} max_rel {v['max_rel']:.2e}" for k, v in report.items()))


@pytest.mark.parametrize("fmt", ["bf16", "nf4", "int8"])
def test_small_backward_matches_oracle(fmt):
    _case(small(fmt))


@pytest.mark.parametrize("r", [8, 32, 48, 64, 128])
def test_backward_lora_ranks(r):
    # Ranks above 32: 32-wide slices of the weight gradients and of dz.
    _case(small("nf4", r=r, alpha=2.0 * r, E=5, k=3, T=300, f=320, d=192))


def test_backward_mixed_lora_ranks_on_tall_tiles():
    w = small("int8", E=4, k=2, T=1100, f=256, d=192, alpha=32.0)
    _case(w, lora=mixed_rank_factors(w, {"w1": 96, "w3": 24, "w2": 64}))


def test_backward_ragged_experts():
    _case(small("int8", T=37, E=64, k=4, d=128, f=128))


def _routes(w, bias=None):
    logits = wl.router_logits(w)
    if bias is not None:
        logits = logits + bias
    idx_np, scores_np = oroute.route_topk(logits.numpy(), w.top_k)
    return torch.from_numpy(idx_np), torch.from_numpy(scores_np)


def _tile_kinds(idx, E):
    """(tall tiles used, experts with a 128-row remainder tile, experts whose
    last rows need a partial 256-row tile) -- the plan's tile rule."""
    counts = torch.bincount(idx.reshape(-1), minlength=E)
    tall = int(counts.sum()) >= 256 * E
    rem = counts % 256
    return tall, int(((rem > 0) & (rem <= 128)).sum()), int((rem > 128).sum())


def _case_routes(w, idx, scores, rows=None):
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    x = wl.tokens(w)
    dy = wl.upstream_grad(w)
    m = build_module(w, dense, lora)
    rows = torch.arange(w.tokens) if rows is None else rows
    _, g = _gpu_grads(m, x[rows], scores[rows], idx[rows], dy[rows])
    _, ref = _oracle_grads(w, dense, lora, x, scores, idx, dy, rows)
    for name, e in ref.items():
        _close(name, g[name], e)


@pytest.mark.parametrize("fmt", ["bf16", "nf4", "int8"])
def test_tall_tile_backward_matches_oracle(fmt):
    # R = 4096 >= 256 * E: 256-row tiles; every gradient over all rows.
    w = small(fmt, T=2048, E=8, k=2, d=256, f=192)
    idx, scores = _routes(w)
    tall, _, _ = _tile_kinds(idx, w.experts)
    assert tall
    _case_routes(w, idx, scores)


def test_tall_tile_remainders_backward_matches_oracle():
    # Skewed routes over 4 experts: remainders of both kinds.
    w = small("nf4", T=700, E=4, k=2, d=192, f=256)
    idx, scores = _routes(w, bias=torch.tensor([1.2, 0.45, 0.0, -0.9]))
    tall, short_rem, long_rem = _tile_kinds(idx, w.experts)
    assert tall and short_rem >= 1 and long_rem >= 1, torch.bincount(idx.reshape(-1))
    _case_routes(w, idx, scores)


def test_c5_full_size_backward_matches_oracle():
    """Full C5 on the GPU (production tiles); oracle on a token subset for d
    tokens / d scores and on each of three experts' routes for their LoRA
    gradients."""
    w = wl.WORKLOADS["c5"]
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    x = wl.tokens(w)
    idx, scores = _routes(w)
    assert _tile_kinds(idx, w.experts)[0]
    dy = wl.upstream_grad(w)
    m = build_module(w, dense, lora)
    _, g = _gpu_grads(m, x, scores, idx, dy)
    rows = torch.arange(0, w.tokens, 64)
    weights = oracle_weights(w, dense, dtype=torch.bfloat16)
    _, ref = _oracle_grads(w, dense, lora, x, scores, idx, dy, rows, weights)
    _close("tokens", g["tokens"][rows.cuda()], ref["tokens"])
    _close("scores", g["scores"][rows.cuda()], ref["scores"])
    for e in (0, 17, 63):
        tok, slot = torch.nonzero(idx == e, as_tuple=True)
        # Expert e alone: its routes as k = 1 problems over its own tokens.
        we = wl.Workload(w.name, w.index, int(tok.numel()), w.hidden, w.ffn, w.experts, 1,
                         w.rank, w.alpha, w.fmt, w.dtype)
        sub = torch.arange(int(tok.numel()))
        _, ref_e = _oracle_grads(we, dense, lora, x[tok], scores[tok, slot].unsqueeze(1),
                                 idx[tok, slot].unsqueeze(1), dy[tok], sub, weights)
        for key in lora:
            for part in ("a", "b"):
                name = f"{key}.{part}"
                _close(f"{name}[{e}]", g[name][e], ref_e[name][e])


def test_c5_backward_on_token_subset():
    w = wl.WORKLOADS["c5"]
    _case(w, rows=torch.arange(0, w.tokens, 32))


def test_c5_full_size_linearity_and_determinism():
    w = wl.WORKLOADS["c5"]
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    x = wl.tokens(w)
    idx_np, scores_np = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    idx, scores = torch.from_numpy(idx_np), torch.from_numpy(scores_np)
    dy = wl.upstream_grad(w)
    m = build_module(w, dense, lora)
    _, g1 = _gpu_grads(m, x, scores, idx, dy)
    _, g1b = _gpu_grads(m, x, scores, idx, dy)
    _, g2 = _gpu_grads(m, x, scores, idx, 2 * dy)
    for name in g1:
        assert torch.equal(g1[name], g1b[name]), f"{name} is not deterministic"
        assert torch.equal(g2[name], 2 * g1[name]), f"{name} is not linear in dY"
        assert torch.isfinite(g1[name]).all(), name


def test_empty_batch_forward_and_backward():
    """Zero tokens (the reference's grouped matmuls over empty tensors): an empty
    output, empty token / score gradients and all-zero LoRA factor gradients."""
    w = small("nf4")
    dense = wl.dense_weights(w)
    m = build_module(w, dense, wl.lora_factors(w))
    x = torch.empty(0, w.hidden, dtype=torch.bfloat16)
    scores = torch.empty(0, w.top_k, dtype=torch.float32)
    idx = torch.empty(0, w.top_k, dtype=torch.int64)
    dy = torch.empty(0, w.hidden, dtype=torch.bfloat16)
    out, grads = _gpu_grads(m, x, scores, idx, dy)
    assert tuple(out.shape) == (0, w.hidden)
    assert tuple(grads["tokens"].shape) == (0, w.hidden)
    assert tuple(grads["scores"].shape) == (0, w.top_k)
    for key, ad in m.expert_lora.items():
        for name in ("a", "b"):
            g = grads[f"{key}.{name}"]
            if g is not None:
                assert not bool(g.abs().gt(0).any()), key + "." + name
    with torch.no_grad():
        assert tuple(m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda()).shape) == (0, w.hidden)


@pytest.mark.parametrize("keys", [("w2",), ("w1",), ("w1", "w3"), ("w3", "w2")])
def test_backward_with_a_subset_of_adapters(keys):
    """LoRA on some projections only (the others frozen without an adapter): the
    absent adapters' columns are skipped in every epilogue and their gradients
    are not produced; tall and remainder tiles both run (R >= 256 E)."""
    w = small("nf4", T=1100, E=4, k=2, d=192, f=256)
    lora = {k: v for k, v in wl.lora_factors(w).items() if k in keys}
    _case(w, lora=lora)


@pytest.mark.parametrize("r", [4, 12, 36])
def test_backward_ranks_off_the_multiple_of_eight(r):
    """Ranks the kernels pad with zero rank rows (to a multiple of 8): the
    padded factors' gradients are cut back to the adapter's own rank."""
    _case(small("nf4", r=r, alpha=2.0 * r, E=5, k=3, T=300, f=320, d=192))


def test_lora_only_backward_when_inputs_need_no_grad():
    """Tokens and scores that do not require gradients (the adapters alone
    train): the LoRA gradients equal those of the full backward."""
    w = small("nf4", T=400, E=6, k=2)
    dense, lora = wl.dense_weights(w), wl.lora_factors(w)
    x = wl.tokens(w)
    idx_np, scores_np = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    idx, scores = torch.from_numpy(idx_np), torch.from_numpy(scores_np)
    dy = wl.upstream_grad(w)
    m = build_module(w, dense, lora)
    _, full = _gpu_grads(m, x, scores, idx, dy)
    for ad in m.expert_lora.values():
        ad.lora_a.grad = None
        ad.lora_b.grad = None
    out = m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda())
    assert out.requires_grad
    out.backward(dy.cuda())
    for key, ad in m.expert_lora.items():
        assert torch.equal(ad.lora_a.grad, full[f"{key}.a"]), key
        assert torch.equal(ad.lora_b.grad, full[f"{key}.b"]), key
