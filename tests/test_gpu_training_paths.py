"""GPU parity of the training paths around the routed layer, against torch
autograd through the CPU oracle:

* grouped_linear (CompressedGroupedExperts.grouped_linear, experts.py:803-827):
  forward and backward (d x, d A, d B) through mx_grouped_linear_backward at
  LoRA ranks 16 and 160, and the reference's residency test pattern
  (tests/test_lingbot_lora_residency.py:1510-1533: silu(gl(w1)) * gl(w3) ->
  gl(w2) -> loss.backward() reaches the lora_b factors);
* the fused LingBot router (transformer_lingbot_video.py:975-1033): d tokens,
  d router weight and d logit_delta through the gating scores, softmax and
  sigmoid, with and without renormalisation and group-limited picks;
* the LingBot block (transformer_lingbot_video.py:2216-2377): d tokens and
  d router weight of the whole block (router + routed experts + shared expert);
* MAGI-2 per-head routing (flash_mh_moe/route.py:28-148): virtual-group
  selection bit-exact with the oracle, and d logits through the probabilities;
* logical expert aliases: zero-score slots dropped (experts.py:2361-2367), and
  token chunking over an aliased module equal to the unchunked layer.

Bounds: the routers' gradients are fp32 products of fp32 values (mean-rel
1e-4; bf16 token gradients 4e-3, one bf16 rounding); gradients through the
expert layer use the layer backward's bounds (mean-rel 5e-3, max 3e-2 of the
oracle's largest magnitude).
"""

import pytest
import torch
import torch.nn.functional as F

from mirai_amd import CompressedGroupedExperts, FusedRouter, route_topk
from mirai_amd import _native as nat
from mirai_amd import workloads as wl
from mirai_amd.chunking import MoETokenChunkPolicy, fused_chunk_runner
from mirai_amd.magi2 import route_topk_heads
from oracle import block as oblock
from oracle import layer as olayer
from oracle import magi2 as om
from oracle import router as orr

from helpers import assert_layer_close, build_module, oracle_loras, oracle_weights

pytestmark = pytest.mark.gpu

MEAN_REL = 5e-3
MAX_REL = 3e-2


def _close(name, actual, expected, mean_rel=MEAN_REL, max_rel=MAX_REL):
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    diff = (a - e).abs()
    scale = float(e.abs().max().clamp_min(1e-30))
    stats = {"mean_rel": float(diff.sum() / e.abs().sum().clamp_min(1e-30)),
             "max_rel": float(diff.max()) / scale}
    print(f"{name}: {stats}")
    assert stats["mean_rel"] <= mean_rel and stats["max_rel"] <= max_rel, (name, stats)
    return stats


# ------------------------------------------------------------ grouped_linear
def _gl_case(fmt, r, *, d=256, f=320, E=4, seed=0):
    w = wl.Workload(f"gl_{fmt}", 7 + seed, 160, d, f, E, 1, r, 2.0 * r, fmt, torch.bfloat16)
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w) if r else None
    m = build_module(w, dense, lora, access="full_dequant")
    return w, dense, lora, m


@pytest.mark.parametrize("fmt,r,key", [("nf4", 16, "w1"), ("int8", 160, "w2"), ("bf16", 16, "w3"),
                                       ("nf4", 0, "w1")])
def test_grouped_linear_backward_matches_oracle_autograd(fmt, r, key):
    w, dense, lora, m = _gl_case(fmt, r)
    counts = torch.tensor([40, 61, 0, 59])
    offsets = counts.cumsum(0).to(torch.int32)
    S = int(counts.sum())
    in_f = w.hidden if key != "w2" else w.ffn
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(S, in_f, generator=g)).to(torch.bfloat16)
    dy = torch.randn(S, w.ffn if key != "w2" else w.hidden, generator=g).to(torch.bfloat16)

    xg = x.cuda().requires_grad_(True)
    out = m.grouped_linear(key, xg, offsets=offsets.cuda())
    out.backward(dy.cuda())

    wts = oracle_weights(w, dense)
    xo = x.clone().requires_grad_(True)
    lo = None
    if lora:
        a, b, s = oracle_loras(w, lora)[key]
        a = a.clone().requires_grad_(True)
        b = b.clone().requires_grad_(True)
        lo = (a, b, s)
    ref = olayer.grouped_linear(xo, counts, wts[key], lo)
    ref.backward(dy)
    assert_layer_close(out.detach().cpu(), ref.detach())
    _close(f"gl {fmt} r{r} dx", xg.grad, xo.grad)
    if lora:
        ad = m.expert_lora[key]
        _close(f"gl {fmt} r{r} dA", ad.lora_a.grad, lo[0].grad)
        _close(f"gl {fmt} r{r} dB", ad.lora_b.grad, lo[1].grad)


def test_grouped_linear_lora_only_gradients():
    # Tokens without a gradient: only the LoRA factors get one, equal to the
    # full backward's (the kernel writes both factor gradients in one pass).
    w, dense, lora, m = _gl_case("nf4", 16, seed=1)
    counts = torch.tensor([30, 30, 30, 30])
    offsets = counts.cumsum(0).to(torch.int32).cuda()
    x = torch.randn(120, w.hidden, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    dy = torch.randn(120, w.ffn, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    ad = m.expert_lora["w1"]

    def grads(x_requires):
        ad.lora_a.grad = ad.lora_b.grad = None
        xx = x.cuda().requires_grad_(x_requires)
        m.grouped_linear("w1", xx, offsets=offsets).backward(dy.cuda())
        return ad.lora_a.grad.clone(), ad.lora_b.grad.clone()

    ga0, gb0 = grads(True)
    ga1, gb1 = grads(False)
    assert torch.equal(ga0, ga1) and torch.equal(gb0, gb1)


def test_grouped_lora_backward_like_the_reference_residency_test():
    """tests/test_lingbot_lora_residency.py:1510-1533 on resident quantised
    experts: the block's grouped path (transformer_lingbot_video.py:1546-1575)
    computes silu(gl(w1)) * gl(w3) -> gl(w2) and loss.backward() must reach the
    lora_b factors with finite gradients. Checked here against the oracle's
    autograd of the same composition as well."""
    w = wl.Workload("gl_res", 3, 128, 256, 192, 4, 1, 16, 16.0, "nf4", torch.bfloat16)
    dense = wl.dense_weights(w)
    m = build_module(w, dense, None, access="full_dequant")
    for key in ("w1", "w3", "w2"):
        m.attach_expert_lora(tensor_name=key, adapter_name="r", rank=16, alpha=16.0)
    for ad in m.expert_lora.values():  # B starts at zero (kaiming A); make the delta live
        with torch.no_grad():
            ad.lora_b.normal_(0.0, 0.02)
        ad.lora_a.requires_grad_(False)
    counts = torch.tensor([32, 32, 32, 32])
    offsets = counts.cumsum(0).to(torch.int32).cuda()
    tokens = torch.randn(128, w.hidden, generator=torch.Generator().manual_seed(8))
    tokens = tokens.to(torch.bfloat16).cuda()
    gate = m.grouped_linear("w1", tokens, offsets=offsets)
    up = m.grouped_linear("w3", tokens, offsets=offsets)
    out = m.grouped_linear("w2", F.silu(gate) * up, offsets=offsets)
    out.float().square().mean().backward()
    grads = {k: ad.lora_b.grad for k, ad in m.expert_lora.items()}
    assert all(g is not None and bool(torch.isfinite(g).all()) for g in grads.values())
    assert all(ad.lora_a.grad is None for ad in m.expert_lora.values())

    wts = oracle_weights(w, dense)
    lo = {}
    for k, ad in m.expert_lora.items():
        lo[k] = (ad.lora_a.detach().cpu().float(),
                 ad.lora_b.detach().cpu().float().requires_grad_(True), ad.scale())
    t = tokens.cpu()
    og = olayer.grouped_linear(t, counts, wts["w1"], lo["w1"])
    ou = olayer.grouped_linear(t, counts, wts["w3"], lo["w3"])
    oo = olayer.grouped_linear(F.silu(og) * ou, counts, wts["w2"], lo["w2"])
    oo.float().square().mean().backward()
    for k in ("w1", "w3", "w2"):
        _close(f"residency dB {k}", grads[k], lo[k][1].grad, mean_rel=1e-2)


# ------------------------------------------------------------ LingBot router
ROUTER_CASES = [
    # score_func, k, norm_topk_prob, n_group, topk_group, token dtype, route_scale
    ("sigmoid", 4, True, None, None, torch.bfloat16, 1.0),
    ("softmax", 4, True, None, None, torch.bfloat16, 2.5),
    ("softmax", 2, False, None, None, torch.float32, 1.0),
    ("sigmoid", 1, True, None, None, torch.float32, 1.0),
    ("sigmoid", 8, True, 8, 4, torch.bfloat16, 1.0),
]


@pytest.mark.parametrize("score_func,k,norm,n_group,topk_group,dtype,scale", ROUTER_CASES)
def test_router_backward_matches_oracle_autograd(score_func, k, norm, n_group, topk_group, dtype,
                                                 scale):
    T, E, d = 300, 64, 256
    g = torch.Generator().manual_seed(31 + k)
    x = torch.randn(T, d, generator=g).to(dtype)
    wt = torch.randn(E, d, generator=g) * 0.05
    bias = torch.randn(E, generator=g) * 0.01
    delta = torch.randn(T, E, generator=g) * 0.1
    gy = torch.randn(T, k, generator=g)
    r = FusedRouter(d, E, k, score_func, norm, n_group, topk_group, scale).cuda()
    with torch.no_grad():
        r.weight.copy_(wt)
        r.e_score_correction_bias.copy_(bias)
    xg = x.cuda().requires_grad_(True)
    dg = delta.cuda().requires_grad_(True)
    idx, top, logits, scores, _ = r(xg, logit_delta=dg)
    assert not logits.requires_grad and not idx.requires_grad
    (top.float() * gy.cuda()).sum().backward()

    xo = x.clone().requires_grad_(True)
    wo = wt.clone().requires_grad_(True)
    do = delta.clone().requires_grad_(True)
    _, otop, _, _, _ = orr.router_forward(xo, wo, k, logit_delta=do, score_func=score_func,
                                          expert_bias=bias, norm_topk_prob=norm, n_group=n_group,
                                          topk_group=topk_group, route_scale=scale,
                                          picks=idx.cpu())
    torch.testing.assert_close(top.float().cpu(), otop.float(), rtol=2**-7, atol=1e-6)
    (otop.float() * gy).sum().backward()
    tok_rel = 4e-3 if dtype == torch.bfloat16 else 1e-4
    _close(f"router {score_func} k{k} dtokens", xg.grad, xo.grad, mean_rel=tok_rel, max_rel=2e-2)
    _close(f"router {score_func} k{k} dweight", r.weight.grad, wo.grad, mean_rel=1e-4,
           max_rel=1e-3)
    _close(f"router {score_func} k{k} ddelta", dg.grad, do.grad, mean_rel=1e-4, max_rel=1e-3)


# ------------------------------------------------------------ LingBot block
def test_block_backward_reaches_tokens_and_router_weight():
    from mirai_amd.block import FusedSparseMoeBlock

    Hd, Fd, Ed, Kd, T = 256, 192, 16, 4, 384
    w = wl.Workload("blk_bwd", 9, T, Hd, Fd, Ed, Kd, 16, 16.0, "nf4", torch.bfloat16)
    g = torch.Generator().manual_seed(2)
    blk = FusedSparseMoeBlock(Hd, 4 * Hd, Ed, Kd, Fd, "sigmoid", True, None, None, 1.0, 1,
                              quant_format="nf4").cuda()
    router_w = torch.randn(Ed, Hd, generator=g) * 0.05
    bias = torch.randn(Ed, generator=g) * 0.01
    with torch.no_grad():
        blk.router.weight.copy_(router_w)
        blk.router.e_score_correction_bias.copy_(bias)
    dense = wl.dense_weights(w)
    for key in ("w1", "w3", "w2"):
        blk.experts.load_dense_weight(key, dense[key].cuda())
    factors = wl.lora_factors(w)
    for key, (a, b) in factors.items():
        ad = blk.experts.attach_expert_lora(tensor_name=key, adapter_name="t", rank=16, alpha=16.0)
        with torch.no_grad():
            ad.lora_a.copy_(a.cuda())
            ad.lora_b.copy_(b.cuda())
    blk.shared_experts.to(torch.bfloat16).requires_grad_(False)
    sh = []
    for lin in (blk.shared_experts.gate_proj, blk.shared_experts.up_proj,
                blk.shared_experts.down_proj):
        wt = (torch.randn(lin.weight.shape, generator=g) * 0.03).to(torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(wt)
        sh.append(wt)
    blk.train()
    x = wl.tokens(w).view(1, T, Hd)
    dy = torch.randn(x.shape, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        idx, _, _, _, _ = blk.router(x.view(-1, Hd).cuda())

    xg = x.cuda().requires_grad_(True)
    out = blk(xg)
    out.backward(dy.cuda())
    assert blk.router.weight.grad is not None

    xo = x.clone().requires_grad_(True)
    wo = router_w.clone().requires_grad_(True)
    want, oidx = oblock.block_forward(xo, wo, Kd, oracle_weights(w, dense),
                                      oracle_loras(w, factors), Ed, shared=tuple(sh),
                                      score_func="sigmoid", expert_bias=bias, route_scale=1.0,
                                      picks=idx.cpu())
    assert torch.equal(oidx, idx.cpu())
    assert_layer_close(out.detach().cpu(), want.detach())
    want.backward(dy)
    _close("block dtokens", xg.grad, xo.grad)
    _close("block drouter", blk.router.weight.grad, wo.grad)


# ------------------------------------------------------------ MAGI-2 routing
@pytest.mark.parametrize("H,S,E,k,nvg,tvg,score_func", [
    (2, 200, 64, 4, 8, 3, "sigmoid"),
    (3, 150, 32, 2, 32, 2, "softmax"),  # groups of one expert
    (1, 300, 256, 8, 16, 16, "sigmoid"),  # every group kept: ungrouped selection
    (2, 100, 48, 6, 4, 1, "softmax"),
])
def test_virtual_group_routing_matches_oracle(H, S, E, k, nvg, tvg, score_func):
    g = torch.Generator().manual_seed(E + nvg)
    logits = torch.randn(H, S, E, generator=g) * 2.0
    bias = torch.randn(H, E, generator=g) * 0.05
    probs, idx = route_topk_heads(logits.cuda(), k, score_func=score_func, expert_bias=bias.cuda(),
                                  num_virtual_group=nvg, topk_virtual_group=tvg)
    oprobs, oidx = om.route_topk_heads(logits, k, score_func=score_func, expert_bias=bias,
                                       num_virtual_group=nvg, topk_virtual_group=tvg)
    assert torch.equal(idx.cpu(), oidx)
    torch.testing.assert_close(probs.cpu(), oprobs, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("layout,score_func,norm", [("heads", "sigmoid", True),
                                                    ("rows", "softmax", True),
                                                    ("rows", "sigmoid", False)])
def test_head_routing_backward_matches_oracle_autograd(layout, score_func, norm):
    H, S, E, k = 3, 120, 32, 4
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(H, S, E, generator=g)
    bias = torch.randn(H, E, generator=g) * 0.05
    lg = logits.cuda().requires_grad_(True)
    probs, idx = route_topk_heads(lg, k, score_func=score_func, expert_bias=bias.cuda(),
                                  route_norm=norm, route_scale=1.7, layout=layout)
    gp = torch.randn(probs.shape, generator=g)
    (probs * gp.cuda()).sum().backward()
    lo = logits.clone().requires_grad_(True)
    if layout == "rows":
        heads = torch.arange(H).view(1, H, 1) * E
        hidx = (idx.cpu().view(S, H, k) - heads).permute(1, 0, 2)
        ghead = gp.view(S, H, k).permute(1, 0, 2)
    else:
        hidx, ghead = idx.cpu(), gp
    op = om.route_probs_for_picks(lo, hidx, score_func=score_func, route_norm=norm,
                                  route_scale=1.7)
    (op * ghead).sum().backward()
    _close(f"heads {layout} {score_func} dlogits", lg.grad, lo.grad, mean_rel=1e-5, max_rel=1e-4)


# ------------------------------------------------------------ aliases
def _aliased_module(seed=0):
    w = wl.Workload("alias", 5, 240, 256, 192, 6, 4, 16, 16.0, "nf4", torch.bfloat16)
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    m = build_module(w, dense, lora)
    aliases = (0, 1, 2, 3, 4, 5, 1, 2, 0, 5, 3, 4)
    m.configure_logical_expert_aliases(aliases)
    g = torch.Generator().manual_seed(40 + seed)
    idx = torch.stack([torch.randperm(len(aliases), generator=g)[:4] for _ in range(w.tokens)])
    scores = torch.rand(w.tokens, 4, generator=g)
    scores[7] = 0.0  # a token the router scored zero: every slot dropped
    return w, dense, lora, m, aliases, idx, scores


def test_aliased_routes_drop_zero_score_slots():
    w, dense, lora, m, aliases, idx, scores = _aliased_module()
    x = wl.tokens(w)
    nat.set_route_check("sync")
    try:
        with torch.no_grad():
            out = m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda())
    finally:
        nat.set_route_check("deferred")
    cs, phys = m._coalesce_logical_routes(scores, idx)
    assert bool((phys == nat.ROUTE_DROPPED).any())
    # The oracle over the routes the reference dispatches: nonzero scores only.
    keep = cs != 0
    oidx = torch.where(keep, phys, torch.full_like(phys, -1))
    want = olayer.layer_forward(x, cs, oidx, oracle_weights(w, dense), oracle_loras(w, lora),
                                w.experts)
    assert_layer_close(out.cpu(), want)
    assert torch.count_nonzero(out[7].cpu()) == 0


def test_token_chunking_over_aliased_experts_equals_the_unchunked_layer():
    w, dense, lora, m, aliases, idx, scores = _aliased_module(seed=1)
    x = wl.tokens(w).cuda()
    dy = torch.randn(x.shape, generator=torch.Generator().manual_seed(9)).to(x.dtype).cuda()

    def run(chunked):
        for ad in m.expert_lora.values():
            ad.lora_a.grad = ad.lora_b.grad = None
        xg = x.clone().requires_grad_(True)
        sg = scores.cuda().requires_grad_(True)
        if chunked:
            out = MoETokenChunkPolicy(token_chunk_size=100).execute(
                xg, sg, idx.cuda(), runner=fused_chunk_runner(m), training=True)
        else:
            out = m.run_direct_routed(xg, sg, idx.cuda())
        out.backward(dy)
        lg = {k: (ad.lora_a.grad.clone(), ad.lora_b.grad.clone())
              for k, ad in m.expert_lora.items()}
        return out.detach(), xg.grad, sg.grad, lg

    o0, gx0, gs0, l0 = run(False)
    o1, gx1, gs1, l1 = run(True)
    assert torch.equal(o0, o1)
    assert torch.equal(gx0, gx1)
    torch.testing.assert_close(gs1, gs0, rtol=1e-6, atol=1e-7)
    for k in l0:
        for a, b in zip(l1[k], l0[k]):
            rel = float((a - b).abs().sum() / b.abs().sum().clamp_min(1e-30))
            assert rel < 1e-5, (k, rel)
