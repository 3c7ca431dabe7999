"""GPU parity of the fused router front end (mx_router_forward) with the
LingBot router oracle.

Three layers of checks:
* the weight planes sum exactly to the fp32 weight;
* the kernel's logits are fp32 dot products: within the oracle's stated
  fp32-accumulation bound of the exact (fp64) logits;
* the selection and scores given the kernel's own logits are bit-exact /
  within fp32 rounding of the oracle, and end to end (oracle logits from the
  CPU's fp32 GEMM) the picks agree on every token whose selection margin
  exceeds what two fp32 summation orders can move.
"""

import pytest
import torch

from mirai_amd import FusedRouter, fused_router_forward, router_weight_planes
from mirai_amd import _native as nat
from oracle import router as orr

pytestmark = pytest.mark.gpu


def _case(T, E, d, seed, *, token_dtype=torch.bfloat16, wstd=0.02):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, d, generator=g).to(token_dtype)
    w = torch.randn(E, d, generator=g) * wstd
    bias = torch.randn(E, generator=g) * 0.01
    return x, w, bias


@pytest.mark.parametrize("E", [8, 64, 100, 128, 256])
def test_weight_planes_sum_exactly_to_the_weight(E):
    g = torch.Generator().manual_seed(E)
    w = torch.randn(E, 128, generator=g) * torch.logspace(-6, 2, 128)
    planes = router_weight_planes(w.cuda()).cpu()
    EP = nat.load_library().mx_router_padded_experts(E)
    p = planes.view(torch.bfloat16).view(3, EP, 128).double()
    assert torch.equal(p[0, :E] + p[1, :E] + p[2, :E], w.double())
    assert torch.count_nonzero(p[:, E:]) == 0
    assert torch.equal(p[0, :E].to(torch.bfloat16), w.to(torch.bfloat16).double().to(torch.bfloat16))


def _margin_ok(keys: torch.Tensor, k: int, slack: torch.Tensor) -> torch.Tensor:
    """Tokens whose k-th and (k+1)-th keys (and consecutive picks) are more
    than `slack` apart: their selection cannot move with the logits' rounding."""
    srt = keys.sort(dim=1, descending=True).values
    gaps = srt[:, :-1] - srt[:, 1:]
    need = gaps[:, :k] if k < keys.shape[1] else gaps[:, : k - 1]
    return (need > slack.unsqueeze(1)).all(dim=1)


CASES = [
    # T, E, d, k, score_func, n_group, topk_group
    (1000, 64, 2048, 4, "softmax", None, None),
    (1000, 64, 2048, 4, "sigmoid", None, None),
    (129, 8, 512, 2, "softmax", None, None),
    (300, 100, 256, 6, "sigmoid", None, None),
    (257, 128, 1024, 8, "sigmoid", 8, 4),
    (200, 256, 512, 8, "sigmoid", None, None),
    (127, 32, 64, 1, "sigmoid", None, None),
    (64, 64, 640, 4, "softmax", 4, 2),
]


@pytest.mark.parametrize("token_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,E,d,k,score_func,n_group,topk_group", CASES)
def test_router_matches_oracle(T, E, d, k, score_func, n_group, topk_group, token_dtype):
    x, w, bias = _case(T, E, d, seed=T + E + d, token_dtype=token_dtype)
    kw = dict(score_func=score_func, expert_bias=bias, norm_topk_prob=True, n_group=n_group,
              topk_group=topk_group, route_scale=2.5)
    planes = router_weight_planes(w.cuda())
    idx, top, logits, scores = fused_router_forward(x.cuda(), planes, E, k,
                                                    score_dtype=torch.float32, **kw)
    idx, top, logits, scores = idx.cpu(), top.cpu(), logits.cpu(), scores.cpu()

    # 1. logits: fp32 dot products
    exact = x.double() @ w.double().t()
    bound = orr.logits_error_bound(x, w)
    err = (logits.double() - exact).abs().max(dim=1).values
    assert bool((err <= bound).all()), float((err / bound).max())
    print(f"T={T} E={E} d={d} {token_dtype}: max |logit err| / bound = {float((err / bound).max()):.3e}")

    # 2. scores of the kernel's logits within fp32 rounding of the oracle's;
    # the selection and gating of the kernel's scores bit-exact / within
    # rounding of the oracle's rule.
    kws = {key: val for key, val in kw.items() if key != "score_func"}
    _, _, rscores, _ = orr.route_from_logits(logits, k, **kw)
    torch.testing.assert_close(scores, rscores, rtol=2e-6, atol=1e-7)
    sidx, stop, _, _ = orr.route_from_scores(scores, k, **kws)
    assert torch.equal(idx, sidx)
    torch.testing.assert_close(top, stop, rtol=3e-6, atol=1e-7)

    # 3. end to end against the oracle's own fp32 logits (the CPU's fp32
    # GEMM sums in another order). With every key of a token within delta of
    # the oracle's, picks separated by more than 2*delta cannot reorder.
    oidx, _, _, oscores, ochoice = orr.router_forward(x, w, k, **kw)
    delta = (scores - oscores).abs().max(dim=1).values
    keys = ochoice
    sure = torch.ones(T, dtype=torch.bool)
    if n_group is not None:
        gs = ochoice.view(T, n_group, E // n_group).topk(2, dim=-1)[0].sum(dim=-1)
        sure &= _margin_ok(gs, topk_group, 4 * delta + 1e-12)
        keys = ochoice.masked_fill(~orr.group_mask(ochoice, n_group, topk_group), float("-inf"))
    sure &= _margin_ok(keys, k, 2 * delta + 1e-12)
    same = (idx == oidx).all(dim=1)
    assert bool(same[sure].all()), int((~same & sure).sum())
    assert int(sure.sum()) >= int(0.98 * T), int(sure.sum())


def test_bf16_scores_logit_delta_and_no_renorm():
    T, E, d, k = 500, 64, 512, 4
    x, w, bias = _case(T, E, d, seed=11)
    delta = torch.randn(T, E, generator=torch.Generator().manual_seed(12)) * 0.1
    planes = router_weight_planes(w.cuda())
    for norm in (True, False):
        idx, top, logits, scores = fused_router_forward(
            x.cuda(), planes, E, k, score_func="sigmoid", expert_bias=bias,
            logit_delta=delta.cuda(), norm_topk_prob=norm, route_scale=1.0)
        assert top.dtype == torch.bfloat16
        exact = x.double() @ w.double().t() + delta.double()
        assert bool(((logits.cpu().double() - exact).abs().max(dim=1).values
                     <= orr.logits_error_bound(x, w) + 1e-7).all())
        ridx, rtop, _, _ = orr.route_from_scores(scores.cpu(), k, expert_bias=bias,
                                                 norm_topk_prob=norm, out_dtype=torch.bfloat16)
        assert torch.equal(idx.cpu(), ridx)
        # bf16 of fp32 values that agree to rounding: equal, or one bf16 ulp apart
        diff = (top.cpu().float() - rtop.float()).abs()
        assert bool((diff <= rtop.float().abs() * 2.0**-7).all())


def test_module_matches_the_reference_router_surface():
    T, E, d = 300, 64, 256
    x, w, bias = _case(T, E, d, seed=21)
    r = FusedRouter(d, E, 4, "sigmoid", True, None, None, 1.0).cuda()
    with torch.no_grad():
        r.weight.copy_(w)
        r.e_score_correction_bias.copy_(bias)
        idx, top, logits, scores, choice = r(x.cuda())
    assert top.dtype == x.dtype and logits.dtype == torch.float32
    torch.testing.assert_close(choice, scores + bias.cuda().unsqueeze(0))
    ridx, _, _, _ = orr.route_from_scores(scores.cpu(), 4, expert_bias=bias)
    assert torch.equal(idx.cpu(), ridx)
    # A changed weight rebuilds the planes.
    with torch.no_grad():
        r.weight.mul_(-1.0)
        idx2, _, logits2, _, _ = r(x.cuda())
    torch.testing.assert_close(logits2, -logits)
    # With a gradient the scores carry one; the picks are unchanged.
    idx3, top3, _, _, _ = r(x.cuda().requires_grad_(True))
    assert top3.requires_grad and torch.equal(idx3, idx2)


def test_empty_and_invalid_inputs():
    w = torch.randn(16, 64).cuda()
    planes = router_weight_planes(w)
    idx, top, _, _ = fused_router_forward(torch.empty(0, 64, dtype=torch.bfloat16, device="cuda"),
                                          planes, 16, 2)
    assert idx.shape == (0, 2) and top.shape == (0, 2)
    x = torch.randn(8, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        fused_router_forward(x, planes, 16, 17)
    with pytest.raises(ValueError):
        fused_router_forward(x, planes, 16, 2, n_group=16, topk_group=2)  # groups of 1
    with pytest.raises(ValueError):
        fused_router_forward(x, planes, 16, 8, n_group=4, topk_group=1)  # k > 1 group of 4
    with pytest.raises(ValueError):
        router_weight_planes(torch.randn(300, 64).cuda())
