"""GPU router parity: indices bit-exact, scores within fp32 tolerance."""

import numpy as np
import pytest
import torch

from mirai_amd import route_topk
from mirai_amd import workloads as wl
from oracle import routing as oroute

pytestmark = pytest.mark.gpu

RENORMS = {"clamp": oroute.RENORM_CLAMP, "eps": oroute.RENORM_EPS, "none": oroute.RENORM_NONE}


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_route_matches_oracle_on_benchmark_logits(name):
    w = wl.WORKLOADS[name]
    logits = wl.router_logits(w)
    idx, scores = route_topk(logits.cuda(), w.top_k, renorm="clamp")
    ref_idx, ref_scores = oroute.route_topk(logits.numpy(), w.top_k)
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
    np.testing.assert_allclose(scores.cpu().numpy(), ref_scores, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("renorm", ["clamp", "eps", "none"])
@pytest.mark.parametrize("experts,k", [(8, 2), (100, 3), (128, 8), (1024, 16), (5, 5), (64, 4),
                                        (40, 6), (36, 16), (48, 1), (16, 4), (12, 3), (24, 6),
                                        (32, 8), (50, 5), (63, 16), (2, 1)])
def test_route_modes_and_shapes(renorm, experts, k):
    g = torch.Generator().manual_seed(experts * 31 + k)
    logits = torch.randn(333, experts, generator=g)
    logits[::7, : experts // 2] = 0.25  # ties: equal logits go to the lower expert id
    logits[3::11, experts // 3:] = -float("inf")  # -inf logits, taken last in id order
    idx, scores = route_topk(logits.cuda(), k, renorm=renorm, route_scale=2.5,
                             score_dtype=torch.float32)
    ref_idx, ref_scores = oroute.route_topk(logits.numpy(), k, renorm=RENORMS[renorm],
                                            route_scale=2.5)
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
    np.testing.assert_allclose(scores.cpu().numpy(), ref_scores, rtol=3e-6, atol=1e-7)


def test_route_bf16_scores_and_backward():
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(257, 64, generator=g)
    idx, s16 = route_topk(logits.cuda(), 4, renorm="eps", score_dtype=torch.bfloat16)
    _, ref = oroute.route_topk(logits.numpy(), 4, renorm=oroute.RENORM_EPS)
    np.testing.assert_allclose(s16.float().cpu().numpy(), ref, rtol=8e-3, atol=1e-6)
    lg = logits.cuda().requires_grad_(True)
    idx, s = route_topk(lg, 4, renorm="clamp", route_scale=1.5)
    gs = torch.randn(s.shape, generator=g)
    s.backward(gs.cuda())
    ref_grad = oroute.route_topk_backward(logits.numpy(), idx.cpu().numpy(), gs.numpy(),
                                          renorm=oroute.RENORM_CLAMP, route_scale=1.5)
    np.testing.assert_allclose(lg.grad.cpu().numpy(), ref_grad, rtol=1e-4, atol=2e-6)


@pytest.mark.parametrize("experts,k", [(64, 4), (40, 6), (16, 4), (32, 8)])
def test_route_misaligned_logits_view(experts, k):
    # A contiguous view one float into its storage: the base is 4-byte but not
    # 16-byte aligned, so the float4 row paths must not be taken.
    g = torch.Generator().manual_seed(experts + k)
    storage = torch.randn(257 * experts + 1, generator=g)
    logits = storage[1:].view(257, experts)
    dev = storage.cuda()[1:].view(257, experts)
    assert dev.data_ptr() % 16 != 0
    idx, scores = route_topk(dev, k, renorm="clamp", score_dtype=torch.float32)
    ref_idx, ref_scores = oroute.route_topk(logits.numpy(), k)
    np.testing.assert_array_equal(idx.cpu().numpy(), ref_idx)
    np.testing.assert_allclose(scores.cpu().numpy(), ref_scores, rtol=3e-6, atol=1e-7)


def test_route_no_tokens_forward_and_backward():
    lg = torch.empty(0, 64, device="cuda").requires_grad_(True)
    idx, s = route_topk(lg, 4, renorm="clamp")
    assert tuple(idx.shape) == (0, 4) and tuple(s.shape) == (0, 4)
    s.sum().backward()
    assert tuple(lg.grad.shape) == (0, 64)
