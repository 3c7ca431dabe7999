"""CPU pin of the block oracle (oracle/block.py) against an independent fp64
per-token formulation of LingBotVideoSparseMoeBlock._forward_once
(mirai/vendors/lingbot_video/transformer_lingbot_video.py:2282-2287 for the
padding-mask renormalisation, :2374-2377 for the shared-expert add,
:491-499 for LingBotVideoMLP).

Per token t, with routes (e_j, s_j), mask m_t and route scale c:
    s'_j = c * (s_j m_t) / (sum_i s_i m_t + 1e-9)          (mask given)
    out_t = sum_j s'_j * MLP_{e_j}(x_t) + MLP_shared(x_t)
computed here in fp64 from the same dequantised weights. The oracle runs in
the reference's bf16 composition, so the two agree to bf16 rounding (a few
roundings of 2^-9 relative each: mean-relative <= 1e-2). Planted
mistakes (the renorm dropped, the route scale dropped, the shared expert's
gate and up swapped) must each move the oracle far outside that bound.
"""

import numpy as np
import torch

from mirai_amd import workloads as wl
from oracle import block as oblock
from oracle import layer as olayer
from oracle import routing as oroute

from helpers import oracle_loras, oracle_weights

H, FF, E, K, T, FS = 128, 192, 6, 2, 48, 160


def _setup(seed=3):
    w = wl.Workload("oblock", 11, T, H, FF, E, K, 8, 16.0, "nf4", torch.bfloat16)
    dense = wl.dense_weights(w)
    lora = wl.lora_factors(w)
    weights = oracle_weights(w, dense)
    loras = oracle_loras(w, lora)
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(2, T // 2, H, generator=g)).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    idx, scores = oroute.route_topk(logits.numpy(), K)
    shared = tuple((torch.randn(shape, generator=g) * 0.05).to(torch.bfloat16)
                   for shape in ((FS, H), (FS, H), (H, FS)))
    mask = (torch.rand(T, generator=g) > 0.25).to(torch.bfloat16)
    return x, torch.from_numpy(idx), torch.from_numpy(scores), weights, loras, shared, mask


def _mlp64(x, gate, up, down, lora=None, e=None):
    """silu(x G^T) * (x U^T) then D^T, all fp64; with per-expert LoRA deltas."""
    def proj(v, wt, key):
        out = v @ wt.double().T
        if lora is not None and key in lora:
            a, b, s = lora[key]
            out = out + (v @ a[e].double().T) @ b[e].double().T * s
        return out
    g = proj(x, gate, "w1")
    u = proj(x, up, "w3")
    h = g / (1.0 + torch.exp(-g)) * u
    return proj(h, down, "w2")


def _reference64(x, idx, scores, weights, loras, shared, mask, route_scale):
    xt = x.reshape(-1, H).double()
    out = torch.zeros_like(xt)
    for t in range(xt.shape[0]):
        s = scores[t].double()
        if mask is not None:
            s = s * float(mask[t])
            s = s / (s.sum() + 1e-9) * route_scale
        for j in range(K):
            e = int(idx[t, j])
            y = _mlp64(xt[t:t + 1], weights["w1"][e], weights["w3"][e], weights["w2"][e],
                       loras, e)
            out[t] += s[j] * y[0]
        if shared is not None:
            out[t] += _mlp64(xt[t:t + 1], *shared)[0]
    return out.reshape(x.shape)


def _err(a, b):
    d = (a.double() - b.double()).abs()
    return float(d.max()), float(d.sum() / b.double().abs().sum())


def _oracle(x, idx, scores, weights, loras, shared, mask, route_scale):
    out, _ = oblock.block_forward(x, None, K, weights, loras, E, shared=shared,
                                  padding_mask=mask, routes=(idx, scores),
                                  route_scale=route_scale)
    return out


def test_block_oracle_matches_fp64_per_token_formulation():
    x, idx, scores, weights, loras, shared, mask = _setup()
    for m, c, sh in ((None, 1.0, shared), (mask, 1.0, shared), (mask, 2.5, shared),
                     (mask, 1.0, None)):
        got = _oracle(x, idx, scores, weights, loras, sh, m, c)
        want = _reference64(x, idx, scores, weights, loras, sh, m, c)
        max_abs, mean_rel = _err(got, want)
        assert max_abs <= 2e-2 and mean_rel <= 1e-2, (m is not None, c, sh is not None,
                                                      max_abs, mean_rel)


def test_masked_tokens_get_only_the_shared_expert():
    x, idx, scores, weights, loras, shared, mask = _setup()
    got = _oracle(x, idx, scores, weights, loras, shared, mask, 1.0).reshape(-1, H)
    shared_only = oblock.shared_mlp(x.reshape(-1, H), *shared)
    off = mask == 0
    assert bool(off.any())
    # Masked tokens: scores become 0 / (0 + 1e-9) = 0, so the routed part is 0.
    torch.testing.assert_close(got[off].float(), shared_only[off].float(), rtol=0, atol=0)


def test_unmasked_renorm_is_the_identity_on_normalised_scores():
    # Softmax top-k scores renormalised to sum 1: the masked path with an
    # all-ones mask and route_scale 1 changes them by at most 1e-9 relative.
    x, idx, scores, weights, loras, shared, _ = _setup()
    ones = torch.ones(T, dtype=torch.bfloat16)
    a = _oracle(x, idx, scores, weights, loras, shared, ones, 1.0)
    b = _oracle(x, idx, scores, weights, loras, shared, None, 1.0)
    max_abs, _ = _err(a, b)
    assert max_abs <= 1e-2


def test_planted_mistakes_are_caught():
    x, idx, scores, weights, loras, shared, mask = _setup()
    # Scores that do not sum to 1, so that the renorm itself matters.
    scores = scores * 0.4
    want = _reference64(x, idx, scores, weights, loras, shared, mask, 2.5)

    def no_renorm():
        s = scores * mask.reshape(-1, 1).float() * 2.5  # renorm dropped, scale kept
        out = olayer.layer_forward(x.reshape(-1, H), s, idx, weights, loras, E)
        return out.view(x.shape) + oblock.shared_mlp(x.reshape(-1, H), *shared).view(x.shape)

    swapped = (shared[1], shared[0], shared[2])
    planted = {
        "renorm dropped": no_renorm(),
        "route scale dropped": _oracle(x, idx, scores, weights, loras, shared, mask, 1.0),
        "shared gate/up swapped": _oracle(x, idx, scores, weights, loras, swapped, mask, 2.5),
    }
    for name, got in planted.items():
        max_abs, mean_rel = _err(got, want)
        assert mean_rel > 5e-2, (name, max_abs, mean_rel)
    np.testing.assert_array_less(
        _err(_oracle(x, idx, scores, weights, loras, shared, mask, 2.5), want)[1], 1e-2)
