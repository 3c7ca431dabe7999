"""GPU parity of the token-chunked routed layer (MoETokenChunkPolicy,
mirai/core/moe/runtime/token_chunking.py:48-118) against torch autograd through
the reference-order oracle, and against the unchunked layer.

Chunking splits the tokens, not the routes: each token's slots stay in one
chunk, so the chunked forward output and token / score gradients are the
unchunked layer's bit for bit; the LoRA factor gradients are fp32 sums over
chunks (order of the sum differs: relative 1e-5). Against the oracle the
layer tolerance holds (max-abs 2e-2 / mean-rel 5e-3) and the gradients meet
the backward bound (mean-rel <= 5e-3, max <= 3e-2 of the oracle's max).
"""

import pytest
import torch

from mirai_amd import MoETokenChunkPolicy, fused_chunk_runner
from mirai_amd import workloads as wl
from oracle import layer as olayer
from oracle import routing as oroute

from helpers import assert_layer_close, build_module, oracle_weights

pytestmark = pytest.mark.gpu

MEAN_REL = 5e-3
MAX_REL = 3e-2


def _close(name, actual, expected):
    a, e = actual.detach().float().cpu(), expected.detach().float().cpu()
    diff = (a - e).abs()
    stats = {"mean_rel": float(diff.sum() / e.abs().sum().clamp_min(1e-30)),
             "max_rel": float(diff.max()) / float(e.abs().max().clamp_min(1e-30))}
    assert stats["mean_rel"] <= MEAN_REL and stats["max_rel"] <= MAX_REL, (name, stats)


def _setup(fmt, T):
    w = wl.Workload(f"chunk_{fmt}", 9, T, 256, 192, 8, 2, 16, 16.0, fmt, torch.bfloat16)
    dense, lora = wl.dense_weights(w), wl.lora_factors(w)
    x = wl.tokens(w)
    idx_np, scores_np = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    return w, dense, lora, x, torch.from_numpy(idx_np), torch.from_numpy(scores_np), \
        wl.upstream_grad(w)


def _run(m, x, scores, idx, dy, policy, runner):
    xg = x.cuda().requires_grad_(True)
    sg = scores.cuda().requires_grad_(True)
    for ad in m.expert_lora.values():
        ad.lora_a.grad = None
        ad.lora_b.grad = None
    if policy is None:
        out = m.run_direct_routed(xg, sg, idx.cuda())
    else:
        out = policy.execute(xg, sg, idx.cuda(), runner=runner, training=True)
    out.backward(dy.cuda())
    grads = {"tokens": xg.grad.detach().clone(), "scores": sg.grad.detach().clone()}
    for key, ad in m.expert_lora.items():
        grads[f"{key}.a"] = ad.lora_a.grad.detach().clone()
        grads[f"{key}.b"] = ad.lora_b.grad.detach().clone()
    return out.detach(), grads


@pytest.mark.parametrize("fmt", ["nf4", "int8"])
def test_chunked_layer_matches_oracle_and_unchunked(fmt):
    # 700 tokens in chunks of 256: three chunks, the last one ragged (188).
    w, dense, lora, x, idx, scores, dy = _setup(fmt, 700)
    m = build_module(w, dense, lora)
    policy = MoETokenChunkPolicy(token_chunk_size=256)
    assert policy.chunk_count(700) == 3
    out_c, g_c = _run(m, x, scores, idx, dy, policy, fused_chunk_runner(m))
    out_u, g_u = _run(m, x, scores, idx, dy, None, None)
    assert torch.equal(out_c, out_u)
    assert torch.equal(g_c["tokens"], g_u["tokens"]) and torch.equal(g_c["scores"], g_u["scores"])
    for k in g_u:
        rel = float((g_c[k] - g_u[k]).abs().sum() / g_u[k].abs().sum().clamp_min(1e-30))
        assert rel < 1e-5, (k, rel)

    xo = x.clone().requires_grad_(True)
    so = scores.clone().requires_grad_(True)
    leaves = {k: (a.clone().float().requires_grad_(True), b.clone().float().requires_grad_(True))
              for k, (a, b) in lora.items()}
    ref = olayer.layer_forward(xo, so, idx, oracle_weights(w, dense),
                               {k: (a, b, wl.lora_scale(w)) for k, (a, b) in leaves.items()},
                               w.experts)
    ref.backward(dy)
    assert_layer_close(out_c.cpu(), ref)
    _close("tokens", g_c["tokens"], xo.grad)
    _close("scores", g_c["scores"], so.grad)
    for k, (a, b) in leaves.items():
        _close(f"{k}.a", g_c[f"{k}.a"], a.grad)
        _close(f"{k}.b", g_c[f"{k}.b"], b.grad)


def test_generic_runner_falls_back_to_checkpointed_chunks():
    # A runner the policy does not recognise (a plain closure over the module)
    # goes through torch's checkpoint per chunk; same results as the fused path.
    w, dense, lora, x, idx, scores, dy = _setup("nf4", 520)
    m = build_module(w, dense, lora)
    policy = MoETokenChunkPolicy(token_chunk_size=200)
    offsets = []

    def runner(t, s, i, off):
        offsets.append(off)
        return m.run_direct_routed(t, s, i)

    out_g, g_g = _run(m, x, scores, idx, dy, policy, runner)
    assert offsets[:3] == [0, 200, 400]  # the forward; the backward replays them
    out_f, g_f = _run(m, x, scores, idx, dy, policy, fused_chunk_runner(m))
    assert torch.equal(out_g, out_f)
    assert torch.equal(g_g["tokens"], g_f["tokens"])
    for k in g_f:
        rel = float((g_g[k] - g_f[k]).abs().sum() / g_f[k].abs().sum().clamp_min(1e-30))
        assert rel < 1e-5, (k, rel)


def test_inference_runs_unchunked():
    w, dense, lora, x, idx, scores, _ = _setup("nf4", 600)
    m = build_module(w, dense, lora)
    policy = MoETokenChunkPolicy(token_chunk_size=128)
    with torch.no_grad():
        out_i = policy.execute(x.cuda(), scores.cuda(), idx.cuda(), runner=fused_chunk_runner(m),
                               training=False)
        out_u = m.run_direct_routed(x.cuda(), scores.cuda(), idx.cuda())
    assert torch.equal(out_i, out_u)
