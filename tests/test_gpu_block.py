"""GPU parity of the LingBot block front end: shared expert, fused router +
routed experts + shared expert overlapped on two streams, padding masks and
token-chunked training, against the block oracle (oracle/block.py)."""

import pytest
import torch

from mirai_amd import workloads as wl
from mirai_amd.block import FusedSparseMoeBlock, SharedExpertMLP
from mirai_amd.chunking import MoETokenChunkPolicy
from oracle import block as oblock

from helpers import assert_layer_close, oracle_loras, oracle_weights

pytestmark = pytest.mark.gpu

H, F, E, K = 256, 192, 16, 4


def _workload(T, fmt="nf4"):
    return wl.Workload(f"block_{fmt}", 9, T, H, F, E, K, 16, 16.0, fmt, torch.bfloat16)


def _block(w, *, shared=True, lora=True, score_func="sigmoid", seed=0):
    g = torch.Generator().manual_seed(seed)
    blk = FusedSparseMoeBlock(H, 4 * H, E, K, F, score_func, True, None, None, 1.0,
                              1 if shared else 0, quant_format=w.fmt).cuda()
    router_w = torch.randn(E, H, generator=g) * 0.05
    bias = torch.randn(E, generator=g) * 0.01
    with torch.no_grad():
        blk.router.weight.copy_(router_w)
        blk.router.e_score_correction_bias.copy_(bias)
    dense = wl.dense_weights(w)
    for key in ("w1", "w3", "w2"):
        blk.experts.load_dense_weight(key, dense[key].cuda())
    factors = wl.lora_factors(w) if lora else None
    if factors:
        for key, (a, b) in factors.items():
            ad = blk.experts.attach_expert_lora(tensor_name=key, adapter_name="t", rank=w.rank,
                                                alpha=w.alpha)
            with torch.no_grad():
                ad.lora_a.copy_(a.cuda())
                ad.lora_b.copy_(b.cuda())
    sh = None
    if shared:
        blk.shared_experts.to(torch.bfloat16).requires_grad_(False)
        sh = []
        for lin in (blk.shared_experts.gate_proj, blk.shared_experts.up_proj,
                    blk.shared_experts.down_proj):
            wt = (torch.randn(lin.weight.shape, generator=g) * 0.03).to(torch.bfloat16)
            with torch.no_grad():
                lin.weight.copy_(wt)
            sh.append(wt)
    ref = dict(router_weight=router_w, expert_weights=oracle_weights(w, dense),
               expert_loras=oracle_loras(w, factors), shared=tuple(sh) if sh else None,
               expert_bias=bias)
    return blk, ref


def test_shared_expert_is_the_bf16_swiglu_mlp():
    g = torch.Generator().manual_seed(3)
    mlp = SharedExpertMLP(H, 320).cuda().to(torch.bfloat16).requires_grad_(False)
    ws = [(torch.randn(lin.weight.shape, generator=g) * 0.05).to(torch.bfloat16)
          for lin in (mlp.gate_proj, mlp.up_proj, mlp.down_proj)]
    with torch.no_grad():
        for lin, wt in zip((mlp.gate_proj, mlp.up_proj, mlp.down_proj), ws):
            lin.weight.copy_(wt)
        x = torch.randn(333, H, generator=g).to(torch.bfloat16)
        out = mlp(x.cuda())
    ref = oblock.shared_mlp(x, *ws)
    print(f"shared expert: {assert_layer_close(out.cpu(), ref)}")


@pytest.mark.parametrize("fmt", ["nf4", "bf16"])
@pytest.mark.parametrize("shared", [True, False])
def test_block_matches_oracle(fmt, shared):
    w = _workload(2 * 160, fmt)
    blk, ref = _block(w, shared=shared)
    x = wl.tokens(w).view(2, 160, H)
    with torch.no_grad():
        out = blk(x.cuda())
        idx, top, _, _, _ = blk.router(x.view(-1, H).cuda())
    assert out.shape == x.shape and out.dtype == x.dtype
    kw = dict(score_func="sigmoid", expert_bias=ref["expert_bias"], norm_topk_prob=True,
              route_scale=1.0)
    # the composition on the kernel's own routes: the whole output
    want, _ = oblock.block_forward(x, ref["router_weight"], K, ref["expert_weights"],
                                   ref["expert_loras"], E, shared=ref["shared"],
                                   routes=(idx.cpu(), top.cpu()), **kw)
    print(f"block {fmt} shared={shared}: {assert_layer_close(out.cpu(), want)}")
    # end to end through the oracle router: tokens routed identically agree
    want2, oidx = oblock.block_forward(x, ref["router_weight"], K, ref["expert_weights"],
                                       ref["expert_loras"], E, shared=ref["shared"], **kw)
    same = (oidx == idx.cpu()).all(dim=1)
    assert int(same.sum()) >= int(0.98 * same.numel())
    assert_layer_close(out.cpu().view(-1, H)[same], want2.view(-1, H)[same])


def test_overlapped_block_equals_sequential_execution():
    w = _workload(512)
    blk, _ = _block(w)
    x = wl.tokens(w).view(1, 512, H).cuda()
    with torch.no_grad():
        out = blk(x)
        tokens = x.view(-1, H)
        idx, top, _, _, _ = blk.router(tokens)
        routed = blk.experts.run_direct_routed(tokens, top, idx)
        seq = routed + blk.shared_experts(tokens)
    assert torch.equal(out.view(-1, H), seq)


def test_padding_mask_renormalises_the_routes():
    w = _workload(2 * 96)
    blk, ref = _block(w, shared=False, lora=False)
    x = wl.tokens(w).view(2, 96, H)
    mask = torch.ones(2 * 96)
    mask[96 + 70:] = 0.0
    with torch.no_grad():
        out = blk(x.cuda(), padding_mask=mask.cuda())
        idx, top, _, _, _ = blk.router(x.view(-1, H).cuda())
    kw = dict(score_func="sigmoid", expert_bias=ref["expert_bias"], route_scale=1.0)
    want, _ = oblock.block_forward(x, ref["router_weight"], K, ref["expert_weights"], {}, E,
                                   padding_mask=mask, routes=(idx.cpu(), top.cpu()), **kw)
    assert_layer_close(out.cpu(), want)
    assert torch.count_nonzero(out.view(-1, H)[96 + 70:].cpu()) == 0


def test_token_chunked_training_matches_unchunked():
    w = _workload(700)
    blk, _ = _block(w)
    blk.train()
    x = wl.tokens(w).view(1, 700, H).cuda()
    dy = torch.randn(x.shape, generator=torch.Generator().manual_seed(5)).to(x.dtype).cuda()

    def run(policy):
        blk.set_token_chunk_policy(policy)
        xg = x.clone().requires_grad_(True)
        out = blk(xg)
        out.backward(dy)
        grads = {f"{k}.{n}": getattr(ad, n).grad.clone()
                 for k, ad in blk.experts.expert_lora.items() for n in ("lora_a", "lora_b")}
        for ad in blk.experts.expert_lora.values():
            ad.lora_a.grad = None
            ad.lora_b.grad = None
        return out.detach(), xg.grad, grads

    out0, gx0, g0 = run(None)
    out1, gx1, g1 = run(MoETokenChunkPolicy(token_chunk_size=256))
    assert MoETokenChunkPolicy(256).chunk_count(700) == 3
    assert torch.equal(out0, out1)
    torch.testing.assert_close(gx1, gx0, rtol=0, atol=0)
    for k in g0:
        rel = float((g1[k] - g0[k]).abs().sum() / g0[k].abs().sum().clamp_min(1e-30))
        assert rel < 1e-5, (k, rel)


def test_empty_batch_through_the_block():
    """A batch with no tokens: router, routed experts and shared expert return
    an empty output, and a training step's backward leaves zero LoRA grads."""
    w = _workload(64)
    blk, _ = _block(w)
    x = torch.empty(2, 0, H, dtype=torch.bfloat16, device="cuda")
    with torch.no_grad():
        assert tuple(blk(x).shape) == (2, 0, H)
    xg = x.clone().requires_grad_(True)
    out = blk(xg)
    out.float().sum().backward()
    assert tuple(xg.grad.shape) == (2, 0, H)
    for ad in blk.experts.expert_lora.values():
        for p in (ad.lora_a, ad.lora_b):
            assert p.grad is None or not bool(p.grad.abs().gt(0).any())
