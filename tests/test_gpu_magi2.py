"""GPU parity of the MAGI-2 multi-head MoE path: per-head routing (bit-exact
indices), the plan over 12 x 256 = 3072 flattened groups, and the routed
swiglu7 expert layer forward and backward vs the oracle (layer tolerance of
the benchmark definition: max-abs 2e-2, mean-rel 5e-3)."""

import numpy as np
import pytest
import torch

from mirai_amd import Magi2FusedMoEBackend, Magi2GroupedExperts, build_dispatch_plan
from mirai_amd import route_topk_heads
from oracle import fastcodec
from oracle import magi2 as om
from oracle import plan as oplan

from helpers import assert_layer_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("score_func", ["softmax", "sigmoid"])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("route_norm", [False, True])
@pytest.mark.parametrize("E,k", [(4, 2), (256, 8), (64, 1)])
def test_route_heads_matches_oracle(score_func, with_bias, route_norm, E, k):
    g = torch.Generator().manual_seed(E + k)
    H, S = 3, 257
    logits = torch.randn(H, S, E, generator=g)
    bias = torch.randn(H, E, generator=g) * 0.05 if with_bias else None
    want_p, want_i = om.route_topk_heads(logits, k, score_func=score_func, expert_bias=bias,
                                         route_norm=route_norm, route_scale=4.9)
    p, i = route_topk_heads(logits.cuda(), k, score_func=score_func,
                            expert_bias=None if bias is None else bias.cuda(),
                            route_norm=route_norm, route_scale=4.9)
    assert torch.equal(i.cpu(), want_i)
    torch.testing.assert_close(p.cpu(), want_p, rtol=2e-6, atol=1e-7)
    pr, ir = route_topk_heads(logits.cuda(), k, score_func=score_func,
                              expert_bias=None if bias is None else bias.cuda(),
                              route_norm=route_norm, route_scale=4.9, layout="rows")
    want_pr, want_ir = om.heads_to_rows(want_p, want_i, E)
    assert torch.equal(ir.cpu(), want_ir)
    torch.testing.assert_close(pr.cpu(), want_pr, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("S,H,E,k", [(300, 12, 256, 2), (64, 16, 512, 4)])
def test_plan_over_flattened_head_expert_groups(S, H, E, k):
    # 3072 and 8192 groups: beyond the 1023-group cap of torch grouped_mm.
    g = torch.Generator().manual_seed(S)
    logits = torch.randn(H, S, E, generator=g)
    probs, idx = om.route_topk_heads(logits, k, score_func="sigmoid")
    p_rows, g_rows = om.heads_to_rows(probs, idx, E)
    top_idx, top_scores = g_rows.numpy(), p_rows.numpy()
    plan = build_dispatch_plan(g_rows.cuda(), p_rows.cuda(), H * E)
    ref = oplan.build_dispatch_plan(top_idx, top_scores, H * E)
    np.testing.assert_array_equal(plan.counts.cpu().numpy(), ref.counts)
    np.testing.assert_array_equal(plan.offsets.cpu().numpy(), ref.offsets)
    np.testing.assert_array_equal(plan.sort_positions.cpu().numpy(), ref.sort_positions)
    np.testing.assert_array_equal(plan.inverse_order.cpu().numpy(), ref.inverse_order)


def _magi2_case(*, H=2, E=4, d=128, f=128, S=64, k=2, seed=0, std=0.05):
    g = torch.Generator().manual_seed(seed)
    G = H * E
    dense = {
        "W_gate": (torch.randn(G, d, f, generator=g) * std).to(torch.bfloat16),
        "W_up": (torch.randn(G, d, f, generator=g) * std).to(torch.bfloat16),
        "W_down": (torch.randn(G, f, d, generator=g) * std).to(torch.bfloat16),
    }
    x = torch.randn(S, H, d, generator=g).to(torch.bfloat16)
    logits = torch.randn(H, S, E, generator=g)
    bias = torch.randn(H, E, generator=g) * 0.05
    probs, idx = om.route_topk_heads(logits, k, score_func="sigmoid", expert_bias=bias,
                                     route_norm=True, route_scale=4.9)
    return dense, x, logits, bias, probs, idx


def _oracle_weights(fmt, dense):
    """The weights the packed module computes with, in the [G, in, out] layout."""
    if fmt == "bf16":
        return dict(dense)
    out = {}
    for key, t in dense.items():
        kt = t.transpose(1, 2).contiguous()  # stored as [G, out, in]
        G, o, i = kt.shape
        bits = kt.view(torch.int16).numpy().view(np.uint16).reshape(G * o, i)
        codes, absmax = fastcodec.nf4_quantize(bits)
        deq = fastcodec.nf4_dequantize(codes, absmax)
        w = torch.from_numpy(deq.view(np.int16).reshape(G, o, i)).view(torch.bfloat16)
        out[key] = w.transpose(1, 2).contiguous()
    return out


@pytest.mark.parametrize("fmt", ["bf16", "nf4"])
def test_reduced_magi2_layer_matches_oracle(fmt):
    # The reduced layer of tests/test_magi2_nf4_experts.py:434-465 (2 heads x 4
    # experts, top-2, sigmoid routing with expert bias, route_scale 4.9).
    dense, x, logits, bias, probs, idx = _magi2_case()
    m = Magi2GroupedExperts.from_dense(*(dense[k].cuda() for k in ("W_gate", "W_up", "W_down")),
                                       num_heads=2, quant_format=fmt)
    with torch.no_grad():
        out = m.execute(x.cuda(), probs.cuda(), idx.cuda())
    ref = om.layer_forward(x, probs, idx, _oracle_weights(fmt, dense), 4)
    stats = assert_layer_close(out.cpu(), ref)
    print(f"magi2 {fmt}: {stats}")
    # Routing on the GPU gives the same result.
    with torch.no_grad():
        out2 = m(x.cuda(), logits.cuda(), top_k=2, score_func="sigmoid", expert_bias=bias.cuda(),
                 route_norm=True, route_scale=4.9)
    assert torch.equal(out2, out)


def test_run_for_loop_with_swiglu7_matches_oracle():
    # run_for_loop over rows already grouped by (head, expert) with the MAGI-2
    # swiglu7 activation (experts.py:1656-1747): the routed layer with one
    # unit-score route per row.
    H, E = 2, 4
    dense, x, _, _, _, _ = _magi2_case(H=H, E=E, seed=5)
    S, d = int(x.shape[0]), int(x.shape[2])
    g = torch.Generator().manual_seed(6)
    idx = torch.randint(0, E, (H, S, 1), generator=g)
    probs = torch.ones(H, S, 1)
    m = Magi2GroupedExperts.from_dense(*(dense[k].cuda() for k in ("W_gate", "W_up", "W_down")),
                                       num_heads=H, quant_format="nf4")
    groups = (idx[:, :, 0] + torch.arange(H).view(H, 1) * E).t().reshape(-1)  # row s*H+h
    order = torch.argsort(groups, stable=True)
    counts = torch.bincount(groups, minlength=H * E)
    rows = x.reshape(S * H, d)[order]
    with torch.no_grad():
        out = m.experts.run_for_loop(rows.cuda(), counts.cuda())
    ref = om.layer_forward(x, probs, idx, _oracle_weights("nf4", dense), E).reshape(S * H, d)
    print(f"magi2 for-loop: {assert_layer_close(out.cpu(), ref[order])}")


def test_magi2_layer_at_production_group_count():
    # 12 heads x 256 experts = 3072 groups in one pass (no segmenting).
    dense, x, _, _, probs, idx = _magi2_case(H=12, E=256, d=64, f=64, S=96, k=2, seed=3)
    m = Magi2GroupedExperts.from_dense(*(dense[k].cuda() for k in ("W_gate", "W_up", "W_down")),
                                       num_heads=12, quant_format="nf4")
    with torch.no_grad():
        out = m.execute(x.cuda(), probs.cuda(), idx.cuda())
    ref = om.layer_forward(x, probs, idx, _oracle_weights("nf4", dense), 256)
    print(f"magi2 3072 groups: {assert_layer_close(out.cpu(), ref)}")


def test_magi2_backward_with_expert_lora_matches_oracle_autograd():
    H, E, d, f, r = 2, 4, 128, 128, 16
    dense, x, _, _, probs, idx = _magi2_case(H=H, E=E, d=d, f=f, S=48, k=2, seed=7, std=0.08)
    m = Magi2GroupedExperts.from_dense(*(dense[k].cuda() for k in ("W_gate", "W_up", "W_down")),
                                       num_heads=H, quant_format="bf16")
    g = torch.Generator().manual_seed(9)
    loras = {}
    for key, (i_f, o_f) in {"W_gate": (d, f), "W_up": (d, f), "W_down": (f, d)}.items():
        a = (torch.randn(H * E, r, i_f, generator=g) * 0.05).to(torch.bfloat16)
        b = (torch.randn(H * E, o_f, r, generator=g) * 0.05).to(torch.bfloat16)
        ad = m.attach_expert_lora(tensor_name=key, adapter_name="t", rank=r, alpha=16.0)
        with torch.no_grad():
            ad.lora_a.copy_(a.cuda())
            ad.lora_b.copy_(b.cuda())
        loras[key] = (a, b)
    dy = torch.randn(x.shape, generator=g).to(torch.bfloat16)
    xg = x.cuda().requires_grad_(True)
    pg = probs.cuda().requires_grad_(True)
    m.execute(xg, pg, idx.cuda()).backward(dy.cuda())

    xo = x.clone().requires_grad_(True)
    po = probs.clone().requires_grad_(True)
    leaves = {k: (a.float().requires_grad_(True), b.float().requires_grad_(True))
              for k, (a, b) in loras.items()}
    ol = {k: (a, b, 1.0) for k, (a, b) in leaves.items()}  # alpha 16 / rank 16
    om.layer_forward(xo, po, idx, dense, E, loras=ol).backward(dy)
    pairs = [("tokens", xg.grad, xo.grad), ("probs", pg.grad, po.grad)]
    for k, (a, b) in leaves.items():
        pairs += [(f"{k}.a", m.experts.expert_lora[k].lora_a.grad, a.grad),
                  (f"{k}.b", m.experts.expert_lora[k].lora_b.grad, b.grad)]
    for name, got, want in pairs:
        rel = float((got.float().cpu() - want.float()).abs().sum() / want.float().abs().sum())
        print(f"magi2 backward {name}: mean_rel={rel:.3e}")
        assert rel <= 1e-2, (name, rel)


def test_backend_seam_executes_attached_experts():
    dense, x, _, _, probs, idx = _magi2_case(seed=4)
    m = Magi2GroupedExperts.from_dense(*(dense[k].cuda() for k in ("W_gate", "W_up", "W_down")),
                                       num_heads=2, quant_format="bf16")
    layer = torch.nn.Module()
    backend = Magi2FusedMoEBackend.attach(layer, m)
    assert layer._mirai_moe_kernel_backend is backend
    with torch.no_grad():
        a = backend.execute(layer, x.cuda(), probs.cuda(), idx.cuda())
        b = m.execute(x.cuda(), probs.cuda(), idx.cuda())
    assert torch.equal(a, b)
    with pytest.raises(RuntimeError, match="attached"):
        backend.execute(torch.nn.Module(), x.cuda(), probs.cuda(), idx.cuda())


def test_empty_sequence_through_the_magi2_layer():
    dense, _, _, bias, _, _ = _magi2_case()
    m = Magi2GroupedExperts.from_dense(*(dense[k].cuda() for k in ("W_gate", "W_up", "W_down")),
                                       num_heads=2, quant_format="nf4")
    x = torch.empty(0, 2, 128, dtype=torch.bfloat16, device="cuda")
    logits = torch.empty(2, 0, 4, device="cuda")
    with torch.no_grad():
        out = m(x, logits, top_k=2, score_func="sigmoid", expert_bias=bias.cuda(),
                route_norm=True, route_scale=4.9)
    assert out.shape[0] == 0 and out.shape[-1] == 128


def _reference_artifact(tmp_path, *, H=2, E=4, d=128, f=192, seed=12):
    """A MAGI-2 artifact as the reference writes it (bitsandbytes double-quant
    per group over [in, out], quantized_experts.py:275-347, packed_experts.py:
    28-78) and the dense bf16 weights [G, in, out] it decodes to (the
    oracle's restatement of bitsandbytes' dequantisation)."""
    from oracle import codec

    from helpers import bnb_group_payload, write_reference_magi2_artifact

    rng = np.random.default_rng(seed)
    table = np.sort(np.concatenate([np.linspace(-1, 1, 255), [0.0]])).astype(np.float32)
    G = H * E
    weights, dense = {}, {}
    for key, (i_f, o_f) in {"W_gate": (d, f), "W_up": (d, f), "W_down": (f, d)}.items():
        w = (rng.standard_normal((G, i_f, o_f)) * 0.05).astype(np.float32)
        bufs, parts = bnb_group_payload(w, table)
        weights[key] = (bufs, (G, i_f, o_f))
        bits = np.stack([codec.bnb_nf4_dequantize(p["packed"], p["absmax"], p["nested_absmax"],
                                                  p["offset"], table, i_f, o_f) for p in parts])
        dense[key] = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    write_reference_magi2_artifact(tmp_path / "artifact", {"blocks.3.moe": weights})
    return tmp_path / "artifact", dense


@pytest.mark.parametrize("S", [80, 1200])  # 128-row tiles; 256-row + remainder tiles
def test_reference_artifact_ingests_without_requantisation(tmp_path, S):
    """The reference's NF4 store loads as stored: the [G, in, out] group payloads
    keep their orientation (blocks along out) and the kernels decode them in
    place (MX_FMT_NF4_F32_KN); the decoded weights equal bitsandbytes'
    dequantisation of the payload (oracle restatement) bit for bit, and the
    layer matches the MAGI-2 oracle on those weights, forward and backward."""
    from mirai_amd import load_reference_magi2_artifact
    from mirai_amd import _native as nat
    from mirai_amd import quant

    H, E, d, f = 2, 4, 128, 192
    path, dense = _reference_artifact(tmp_path, H=H, E=E, d=d, f=f)
    layer = Magi2GroupedExperts(num_heads=H, num_experts=E, quant_format="nf4")
    load_reference_magi2_artifact(path, {"blocks.3.moe": layer})
    assert layer.is_fully_loaded()
    assert layer.expert_weight_shape("W_down") == (H * E, f, d)
    for key in ("W_gate", "W_up", "W_down"):
        pw = layer.experts.packed_weight(key)
        assert pw.layout == "in_out" and pw.format_code() == nat.FMT_NF4_F32_KN
        deq = quant.dequantize(pw)  # [G, out, in]
        assert torch.equal(deq.transpose(1, 2).cpu(), dense[key])

    _, x, _, _, probs, idx = _magi2_case(H=H, E=E, d=d, f=f, S=S, k=2, seed=13)
    with torch.no_grad():
        out = layer.execute(x.cuda(), probs.cuda(), idx.cuda())
    ref = om.layer_forward(x, probs, idx, dense, E)
    print(f"magi2 reference artifact forward: {assert_layer_close(out.cpu(), ref)}")

    # Backward with expert LoRA on every weight (the ingested weights stay frozen).
    g = torch.Generator().manual_seed(21)
    r = 16
    leaves = {}
    for key, (i_f, o_f) in {"W_gate": (d, f), "W_up": (d, f), "W_down": (f, d)}.items():
        a = (torch.randn(H * E, r, i_f, generator=g) * 0.05).to(torch.bfloat16)
        b = (torch.randn(H * E, o_f, r, generator=g) * 0.05).to(torch.bfloat16)
        ad = layer.attach_expert_lora(tensor_name=key, adapter_name="t", rank=r, alpha=32.0)
        with torch.no_grad():
            ad.lora_a.copy_(a.cuda())
            ad.lora_b.copy_(b.cuda())
        leaves[key] = (a.float().requires_grad_(True), b.float().requires_grad_(True))
    dy = torch.randn(x.shape, generator=g).to(torch.bfloat16)
    xg = x.cuda().requires_grad_(True)
    pg = probs.cuda().requires_grad_(True)
    layer.execute(xg, pg, idx.cuda()).backward(dy.cuda())
    xo = x.clone().requires_grad_(True)
    po = probs.clone().requires_grad_(True)
    ol = {k: (a, b, 2.0) for k, (a, b) in leaves.items()}  # alpha 32 / rank 16
    om.layer_forward(xo, po, idx, dense, E, loras=ol).backward(dy)
    pairs = [("tokens", xg.grad, xo.grad), ("probs", pg.grad, po.grad)]
    for k, (a, b) in leaves.items():
        pairs += [(f"{k}.a", layer.experts.expert_lora[k].lora_a.grad, a.grad),
                  (f"{k}.b", layer.experts.expert_lora[k].lora_b.grad, b.grad)]
    for name, got, want in pairs:
        rel = float((got.float().cpu() - want.float()).abs().sum() / want.float().abs().sum())
        print(f"magi2 reference artifact backward {name}: mean_rel={rel:.3e}")
        assert rel <= 1e-2, (name, rel)


@pytest.mark.parametrize("S", [300])
def test_reference_artifact_two_level_absmax_equals_the_fp32_absmax(tmp_path, S):
    """The same reference artifact ingested with its two-level absmax kept as
    stored (MX_FMT_NF4_DQ_KN, decoded by the GEMMs per K step) and decoded at
    load (MX_FMT_NF4_F32_KN): the same absmax arithmetic, so the dequantised
    weights, the forward and the backward (LoRA on every weight) agree bit for
    bit."""
    from mirai_amd import load_reference_magi2_artifact
    from mirai_amd import _native as nat
    from mirai_amd import quant

    H, E, d, f = 2, 4, 128, 192
    path, dense = _reference_artifact(tmp_path, H=H, E=E, d=d, f=f)
    layers = {}
    for two in (False, True):
        layer = Magi2GroupedExperts(num_heads=H, num_experts=E, quant_format="nf4")
        load_reference_magi2_artifact(path, {"blocks.3.moe": layer}, two_level=two)
        layers[two] = layer
    for key in ("W_gate", "W_up", "W_down"):
        pq = layers[True].experts.packed_weight(key)
        pf = layers[False].experts.packed_weight(key)
        assert pq.format_code() == nat.FMT_NF4_DQ_KN and pf.format_code() == nat.FMT_NF4_F32_KN
        assert torch.equal(quant.dequantize(pq), quant.dequantize(pf))
    _, x, _, _, probs, idx = _magi2_case(H=H, E=E, d=d, f=f, S=S, k=2, seed=14)
    g = torch.Generator().manual_seed(22)
    r = 16
    facs = {key: ((torch.randn(H * E, r, i_f, generator=g) * 0.05).to(torch.bfloat16),
                  (torch.randn(H * E, o_f, r, generator=g) * 0.05).to(torch.bfloat16))
            for key, (i_f, o_f) in {"W_gate": (d, f), "W_up": (d, f), "W_down": (f, d)}.items()}
    dy = torch.randn(x.shape, generator=g).to(torch.bfloat16)
    res = {}
    for two, layer in layers.items():
        with torch.no_grad():
            out = layer.execute(x.cuda(), probs.cuda(), idx.cuda())
        for key, (a, b) in facs.items():
            ad = layer.attach_expert_lora(tensor_name=key, adapter_name="t", rank=r, alpha=32.0)
            with torch.no_grad():
                ad.lora_a.copy_(a.cuda())
                ad.lora_b.copy_(b.cuda())
        xg = x.cuda().requires_grad_(True)
        pg = probs.cuda().requires_grad_(True)
        layer.execute(xg, pg, idx.cuda()).backward(dy.cuda())
        res[two] = [out, xg.grad, pg.grad] + [
            p.grad for k in facs for p in (layer.experts.expert_lora[k].lora_a,
                                           layer.experts.expert_lora[k].lora_b)]
    for a, b in zip(res[True], res[False]):
        assert torch.equal(a, b)
    ref = om.layer_forward(x, probs, idx, dense, E)
    print(f"magi2 two-level artifact forward: {assert_layer_close(res[True][0].cpu(), ref)}")
