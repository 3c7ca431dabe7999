"""Host-side behaviour of the drop-in module (CPU only): argument validation
and error types of CompressedGroupedExperts, LoRA adapter state, policy
normalisation, and that the product path refuses to run without the GPU
library instead of falling back to a CPU path.

Error types and messages follow
mirai/core/models/compressed_weights/execution/experts.py:189-196, 544-558,
756-769, 1662-1666 and 1755-1769.
"""

import pytest
import torch

from mirai_amd._native import ROUTE_DROPPED

from mirai_amd import CompressedGroupedExperts, route_topk
from mirai_amd import _native as nat
from mirai_amd import quant
from mirai_amd.lora import ActiveExpertLoRA, lora_scale
from mirai_amd.specs import ExpertMLPExecutionSpec, normalize_expert_weight_access_policy


def _module(**kw):
    kw.setdefault("num_experts", 4)
    kw.setdefault("expert_weight_access", "chunked_dequant")
    kw.setdefault("expert_dequant_chunk_size", 2)
    kw.setdefault("quant_format", "nf4")
    return CompressedGroupedExperts.from_empty(**kw)


def test_from_empty_validation():
    with pytest.raises(ValueError):
        _module(num_experts=0)
    with pytest.raises(ValueError):
        _module(num_experts=8193)  # the plan takes up to 8192 (flattened MAGI-2 groups)
    with pytest.raises(ValueError):
        _module(nf4_blocksize=128)
    with pytest.raises(ValueError):
        _module(quant_format="fp8")
    with pytest.raises(TypeError):
        _module(execution_spec=object())


def test_access_policy_rules():
    m = _module(expert_weight_access="full_dequant", expert_dequant_chunk_size=0)
    assert not m.prefers_for_loop()
    with pytest.raises(ValueError, match="expert_dequant_chunk_size > 0"):
        m.set_expert_weight_access_policy(expert_weight_access="chunked_dequant",
                                          expert_dequant_chunk_size=0)
    m.set_expert_weight_access_policy(expert_weight_access="chunked_dequant",
                                      expert_dequant_chunk_size=8)
    assert m.prefers_for_loop() and m.expert_dequant_chunk_size == 8
    m.set_expert_weight_access_policy(expert_weight_access="active_dequant")
    assert m.prefers_for_loop()
    # A module built with a chunked policy and no chunk size gets the default.
    assert _module(expert_dequant_chunk_size=0).expert_dequant_chunk_size > 0
    assert normalize_expert_weight_access_policy("auto") == "auto"
    with pytest.raises(ValueError):
        normalize_expert_weight_access_policy("nonsense")


def test_run_direct_routed_validation_order():
    tokens = torch.zeros(6, 64)
    scores = torch.zeros(6, 2)
    idx = torch.zeros(6, 2, dtype=torch.long)
    full = _module(expert_weight_access="full_dequant", expert_dequant_chunk_size=0)
    with pytest.raises(RuntimeError, match="requires active_dequant"):
        full.run_direct_routed(tokens, scores, idx)
    m = _module()
    with pytest.raises(ValueError, match="matching"):
        m.run_direct_routed(tokens, scores[:, :1], idx)
    with pytest.raises(ValueError, match="token count"):
        m.run_direct_routed(tokens[:5], scores, idx)
    with pytest.raises(RuntimeError, match="missing weights"):
        m.run_direct_routed(tokens, scores, idx)
    with pytest.raises(RuntimeError, match="missing weights"):
        m.run_for_loop(tokens, torch.tensor([6, 0, 0, 0]))


def test_attach_lora_validation():
    m = _module()
    with pytest.raises(ValueError, match="Unknown grouped expert LoRA tensor"):
        m.attach_expert_lora(tensor_name="w9", adapter_name="a", rank=8, alpha=16)
    with pytest.raises(AttributeError):
        m.attach_expert_lora(tensor_name="w1", adapter_name="a", rank=8, alpha=16)  # not loaded


def test_quantisation_needs_the_gpu_and_fails_loudly():
    m = _module()
    with pytest.raises(nat.NativeLibraryError):
        m.load_dense_weight("w1", torch.zeros(4, 128, 64))
    with pytest.raises(ValueError):
        quant.quantize(torch.zeros(4, 128, 96), "nf4")  # in_features % 64
    with pytest.raises(ValueError):
        m.load_dense_weight("w7", torch.zeros(4, 128, 64))


def test_routing_refuses_cpu_tensors():
    with pytest.raises((nat.NativeLibraryError, ValueError)):
        route_topk(torch.randn(8, 16), 2)


def test_active_expert_lora_state():
    ad = ActiveExpertLoRA(adapter_name="a", num_experts=3, in_features=64, out_features=32,
                          rank=12, alpha=24.0)
    assert ad.lora_a.shape == (3, 12, 64) and ad.lora_b.shape == (3, 32, 12)
    assert torch.count_nonzero(ad.lora_b) == 0 and torch.count_nonzero(ad.lora_a) > 0
    assert ad.scale() == pytest.approx(2.0)
    assert ad.padded_rank() == 16
    a, b = ad.kernel_factors(torch.device("cpu"))
    assert a.dtype == torch.bfloat16 and a.shape == (3, 16, 64) and b.shape == (3, 32, 16)
    assert torch.count_nonzero(a[:, 12:]) == 0 and torch.count_nonzero(b[:, :, 12:]) == 0
    assert torch.equal(a[:, :12], ad.lora_a.detach().to(torch.bfloat16))
    rs = ActiveExpertLoRA(adapter_name="r", num_experts=1, in_features=64, out_features=64,
                          rank=16, alpha=16.0, use_rslora=True)
    assert rs.scale() == pytest.approx(4.0)
    wide = ActiveExpertLoRA(adapter_name="w", num_experts=2, in_features=64, out_features=32,
                            rank=100, alpha=1.0)
    assert wide.padded_rank() == 104  # ranks above 32 run as extra 32-wide K chunks
    assert wide.kernel_factors(torch.device("cpu"))[0].shape == (2, 104, 64)
    with pytest.raises(ValueError):
        ActiveExpertLoRA(adapter_name="x", num_experts=1, in_features=64, out_features=64,
                         rank=260, alpha=1.0)
    with pytest.raises(ValueError):
        lora_scale(1.0, 0, use_rslora=False)


def test_execution_spec_surface():
    spec = _module().expert_mlp_spec
    assert isinstance(spec, ExpertMLPExecutionSpec)
    assert spec.tensor_for_role("gate") == "w1"
    assert spec.tensor_for_role("up") == "w3"
    assert spec.tensor_for_role("down") == "w2"


# A spec class that is not this package's: the reference's own
# ExpertMLPExecutionSpec (mirai/core/moe/runtime/specs.py:111-231) reaches the
# module this way from provider code (prepare.py:137-151,
# lingbot_video/pipeline.py:1678).
from dataclasses import dataclass as _dataclass


@_dataclass(frozen=True)
class _ForeignRole:
    role: str
    tensor_name: str


@_dataclass(frozen=True)
class _ForeignSpec:
    projections: tuple
    activation: str = "silu"
    combiner: str = "gated_product"


_FOREIGN = _ForeignSpec((_ForeignRole("gate", "gate_proj"), _ForeignRole("up", "up_proj"),
                         _ForeignRole("down", "down_proj")))


def test_foreign_spec_objects_are_accepted_by_fields():
    m = _module(execution_spec=_FOREIGN)
    # The provider's object is kept as given; the module works from its fields.
    assert m.mirai_expert_mlp_spec is _FOREIGN and m.expert_mlp_spec is _FOREIGN
    assert m.projection_for_role("gate") == "gate_proj"
    assert m.projection_for_role("down") == "down_proj"
    with pytest.raises(ValueError, match="Unknown compressed_weights grouped expert tensor"):
        m.load_dense_weight("w1", torch.zeros(4, 64, 64))
    assert not m.is_fully_loaded()
    # Field validation still applies to foreign specs.
    with pytest.raises(ValueError):
        _module(execution_spec=_ForeignSpec(_FOREIGN.projections, activation="tanh"))
    with pytest.raises(ValueError):
        _module(execution_spec=_ForeignSpec(_FOREIGN.projections[:2]))
    with pytest.raises(TypeError):
        _module(execution_spec=_ForeignSpec(projections=(object(),)))


def test_foreign_spec_through_the_base_module_constructor():
    class Base(torch.nn.Module):
        num_experts = 4
        mirai_expert_mlp_spec = _FOREIGN

        def __init__(self):
            super().__init__()
            self.gate_proj = torch.zeros(4, 64, 64)
            self.up_proj = torch.zeros(4, 64, 64)
            self.down_proj = torch.zeros(4, 64, 64)

    # Construction reads the foreign spec and goes on to quantise its tensors,
    # which needs the GPU library: without a GPU the error is the library's,
    # not a TypeError about the spec class.
    if torch.cuda.is_available():
        m = CompressedGroupedExperts(Base(), quant_format="nf4",
                                     expert_weight_access="chunked_dequant",
                                     expert_dequant_chunk_size=2)
        assert m.is_fully_loaded() and m.expert_mlp_spec is _FOREIGN
    else:
        with pytest.raises(nat.NativeLibraryError):
            CompressedGroupedExperts(Base(), quant_format="nf4",
                                     expert_weight_access="chunked_dequant",
                                     expert_dequant_chunk_size=2)


def test_token_chunk_policy_surface():
    from mirai_amd.chunking import MoETokenChunkPolicy

    with pytest.raises(ValueError):
        MoETokenChunkPolicy(-1)
    p = MoETokenChunkPolicy(100)
    assert p.enabled and not MoETokenChunkPolicy(0).enabled
    assert [p.chunk_count(n) for n in (0, 1, 100, 101, 250)] == [1, 1, 1, 2, 3]
    calls = []

    def runner(t, s, i, off):
        calls.append((int(t.shape[0]), off))
        return t * 2

    x = torch.arange(250.0).view(250, 1)
    s, i = torch.ones(250, 2), torch.zeros(250, 2, dtype=torch.long)
    with torch.no_grad():
        out = p.execute(x, s, i, runner=runner, training=True)
    assert calls == [(100, 0), (100, 100), (50, 200)] and torch.equal(out, x * 2)
    calls.clear()
    p.execute(x, s, i, runner=runner, training=False)  # eval: one call
    assert calls == [(250, 0)]
    with pytest.raises(ValueError):
        p.execute(x, s[:, :1], i, runner=runner, training=True)


def test_block_builds_the_reference_submodules():
    from mirai_amd.block import FusedSparseMoeBlock

    blk = FusedSparseMoeBlock(128, 512, 8, 2, 64, "sigmoid", True, None, None, 1.0, 1)
    assert blk.router.weight.shape == (8, 128) and blk.router.weight.dtype == torch.float32
    assert blk.router.e_score_correction_bias.shape == (8,)
    assert blk.shared_experts.gate_proj.weight.shape == (64, 128)
    assert blk.shared_experts.down_proj.weight.shape == (128, 64)
    assert blk.experts.num_experts == 8
    assert FusedSparseMoeBlock(128, 512, 8, 2, 64, "softmax", True, None, None, 1.0,
                               0).shared_experts is None
    with pytest.raises((nat.NativeLibraryError, ValueError)):
        blk(torch.zeros(1, 4, 128))


def test_lora_scale_follows_alpha_buffer_updates():
    ad = ActiveExpertLoRA(adapter_name="a", num_experts=2, in_features=64, out_features=32,
                          rank=8, alpha=16.0)
    assert ad.scale() == pytest.approx(2.0)
    with torch.no_grad():
        ad.lora_alpha.fill_(32.0)  # in place: the cached value must not go stale
    assert ad.scale() == pytest.approx(4.0)
    ad.load_state_dict({**ad.state_dict(), "lora_alpha": torch.tensor(8.0)})
    assert ad.scale() == pytest.approx(1.0)


def _coalesce_brute(scores, idx, aliases):
    """coalesce_alias_routes (storage/aliases.py:156-199) one slot at a time,
    then every slot whose coalesced score is zero left out of the dispatch
    (experts.py:2361-2367: only nonzero scores are routed with aliases)."""
    T, k = idx.shape
    phys = torch.tensor([[aliases[int(idx[t, j])] for j in range(k)] for t in range(T)])
    out = torch.zeros_like(scores)
    for t in range(T):
        for j in range(k):
            first = min(i for i in range(k) if phys[t, i] == phys[t, j])
            out[t, first] += scores[t, j]
    for t in range(T):
        for j in range(k):
            if float(out[t, j]) == 0.0:
                phys[t, j] = ROUTE_DROPPED
    return out, phys


def test_logical_alias_coalescing_matches_slot_by_slot_rule():
    m = _module(num_experts=4)
    aliases = (0, 1, 2, 3, 1, 2, 0, 3, 2)
    m.configure_logical_expert_aliases(aliases)
    assert m.has_logical_expert_aliases() and m.logical_num_experts == 9
    assert m.prototype_logical_ids == (0, 1, 2, 3)
    g = torch.Generator().manual_seed(4)
    idx = torch.stack([torch.randperm(9, generator=g)[:4] for _ in range(200)])
    scores = torch.rand(200, 4, generator=g, dtype=torch.float64).float()
    got_s, got_p = m._coalesce_logical_routes(scores, idx)
    want_s, want_p = _coalesce_brute(scores, idx, aliases)
    assert torch.equal(got_p, want_p)
    torch.testing.assert_close(got_s, want_s, rtol=0, atol=1e-7)
    # At least one token must have had two slots on one physical expert; the
    # later slots are dropped, not routed with score 0.
    assert bool((got_s == 0).any())
    assert bool((got_p[got_s == 0] == ROUTE_DROPPED).all())
    # A route the router itself scored zero is dropped too.
    zs = scores.clone()
    zs[3, :] = 0.0
    _, zp = m._coalesce_logical_routes(zs, idx)
    assert bool((zp[3] == ROUTE_DROPPED).all())
    # Out-of-range logical ids become invalid physical ids (reported by the plan).
    bad = idx.clone()
    bad[5, 1] = 9
    bad[7, 0] = -2
    _, p = m._coalesce_logical_routes(scores, bad)
    assert int(p[5, 1]) == -1 and int(p[7, 0]) == -1
    # Gradients reach the scores through the coalescing.
    sg = scores.clone().requires_grad_(True)
    out, _ = m._coalesce_logical_routes(sg, idx)
    out.sum().backward()
    assert torch.equal(sg.grad, torch.ones_like(scores))


def test_configure_logical_expert_aliases_validation():
    m = _module(num_experts=4)
    with pytest.raises(ValueError, match="more logical than physical"):
        m.configure_logical_expert_aliases((0, 1, 2, 3))
    with pytest.raises(ValueError, match="invalid ids"):
        m.configure_logical_expert_aliases((0, 1, 2, 3, 4))
    with pytest.raises(ValueError, match="does not reference"):
        m.configure_logical_expert_aliases((0, 1, 2, 2, 1))
    with pytest.raises(ValueError, match="corresponding physical id"):
        m.configure_logical_expert_aliases((0, 1, 2, 3, 1), prototype_logical_ids=(0, 4, 2, 1))
    assert not m.has_logical_expert_aliases()


def test_route_check_modes():
    assert nat.route_check_mode() in nat.ROUTE_CHECK_MODES
    with pytest.raises(ValueError):
        nat.set_route_check("loud")
    assert issubclass(nat.RouteIndexError, ValueError)
    nat.check_route_errors()  # nothing pending: returns
