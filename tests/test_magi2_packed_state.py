"""MAGI-2 packed-store persistence on the CPU: descriptor, validated restore and
the versioned safetensors artifact (the surface of
mirai/core/models/magi2_preview/quantized_experts.py:140-219 and
packed_experts.py:28-183; the payload is this build's packed layout).

No kernel runs here: the payload tensors are built with the layouts
``mirai_amd.quant.quantize`` produces and only moved in and out of modules.
The GPU round trip through real quantisation and the fused layer is in
tests/test_gpu_magi2.py."""

import json

import pytest
import torch

from mirai_amd import (
    Magi2GroupedExperts,
    Magi2PackedExpertStateError,
    Magi2QuantizedExpertError,
    load_magi2_packed_state,
    save_magi2_packed_state,
)

H, E, D_HEAD, D_EXPERT = 2, 3, 64, 128
G = H * E
# The reference layer's [G, in, out] shapes.
SHAPES = {"W_gate": (G, D_HEAD, D_EXPERT), "W_up": (G, D_HEAD, D_EXPERT),
          "W_down": (G, D_EXPERT, D_HEAD)}


def _payload(fmt: str, seed: int = 0) -> dict[str, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    out = {}
    for key, (groups, rows, cols) in SHAPES.items():
        o, i = cols, rows  # stored as [G, out, in]
        if fmt == "nf4":
            out[f"{key}_nf4"] = torch.randint(0, 256, (groups, o, i // 2), generator=g,
                                              dtype=torch.uint8)
            out[f"{key}_nf4_absmax"] = torch.rand((groups, o, i // 64), generator=g).to(torch.bfloat16)
        elif fmt == "int8":
            out[f"{key}_int8"] = torch.randint(-127, 128, (groups, o, i), generator=g,
                                               dtype=torch.int8)
            out[f"{key}_scale"] = torch.rand((groups, o), generator=g).to(torch.bfloat16)
        else:
            out[f"{key}_bf16"] = torch.randn((groups, o, i), generator=g).to(torch.bfloat16)
    return out


def _descriptor(fmt: str, payload: dict) -> dict:
    meta = {"format": fmt, "blocksize": 64}
    if fmt == "nf4":
        meta["absmax_dtype"] = "bfloat16"
    return {"num_groups": G, "blocksize": 64,
            "expert_shapes": {k: list(v) for k, v in SHAPES.items()},
            "expert_dtypes": {k: "bfloat16" for k in SHAPES},
            "packed_meta": meta, "buffers": sorted(payload)}


def _module(fmt: str = "nf4") -> Magi2GroupedExperts:
    return Magi2GroupedExperts(num_heads=H, num_experts=E, quant_format=fmt)


@pytest.mark.parametrize("fmt", ["nf4", "int8", "bf16"])
def test_restore_then_describe_round_trips(fmt):
    payload = _payload(fmt)
    desc = _descriptor(fmt, payload)
    m = _module(fmt)
    assert not m.is_fully_loaded()
    m.restore_packed_state(descriptor=desc, buffers=payload)
    assert m.is_fully_loaded()
    assert m.packed_state_descriptor() == desc
    for name, value in m.packed_buffers().items():
        assert torch.equal(value, payload[name])
    for key, shape in SHAPES.items():
        assert m.expert_weight_shape(key) == shape
        assert m.expert_weight_dtype(key) == torch.bfloat16
        # The kernels' view: [G, out, in].
        assert m.experts.expert_weight_shape(key) == (shape[0], shape[2], shape[1])
    assert m.payload_bytes() == sum(t.numel() * t.element_size() for t in payload.values())
    assert m.quantized_numel() == sum(a * b * c for a, b, c in SHAPES.values())


def test_incomplete_store_cannot_be_persisted():
    with pytest.raises(Magi2QuantizedExpertError, match="must be complete"):
        _module().packed_state_descriptor()


@pytest.mark.parametrize("edit,message", [
    (lambda d, b: d.update(num_groups=G + 1), "incompatible groups"),
    (lambda d, b: d.update(blocksize=32), "incompatible NF4 blocksize"),
    (lambda d, b: d.pop("expert_shapes"), "incomplete tensor metadata"),
    (lambda d, b: d["expert_dtypes"].pop("W_up"), "incomplete expert metadata"),
    (lambda d, b: d.pop("packed_meta"), "no NF4 metadata"),
    (lambda d, b: d["packed_meta"].update(format="int8"), "holds 'int8' weights"),
    (lambda d, b: d["expert_dtypes"].update(W_up="bfloat17"), "unknown dtype 'bfloat17'"),
    (lambda d, b: b.pop("W_down_nf4_absmax"), "buffer inventory does not match"),
    (lambda d, b: d["expert_shapes"].update(W_gate=[G, D_HEAD]), "gives W_gate the shape"),
])
def test_restore_rejects_mismatched_payloads(edit, message):
    payload = _payload("nf4")
    desc = _descriptor("nf4", payload)
    edit(desc, payload)
    with pytest.raises(Magi2QuantizedExpertError, match=message):
        _module().restore_packed_state(descriptor=desc, buffers=payload)


def test_restore_checks_each_buffer_layout():
    payload = _payload("nf4")
    desc = _descriptor("nf4", payload)
    payload["W_up_nf4"] = payload["W_up_nf4"][:, :, :-1].contiguous()
    with pytest.raises(Magi2QuantizedExpertError, match="W_up_nf4"):
        _module().restore_packed_state(descriptor=desc, buffers=payload)
    payload = _payload("nf4")
    payload["W_gate_nf4_absmax"] = payload["W_gate_nf4_absmax"].to(torch.float16)
    with pytest.raises(Magi2QuantizedExpertError, match="W_gate_nf4_absmax"):
        _module().restore_packed_state(descriptor=desc, buffers=payload)
    # An fp32 absmax (ingested bitsandbytes payloads) is a valid NF4 layout.
    payload = _payload("nf4")
    for key in SHAPES:
        payload[f"{key}_nf4_absmax"] = payload[f"{key}_nf4_absmax"].float()
    m = _module()
    m.restore_packed_state(descriptor=desc, buffers=payload)
    assert m.packed_state_descriptor()["packed_meta"]["absmax_dtype"] == "float32"


def _saved(tmp_path, fmt="nf4", metadata=None):
    layers = {}
    for i in range(2):
        payload = _payload(fmt, seed=i)
        m = _module(fmt)
        m.restore_packed_state(descriptor=_descriptor(fmt, payload), buffers=payload)
        layers[f"blocks.{i}.moe"] = m
    path = save_magi2_packed_state(tmp_path / "packed", layers, metadata=metadata)
    return path, layers


def test_artifact_round_trip(tmp_path):
    path, layers = _saved(tmp_path, metadata={"base": "magi2-test"})
    fresh = {name: _module() for name in layers}
    load_magi2_packed_state(path, fresh, expected_metadata={"base": "magi2-test"}, device="cpu")
    for name, layer in layers.items():
        assert fresh[name].packed_state_descriptor() == layer.packed_state_descriptor()
        for k, v in layer.packed_buffers().items():
            assert torch.equal(fresh[name].packed_buffers()[k], v)
    manifest = json.loads((path / "manifest.json").read_text())
    assert manifest["schema_version"] == 1 and set(manifest["layers"]) == set(layers)


def test_artifact_rejects_mismatches(tmp_path):
    path, layers = _saved(tmp_path, metadata={"base": "a"})
    with pytest.raises(FileExistsError):
        save_magi2_packed_state(path, layers)
    with pytest.raises(Magi2PackedExpertStateError, match="incompatible base"):
        load_magi2_packed_state(path, {n: _module() for n in layers},
                                expected_metadata={"base": "b"}, device="cpu")
    with pytest.raises(Magi2PackedExpertStateError, match="layer inventory"):
        load_magi2_packed_state(path, {"blocks.0.moe": _module()}, device="cpu")
    manifest_path = path / "manifest.json"
    manifest = json.loads(manifest_path.read_text())
    manifest["schema_version"] = 99
    manifest_path.write_text(json.dumps(manifest))
    with pytest.raises(Magi2PackedExpertStateError, match="unsupported schema"):
        load_magi2_packed_state(path, {n: _module() for n in layers}, device="cpu")
    manifest["schema_version"] = 1
    manifest["layers"]["blocks.1.moe"]["shard"] = "../escape.safetensors"
    manifest_path.write_text(json.dumps(manifest))
    with pytest.raises(Magi2PackedExpertStateError, match="invalid shard path"):
        load_magi2_packed_state(path, {n: _module() for n in layers}, device="cpu")
    with pytest.raises(FileNotFoundError):
        load_magi2_packed_state(tmp_path / "absent", {n: _module() for n in layers}, device="cpu")
