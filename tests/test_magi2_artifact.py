"""CPU checks of the reader of the reference's MAGI-2 NF4 expert artifacts
(manifest + safetensors shards, packed_experts.py:28-78): what it returns for
a well-formed artifact, and that it refuses what it cannot ingest. The GPU
ingestion and the layer parity are in tests/test_gpu_magi2.py."""

import json

import numpy as np
import pytest
import torch

from mirai_amd import read_reference_magi2_artifact
from mirai_amd.magi2 import Magi2QuantizedExpertError

from helpers import MAGI2_KEYS, bnb_group_payload, write_reference_magi2_artifact

TABLE = np.sort(np.concatenate([np.linspace(-1, 1, 255), [0.0]])).astype(np.float32)


def _layers(G=4, d=64, f=128, seed=0):
    rng = np.random.default_rng(seed)
    out = {}
    for name in ("blocks.0.moe", "blocks.1.moe"):
        weights = {}
        for key in MAGI2_KEYS:
            shape = (G, d, f) if key != "W_down" else (G, f, d)
            w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
            bufs, _ = bnb_group_payload(w, TABLE)
            weights[key] = (bufs, shape)
        out[name] = weights
    return out


def test_reader_returns_every_layer_buffer_and_shape(tmp_path):
    layers = _layers()
    write_reference_magi2_artifact(tmp_path, layers)
    got = read_reference_magi2_artifact(tmp_path)
    assert set(got) == set(layers)
    for name, weights in layers.items():
        for key, (bufs, shape) in weights.items():
            assert got[name]["shapes"][key] == shape
            assert got[name]["dtypes"][key] == torch.bfloat16
            for field, value in bufs.items():
                np.testing.assert_array_equal(got[name]["buffers"][f"{key}_{field}"].numpy(),
                                              value)


def test_reader_refuses_what_it_cannot_ingest(tmp_path):
    layers = _layers()
    with pytest.raises(Magi2QuantizedExpertError, match="manifest"):
        read_reference_magi2_artifact(tmp_path / "absent")
    write_reference_magi2_artifact(tmp_path / "v1", layers, schema=("mirai.magi2_preview.nf4_experts", 1))
    with pytest.raises(Magi2QuantizedExpertError, match="this reader takes"):
        read_reference_magi2_artifact(tmp_path / "v1")
    write_reference_magi2_artifact(tmp_path / "bs", layers, blocksize=128)
    with pytest.raises(Magi2QuantizedExpertError, match="64 / 256"):
        read_reference_magi2_artifact(tmp_path / "bs")
    # A shard path that leaves the artifact directory, and a missing shard.
    root = tmp_path / "ok"
    write_reference_magi2_artifact(root, layers)
    manifest = json.loads((root / "manifest.json").read_text())
    manifest["layers"]["blocks.0.moe"]["shard"] = "../escape.safetensors"
    (root / "manifest.json").write_text(json.dumps(manifest))
    with pytest.raises(Magi2QuantizedExpertError, match="not a file"):
        read_reference_magi2_artifact(root)
    # A shard without one of the six buffers of a weight.
    part = {"only": {k: v for k, v in _layers()["blocks.0.moe"].items()}}
    bufs, shape = part["only"]["W_up"]
    part["only"]["W_up"] = ({k: v for k, v in bufs.items() if k != "nf4_nabsmax"}, shape)
    write_reference_magi2_artifact(tmp_path / "miss", part)
    with pytest.raises(Magi2QuantizedExpertError, match="W_up_nf4_nabsmax"):
        read_reference_magi2_artifact(tmp_path / "miss")
