"""One-expert hosts of the reference's mixed-precision expert pool.

MixedPrecisionGroupedExperts (mirai/core/models/compressed_weights/execution/
mixed_precision.py:93-246, schema-v1 plans) gives every expert a
CompressedGroupedExperts of its own: num_experts=1,
expert_weight_access="active_dequant", the expert's own quant_format
(:189-202). Its dispatcher then calls, per expert, host.run_direct_routed on
the expert's token rows with unit scores and expert id 0. It weights the
result by the route scores and index_adds it into the output (:218-241).

The dispatcher is restated below in plain torch, the same code on both sides.
One side runs this package's hosts on the GPU. The other side runs the
oracle's one-expert layer over each expert's dequantised weights. The hosts
here mix NF4 and INT8 experts. Some experts get 0, 1 or a few rows; one
takes most of them.
"""

import numpy as np
import pytest
import torch

from mirai_amd import workloads as wl
from oracle import layer as olayer

from helpers import assert_layer_close, oracle_payload

pytestmark = pytest.mark.gpu


def _pool_forward(hosts, tokens, scores, idx):
    """The pool's forward (mixed_precision.py:205-246) over callables
    host(rows, ones, zeros) -> rows' expert outputs."""
    output = torch.zeros_like(tokens)
    for e, host in enumerate(hosts):
        positions = torch.nonzero(idx == e, as_tuple=False)
        if positions.numel() == 0:
            continue
        token_ids, slots = positions[:, 0], positions[:, 1]
        selected = tokens.index_select(0, token_ids)
        ones = torch.ones((selected.shape[0], 1), dtype=scores.dtype, device=scores.device)
        zeros = torch.zeros((selected.shape[0], 1), dtype=torch.long, device=idx.device)
        routed = host(selected, ones, zeros)
        weighted = routed * scores[token_ids, slots].unsqueeze(-1)
        output.index_add_(0, token_ids, weighted)
    return output


def test_one_expert_hosts_of_a_mixed_precision_pool():
    from mirai_amd import CompressedGroupedExperts

    E, T, k, d, f = 7, 300, 2, 256, 384
    formats = ["nf4", "int8", "nf4", "int8", "nf4", "int8", "nf4"]
    w = wl.Workload("mixed", 31, T, d, f, E, k, 16, 16.0, "nf4", torch.bfloat16)
    dense = wl.dense_weights(w)
    x = wl.tokens(w)
    # Skewed routes: expert 0 takes most rows, expert 6 none, expert 5 one.
    rng = np.random.default_rng(7)
    p = np.array([0.5, 0.15, 0.12, 0.1, 0.08, 0.05, 0.0])
    idx = np.stack([rng.choice(E, size=k, replace=False, p=p) for _ in range(T)])
    idx[idx == 5] = 4
    idx[0] = [5, 0]
    idx = torch.from_numpy(idx.astype(np.int64))
    s = torch.from_numpy(rng.random((T, k)).astype(np.float32) + 0.1)
    scores = (s / s.sum(dim=1, keepdim=True)).to(torch.bfloat16)
    assert int((idx == 6).sum()) == 0 and int((idx == 5).sum()) == 1

    gpu_hosts, oracle_hosts = [], []
    for e, fmt in enumerate(formats):
        host = CompressedGroupedExperts.from_empty(num_experts=1, expert_weight_access="active_dequant",
                                                   quant_format=fmt)
        weights = {}
        for key in ("w1", "w3", "w2"):
            one = dense[key][e:e + 1].contiguous()
            host.load_dense_weight(key, one.cuda())
            weights[key] = olayer.dense_weight(fmt, oracle_payload(fmt, one), tuple(one.shape),
                                               dtype=torch.bfloat16)
        gpu_hosts.append(host.run_direct_routed)
        oracle_hosts.append(lambda rows, ones, zeros, wts=weights:
                            olayer.layer_forward(rows, ones, zeros, wts, {}, 1))

    with torch.no_grad():
        out = _pool_forward(gpu_hosts, x.cuda(), scores.cuda(), idx.cuda())
    ref = _pool_forward(oracle_hosts, x, scores, idx)
    stats = assert_layer_close(out.cpu(), ref)
    print(f"mixed-precision pool of one-expert hosts: {stats}")
