"""The inference step (routing + fused layer) captured as one HIP graph:
every replay equals the eager result, with eager work and synchronisations
between the replays, and the graph keeps working after other launches."""

import pytest
import torch

from mirai_amd import route_topk
from mirai_amd import workloads as wl

from helpers import build_module

pytestmark = pytest.mark.gpu


def test_captured_forward_replays_match_eager():
    w = wl.Workload("graph_nf4", 21, 700, 256, 192, 16, 4, 16, 16.0, "nf4", torch.bfloat16)
    m = build_module(w, wl.dense_weights(w), wl.lora_factors(w), access="fused_kernel")
    x = wl.tokens(w).cuda()
    logits = wl.router_logits(w).cuda()
    state = {}

    def forward():
        with torch.no_grad():
            idx, scores = route_topk(logits, w.top_k, renorm="clamp", score_dtype=torch.bfloat16)
            state["out"] = m.run_direct_routed(x, scores, idx)

    forward()
    torch.cuda.synchronize()
    eager = state["out"].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        forward()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        forward()
    captured = state["out"]
    other = wl.tokens(wl.Workload("graph_other", 22, 300, 256, 192, 16, 4, 16, 16.0, "nf4",
                                  torch.bfloat16)).cuda()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {i}"
        # eager work between replays: a different routed batch through the same module
        with torch.no_grad():
            idx = torch.randint(0, 16, (300, 4), device="cuda")
            sc = torch.rand(300, 4, device="cuda")
            m.run_direct_routed(other, sc, idx)
        torch.cuda.synchronize()
