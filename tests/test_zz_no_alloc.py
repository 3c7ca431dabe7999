"""GPU check of the allocation-free forward entry point mx_moe_forward_static
against mx_moe_forward_act with a caller workspace, through the C ABI: the
same kernels on the same inputs, so the outputs must be bit-identical. Two
calls in a row (the second smaller) share the static device scratch; a call
too large for it must fail cleanly before launching anything."""

import pytest
import torch

from mirai_amd import _native as nat
from mirai_amd import workloads as wl
from mirai_amd.fused import _lora_descriptors, _weight_descriptors, lora_rank
from oracle import routing as oroute

from helpers import build_module

pytestmark = pytest.mark.gpu


def _args(m, x, idx, scores, out):
    device = x.device
    (w1, w3, w2), packed = _weight_descriptors(m, device)
    lora, keep = _lora_descriptors(m, device)
    T, d = (int(v) for v in x.shape)
    f = int(packed[0].shape[1])
    common = (x.data_ptr(), idx.data_ptr(), scores.data_ptr(), nat.dtype_code(scores.dtype), T,
              int(idx.shape[1]), m.num_experts, d, f, nat.ACT_SILU, w1, w3, w2, lora[0], lora[1],
              lora[2], out.data_ptr(), nat.dtype_code(out.dtype))
    return common, keep, (T, int(idx.shape[1]), m.num_experts, d, f, lora_rank(m))


def _both(m, x, idx, scores):
    a = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    b = torch.empty_like(a)
    common, keep, sizes = _args(m, x, idx, scores, a)
    nat.call("mx_moe_forward_static", *common, nat.stream(x.device))
    common_b, keep_b, _ = _args(m, x, idx, scores, b)
    lib = nat.load_library()
    ws = nat.workspace(lib.mx_moe_workspace_size(*sizes), x.device)
    nat.call("mx_moe_forward_act", *common_b, None, None, None, None, None, ws.data_ptr(),
             nat.stream(x.device))
    torch.cuda.synchronize()
    del keep, keep_b
    return a, b


def test_static_scratch_forward_matches_the_workspace_forward():
    w = wl.Workload("noalloc", 12, 600, 256, 192, 8, 4, 16, 16.0, "nf4", torch.bfloat16)
    m = build_module(w, wl.dense_weights(w), wl.lora_factors(w))
    x = wl.tokens(w).cuda()
    idx_np, scores_np = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    idx = torch.from_numpy(idx_np).cuda()
    scores = torch.from_numpy(scores_np).cuda()
    for rows in (600, 150):  # the second call is smaller and reuses the array
        a, b = _both(m, x[:rows].contiguous(), idx[:rows].contiguous(),
                     scores[:rows].contiguous())
        assert torch.equal(a, b), rows
        assert torch.isfinite(a.float()).all()
    # Too large for the static array: refused before any launch.
    big = nat.STATIC_SCRATCH_BYTES // (2 * (256 + 192 + 96)) + 1
    lib = nat.load_library()
    assert lib.mx_moe_workspace_size(big, 1, 8, 256, 192, 16) > nat.STATIC_SCRATCH_BYTES
    xb = torch.empty((big, 256), dtype=torch.bfloat16, device="cuda")
    ib = torch.zeros((big, 1), dtype=torch.int64, device="cuda")
    sb = torch.ones((big, 1), dtype=torch.float32, device="cuda")
    out = torch.empty_like(xb)
    common, keep, _ = _args(m, xb, ib, sb, out)
    with pytest.raises(ValueError, match="static"):
        nat.call("mx_moe_forward_static", *common, nat.stream(xb.device))
    del keep


def test_static_forward_allocates_nothing_and_replays_in_a_graph():
    """After one warm-up call (which resolves the device's scratch address),
    the static forward allocates no device memory and can be captured into a
    HIP graph; every replay, with eager work and synchronisation between the
    replays, reproduces the workspace forward bit for bit."""
    w = wl.Workload("noalloc_graph", 13, 300, 256, 192, 8, 4, 16, 16.0, "nf4", torch.bfloat16)
    m = build_module(w, wl.dense_weights(w), wl.lora_factors(w))
    x = wl.tokens(w).cuda()
    idx_np, scores_np = oroute.route_topk(wl.router_logits(w).numpy(), w.top_k)
    idx = torch.from_numpy(idx_np).cuda()
    scores = torch.from_numpy(scores_np).cuda()
    _, want = _both(m, x, idx, scores)  # also the warm-up of the static entry point
    out = torch.empty_like(want)
    common, keep, _ = _args(m, x, idx, scores, out)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    nat.call("mx_moe_forward_static", *common, nat.stream(x.device))
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    assert torch.equal(out, want)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out.zero_()
        with torch.cuda.graph(graph, stream=side):
            nat.call("mx_moe_forward_static", *common, nat.stream(x.device))
    torch.cuda.current_stream().wait_stream(side)
    for i in range(3):
        out.fill_(float(i + 1))  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), i
    del graph, keep
