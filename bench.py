#!/usr/bin/env python3
"""Benchmark of the MI355X routed expert layer (one GPU).

A step is one pass of the hot path over one batch: fp32 router logits in ->
softmax top-k routing -> dispatch plan -> gathered gate/up grouped GEMM (NF4
decode, LoRA, SwiGLU) -> down grouped GEMM (LoRA) -> gate-weighted combine ->
[T, d] bf16 out. Inputs are seeded synthetic tensors already resident in HBM
when the timed region starts. Default workload: the C2 geometry (NF4, E=64,
top-4, d=2048, ffn=1408, LoRA r=16) at T=32768 tokens.

Prints one JSON line. ``value`` is routed tokens/s (T*k / step time).
``roofline`` describes the dominant kernel (the gate/up grouped GEMM) from HIP
events recorded on the library's stream around that kernel; ``cpu_baseline``
times the oracle's restatement of the reference CPU expert path on a bounded
token sample on the host cores.

The headline's step time is the mean of exactly ``--steps`` back-to-back
steps (synchronised before and after); ``median_ms`` / ``p95_ms`` / ``min_ms``
come from events recorded between those steps on the same stream. The line
also nests one record per benchmark configuration (``configs``: C1-C5 at their
own shapes; ``--no-configs`` skips them) with the same timing summary, TFLOP/s,
the fraction of the bf16 MFMA peak and of the roofline bound
min(P_mfma, AI * BW_hbm) on algorithmic bytes, and the HBM rate of those bytes.

``--config c5`` (adapter training) times forward + backward per step: the
forward keeps its activations, the backward produces d tokens, d scores and the
LoRA factor gradients from dY ~ N(0, 1); forward and backward are also timed
apart, and the backward's stages are reported next to the forward's.

``--path`` measures the paths next to the layer on the same geometry (one JSON
line each, not the headline): ``router`` (the fused router front end, tokens ->
routes, LingBot's sigmoid router with correction bias), ``block`` (LingBot's
sparse-MoE block: fused router, routed layer, and a shared expert of the same
width overlapped on a side stream), ``expert_choice`` (the same experts under
expert-choice routes with capacity T * k / E).
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
STAGES = ("plan", "lora_down_gate_up", "gate_up_gemm", "lora_down_down", "down_gemm", "combine")
BACK_STAGES = ("plan_and_combine_bwd", "lora_dz_down", "dh_gemm",
               "lora_grads_swiglu_bwd_and_lora_dz_gate_up", "dx_gemm", "dx_sum")


def _parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="target",
                    help="workload key: target (default), c2, c3, c4")
    ap.add_argument("--weights", choices=("nf4", "int8", "bf16"), default=None,
                    help="override the workload's frozen-weight format")
    ap.add_argument("--tokens", type=int, default=None, help="override the token count")
    ap.add_argument("--lora-rank", type=int, default=None,
                    help="override the workload's LoRA rank (0: no adapters; alpha = 2 * rank)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="approximate CPU time budget of the baseline sample")
    ap.add_argument("--graph", action="store_true",
                    help="inference configs: also replay the step as one HIP graph and report "
                         "that time (the graph's output is checked against the eager step)")
    ap.add_argument("--path", choices=("layer", "router", "block", "expert_choice"),
                    default="layer", help="the path to time (layer: the headline)")
    ap.add_argument("--settle-seconds", type=float, default=1.0,
                    help="untimed steps for about this long after setup, before the warmup "
                         "steps (clocks and power state settle)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the nested per-configuration records (C1-C5)")
    ap.add_argument("--config-steps", type=int, default=30,
                    help="timed steps of each nested configuration record")
    ap.add_argument("--config-warmup", type=int, default=5)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the run, copy this many MiB device-to-device once: a kernel "
                         "of known traffic that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return ap.parse_args()


def _build_module(w, device):
    import torch

    from mirai_amd import CompressedGroupedExperts
    from mirai_amd import workloads as wl

    m = CompressedGroupedExperts.from_empty(num_experts=w.experts, quant_format=w.fmt,
                                            expert_weight_access="fused_kernel",
                                            expert_dequant_chunk_size=16)
    dense = wl.dense_weights(w, device=device)
    for key in ("w1", "w3", "w2"):
        m.load_dense_weight(key, dense[key])
    del dense
    factors = wl.lora_factors(w, device=device) if w.rank > 0 else {}
    for key, (a, b) in factors.items():
        ad = m.attach_expert_lora(tensor_name=key, adapter_name="bench", rank=w.rank,
                                  alpha=w.alpha)
        with torch.no_grad():
            ad.lora_a.copy_(a)
            ad.lora_b.copy_(b)
    torch.cuda.synchronize()
    return m


def _stage_times(step, n, device, names=STAGES):
    """Average duration (ms) of each layer stage, from events on the library stream.

    The library records the seven events at its stage boundaries on every
    forward / backward call; with both in one step the backward's records win.
    """
    import ctypes

    import torch

    from mirai_amd import _native as nat

    events = [torch.cuda.Event(enable_timing=True) for _ in range(7)]
    for ev in events:
        ev.record()  # materialise the underlying hipEvent_t
    torch.cuda.synchronize()
    handles = (ctypes.c_void_p * 7)(*[ev.cuda_event for ev in events])
    lib = nat.load_library()
    sums = [0.0] * 6
    try:
        nat.call("mx_set_stage_events", handles, 7)
        for _ in range(n):
            step()
            torch.cuda.synchronize()
            for i in range(6):
                sums[i] += events[i].elapsed_time(events[i + 1])
    finally:
        lib.mx_set_stage_events(None, 0)
    return {name: sums[i] / n for i, name in enumerate(names)}


def _profiled_traffic(kernel: str, workload: str):
    """HBM bytes per dispatch of `kernel` on `workload` from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summaries (calibrated against a copy of
    known size), or None when that pair was not profiled."""
    pat = re.compile(r"^traffic_bytes_per_dispatch:\s*(\S+)\s+(\S+)\s*=\s*(\d+)\s*$")
    for path in sorted((ROOT / "profiles").glob("*.md")):
        for line in path.read_text().splitlines():
            m = pat.match(line.strip())
            if m and m.group(1) == kernel and m.group(2) == workload:
                return int(m.group(3))
    return None


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_baseline(w, module, logits_cpu, tokens_cpu, budget_s):
    """Reference-style CPU expert path (oracle restatement) on a token sample.

    Per call: softmax top-k routing, dequantisation of every projection from
    the packed format (the reference re-dequantises per call), per-expert
    gather + bf16 matmuls + LoRA + SwiGLU, fp32 index_add combine.
    """
    import numpy as np
    import torch

    from mirai_amd import workloads as wl
    from oracle import layer as olayer
    from oracle import routing as oroute

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    payloads = {}
    for key in ("w1", "w3", "w2"):
        p = module.packed_weight(key)
        if p.fmt == "nf4":
            payloads[key] = (p.data.cpu().numpy(), p.scale.cpu().view(torch.int16).numpy()
                             .view(np.uint16))
        elif p.fmt == "int8":
            payloads[key] = (p.data.cpu().numpy(), p.scale.cpu().view(torch.int16).numpy()
                             .view(np.uint16))
        elif p.fmt == "fp32":  # bf16 planes -> the fp32 weight (hi + lo)
            from mirai_amd import quant
            payloads[key] = quant.dequantize(p, dtype=torch.float32).cpu()
        else:
            payloads[key] = p.data.cpu()
    shapes = {k: module.packed_weight(k).shape for k in payloads}
    loras = {}
    for key in ("w1", "w3", "w2"):
        ad = module.expert_lora[key]
        loras[key] = (ad.lora_a.detach().cpu(), ad.lora_b.detach().cpu(), ad.scale())

    dy_cpu = wl.upstream_grad(w) if w.backward else None

    def run(n_tok):
        lg = logits_cpu[:n_tok].numpy()
        idx, scores = oroute.route_topk(lg, w.top_k)
        weights = {k: olayer.dense_weight(w.fmt, payloads[k], shapes[k]) for k in payloads}
        if not w.backward:
            with torch.no_grad():
                olayer.layer_forward(tokens_cpu[:n_tok], torch.from_numpy(scores).to(w.dtype),
                                     torch.from_numpy(idx), weights, loras, w.experts)
            return
        x = tokens_cpu[:n_tok].clone().requires_grad_(True)
        sc = torch.from_numpy(scores).requires_grad_(True)
        lr = {k: (a.clone().requires_grad_(True), b.clone().requires_grad_(True), s)
              for k, (a, b, s) in loras.items()}
        out = olayer.layer_forward(x, sc, torch.from_numpy(idx), weights, lr, w.experts)
        out.backward(dy_cpu[:n_tok])

    n_tok = min(256, w.tokens)
    t0 = time.perf_counter()
    run(n_tok)  # warmup + probe
    probe = time.perf_counter() - t0
    # Scale the sample so that ~3 timed calls fit the budget.
    target = max(1.0, budget_s / 3.0)
    if probe < target:
        n_tok = int(min(w.tokens, n_tok * target / max(probe, 1e-3)))
        n_tok = max(64, n_tok // 64 * 64)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run(n_tok)
        times.append(time.perf_counter() - t0)
    sec = statistics.median(times)
    return {
        "value": n_tok * w.top_k / sec,
        "unit": "routed tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{n_tok} of {w.tokens} tokens (x top-{w.top_k} routes), same weights and "
                   f"LoRA; median of 3 calls incl. per-call dequantisation"
                   f"{' and the autograd backward' if w.backward else ''}; torch CPU bf16, "
                   f"{threads} threads on {_cpu_model()}"),
        "ms_per_call": sec * 1e3,
    }


def _timed(fn, steps, warmup):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def _bench_path(args, w, device) -> dict:
    """One JSON record for a path next to the layer (see the module docstring)."""
    import torch

    from mirai_amd import fused_router_forward, router_weight_planes
    from mirai_amd import workloads as wl

    T, d, E, k = w.tokens, w.hidden, w.experts, w.top_k
    g = torch.Generator(device=device).manual_seed(7)
    x = wl.tokens(w).to(device)
    router_w = torch.randn(E, d, generator=g, device=device) * 0.02
    bias = torch.randn(E, generator=g, device=device) * 0.01
    base = {"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) tokens, N(0,0.02) weights)"}
    if args.path == "router":
        planes = router_weight_planes(router_w)

        def fused():
            fused_router_forward(x, planes, E, k, score_func="sigmoid", expert_bias=bias,
                                 return_logits=False, return_scores=False)

        ms = _timed(fused, args.steps, args.warmup)

        def unfused():  # torch's fp32 GEMM, then the routing kernel
            from mirai_amd import route_topk
            route_topk(torch.nn.functional.linear(x.float(), router_w), k, renorm="eps")

        ms_unfused = _timed(unfused, args.steps, args.warmup)
        EP = 32 * -(-E // 32)
        traffic = T * d * 2 + 3 * EP * d * 2 + T * k * (8 + 2)
        gbs = traffic / (ms * 1e-3) / 1e9
        return {**base, "metric": "router tokens/s (fused router front end), 1 GPU",
                "value": T / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms,
                "config": {"workload": f"router_{w.name}", "tokens": T, "hidden": d,
                           "experts": E, "top_k": k, "score_func": "sigmoid"},
                "unfused_torch_gemm_plus_route_ms": ms_unfused,
                "roofline": {"kernel": "router_fused_kernel", "bound": "hbm", "achieved": gbs,
                             "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": gbs / PEAK_HBM_GBS,
                             "traffic": None}}
    module = _build_module(w, device)
    if args.path == "block":
        from mirai_amd.block import FusedSparseMoeBlock

        blk = FusedSparseMoeBlock(d, 4 * d, E, k, w.ffn, "sigmoid", True, None, None, 1.0, 1,
                                  quant_format=w.fmt).to(device)
        blk.experts = module
        with torch.no_grad():
            blk.router.weight.copy_(router_w)
            blk.router.e_score_correction_bias.copy_(bias)
        blk.shared_experts.to(torch.bfloat16).requires_grad_(False)
        for lin in (blk.shared_experts.gate_proj, blk.shared_experts.up_proj,
                    blk.shared_experts.down_proj):
            with torch.no_grad():
                lin.weight.copy_(torch.randn(lin.weight.shape, generator=g, device=device) * 0.02)
        hs = x.view(1, T, d)
        with torch.no_grad():
            ms = _timed(lambda: blk(hs), args.steps, args.warmup)
            idx, top, _, _, _ = blk.router(x)
            ms_routed = _timed(lambda: module.run_direct_routed(x, top, idx), args.steps,
                               args.warmup)
            ms_shared = _timed(lambda: blk.shared_experts(x), args.steps, args.warmup)
            ms_router = _timed(lambda: blk.router(x), args.steps, args.warmup)
        flops = w.flops() + 2 * T * 3 * d * w.ffn + 2 * T * d * E  # routed + shared + router
        return {**base, "metric": "tokens/s (LingBot sparse-MoE block: router + routed NF4 "
                "experts + shared expert), 1 GPU",
                "value": T / (ms * 1e-3), "unit": "tokens/s", "ms_per_step": ms,
                "config": {"workload": f"block_{w.name}", "tokens": T, "hidden": d,
                           "experts": E, "top_k": k, "ffn": w.ffn, "shared_ffn": w.ffn,
                           "weights": w.fmt, "lora_rank": w.rank},
                "tflops": flops / (ms * 1e-3) / 1e12,
                "parts_ms": {"router": ms_router, "routed_layer": ms_routed,
                             "shared_expert": ms_shared,
                             "sum": ms_router + ms_routed + ms_shared}}
    # expert choice: capacity T * k / E per expert, one sample
    C = T * k // E
    gi = torch.Generator().manual_seed(11)
    idx = torch.stack([torch.randperm(T, generator=gi)[:C] for _ in range(E)]).view(1, E, C)
    scores = torch.rand(1, E, C, generator=gi)
    idx, scores = idx.to(device), scores.to(device)
    with torch.no_grad():
        ms = _timed(lambda: module.run_expert_choice_routed(x, scores, idx, tokens_per_sample=T),
                    args.steps, args.warmup)
    R = E * C
    flops = 2 * R * 3 * d * w.ffn + 2 * R * w.rank * 3 * (d + w.ffn)
    return {**base, "metric": "routed slots/s (expert-choice routes, NF4 experts + LoRA), 1 GPU",
            "value": R / (ms * 1e-3), "unit": "routed slots/s", "ms_per_step": ms,
            "config": {"workload": f"expert_choice_{w.name}", "tokens": T, "hidden": d,
                       "experts": E, "capacity": C, "ffn": w.ffn, "weights": w.fmt,
                       "lora_rank": w.rank},
            "tflops": flops / (ms * 1e-3) / 1e12,
            "pct_bf16_peak": 100.0 * flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS}


def _settle(fn, seconds):
    """Untimed steps for about `seconds` before a measurement: the GPU's clocks
    and power state take a few hundred steps to settle after setup (a run
    without this showed a 24 ms step and some 15 slow steps after it)."""
    import torch

    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(5):
            fn()
        torch.cuda.synchronize()


def _step_times(fn, steps, warmup):
    """Mean ms per step over exactly `steps` back-to-back steps (synchronised on
    both sides), plus each step's own duration from an event recorded between
    steps on the same stream (no synchronisation inside the timed region).
    Python's garbage collector is off while the steps are issued."""
    import gc

    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    events = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    gc_was_on = gc.isenabled()
    gc.disable()
    try:
        events[0].record()
        for i in range(steps):
            fn()
            events[i + 1].record()
        torch.cuda.synchronize()
    finally:
        if gc_was_on:
            gc.enable()
    per = [events[i].elapsed_time(events[i + 1]) for i in range(steps)]
    return events[0].elapsed_time(events[-1]) / steps, per


def _summary(per):
    s = sorted(per)
    p95 = s[min(len(s) - 1, max(0, int(round(0.95 * (len(s) - 1)))))]
    return {"median_ms": statistics.median(s), "p95_ms": p95, "min_ms": s[0]}


def _flops(w):
    """Algorithmic FLOPs of one step: the forward (base 2*R*3*d*f plus LoRA
    2*R*r*3*(d+f)); with the backward, dX through the re-decoded base
    (2*R*3*d*f) plus about twice the forward's LoRA FLOPs (dz, dA, dB and the
    LoRA part of dX)."""
    R = w.routed_rows
    flops = w.flops()
    if w.backward:
        flops += 2 * R * 3 * w.hidden * w.ffn + 2 * (2 * R * w.rank * 3 * (w.hidden + w.ffn))
    return flops


class _Layer:
    """One workload's module, inputs and step functions on the GPU."""

    def __init__(self, w, device):
        import torch

        from mirai_amd import route_topk
        from mirai_amd import workloads as wl

        self.w = w
        self.logits_cpu = wl.router_logits(w)
        self.tokens_cpu = wl.tokens(w)
        self.logits = self.logits_cpu.to(device)
        self.x = self.tokens_cpu.to(device)
        self.module = _build_module(w, device)
        self.dy = wl.upstream_grad(w, device=device) if w.backward else None
        self.lora_params = [p for ad in self.module.expert_lora.values()
                            for p in (ad.lora_a, ad.lora_b)]
        self.state = {}
        self._route = route_topk

    def routes(self):
        import torch

        with torch.no_grad():
            return self._route(self.logits, self.w.top_k, renorm="clamp", score_dtype=self.w.dtype)

    def forward_only(self):
        import torch

        with torch.no_grad():
            idx, scores = self.routes()
            self.state["out"] = self.module.run_direct_routed(self.x, scores, idx)
            self.state["idx"] = idx

    def forward_train(self):
        # Routing stays outside the graph here: its backward (d logits) is a
        # separate, tiny kernel; d scores is what the expert op produces.
        idx, scores = self.routes()
        xg = self.x.detach().requires_grad_(True)
        sg = scores.detach().requires_grad_(True)
        for p in self.lora_params:
            p.grad = None
        out = self.module.run_direct_routed(xg, sg, idx)
        self.state["idx"] = idx
        return out

    def step(self):
        if not self.w.backward:
            self.forward_only()
            return
        self.forward_train().backward(self.dy)

    def counts(self):
        import torch

        return torch.bincount(self.state["idx"].reshape(-1), minlength=self.w.experts).cpu()


def _config_record(w, device, steps, warmup, args_settle=0.5):
    """Nested per-configuration record: step time (mean, median, p95), routed
    tokens/s, TFLOP/s, the fraction of the bf16 MFMA peak and of the roofline
    attainable = min(P_mfma, AI * BW_hbm) on algorithmic bytes, and the HBM rate
    of those bytes (the weight-streaming view of light experts)."""
    from mirai_amd import workloads as wl

    layer = _Layer(w, device)
    _settle(layer.step, args_settle)
    ms, per = _step_times(layer.step, steps, warmup)
    counts = layer.counts()
    flops = _flops(w)
    nbytes = wl.algorithmic_bytes(w, counts)
    attainable = min(PEAK_BF16_TFLOPS * 1e12, flops / nbytes * PEAK_HBM_GBS * 1e9)
    rate = flops / (ms * 1e-3)
    rec = {"workload": w.name, **{k: v for k, v in wl.describe(w).items() if k != "workload"},
           "backward": w.backward, "steps": steps, "warmup": warmup, "ms_per_step": ms,
           **_summary(per), "routed_tokens_per_s": w.routed_rows / (ms * 1e-3),
           "tflops": rate / 1e12, "pct_bf16_peak": 100.0 * rate / 1e12 / PEAK_BF16_TFLOPS,
           "algorithmic_bytes": nbytes, "hbm_gbs_of_algorithmic_bytes": nbytes / (ms * 1e-3) / 1e9,
           "roofline_attainable_tflops": attainable / 1e12, "roofline_frac": rate / attainable,
           "empty_experts": int((counts == 0).sum()),
           "rows_per_expert": {"min": int(counts.min()), "median": int(counts.median()),
                               "max": int(counts.max())}}
    del layer
    return rec


def main() -> int:
    args = _parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the routed expert layer is built and measured on a "
              "single MI355X in this build.", file=sys.stderr)
        return 2

    import torch

    from mirai_amd import workloads as wl

    if args.config not in wl.WORKLOADS:
        print(f"unknown config {args.config!r}; choose from {sorted(wl.WORKLOADS)}",
              file=sys.stderr)
        return 2
    w = wl.WORKLOADS[args.config]
    if args.weights:
        w = dataclasses.replace(w, fmt=args.weights, name=f"{w.name}_{args.weights}")
    if args.tokens:
        w = dataclasses.replace(w.with_tokens(args.tokens), name=f"{w.name}_T{args.tokens}")
    if args.lora_rank is not None:
        r = int(args.lora_rank)
        w = dataclasses.replace(w, rank=r, alpha=2.0 * r if r > 0 else w.alpha,
                                name=f"{w.name}_r{r}")
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.path != "layer":
        print(json.dumps(_bench_path(args, w, device)))
        return 0

    layer = _Layer(w, device)
    _settle(layer.step, args.settle_seconds)
    eager_ms, per_step = _step_times(layer.step, args.steps, args.warmup)
    ms = eager_ms
    execution = "eager"
    if not w.backward and args.graph:
        # The inference step (route + layer: about a dozen kernels) replayed as
        # one HIP graph: the same kernels on the same inputs, without the
        # per-launch gaps. Nothing on this path records a memset.
        layer.forward_only()
        torch.cuda.synchronize()
        eager_out = layer.state["out"].clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                layer.forward_only()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            layer.forward_only()
        ms, per_step = _step_times(graph.replay, args.steps, args.warmup)
        if not torch.equal(layer.state["out"], eager_out):
            print("graph replay differs from the eager step", file=sys.stderr)
            return 1
        execution = "hip_graph"

    # Routing kernel alone, then the library stages (separate, synchronised passes).
    route_ms, _ = _step_times(layer.routes, args.steps, 1)
    stages = _stage_times(layer.forward_only if not w.backward else layer.forward_train,
                          max(3, args.steps // 2), device)
    back = {}
    if w.backward:
        fwd_ms, _ = _step_times(layer.forward_train, args.steps, 1)
        back = {
            "forward_ms": fwd_ms,
            "backward_ms": ms - fwd_ms,
            "backward_stage_ms": _stage_times(layer.step, max(3, args.steps // 2), device,
                                              BACK_STAGES),
        }

    counts = layer.counts()
    R = w.routed_rows
    flops = _flops(w)
    tflops = flops / (ms * 1e-3) / 1e12
    gate_up_flops = 2 * R * 2 * w.hidden * w.ffn + 2 * R * 2 * w.ffn * w.rank
    gu_ms = stages["gate_up_gemm"]
    achieved = gate_up_flops / (gu_ms * 1e-3) / 1e12
    down_flops = 2 * R * w.ffn * w.hidden + 2 * R * w.hidden * w.rank
    if w.backward:
        bst = back["backward_stage_ms"]
        dx_flops = 2 * R * 2 * w.ffn * w.hidden + 2 * R * 2 * w.rank * w.hidden
        back["dx_gemm_tflops"] = dx_flops / (bst["dx_gemm"] * 1e-3) / 1e12
        dh_flops = 2 * R * w.hidden * w.ffn + 2 * R * w.rank * w.ffn
        back["dh_gemm_tflops"] = dh_flops / (bst["dh_gemm"] * 1e-3) / 1e12
    result = {
        "metric": "routed tokens/s + TFLOP/s (% bf16 MFMA peak) for NF4 MoE+LoRA layer, 1 GPU",
        "value": R / (ms * 1e-3),
        "unit": "routed tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) tokens and logits, N(0,0.02) weights and LoRA)",
        "config": {**wl.describe(w), "lora_alpha": w.alpha, "parallelism": "single_gpu"},
        **_summary(per_step),
        "tflops": tflops,
        "pct_bf16_peak": 100.0 * tflops / PEAK_BF16_TFLOPS,
        "tokens_per_s": w.tokens / (ms * 1e-3),
        "algorithmic_gflop": flops / 1e9,
        "empty_experts": int((counts == 0).sum()),
        "execution": execution,
        "eager_ms_per_step": eager_ms,
        "stage_ms": {"route": route_ms, **stages},
        "down_gemm_tflops": down_flops / (stages["down_gemm"] * 1e-3) / 1e12,
        **back,
        "roofline": {
            "kernel": "grouped_gemm_dual_kernel<NF4, SWIGLU, LoRA> (gate/up)",
            "bound": "mfma",
            "achieved": achieved,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / PEAK_BF16_TFLOPS,
            "traffic": _profiled_traffic("gate_up", w.name),
        },
    }
    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        result["copy_probe_bytes"] = {"read": n * 4, "write": n * 4}
        del src, dst
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = _cpu_baseline(w, layer.module, layer.logits_cpu,
                                               layer.tokens_cpu, args.cpu_seconds)
    del layer
    if not args.no_configs:
        # The benchmark definition's other configurations, as nested records
        # (not the headline): C1 fp32, C2 at its own T = 4096, C3 Zipf-skewed,
        # C4 INT8, C5 forward + backward.
        result["configs"] = {}
        for key in ("c1", "c2", "c3", "c4", "c5"):
            torch.cuda.empty_cache()
            result["configs"][key] = _config_record(wl.WORKLOADS[key], device,
                                                    args.config_steps, args.config_warmup)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
