"""ctypes binding of libmirai_moe.so (the gfx950 HIP kernels behind a C ABI).

The library is loaded from ``mirai_amd/lib/``; it is built in-tree by
``mirai_amd.csrc.build``. There is no fallback: every product entry point
raises :class:`NativeLibraryError` when the library or a GPU is missing.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path
from typing import Any

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmirai_moe.so"

MX_OK = 0
MX_ERR_INVALID = 1
MX_ERR_HIP = 2

DTYPE_F32 = 0
DTYPE_BF16 = 1

FMT_BF16 = 0
FMT_NF4 = 1
FMT_INT8 = 2
FMT_F32X3 = 3      # fp32 weights as bf16 planes [hi | lo | hi] along in_features
FMT_NF4_F32 = 4    # NF4 codes with an fp32 block absmax (ingested bitsandbytes payloads)
FMT_NF4_F32_KN = 5  # the same, stored [E, in, out] with the blocks along out (MAGI-2 groups)
FMT_NF4_DQ = 6     # NF4 codes with a bitsandbytes two-level absmax decoded in the GEMMs
FMT_NF4_DQ_KN = 7  # the same, stored [E, in, out]

SPLIT_ACT = 0      # mx_split_f32 plane orders
SPLIT_WEIGHT = 1

RENORM_NONE = 0
RENORM_CLAMP = 1
RENORM_EPS = 2

ACT_SILU = 0       # expert activations
ACT_SWIGLU7 = 1
ACT_FLAG_BF16_COMBINE = 0x100  # or-ed into act: bf16 terms and sums in the combine (MAGI-2)

SCORE_SOFTMAX = 0  # mx_route_topk_heads score functions and output layouts
SCORE_SIGMOID = 1
ROUTE_LAYOUT_HEADS = 0
ROUTE_LAYOUT_ROWS = 1

# A route slot whose expert id is ROUTE_DROPPED is left out of the layer
# without counting as an invalid route (zero-score slots of coalesced aliases).
ROUTE_DROPPED = -(1 << 63)

# mx_abi_version() of the library these bindings describe.
ABI_VERSION = 9

PLAN_MAX_EXPERTS = 8192
STATIC_SCRATCH_BYTES = 64 << 20  # MX_STATIC_SCRATCH_BYTES
ROUTER_MAX_EXPERTS = 256  # mx_router_forward


class NativeLibraryError(RuntimeError):
    """The HIP library is not built, not loadable, or no GPU is present."""


class MxWeight(ctypes.Structure):
    _fields_ = [
        ("format", c_int),
        ("data", c_void_p),
        ("scale", c_void_p),
        ("out_features", c_int64),
        ("in_features", c_int64),
    ]


class MxNf4Dq(ctypes.Structure):
    """mx_nf4_dq: the two-level absmax of an NF4_DQ weight (device pointers)."""
    _fields_ = [
        ("absmax_q", c_void_p),
        ("nested_absmax", c_void_p),
        ("offsets", c_void_p),
        ("code", c_void_p),
        ("nested_per_expert", c_int64),
    ]


class MxLora(ctypes.Structure):
    _fields_ = [("a", c_void_p), ("b", c_void_p), ("rank", c_int), ("scale", c_float)]


_P = c_void_p
_W = POINTER(MxWeight)
_L = POINTER(MxLora)

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "mx_last_error": (ctypes.c_char_p, []),
    "mx_abi_version": (c_int, []),
    "mx_route_topk": (c_int, [_P, c_int64, c_int, c_int, c_int, c_float, _P, _P, c_int, _P]),
    "mx_route_topk_backward": (
        c_int, [_P, c_int64, c_int, c_int, c_int, c_float, _P, _P, _P, _P]),
    "mx_route_scores_backward": (
        c_int, [_P, c_int64, c_int, c_int, c_int, c_int, c_float, c_float, _P, _P, _P, _P]),
    "mx_route_topk_heads": (
        c_int,
        [_P, c_int, c_int64, c_int, c_int, c_int, _P, c_int, c_float, c_float, c_int, c_int,
         c_int, _P, _P, c_int, _P]),
    "mx_router_padded_experts": (c_int, [c_int]),
    "mx_router_planes_size": (c_size_t, [c_int, c_int64]),
    "mx_router_weight_planes": (c_int, [_P, c_int, c_int64, _P, _P]),
    "mx_router_forward": (
        c_int,
        [_P, c_int, c_int64, c_int64, c_int, _P, _P, _P, c_int, c_int, c_int, c_int, c_int,
         c_float, _P, _P, _P, _P, c_int, _P]),
    "mx_expert_choice_plan_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int]),
    "mx_build_expert_choice_plan": (
        c_int, [_P, _P, c_int, c_int, c_int, c_int, c_int64, _P, c_int, _P, _P, _P, _P, _P, _P,
                _P, _P, _P]),
    "mx_moe_expert_choice_workspace_size": (
        c_size_t, [c_int, c_int, c_int, c_int64, c_int, c_int64, c_int64, c_int]),
    "mx_moe_forward_expert_choice": (
        c_int,
        [_P, _P, _P, c_int, c_int, c_int, c_int, c_int64, _P, _P, c_int, c_int64, c_int64, c_int,
         _W, _W, _W, _L, _L, _L, _P, c_int, _P, _P]),
    "mx_moe_forward_expert_choice_ex": (
        c_int,
        [_P, _P, _P, c_int, c_int, c_int, c_int, c_int64, _P, _P, c_int, c_int64, c_int64, c_int,
         _W, _W, _W, _L, _L, _L, _P, c_int, _P, _P, _P, _P, _P, _P, _P]),
    "mx_moe_backward_expert_choice_workspace_size": (
        c_size_t, [c_int, c_int, c_int, c_int64, c_int, c_int64, c_int64, c_int]),
    "mx_moe_backward_expert_choice": (
        c_int,
        [_P, c_int, _P, _P, _P, c_int, c_int, c_int, c_int, c_int64, _P, _P, c_int, c_int64,
         c_int64, c_int, _W, _W, _W, _L, _L, _L, _P, _P, _P, _P, _P, _P, c_int, _P, _P, _P, _P,
         _P, _P, _P, _P, _P]),
    "mx_plan_workspace_size": (c_size_t, [c_int64, c_int, c_int]),
    "mx_build_plan": (
        c_int, [_P, _P, c_int, c_int64, c_int, c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "mx_plan_from_counts": (c_int, [_P, c_int64, c_int, _P, _P]),
    "mx_plan_error_counter": (POINTER(c_int32), [_P]),
    "mx_gather_rows": (c_int, [_P, c_int64, _P, c_int64, c_int64, c_int, _P, _P]),
    "mx_scatter_add_rows": (c_int, [_P, _P, _P, c_int64, c_int64, c_int, c_int64, _P, _P]),
    "mx_combine": (c_int, [_P, _P, _P, c_int, c_int64, c_int, c_int, c_int64, _P, c_int, _P]),
    "mx_combine_backward": (
        c_int, [_P, c_int, _P, _P, _P, c_int, c_int64, c_int, c_int, c_int64, _P, _P, _P]),
    "mx_nf4_quantize": (c_int, [_P, c_int, c_int64, c_int64, _P, _P, _P]),
    "mx_nf4_dequantize": (c_int, [_P, _P, c_int64, c_int64, _P, c_int, _P]),
    "mx_nf4_dequantize_ex": (c_int, [_P, _P, c_int, c_int64, c_int64, _P, c_int, _P]),
    "mx_nf4_from_bnb": (
        c_int, [_P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P, _P, _P]),
    "mx_nf4_dq_absmax": (c_int, [POINTER(MxNf4Dq), c_int64, c_int64, _P, _P]),
    "mx_int8_quantize": (c_int, [_P, c_int, c_int64, c_int64, _P, _P, _P]),
    "mx_int8_dequantize": (c_int, [_P, _P, c_int64, c_int64, _P, c_int, _P]),
    "mx_set_stage_events": (c_int, [POINTER(c_void_p), c_int]),
    "mx_moe_workspace_size": (c_size_t, [c_int64, c_int, c_int, c_int64, c_int64, c_int]),
    "mx_moe_f32x3_workspace_size": (c_size_t, [c_int64, c_int, c_int, c_int64, c_int64]),
    "mx_split_f32": (c_int, [_P, c_int64, c_int64, c_int, _P, _P]),
    "mx_moe_forward": (
        c_int,
        [_P, _P, _P, c_int, c_int64, c_int, c_int, c_int64, c_int64, _W, _W, _W, _L, _L, _L,
         _P, c_int, _P, _P, _P, _P, _P, _P, _P]),
    "mx_moe_forward_act": (
        c_int,
        [_P, _P, _P, c_int, c_int64, c_int, c_int, c_int64, c_int64, c_int, _W, _W, _W, _L, _L,
         _L, _P, c_int, _P, _P, _P, _P, _P, _P, _P]),
    "mx_moe_forward_ex": (
        c_int,
        [_P, _P, _P, c_int, c_int64, c_int, c_int, c_int64, c_int64, c_int, _W, _W, _W, _L, _L,
         _L, _P, c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "mx_moe_forward_static": (
        c_int,
        [_P, _P, _P, c_int, c_int64, c_int, c_int, c_int64, c_int64, c_int, _W, _W, _W, _L, _L,
         _L, _P, c_int, _P]),
    "mx_moe_for_loop": (
        c_int, [_P, _P, c_int64, c_int, c_int64, c_int64, _W, _W, _W, _L, _L, _L, _P, _P, _P]),
    "mx_moe_for_loop_act": (
        c_int, [_P, _P, c_int64, c_int, c_int64, c_int64, c_int, _W, _W, _W, _L, _L, _L, _P, _P,
                _P]),
    "mx_grouped_linear": (c_int, [_P, _P, c_int64, c_int, _W, _L, _P, _P, _P]),
    "mx_grouped_linear_backward_workspace_size": (
        c_size_t, [c_int64, c_int, c_int64, c_int64, c_int]),
    "mx_grouped_linear_backward": (
        c_int, [_P, _P, _P, c_int64, c_int, _W, _L, _P, _P, _P, _P, _P]),
    "mx_moe_backward_workspace_size": (c_size_t,
                                       [c_int64, c_int, c_int, c_int64, c_int64, c_int]),
    "mx_moe_backward": (
        c_int,
        [_P, c_int, _P, _P, _P, c_int, c_int64, c_int, c_int, c_int64, c_int64, _W, _W, _W,
         _L, _L, _L, _P, _P, _P, _P, _P, _P, c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "mx_moe_backward_act": (
        c_int,
        [_P, c_int, _P, _P, _P, c_int, c_int64, c_int, c_int, c_int64, c_int64, c_int, _W, _W,
         _W, _L, _L, _L, _P, _P, _P, _P, _P, _P, c_int, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
}

_lib: ctypes.CDLL | None = None


def load_library() -> ctypes.CDLL:
    """Load (once) and return the native library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise NativeLibraryError(
            f"{LIB_PATH} is not built; run `python -m mirai_amd.csrc.build` "
            "(hipcc --offload-arch=gfx950)."
        )
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:  # pragma: no cover - depends on the ROCm install
        raise NativeLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
    version = getattr(lib, "mx_abi_version", None)
    found = int(version()) if version is not None else -1
    if found != ABI_VERSION:
        raise NativeLibraryError(
            f"{LIB_PATH} has ABI version {found}, these bindings need {ABI_VERSION}; rebuild "
            "with `python -m mirai_amd.csrc.build`.")
    missing = [name for name in SIGNATURES if getattr(lib, name, None) is None]
    if missing:
        raise NativeLibraryError(
            f"{LIB_PATH} lacks {', '.join(missing[:4])}; rebuild with "
            "`python -m mirai_amd.csrc.build`.")
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def last_error() -> str:
    msg = load_library().mx_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> None:
    """Invoke ``name``; translate a non-zero status into a Python exception."""
    fn = getattr(load_library(), name)
    rc = fn(*args)
    if rc == MX_OK:
        return
    msg = last_error() or f"{name} failed with status {rc}"
    if rc == MX_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(msg)


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """Device of the given tensors; raises unless they share one ROCm GPU."""
    load_library()
    devices = {t.device for t in tensors if t is not None}
    if not torch.cuda.is_available():
        raise NativeLibraryError("mirai_amd kernels need a ROCm GPU (torch.cuda is unavailable).")
    if len(devices) != 1:
        raise ValueError(f"all tensors must live on one device, got {sorted(map(str, devices))}")
    device = devices.pop()
    if device.type != "cuda":
        raise ValueError(f"mirai_amd kernels run on the GPU; got a {device.type} tensor")
    return device


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    if dtype == torch.float32:
        return DTYPE_F32
    raise ValueError(f"unsupported dtype {dtype}; expected bfloat16 or float32")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


# --------------------------------------------------------- route errors
# The dispatch plan counts route slots whose expert id lies outside
# [0, num_experts) (and, for count-driven plans, counts that do not add up)
# into the workspace's error counter; such slots are left out of every
# expert. The reference's torch.bincount raises on such ids
# (dispatch_preprocess.py:155-157). Reading the counter needs the GPU to have
# run the plan, so by default ("deferred") each call copies it into a pinned
# host slot on its stream and the count is read once that copy has landed:
# at the start of a later call, or by check_route_errors(), which waits. With
# "sync" the call itself waits for its plan and raises; "off" skips the copy.
# Calls captured into a HIP graph are not watched.
ROUTE_CHECK_MODES = ("deferred", "sync", "off")
_route_check = os.environ.get("MIRAI_ROUTE_CHECK", "deferred").strip().lower()
if _route_check not in ROUTE_CHECK_MODES:  # pragma: no cover - environment
    _route_check = "deferred"
_SLOTS = 256
_slot_buf: torch.Tensor | None = None
_slot_next = 0
_pending: list = []  # (event, slot index, what)


class RouteIndexError(ValueError):
    """Routed expert ids outside [0, num_experts) reached the dispatch plan."""


def set_route_check(mode: str) -> None:
    """Select how invalid route ids are reported: "deferred" (default),
    "sync" (raise at the call, after a wait for its plan) or "off"."""
    global _route_check
    mode = str(mode).strip().lower()
    if mode not in ROUTE_CHECK_MODES:
        raise ValueError(f"route check mode must be one of {ROUTE_CHECK_MODES}.")
    _route_check = mode


def route_check_mode() -> str:
    return _route_check


def _raise_for(count: int, what: str, deferred: bool) -> None:
    when = "an earlier " if deferred else ""
    raise RouteIndexError(
        f"{count} route slot(s) of {when}{what} carry an expert id outside "
        f"[0, num_experts) or counts that do not match the rows; those slots were left "
        f"out of the expert computation.")


def _drain(block: bool) -> None:
    while _pending:
        event, slot, what = _pending[0]
        if block:
            event.synchronize()
        elif not event.query():
            return
        _pending.pop(0)
        count = int(_slot_buf[slot])
        if count:
            _pending.clear()
            _raise_for(count, what, deferred=True)


def poll_route_errors() -> None:
    """Raise for an earlier call whose plan found invalid routes (no wait)."""
    if _pending and not torch.cuda.is_current_stream_capturing():
        _drain(block=False)


def check_route_errors() -> None:
    """Wait for every watched call's plan and raise if any found invalid routes."""
    _drain(block=True)


def watch_plan_errors(workspace: torch.Tensor, device: torch.device, what: str) -> None:
    """Queue the plan error counter at the head of ``workspace`` for reading
    (see ROUTE_CHECK_MODES); in "sync" mode wait for it and raise now."""
    global _slot_buf, _slot_next
    # Calls captured into a HIP graph are not watched: a capture may neither
    # query events nor wait, and a replay would not refresh the slot.
    if _route_check == "off" or torch.cuda.is_current_stream_capturing():
        return
    if _slot_buf is None:
        _slot_buf = torch.zeros(_SLOTS, dtype=torch.int32, pin_memory=True)
    slot = _slot_next
    _slot_next = (_slot_next + 1) % _SLOTS
    # A slot is reused only after its previous copy has been read.
    while any(p[1] == slot for p in _pending):
        _drain(block=True)
    counter = workspace[:4].view(torch.int32)
    _slot_buf[slot:slot + 1].copy_(counter, non_blocking=True)
    event = torch.cuda.Event()
    event.record(torch.cuda.current_stream(device))
    if _route_check == "sync":
        event.synchronize()
        count = int(_slot_buf[slot])
        if count:
            _raise_for(count, what, deferred=False)
        return
    _pending.append((event, slot, what))
