"""ctypes binding of `libmtpk.so` (include/mtpk.h), the C ABI every device op here goes through.

The library is built in-tree (`build_lib.py`) and loaded from this directory. When it is
missing or does not load, every device entry point raises: there is no silent fallback.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_int, c_int64, c_void_p
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("MTPK_LIB", str(HERE / "libmtpk.so")))
"""The in-tree build; `MTPK_LIB` points the binding at another build of the same sources."""

F32, BF16, I32, I64, U8 = 0, 1, 2, 3, 4
EINVAL, ENODEV, ETOOBIG = -1, -2, -3
MOE_STATIC_SCRATCH = 64 << 20
ABI_VERSION = 4
MAX_TOP_K = 32
MAX_EXPERTS = 4096
MAX_ROUTER_EXPERTS = 1024
UNIT_TOKENS = 16

_SIGNATURES: dict[str, tuple[object, list]] = {
    "mtpk_status_string": (ctypes.c_char_p, [c_int]),
    "mtpk_abi_version": (c_int, []),
    "mtpk_dequant_mxfp4": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int, c_void_p, c_void_p]),
    "mtpk_scale_scan": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "mtpk_fused_moe_static": (
        c_int,
        [c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
         c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p, c_int,
         c_int64, c_void_p, c_void_p],
    ),
    "mtpk_moe_max_units": (c_int64, [c_int64, c_int64]),
    "mtpk_moe_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int64, c_int]),
    "mtpk_moe_prep": (
        c_int,
        [c_void_p, c_int, c_void_p, c_int, c_int64, c_int, c_int, c_void_p, c_void_p, c_int64,
         c_void_p, c_void_p],
    ),
    "mtpk_moe_gate_up": (
        c_int,
        [c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p,
         c_void_p, c_void_p, c_int64, c_int, c_void_p, c_int, c_int64, c_void_p],
    ),
    "mtpk_moe_down": (
        c_int,
        [c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p,
         c_void_p, c_void_p, c_int64, c_void_p, c_void_p],
    ),
    "mtpk_moe_direct_max_tokens": (c_int, []),
    "mtpk_moe_gate_up_direct": (
        c_int,
        [c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p,
         c_int, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p],
    ),
    "mtpk_moe_down_combine": (
        c_int,
        [c_void_p, c_int, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int,
         c_void_p, c_int, c_int64, c_int, c_int, c_int, c_void_p, c_int, c_void_p],
    ),
    "mtpk_moe_combine": (
        c_int,
        [c_void_p, c_void_p, c_int, c_void_p, c_int, c_int64, c_int, c_int64, c_int, c_int,
         c_void_p, c_int, c_void_p],
    ),
    "mtpk_moe_combine_rows": (
        c_int,
        [c_void_p, c_int, c_void_p, c_int, c_void_p, c_int, c_int64, c_int, c_int64, c_int, c_int,
         c_void_p, c_int, c_void_p, c_int, c_int64, c_void_p, c_int, c_void_p],
    ),
    "mtpk_split_planes": (c_int, [c_void_p, c_int64, c_int, c_void_p, c_void_p]),
    "mtpk_fused_moe": (
        c_int,
        [c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
         c_int64, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int64,
         c_void_p, c_void_p],
    ),
    "mtpk_fused_moe_shared": (
        c_int,
        [c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
         c_int64, c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int,
         c_void_p, c_int, c_int64, c_void_p, c_int64, c_void_p, c_void_p],
    ),
    "mtpk_moe_layer_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int, c_int64, c_int64]),
    "mtpk_moe_layer": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
         c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_void_p, c_void_p,
         c_void_p, c_int64, c_void_p, c_void_p],
    ),
    "mtpk_moe_layer_add_norm": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
         c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int, c_void_p, c_void_p,
         c_void_p, c_int64, c_void_p, c_void_p, ctypes.c_float, c_void_p, c_void_p, c_void_p],
    ),
    "mtpk_moe_layer_supported": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
         c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int, c_int, c_int],
    ),
    "mtpk_paged_attention_gated": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64,
         c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, ctypes.c_float, c_int,
         c_void_p, c_int64, c_void_p, c_void_p, c_void_p],
    ),
    "mtpk_kv_write": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
         c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p],
    ),
    "mtpk_deltanet_prep": (
        c_int,
        [c_void_p, c_int, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64,
         c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, ctypes.c_float, ctypes.c_float, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "mtpk_conv_commit": (
        c_int,
        [c_void_p, c_int, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64,
         c_int64, c_void_p],
    ),
    "mtpk_deltanet_commit": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_void_p,
         c_int64, c_void_p, c_int64, c_int64, c_void_p],
    ),
    "mtpk_moe_dense_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int64]),
    "mtpk_moe_dense": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int,
         c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_int64, c_void_p, c_void_p],
    ),
    "mtpk_gemm_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int]),
    "mtpk_gemm_bf16": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int, c_void_p, c_int, c_void_p, c_int64,
         c_void_p],
    ),
    "mtpk_rownorm": (
        c_int,
        [c_void_p, c_int, c_int64, c_int64, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int,
         ctypes.c_float, ctypes.c_float, c_void_p, c_int, c_int64, c_int64, c_void_p, c_void_p,
         c_void_p, c_int, c_void_p, c_int, c_int64, c_int, c_int, c_void_p, c_int64, c_int64,
         c_int64, c_void_p],
    ),
    "mtpk_route_topk": (
        c_int,
        [c_void_p, c_int, c_int64, c_int64, c_int, c_int, c_void_p, c_void_p, c_int, c_void_p],
    ),
    "mtpk_argmax_partials": (c_int64, [c_int64, c_int64]),
    "mtpk_argmax_rows": (
        c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p]
    ),
    "mtpk_greedy_accept": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
         c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "mtpk_greedy_accept_keys": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
         c_void_p, c_int, c_void_p, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "mtpk_round_fill": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int, c_void_p,
         c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "mtpk_draft_feed": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p],
    ),
    "mtpk_copy_rows": (
        c_int,
        [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64,
         c_void_p],
    ),
    "mtpk_argmax_keys": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "mtpk_rejection_workspace_bytes": (c_int64, [c_int64, c_int, c_int64]),
    "mtpk_rejection_sample": (
        c_int,
        [c_void_p, c_void_p, c_int, c_int64, c_int, c_int64, c_void_p, c_void_p, c_void_p,
         ctypes.c_float, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "mtpk_rejection_accept": (
        c_int,
        [c_void_p, c_void_p, c_int, c_int64, c_int, c_int64, c_void_p, c_void_p, c_void_p,
         ctypes.c_float, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "mtpk_sample_workspace_bytes": (c_int64, [c_int64, c_int64]),
    "mtpk_sample_rows": (
        c_int,
        [c_void_p, c_int, c_int64, c_int64, ctypes.c_float, c_void_p, c_void_p, c_int64, c_void_p,
         c_void_p],
    ),
    "mtpk_probe_mfma_16x16x32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "mtpk_probe_stream": (c_int, [c_void_p, c_int64, c_int, c_int, c_void_p, c_void_p]),
    "mtpk_delta_rule": (
        c_int,
        [c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p,
         c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "mtpk_attention_splits": (c_int, [c_int64, c_int64, c_int64, c_int64, c_int64, c_int64]),
    "mtpk_attention_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int64, c_int]),
    "mtpk_paged_attention": (
        c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
         c_int64, c_void_p, ctypes.c_float, c_int, c_void_p, c_int64, c_void_p, c_void_p],
    ),
}

EXPORTED = tuple(_SIGNATURES)
"""Every entry point `include/mtpk.h` declares."""

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises `RuntimeError` if it is not built or does not load."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"libmtpk.so is not built at {LIB_PATH}; run `python __graft_entry__.py build` "
            "(or build_lib.py) first"
        )
    try:
        handle = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        raise RuntimeError(f"libmtpk.so failed to load: {exc}") from exc
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if handle.mtpk_abi_version() != ABI_VERSION:
        raise RuntimeError(
            f"libmtpk.so at {LIB_PATH} has ABI version {handle.mtpk_abi_version()}, the binding "
            f"expects {ABI_VERSION}: rebuild it (`python __graft_entry__.py build`)"
        )
    _lib = handle
    return handle


def check(status: int, what: str) -> None:
    """Raise on a nonzero status; the message names the entry point and the cause."""
    if status != 0:
        text = lib().mtpk_status_string(status).decode()
        if status in (EINVAL, ETOOBIG):
            raise ValueError(f"{what}: {text}")
        raise RuntimeError(f"{what}: {text} (status {status})")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def row_stride(x: torch.Tensor) -> int | None:
    """Element stride between consecutive rows of `x` `[B, t, ...]` read as `B * t` rows, or
    None when the two leading dims do not collapse to one stride. A size-1 dim's stride is
    arbitrary (views and reshapes set it freely), so it neither sets nor checks the stride."""
    b, t = x.shape[0], x.shape[1]
    if t == 1:
        return x.stride(0)
    if b > 1 and x.stride(0) != t * x.stride(1):
        return None
    return x.stride(1)


def stream_of(device: torch.device) -> int:
    """Handle of torch's current stream on `device` (what the kernels launch on)."""
    return torch.cuda.current_stream(device).cuda_stream


def float_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return F32
    if dtype == torch.bfloat16:
        return BF16
    raise ValueError(f"unsupported float dtype {dtype} (float32 or bfloat16)")


def index_code(dtype: torch.dtype) -> int:
    if dtype == torch.int32:
        return I32
    if dtype == torch.int64:
        return I64
    raise ValueError(f"unsupported index dtype {dtype} (int32 or int64)")


def require_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one HIP device; returns it. CPU tensors are a caller error here."""
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise ValueError("libmtpk entry points take device tensors")
        if t.device != dev:
            raise ValueError("all tensors must be on the same device")
    return dev
