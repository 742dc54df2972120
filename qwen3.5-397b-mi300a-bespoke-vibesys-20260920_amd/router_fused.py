"""Fused router — the reference's `router_fused` interface (`router_fused.py:36-151`) on the
gfx950 kernel `mtpk_route_topk` (csrc/mtpk_router.hip).

`route(routing, experts_out, top_k)` = `softmax(routing[:, :experts_out]).topk(top_k)`,
renormalised, in one launch: one wave per token, the row's logits in registers. Selection
ranks by logit (the exact softmax order), ties to the lower expert index, so the selected set
never depends on how the fp32 exponentials round. Weights follow the reference arithmetic
(fp32 softmax, then each selected probability over the sum of the selected ones).
"""

from __future__ import annotations

import torch

import _mtpk

MAX_TOP_K = _mtpk.MAX_TOP_K
"""Largest `top_k` accepted (`router_fused.py:37-40`). The real model's is 10."""

MAX_EXPERTS_OUT = _mtpk.MAX_ROUTER_EXPERTS
"""Widest softmax row one wave holds in registers (16 logits per lane)."""


def available(device: torch.device) -> bool:
    """True on a HIP device (loading the library, raising if it is missing); False on CPU."""
    if device.type != "cuda":
        return False
    _mtpk.lib()
    return True


def route(
    routing: torch.Tensor,
    experts_out: int,
    top_k: int,
    *,
    index_dtype: torch.dtype = torch.int64,
) -> tuple[torch.Tensor, torch.Tensor]:
    """`(top_w fp32 [t, top_k], top_i index_dtype [t, top_k])`, highest weight first.

    `routing` is `[t, >= experts_out]` f32 or bf16 with unit column stride; only its row stride
    matters, so a row that also carries the shared-expert gate is read in place.
    """
    if top_k > MAX_TOP_K:
        raise ValueError(f"route: top_k {top_k} exceeds MAX_TOP_K {MAX_TOP_K}")
    if index_dtype not in (torch.int64, torch.int32):
        raise ValueError(f"route: index_dtype must be int32 or int64, got {index_dtype}")
    if experts_out > MAX_EXPERTS_OUT:
        raise ValueError(f"route: experts_out {experts_out} exceeds {MAX_EXPERTS_OUT}")
    if routing.dim() != 2 or routing.shape[1] < experts_out or routing.stride(1) != 1:
        raise ValueError("route: routing must be [t, >= experts_out] with unit column stride")
    device = _mtpk.require_device(routing)
    t = routing.shape[0]
    top_w = torch.empty(t, top_k, dtype=torch.float32, device=device)
    top_i = torch.empty(t, top_k, dtype=index_dtype, device=device)
    _mtpk.check(
        _mtpk.lib().mtpk_route_topk(
            routing.data_ptr(), _mtpk.float_code(routing.dtype), t, routing.stride(0),
            experts_out, top_k, top_w.data_ptr(), top_i.data_ptr(), _mtpk.index_code(index_dtype),
            _mtpk.stream_of(device),
        ),
        "mtpk_route_topk",
    )  # fmt: skip
    return top_w, top_i
