"""The hot path's device entry points as PyTorch custom ops, namespace `mtpk`.

Each op is a `torch.library.custom_op` over the same C-ABI call the Python wrapper makes
(`mxfp4_gemv.fused_moe`, `mxfp4_gemv.fused_moe_layer`, `router_fused.route`, `mtp.argmax_rows`,
`graph_mtp.greedy_accept`, `graph_mtp.rejection_sample`), registered for HIP devices only, with a fake kernel that gives
the output shapes and dtypes without running anything. That puts the ops in the dispatcher:
`torch.compile` traces through them as single nodes, FakeTensor / meta propagation works, and a
HIP graph captures them like any other launch. There is no CPU kernel: a call on CPU tensors
fails in the dispatcher.

The reference reaches its kernels through a pybind extension of plain functions
(`moe_hip.py:134-190`); the argument meanings here follow the Python wrappers above, flattened
into tensors and scalars (the expert dict becomes its four payload tensors, the routing pair
two tensors, the expert range two ints).
"""

from __future__ import annotations

import torch
from torch import Tensor
from torch.library import custom_op

import graph_mtp
import mtp
import mxfp4_gemv
import router_fused

# ---------------------------------------------------------------- routed MXFP4 experts


@custom_op("mtpk::fused_moe", mutates_args=(), device_types="cuda")
def fused_moe(x: Tensor, gate_up: Tensor, gate_up_scale: Tensor, down: Tensor, down_scale: Tensor,
              a_expert: Tensor, a_weight: Tensor, top_k: int, expert_lo: int, expert_hi: int,
              shared: Tensor | None = None, shared_gate: Tensor | None = None) -> Tensor:
    """`mxfp4_gemv.fused_moe(x, experts, (a_expert, a_weight), top_k, (expert_lo, expert_hi),
    shared=, shared_gate=)`: the routed experts' output `[T, hidden]` in x's dtype, plus
    `sigmoid(shared_gate) * shared` when both are given."""
    experts = {"gate_up": gate_up, "gate_up_scale": gate_up_scale, "down": down,
               "down_scale": down_scale}
    return mxfp4_gemv.fused_moe(x, experts, (a_expert, a_weight), top_k, (expert_lo, expert_hi),
                                shared=shared, shared_gate=shared_gate)


@fused_moe.register_fake
def _(x, gate_up, gate_up_scale, down, down_scale, a_expert, a_weight, top_k, expert_lo,
      expert_hi, shared=None, shared_gate=None):
    torch._check(x.dim() == 2, lambda: "x must be [T, hidden]")
    torch._check(a_expert.numel() == x.shape[0] * top_k, lambda: "one expert id per (token, slot)")
    return x.new_empty(x.shape)


# ---------------------------------------------------------------- whole MoE layer


@custom_op("mtpk::moe_layer", mutates_args=(), device_types="cuda")
def moe_layer(h: Tensor, router_gate: Tensor, shared_gate_up: Tensor, shared_down: Tensor,
              gate_up: Tensor, gate_up_scale: Tensor, down: Tensor, down_scale: Tensor, top_k: int,
              expert_lo: int, expert_hi: int) -> tuple[Tensor, Tensor, Tensor]:
    """`mxfp4_gemv.fused_moe_layer`: `(out [T, hidden] bf16, top_w f32 [T, top_k], top_i int32
    [T, top_k])` -- the layer output and the routing it chose."""
    experts = {"gate_up": gate_up, "gate_up_scale": gate_up_scale, "down": down,
               "down_scale": down_scale}
    t = h.shape[0]
    tw = torch.empty(t, top_k, dtype=torch.float32, device=h.device)
    ti = torch.empty(t, top_k, dtype=torch.int32, device=h.device)
    out = mxfp4_gemv.fused_moe_layer(h, router_gate, shared_gate_up, shared_down, experts, top_k,
                                     (expert_lo, expert_hi), routing_out=(tw, ti))
    return out, tw, ti


@moe_layer.register_fake
def _(h, router_gate, shared_gate_up, shared_down, gate_up, gate_up_scale, down, down_scale, top_k,
      expert_lo, expert_hi):
    torch._check(h.dim() == 2, lambda: "h must be [T, hidden]")
    t = h.shape[0]
    return (h.new_empty(h.shape), h.new_empty(t, top_k, dtype=torch.float32),
            h.new_empty(t, top_k, dtype=torch.int32))


# ---------------------------------------------------------------- router top-k


@custom_op("mtpk::route", mutates_args=(), device_types="cuda")
def route(routing: Tensor, experts_out: int, top_k: int,
          index_dtype: torch.dtype = torch.int64) -> tuple[Tensor, Tensor]:
    """`router_fused.route`: `(top_w f32 [t, top_k], top_i [t, top_k])`, highest weight first,
    weights renormalised over the top-k."""
    return router_fused.route(routing, experts_out, top_k, index_dtype=index_dtype)


@route.register_fake
def _(routing, experts_out, top_k, index_dtype=torch.int64):
    t = routing.shape[0]
    return (routing.new_empty(t, top_k, dtype=torch.float32),
            routing.new_empty(t, top_k, dtype=index_dtype))


# ---------------------------------------------------------------- greedy token


@custom_op("mtpk::argmax_rows", mutates_args=(), device_types="cuda")
def argmax_rows(logits: Tensor) -> Tensor:
    """`mtp.argmax_rows`: first-occurrence argmax over the last dim, int64 `logits.shape[:-1]`."""
    return mtp.argmax_rows(logits)


@argmax_rows.register_fake
def _(logits):
    return logits.new_empty(logits.shape[:-1], dtype=torch.int64)


# ---------------------------------------------------------------- acceptance


@custom_op("mtpk::greedy_accept", mutates_args=(), device_types="cuda")
def greedy_accept(step_argmax: Tensor, draft: Tensor, active: Tensor, pos: Tensor, budget: Tensor,
                  stops: Tensor, conv_k1: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                                        Tensor, Tensor, Tensor, Tensor, Tensor]:
    """`graph_mtp.greedy_accept` as new tensors, in `AcceptResult`'s field order: accept_len,
    lengths, packed_src, packed_cu, conv_idx, keep, bonus, next_pos, budget_left, live,
    hidden_src."""
    r = graph_mtp.greedy_accept(step_argmax, draft, active, pos, budget, stops, conv_k1)
    return (r.accept_len, r.lengths, r.packed_src, r.packed_cu, r.conv_idx, r.keep, r.bonus,
            r.next_pos, r.budget_left, r.live, r.hidden_src)


@greedy_accept.register_fake
def _(step_argmax, draft, active, pos, budget, stops, conv_k1):
    b, t = step_argmax.shape
    i64 = dict(dtype=torch.int64)
    return (step_argmax.new_empty(b, **i64), step_argmax.new_empty(b, **i64),
            step_argmax.new_empty(b * t, **i64), step_argmax.new_empty(b + 1, dtype=torch.int32),
            step_argmax.new_empty(b, conv_k1, **i64), step_argmax.new_empty(b, t, dtype=torch.bool),
            step_argmax.new_empty(b, **i64), step_argmax.new_empty(b, **i64),
            step_argmax.new_empty(b, **i64), step_argmax.new_empty(b, dtype=torch.bool),
            step_argmax.new_empty(b, **i64))


@custom_op("mtpk::rejection_sample", mutates_args=(), device_types="cuda")
def rejection_sample(target_logits: Tensor, draft_logits: Tensor, draft_tokens: Tensor,
                     u_accept: Tensor, u_sample: Tensor,
                     temperature: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """`graph_mtp.rejection_sample(..., with_margin=True)`: `(accept_len i64 [B], token i64 [B],
    emitted i64 [B, k+1], margin f32 [B, k])`."""
    acc, tok, emitted, margin = graph_mtp.rejection_sample(
        target_logits, draft_logits, draft_tokens, u_accept, u_sample, temperature, with_margin=True)
    return acc, tok, emitted, margin.contiguous()


@rejection_sample.register_fake
def _(target_logits, draft_logits, draft_tokens, u_accept, u_sample, temperature):
    b, t, _ = target_logits.shape
    i64 = dict(dtype=torch.int64)
    return (target_logits.new_empty(b, **i64), target_logits.new_empty(b, **i64),
            target_logits.new_empty(b, t, **i64),
            target_logits.new_empty(b, t - 1, dtype=torch.float32))
