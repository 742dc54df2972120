"""Gated DeltaNet recurrence on the device through `mtpk_delta_rule` (include/mtpk.h).

One call runs `t` gated delta-rule steps per row over a pool of fp32 recurrent states:

    S <- exp(g) S;   S <- S + k ((v - S^T k) beta)^T;   out = S^T q

In verify mode (`lengths is None`) the rows start from their slots' committed state, every
step's output is returned and the state is left as it was (`deltanet_verify_static`,
`graph_mtp.py:227-344`). In commit mode each row advances its slot in place by its accepted
prefix `min(lengths[j], t)` (`deltanet_verify_rollback_static`, `graph_mtp.py:347-437`). Both
replace `deltanet_fused.delta_rule_verify_exact` (`deltanet_fused.py:1090-1176`); the argument
checks follow that function's.
"""

from __future__ import annotations

import torch

import _mtpk


def delta_rule(state: torch.Tensor, slots: torch.Tensor | None, q: torch.Tensor, k: torch.Tensor,
               v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
               lengths: torch.Tensor | None = None, *, want_out: bool = True) -> torch.Tensor | None:
    """`state` f32 `[slots_total, heads, k_dim, v_dim]` (contiguous, updated in place in commit
    mode); `slots` int64 `[B]` (distinct) or None for row j -> slot j; `q`, `k` f32
    `[B, t, qk_heads, k_dim]` (normalised, q scaled; head h reads q/k head
    `h // (heads // qk_heads)`); `v` f32 `[B, t, heads, v_dim]`; `g` (log decay), `beta` f32
    `[B, t, heads]`; `lengths` int64 `[B]` selects commit mode. Returns the per-step outputs
    f32 `[B, t, heads, v_dim]`, or None when `want_out` is False in commit mode."""
    device = _mtpk.require_device(state, q, k, v, g, beta)
    if state.dtype != torch.float32 or state.dim() != 4 or not state.is_contiguous():
        raise ValueError("state must be a contiguous f32 [slots, heads, k_dim, v_dim] tensor")
    n_slots, heads, k_dim, v_dim = state.shape
    if q.dim() != 4 or q.shape != k.shape:
        raise ValueError(f"q/k must have matching [B, t, heads, dim]; got {tuple(q.shape)}/{tuple(k.shape)}")
    rows, t, qk_heads, qk_dim = q.shape
    if qk_dim != k_dim or t < 1:
        raise ValueError(f"q/k must be [B, t >= 1, heads, {k_dim}], got {tuple(q.shape)}")
    if heads % qk_heads:
        raise ValueError(f"state heads {heads} is not a multiple of q/k heads {qk_heads}")
    if tuple(v.shape) != (rows, t, heads, v_dim):
        raise ValueError(f"v must be [{rows}, {t}, {heads}, {v_dim}], got {tuple(v.shape)}")
    if tuple(g.shape) != (rows, t, heads) or tuple(beta.shape) != (rows, t, heads):
        raise ValueError(f"g/beta must be [{rows}, {t}, {heads}], got {tuple(g.shape)}/{tuple(beta.shape)}")
    if k_dim not in (16, 32, 64, 128):
        raise ValueError(f"k_dim must be 16, 32, 64 or 128, got {k_dim}")
    if slots is not None:
        if tuple(slots.shape) != (rows,):
            raise ValueError(f"slots must be [{rows}], got {tuple(slots.shape)}")
        slots = slots.to(device, torch.int64).contiguous()
    elif n_slots < rows:
        raise ValueError(f"{rows} rows need {rows} state slots, the pool has {n_slots}")
    if lengths is not None:
        if tuple(lengths.shape) != (rows,):
            raise ValueError(f"lengths must be [{rows}], got {tuple(lengths.shape)}")
        lengths = lengths.to(device, torch.int64).contiguous()
    elif not want_out:
        raise ValueError("verify mode (no lengths) produces only outputs")
    f32 = [x.to(torch.float32).contiguous() for x in (q, k, v, g, beta)]
    out = torch.empty(rows, t, heads, v_dim, dtype=torch.float32, device=device) if want_out else None
    _mtpk.check(
        _mtpk.lib().mtpk_delta_rule(
            state.data_ptr(), n_slots, _mtpk.ptr(slots), rows, t, heads, qk_heads, k_dim, v_dim,
            *(x.data_ptr() for x in f32), _mtpk.ptr(lengths), _mtpk.ptr(out), _mtpk.stream_of(device)),
        "mtpk_delta_rule",
    )
    return out
