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


def commit(state: torch.Tensor, conv_state: torch.Tensor, slots: torch.Tensor, q: torch.Tensor,
           k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
           lengths: torch.Tensor, proj: torch.Tensor, idx: torch.Tensor, channels: int) -> None:
    """`delta_rule(state, slots, q, k, v, g, beta, lengths, want_out=False)` and
    `conv_commit(conv_state, slots, proj, idx, channels)` as one launch where the layer's sizes
    allow it (`mtpk_deltanet_commit`); same arguments, same results."""
    device = _mtpk.require_device(state, conv_state, slots, q, k, v, g, beta, lengths, proj, idx)
    if state.dtype != torch.float32 or state.dim() != 4 or not state.is_contiguous():
        raise ValueError("state must be a contiguous f32 [slots, heads, k_dim, v_dim] tensor")
    n_slots, heads, k_dim, v_dim = state.shape
    rows, t, qk_heads, qk_dim = q.shape
    if k.shape != q.shape or qk_dim != k_dim or heads % qk_heads or k_dim not in (16, 32, 64, 128):
        raise ValueError("q/k do not match the state")
    if (tuple(v.shape) != (rows, t, heads, v_dim) or tuple(g.shape) != (rows, t, heads)
            or tuple(beta.shape) != (rows, t, heads)):
        raise ValueError("v/g/beta do not match q and the state")
    if tuple(slots.shape) != (rows,) or tuple(lengths.shape) != (rows,):
        raise ValueError(f"slots and lengths must be [{rows}]")
    rs = _mtpk.row_stride(proj)
    if proj.shape[:2] != (rows, t) or proj.stride(2) != 1 or rs is None:
        raise ValueError("proj must be [B, t, P] with contiguous rows")
    if proj.dtype != conv_state.dtype or not conv_state.is_contiguous():
        raise ValueError("conv_state must be contiguous and of proj's dtype")
    k1 = conv_state.shape[-1]
    ix = idx.to(torch.int64).contiguous()
    if ix.shape != (rows, k1):
        raise ValueError(f"idx must be [{rows}, {k1}]")
    sl = slots.to(device, torch.int64).contiguous()
    ln = lengths.to(device, torch.int64).contiguous()
    f32 = [x.to(torch.float32).contiguous() for x in (q, k, v, g, beta)]
    _mtpk.check(_mtpk.lib().mtpk_deltanet_commit(
        state.data_ptr(), n_slots, sl.data_ptr(), rows, t, heads, qk_heads, k_dim, v_dim,
        *(x.data_ptr() for x in f32), ln.data_ptr(), conv_state.data_ptr(),
        _mtpk.float_code(conv_state.dtype), conv_state.shape[0], proj.data_ptr(), rs, ix.data_ptr(),
        channels, k1, _mtpk.stream_of(device)), "mtpk_deltanet_commit")  # fmt: skip


def prep(proj: torch.Tensor, conv_state: torch.Tensor, slots: torch.Tensor, conv_w: torch.Tensor,
         a_log: torch.Tensor, dt_bias: torch.Tensor, k_heads: int, k_dim: int, v_heads: int,
         v_dim: int, eps: float = 1e-6) -> tuple[torch.Tensor, ...]:
    """The verify rows' recurrence inputs from the in-projection in one launch
    (`mtpk_deltanet_prep`): `proj` `[B, t, P]` (last dim contiguous: qkv, z, b, a), the stored
    conv windows `conv_state` `[slots_total, C, conv_k - 1]` read at `slots` `[B]`, `conv_w`
    `[C, conv_k]` of the model dtype, `a_log` / `dt_bias` `[v_heads]` (taken in fp32). Returns fp32
    `q`, `k` `[B, t, k_heads, k_dim]` (L2-normalised, q scaled by k_dim^-1/2), `v`
    `[B, t, v_heads, v_dim]`, `g`, `beta` `[B, t, v_heads]`."""
    device = _mtpk.require_device(proj, conv_state, slots, conv_w, a_log, dt_bias)
    b, t, width = proj.shape
    rs = _mtpk.row_stride(proj)
    if proj.stride(2) != 1 or rs is None:
        raise ValueError("proj must be [B, t, P] with contiguous rows")
    dt = proj.dtype
    for name, ten in (("conv_state", conv_state), ("conv_w", conv_w)):
        if ten.dtype != dt or not ten.is_contiguous():
            raise ValueError(f"{name} must be contiguous {dt}")
    a_log = a_log.float().contiguous()
    dt_bias = dt_bias.float().contiguous()
    f32 = dict(dtype=torch.float32, device=device)
    q = torch.empty(b, t, k_heads, k_dim, **f32)
    k = torch.empty(b, t, k_heads, k_dim, **f32)
    v = torch.empty(b, t, v_heads, v_dim, **f32)
    g = torch.empty(b, t, v_heads, **f32)
    beta = torch.empty(b, t, v_heads, **f32)
    sl = slots.to(torch.int64).contiguous()
    _mtpk.check(_mtpk.lib().mtpk_deltanet_prep(
        proj.data_ptr(), _mtpk.float_code(dt), rs, conv_state.data_ptr(), sl.data_ptr(),
        conv_state.shape[0], conv_w.data_ptr(), a_log.data_ptr(), dt_bias.data_ptr(), b, t, k_heads, k_dim, v_heads, v_dim,
        conv_w.shape[1], float(eps), float(k_dim) ** -0.5, q.data_ptr(), k.data_ptr(), v.data_ptr(),
        g.data_ptr(), beta.data_ptr(), _mtpk.stream_of(device)), "mtpk_deltanet_prep")  # fmt: skip
    return q, k, v, g, beta


def conv_commit(conv_state: torch.Tensor, slots: torch.Tensor, proj: torch.Tensor,
                idx: torch.Tensor, channels: int) -> None:
    """Slot `slots[b]`'s conv window `conv_state[slot]` `[C, k1]` becomes columns `idx[b]`
    `[k1]` of [stored window | the t new raw columns], the raw columns being `proj[b, :, :C]`
    (`mtpk_conv_commit`)."""
    device = _mtpk.require_device(conv_state, slots, proj, idx)
    b, t, _ = proj.shape
    rs = _mtpk.row_stride(proj)
    if proj.stride(2) != 1 or rs is None:
        raise ValueError("proj must be [B, t, P] with contiguous rows")
    if proj.dtype != conv_state.dtype or not conv_state.is_contiguous():
        raise ValueError("conv_state must be contiguous and of proj's dtype")
    k1 = conv_state.shape[-1]
    ix = idx.to(torch.int64).contiguous()
    if ix.shape != (b, k1):
        raise ValueError(f"idx must be [{b}, {k1}]")
    sl = slots.to(torch.int64).contiguous()
    _mtpk.check(_mtpk.lib().mtpk_conv_commit(
        conv_state.data_ptr(), _mtpk.float_code(conv_state.dtype), sl.data_ptr(), conv_state.shape[0],
        proj.data_ptr(),
        rs, ix.data_ptr(), b, channels, k1, t, _mtpk.stream_of(device)),
        "mtpk_conv_commit")  # fmt: skip
