"""Row normalisations of the verify / draft forward on the device (`mtpk_rownorm`).

Each call is one launch in place of the chain of elementwise and reduction kernels the torch
spelling takes (`model.py:587-604` RMSNorm with `1 + w`, `model.py:613-619` the DeltaNet
output norm, the DeltaNet q/k L2 norm, `model.py:631-635` rotate-half RoPE). The inputs may be
head slices of a projection output (last dim contiguous, one stride per head and one per
token); outputs are new contiguous tensors. Device tensors only: the model keeps the torch
spelling for CPU tensors.
"""

from __future__ import annotations

import torch

import _mtpk

RMS, GATED, L2 = 0, 1, 2


def _layout(x: torch.Tensor, heads: bool) -> tuple[int, int, int, int]:
    """(token stride, head stride, heads per token, rows) of `x` `[..., dim]` or, with
    `heads`, `[..., heads, dim]`, in elements."""
    if x.stride(-1) != 1:
        raise ValueError("the normalised dim must be contiguous")
    dim = x.shape[-1]
    if not heads:
        lead = x.shape[:-1]
        strides = x.stride()[:-1]
        hpt, hs = 1, dim
    else:
        lead = x.shape[:-2]
        strides = x.stride()[:-2]
        hpt, hs = x.shape[-2], x.stride(-2)
    # A size-1 dim's stride is arbitrary (views and reshapes set it freely), so only the dims
    # of size > 1 set and check the token stride.
    kept = [(n, s) for n, s in zip(lead, strides, strict=True) if n != 1]
    ts = kept[-1][1] if kept else hpt * hs
    for (_, s_outer), (n_inner, s_inner) in zip(kept, kept[1:]):
        if s_outer != s_inner * n_inner:
            raise ValueError("leading dims of the input do not collapse to one token stride")
    tokens = 1
    for n in lead:
        tokens *= n
    return ts, hs, hpt, tokens * hpt


def _launch(x, *, kind, w=None, eps=0.0, scale=1.0, gate=None, heads=False, res=None,
            rope=None, out_dtype=None, gather=None, out=None):
    dev = _mtpk.require_device(x)
    dim = x.shape[-1]
    ts, hs, hpt, rows = _layout(x, heads)
    shape, gp, g_stride, g_rows = x.shape, None, 0, 0
    if gather is not None:
        if heads or res is not None or gate is not None or x.dim() != 2:
            raise ValueError("a gather reads whole rows of a [rows, dim] table")
        if gather.dtype != torch.int64 or gather.device != dev:
            raise ValueError("gather must be an int64 device tensor")
        gp = gather.reshape(-1)
        shape, rows, g_stride, g_rows = (*gather.shape, dim), gp.numel(), gp.stride(0), x.shape[0]
    o_ts = 0
    if out is None:
        out = torch.empty(shape, dtype=out_dtype or x.dtype, device=dev)
    else:
        if out.shape != shape or out.dtype != (out_dtype or x.dtype) or out.device != dev:
            raise ValueError(f"out must be {tuple(shape)} {out_dtype or x.dtype} on {dev}")
        o_ts, o_hs, _, _ = _layout(out, heads)
        if heads and o_hs != dim:
            raise ValueError("out's heads must be packed")
    g_ts = g_hs = 0
    if gate is not None:
        if gate.shape != x.shape:
            raise ValueError("gate must match x's shape")
        g_ts, g_hs, _, _ = _layout(gate, heads)
    sum_out = None
    if res is not None:
        if res.shape != x.shape or not res.is_contiguous() or not x.is_contiguous():
            raise ValueError("the residual form takes contiguous x and res of one shape")
        sum_out = torch.empty_like(x)
    cos = sin = pos = None
    rot = 0
    if rope is not None:
        cos, sin, pos = rope
        rot = cos.shape[-1]
        pos = pos.to(torch.int64).contiguous()
    lib = _mtpk.lib()
    _mtpk.check(lib.mtpk_rownorm(
        x.data_ptr(), _mtpk.float_code(x.dtype), ts, hs,
        _mtpk.ptr(res), _mtpk.float_code(res.dtype) if res is not None else 0, _mtpk.ptr(sum_out),
        _mtpk.ptr(w), _mtpk.float_code(w.dtype) if w is not None else 0, kind, float(eps), float(scale),
        _mtpk.ptr(gate), _mtpk.float_code(gate.dtype) if gate is not None else 0, g_ts, g_hs,
        _mtpk.ptr(cos), _mtpk.ptr(sin), _mtpk.ptr(pos), rot,
        out.data_ptr(), _mtpk.float_code(out.dtype), rows, hpt, dim, _mtpk.ptr(gp), g_stride, g_rows,
        o_ts, _mtpk.stream_of(dev),
    ), "mtpk_rownorm")  # fmt: skip
    return out if res is None else (sum_out, out)


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, *, heads: bool = False,
            rope: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
            gather: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """`x * rsqrt(mean(x^2) + eps) * (1 + w)` in fp32, x's dtype out. `rope = (cos, sin, pos)`
    then rotates the first `cos.shape[-1]` channels at `pos[token]` (fp32 tables
    `[positions, rot]`; `pos` one entry per token, i.e. per `x.shape[:-2]` element with
    `heads`). `gather` (int64, any shape and strides): normalise rows `x[gather]` of the table
    `x` `[rows, dim]` (the embedding lookup fused; ids are clamped into the table, so callers
    check them). `out`: write into this tensor (last dim contiguous, rows at one stride, e.g.
    one half of a concatenated row) instead of a new one; returned."""
    return _launch(x, kind=RMS, w=w, eps=eps, heads=heads, rope=rope, gather=gather, out=out)


def add_rmsnorm(x: torch.Tensor, res: torch.Tensor, w: torch.Tensor,
                eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """`s = x + res` (x's dtype) and `rmsnorm(s, w, eps)`, in one launch: returns `(s, normed)`."""
    return _launch(x, kind=RMS, w=w, eps=eps, res=res)


def gated_rmsnorm(x: torch.Tensor, gate: torch.Tensor, w: torch.Tensor, eps: float,
                  dtype: torch.dtype) -> torch.Tensor:
    """`x * rsqrt(mean(x^2) + eps) * w * silu(gate)` over `[..., heads, dim]`, `dtype` out."""
    return _launch(x, kind=GATED, w=w, eps=eps, gate=gate, heads=True, out_dtype=dtype)


def l2norm(x: torch.Tensor, eps: float = 1e-6, scale: float = 1.0,
           out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """`x * rsqrt(sum(x^2) + eps) * scale` over `[..., heads, dim]`."""
    return _launch(x, kind=L2, eps=eps, scale=scale, heads=True, out_dtype=out_dtype)
