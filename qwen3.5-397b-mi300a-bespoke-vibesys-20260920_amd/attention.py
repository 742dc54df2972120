"""Paged causal GQA attention of the verify rows on the device, through
`mtpk_paged_attention` (include/mtpk.h): the role of `verify_attention_paged`
(`model.py:1120-1205`) and, at t = 1, of the MTP draft step's attention (`mtp.py:233-279`).

q bf16 `[B, heads, t, hd]`; the K pool bf16 `[pool_rows, kv_heads, hd]` and the V pool bf16
`[pool_rows / 16, kv_heads, hd, 16]` of 16-row blocks: V is kept transposed inside each block
(`v_blocks`), so the kernel stages a V tile with contiguous reads and no transposition.
`block_table` int32 `[B, blocks]` (the lanes' own tables); `base_pos` int64 `[B]`: query row s
of lane b sits at `base_pos[b] + s` and sees every cached position up to its own. The output is
bf16 `[B, heads, t, hd]`.
"""

from __future__ import annotations

import ctypes

import torch

import _mtpk

BLOCK = 16
HEAD_DIMS = (64, 128, 256)


def v_blocks(v: torch.Tensor, block: int = BLOCK) -> torch.Tensor:
    """V rows `[rows, kv_heads, hd]` -> the V cache layout `[rows / block, kv_heads, hd, block]`."""
    rows, kvh, hd = v.shape
    return v.view(rows // block, block, kvh, hd).permute(0, 2, 3, 1).contiguous()


def v_rows(vt: torch.Tensor) -> torch.Tensor:
    """The V cache layout `[blocks, kv_heads, hd, block]` -> V rows `[blocks * block, kv_heads, hd]`."""
    nb, kvh, hd, bs = vt.shape
    return vt.permute(0, 3, 1, 2).reshape(nb * bs, kvh, hd)


def write_v(vt: torch.Tensor, rows: torch.Tensor, v: torch.Tensor) -> None:
    """Store V rows `v` `[n, kv_heads, hd]` at pool rows `rows` `[n]` of the V cache `vt`."""
    bs = vt.shape[-1]
    vt[rows // bs, :, :, rows % bs] = v


def read_v(vt: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """V rows at pool rows `rows` (any shape) of the V cache: `[*rows.shape, kv_heads, hd]`."""
    bs = vt.shape[-1]
    return vt[rows // bs, :, :, rows % bs]


def supported(q: torch.Tensor, block_size: int) -> bool:
    """Shapes the kernel takes: bf16 device tensors, 16-row blocks, head_dim 64/128/256."""
    return q.device.type == "cuda" and q.dtype == torch.bfloat16 and block_size == BLOCK and \
        q.shape[-1] in HEAD_DIMS


def paged_attention(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                    block_table: torch.Tensor, base_pos: torch.Tensor, ctx_len: int,
                    scale: float) -> torch.Tensor:
    """`ctx_len` is a host bound on `max(base_pos) + t`; it only sizes the key splits."""
    device = _mtpk.require_device(q, k_pool, v_pool, block_table, base_pos)
    if q.dim() != 4 or q.dtype != torch.bfloat16:
        raise ValueError(f"q must be bf16 [B, heads, t, hd], got {q.dtype} {tuple(q.shape)}")
    b, heads, t, hd = q.shape
    if k_pool.dim() != 3 or k_pool.shape[2] != hd or k_pool.shape[0] % BLOCK:
        raise ValueError(f"k_pool must be [rows, kv_heads, {hd}] of {BLOCK}-row blocks, got {tuple(k_pool.shape)}")
    if tuple(v_pool.shape) != (k_pool.shape[0] // BLOCK, k_pool.shape[1], hd, BLOCK):
        raise ValueError(f"v_pool must be [{k_pool.shape[0] // BLOCK}, {k_pool.shape[1]}, {hd}, {BLOCK}] "
                         f"(V transposed per block), got {tuple(v_pool.shape)}")
    if k_pool.dtype != torch.bfloat16 or v_pool.dtype != torch.bfloat16:
        raise ValueError("pools must be bf16")
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("pools must be contiguous")
    kvh = k_pool.shape[1]
    if heads % kvh:
        raise ValueError(f"{heads} q heads are not a multiple of {kvh} kv heads")
    if block_table.dim() != 2 or block_table.shape[0] != b:
        raise ValueError(f"block_table must be [{b}, blocks], got {tuple(block_table.shape)}")
    if tuple(base_pos.shape) != (b,):
        raise ValueError(f"base_pos must be [{b}], got {tuple(base_pos.shape)}")
    if int(ctx_len) > block_table.shape[1] * BLOCK:
        raise ValueError(f"context bound {ctx_len} exceeds the table's {block_table.shape[1]} blocks")
    q = q.contiguous()
    table = block_table.to(torch.int32).contiguous()
    pos = base_pos.to(torch.int64).contiguous()
    lib = _mtpk.lib()
    n_split = int(lib.mtpk_attention_splits(b, t, heads, kvh, hd, max(int(ctx_len), 1)))
    ws_bytes = int(lib.mtpk_attention_workspace_bytes(b, t, heads, kvh, hd, n_split))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    out = torch.empty_like(q)
    _mtpk.check(
        lib.mtpk_paged_attention(q.data_ptr(), b, t, heads, kvh, hd, k_pool.data_ptr(), v_pool.data_ptr(),
                                 k_pool.shape[0], table.data_ptr(), table.shape[1], pos.data_ptr(),
                                 float(scale), n_split, ws.data_ptr(), ws_bytes, out.data_ptr(),
                                 _mtpk.stream_of(device)),
        "mtpk_paged_attention",
    )
    return out


def _strides(x: torch.Tensor) -> ctypes.Array:
    """(lane, head, step) element strides of a `[B, t, heads, hd]` tensor, as int64[3]."""
    return (ctypes.c_int64 * 3)(x.stride(0), x.stride(2), x.stride(1))


def paged_attention_gated(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                          block_table: torch.Tensor, base_pos: torch.Tensor, ctx_len: int,
                          scale: float, gate: torch.Tensor | None = None) -> torch.Tensor:
    """`paged_attention` on q `[B, t, heads, hd]` (the q-norm output's layout: any strides,
    unit stride over hd), output `[B, t, heads, hd]` contiguous, times `sigmoid(gate)` when
    `gate` `[B, t, heads, hd]` is given (`mtpk_paged_attention_gated`), with the unfused bf16
    ops' rounding."""
    device = _mtpk.require_device(q, k_pool, v_pool, block_table, base_pos)
    if q.dim() != 4 or q.dtype != torch.bfloat16 or q.stride(3) != 1:
        raise ValueError(f"q must be bf16 [B, t, heads, hd] with unit stride over hd, got {tuple(q.shape)}")
    b, t, heads, hd = q.shape
    if gate is not None and (gate.shape != q.shape or gate.dtype != torch.bfloat16 or gate.stride(3) != 1):
        raise ValueError("gate must be bf16 of q's shape with unit stride over hd")
    if k_pool.dim() != 3 or k_pool.shape[2] != hd or k_pool.shape[0] % BLOCK:
        raise ValueError(f"k_pool must be [rows, kv_heads, {hd}] of {BLOCK}-row blocks, got {tuple(k_pool.shape)}")
    if tuple(v_pool.shape) != (k_pool.shape[0] // BLOCK, k_pool.shape[1], hd, BLOCK):
        raise ValueError(f"v_pool must be [{k_pool.shape[0] // BLOCK}, {k_pool.shape[1]}, {hd}, {BLOCK}] "
                         f"(V transposed per block), got {tuple(v_pool.shape)}")
    if k_pool.dtype != torch.bfloat16 or v_pool.dtype != torch.bfloat16 or not (
            k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("pools must be contiguous bf16")
    kvh = k_pool.shape[1]
    if heads % kvh:
        raise ValueError(f"{heads} q heads are not a multiple of {kvh} kv heads")
    if block_table.dim() != 2 or block_table.shape[0] != b or tuple(base_pos.shape) != (b,):
        raise ValueError("block_table must be [B, blocks] and base_pos [B]")
    if int(ctx_len) > block_table.shape[1] * BLOCK:
        raise ValueError(f"context bound {ctx_len} exceeds the table's {block_table.shape[1]} blocks")
    table = block_table.to(torch.int32).contiguous()
    pos = base_pos.to(torch.int64).contiguous()
    lib = _mtpk.lib()
    n_split = int(lib.mtpk_attention_splits(b, t, heads, kvh, hd, max(int(ctx_len), 1)))
    ws_bytes = int(lib.mtpk_attention_workspace_bytes(b, t, heads, kvh, hd, n_split))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    out = torch.empty(b, t, heads, hd, dtype=torch.bfloat16, device=device)
    qs, os_ = _strides(q), _strides(out)
    gs = _strides(gate) if gate is not None else None
    _mtpk.check(
        lib.mtpk_paged_attention_gated(
            q.data_ptr(), ctypes.addressof(qs), _mtpk.ptr(gate), ctypes.addressof(gs) if gs else None,
            b, t, heads, kvh, hd, k_pool.data_ptr(), v_pool.data_ptr(), k_pool.shape[0], table.data_ptr(),
            table.shape[1], pos.data_ptr(), float(scale), n_split, ws.data_ptr(), ws_bytes,
            out.data_ptr(), ctypes.addressof(os_), _mtpk.stream_of(device)),
        "mtpk_paged_attention_gated",
    )  # fmt: skip
    return out


def kv_write(k_pool: torch.Tensor, v_pool: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             block_table: torch.Tensor, base_pos: torch.Tensor, keep: torch.Tensor | None = None) -> None:
    """Store K/V rows `k`, `v` `[B, t, kv_heads, hd]` (inner two dims contiguous, rows at any
    stride) at positions `base_pos[b] + s` through the lanes' `block_table` `[B, blocks]` into
    the K pool and the block-transposed V pool (`mtpk_kv_write`); rows with `keep[b, s]` False
    are left as they are."""
    device = _mtpk.require_device(k_pool, v_pool, k, v, block_table, base_pos)
    b, t, kvh, hd = k.shape
    for name, x in (("k", k), ("v", v)):
        if x.dtype != torch.bfloat16 or x.shape != (b, t, kvh, hd) or x.stride(3) != 1 or x.stride(2) != hd \
                or _mtpk.row_stride(x) is None:
            raise ValueError(f"{name} must be bf16 [B, t, kv_heads, hd] with contiguous rows")
    if k_pool.shape[1:] != (kvh, hd) or v_pool.shape[1:] != (kvh, hd, BLOCK):
        raise ValueError("pools do not match the rows' kv_heads / head_dim")
    table = block_table.to(torch.int32).contiguous()
    pos = base_pos.to(torch.int64).contiguous()
    kp, kb, ks = None, 0, 0
    if keep is not None:
        if keep.numel() != b * t:
            raise ValueError("keep must have B * t entries")
        # read in place through its strides (a per-lane mask broadcast over t has stride 0);
        # a bool tensor's bytes are its 0 / 1 values
        kp = keep.to(device).reshape(b, t)
        kp = kp.view(torch.uint8) if kp.dtype == torch.bool else kp.to(torch.uint8)
        kb, ks = kp.stride()
    _mtpk.check(_mtpk.lib().mtpk_kv_write(
        k.data_ptr(), _mtpk.row_stride(k), v.data_ptr(), _mtpk.row_stride(v), k_pool.data_ptr(), v_pool.data_ptr(),
        k_pool.shape[0], table.data_ptr(), table.shape[1], pos.data_ptr(), _mtpk.ptr(kp), kb, ks, b, t,
        kvh, hd, _mtpk.stream_of(device)), "mtpk_kv_write")  # fmt: skip
