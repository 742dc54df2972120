"""The HIP paged verify attention (`attention.paged_attention` -> `mtpk_paged_attention`)
against the float64 oracle (`oracle/attention_ref.py`) on bf16 inputs.

Bar: the kernel computes scores and softmax in fp32 but feeds bf16 probabilities to the PV
MFMA and stores bf16, so outputs agree to rel-L2 <= 4e-3 over the whole output and max |diff|
<= 2e-2 (values are O(1)). Cases: config 5's shapes (32 q / 2 kv heads of 256, t = 4 verify and
t = 1 draft), ragged contexts across lanes (single-split and multi-split paths), head_dim 64
and 128, more than 64 query rows per kv head, and shuffled block tables."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import attention
from oracle import attention_ref as ar

pytestmark = pytest.mark.gpu

REL_L2, MAX_ABS = 4e-3, 2e-2


def _case(seed, b, heads, kvh, hd, t, base, max_blocks):
    rng = np.random.default_rng(seed)
    pool_rows = (b * max_blocks + 1) * 16
    perm = rng.permutation(np.arange(1, b * max_blocks + 1))  # block 0 stays unused
    table = perm.reshape(b, max_blocks).astype(np.int32)
    to_bf = lambda a: torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16)
    q = to_bf(rng.standard_normal((b, heads, t, hd)))
    k = to_bf(rng.standard_normal((pool_rows, kvh, hd)))
    v = to_bf(rng.standard_normal((pool_rows, kvh, hd)))
    return q, k, v, table, np.asarray(base, np.int64)


def _check(dev, q, k, v, table, base, scale):
    t = q.shape[2]
    ctx = int(base.max()) + t
    got = attention.paged_attention(q.to(dev), k.to(dev), attention.v_blocks(v).to(dev),
                                    torch.from_numpy(table).to(dev),
                                    torch.from_numpy(base).to(dev), ctx, scale)
    want = ar.paged_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), table, base, scale)
    got = got.float().cpu().numpy()
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel <= REL_L2, rel
    assert np.abs(got - want).max() <= MAX_ABS


@pytest.mark.parametrize("t", [4, 1])
def test_config5_heads_ragged_lanes(dev, t) -> None:
    """32 q / 2 kv heads of 256; lanes at 0, 17, 300 and 1100 cached positions."""
    q, k, v, table, base = _case(t, 4, 32, 2, 256, t, [0, 17, 300, 1100], 72)
    _check(dev, q, k, v, table, base, 256 ** -0.5)


@pytest.mark.parametrize("hd", [64, 128])
def test_other_head_dims(dev, hd) -> None:
    q, k, v, table, base = _case(hd, 3, 8, 2, hd, 3, [40, 5, 700], 48)
    _check(dev, q, k, v, table, base, hd ** -0.5)


def test_many_rows_per_kv_head(dev) -> None:
    """16 q heads per kv head x t = 8 = 128 query rows: two row groups per (lane, kv head)."""
    q, k, v, table, base = _case(5, 2, 16, 1, 128, 8, [90, 400], 32)
    _check(dev, q, k, v, table, base, 0.09)


def test_long_context_splits(dev) -> None:
    """8192-position contexts at config 5's batch-48 shape for 2 lanes: many key splits."""
    q, k, v, table, base = _case(6, 2, 32, 2, 256, 4, [8188, 6000], 513)
    _check(dev, q, k, v, table, base, 256 ** -0.5)


def test_rejects_bad_arguments(dev) -> None:
    q, k, v, table, base = _case(7, 1, 4, 2, 64, 1, [3], 2)
    args = dict(block_table=torch.from_numpy(table).to(dev), base_pos=torch.from_numpy(base).to(dev),
                ctx_len=4, scale=0.1)
    with pytest.raises(ValueError):
        attention.paged_attention(q.to(dev).float(), k.to(dev), v.to(dev), **args)
    with pytest.raises(ValueError):
        attention.paged_attention(q.to(dev), k.to(dev)[:, :1].contiguous(), v.to(dev), **args)
    with pytest.raises(ValueError):
        attention.paged_attention(q.to(dev)[..., :32].contiguous(), k.to(dev)[..., :32].contiguous(),
                                  v.to(dev)[..., :32].contiguous(), **args)


@pytest.mark.parametrize("keep_some", [False, True, "lanes"])
def test_kv_write_matches_the_indexed_writes(dev, keep_some) -> None:
    """`attention.kv_write` (positions mapped through the block tables in the kernel) stores
    exactly what the indexed K write and `write_v` store, and nothing else; `keep` per row, or
    a per-lane mask broadcast over the round's rows (read in place, stride 0)."""
    import verify_model as vm

    b, t, kvh, hd, lanes_total = 3, 4, 2, 256, 5
    blocks = vm.BlockTables(lanes_total, 64, 16, dev, seed=3)
    lanes = torch.tensor([4, 0, 2], device=dev)
    base = torch.tensor([13, 0, 30], device=dev)  # block crossings inside the round
    for lane, p in zip(lanes.tolist(), base.tolist(), strict=True):
        blocks.grow(lane, p + t)
    g = torch.Generator(device="cpu").manual_seed(5)
    k = torch.randn(b, t, kvh, hd, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(b, t, kvh, hd, generator=g).to(torch.bfloat16).to(dev)
    kp = torch.randn(blocks.rows, kvh, hd, generator=g).to(torch.bfloat16).to(dev)
    vp = torch.randn(blocks.rows // 16, kvh, hd, 16, generator=g).to(torch.bfloat16).to(dev)
    keep = None
    if keep_some == "lanes":
        keep = torch.tensor([True, False, True], device=dev)[:, None].expand(b, t)
    elif keep_some:
        keep = torch.arange(t, device=dev)[None, :] <= torch.tensor([0, 3, 1], device=dev)[:, None]
    want_k, want_v = kp.clone(), vp.clone()
    pos = base[:, None] + torch.arange(t, device=dev)[None, :]
    rows = blocks.physical_rows(lanes, pos).reshape(-1)
    sel = torch.ones(b * t, dtype=torch.bool, device=dev) if keep is None else keep.reshape(-1)
    want_k[rows[sel]] = k.reshape(-1, kvh, hd)[sel]
    attention.write_v(want_v, rows[sel], v.reshape(-1, kvh, hd)[sel])
    attention.kv_write(kp, vp, k, v, blocks.table[lanes], base, keep)
    assert torch.equal(kp, want_k)
    assert torch.equal(vp, want_v)


@pytest.mark.parametrize("t,ctx", [(4, 200), (1, 8192), (4, 8192)])
def test_gated_layout_equals_the_unfused_ops(dev, t, ctx) -> None:
    """`paged_attention_gated` on the q-norm layout with the gate in the epilogue equals the
    transposes + `paged_attention` + `out * sigmoid(gate)` as bf16 torch ops, bit for bit (one
    key split and several)."""
    import verify_model as vm

    b, heads, kvh, hd = 3, 32, 2, 256
    blocks = vm.BlockTables(b, ctx + t, 16, dev, seed=2)
    base = torch.tensor([ctx - t, ctx // 3, 7], device=dev)
    for lane in range(b):
        blocks.grow(lane, int(base[lane]) + t)
    g = torch.Generator(device="cpu").manual_seed(t)
    kp = torch.randn(blocks.rows, kvh, hd, generator=g).to(torch.bfloat16).to(dev)
    vp = torch.randn(blocks.rows // 16, kvh, hd, 16, generator=g).to(torch.bfloat16).to(dev)
    qg = torch.randn(b, t, heads, 2 * hd, generator=g).to(torch.bfloat16).to(dev)
    q, gate = qg[..., :hd], qg[..., hd:]  # strided views, as the model holds them
    table, lanes = blocks.table, torch.arange(b, device=dev)
    want = attention.paged_attention(q.transpose(1, 2), kp, vp, table[lanes], base, ctx + t, hd ** -0.5)
    want = want.transpose(1, 2) * torch.sigmoid(gate)
    got = attention.paged_attention_gated(q, kp, vp, table[lanes], base, ctx + t, hd ** -0.5, gate)
    assert got.is_contiguous() and torch.equal(got, want)
    plain = attention.paged_attention_gated(q, kp, vp, table[lanes], base, ctx + t, hd ** -0.5)
    ref = attention.paged_attention(q.transpose(1, 2), kp, vp, table[lanes], base, ctx + t, hd ** -0.5)
    assert torch.equal(plain, ref.transpose(1, 2))
