"""Host-side pieces of `mxfp4_gemv` that run on CPU tensors: `align_blocks` (the reference test's
partition property, `test_mxfp4_fused_gemv.py:430-459`, plus block contiguity) and the torch
`reference_moe` path against the fp64 oracle."""

import numpy as np
import pytest
import torch

import mxfp4
import mxfp4_gemv
from oracle import moe_ref
from tests.moe_inputs import random_experts, random_routing


@pytest.mark.parametrize("assignments,experts,block_m", [(30, 4, 16), (12, 3, 16), (7, 2, 32), (0, 3, 16),
                                                         (200, 9, 16), (64, 1, 16)])
def test_align_blocks_partition(assignments, experts, block_m):
    g = torch.Generator().manual_seed(assignments + experts)
    a_expert = torch.randint(0, experts, (assignments,), dtype=torch.int32, generator=g)
    a_weight = torch.rand(assignments, generator=g)
    a_weight[::5] = 0.0
    slot, block_expert = mxfp4_gemv.align_blocks(a_expert, a_weight, (0, experts), block_m)
    assert block_expert.numel() == mxfp4_gemv.grouped_block_count(assignments, experts, block_m)
    assert slot.numel() == block_expert.numel() * block_m
    assert sorted(slot[slot >= 0].tolist()) == list(range(assignments))
    live = a_weight != 0
    for b in range(block_expert.numel()):
        e = int(block_expert[b])
        rows = slot[b * block_m : (b + 1) * block_m]
        held = rows[rows >= 0]
        # a block's rows are filled from the front, in assignment order
        assert (rows[: held.numel()] >= 0).all() and torch.equal(held, held.sort().values)
        for r in held.tolist():
            assert (int(a_expert[r]) == e) if live[r] else (e == experts)
    # each bucket's blocks are consecutive, in bucket order
    owners = block_expert.tolist()
    assert owners == sorted(owners)


def test_align_blocks_expert_range_offset():
    a_expert = torch.tensor([5, 6, 9, 5, 7, 6], dtype=torch.int64)
    a_weight = torch.ones(6)
    slot, owner = mxfp4_gemv.align_blocks(a_expert, a_weight, (5, 8), 2)
    # experts 5, 6, 7 are local 0, 1, 2; id 9 is unowned and lands in the sentinel bucket 3
    got = {int(owner[b]): sorted(v for v in slot[2 * b : 2 * b + 2].tolist() if v >= 0)
           for b in range(owner.numel()) if (slot[2 * b : 2 * b + 2] >= 0).any()}
    assert got == {0: [0, 3], 1: [1, 5], 2: [4], 3: [2]}


@pytest.mark.parametrize("seed", [0, 1])
def test_reference_moe_matches_the_fp64_oracle(seed):
    ex = random_experts(6, 64, 32, seed=seed)
    a_e, a_w = random_routing(5, 6, 2, seed=seed + 10, zero_rows=(3,))
    x = np.random.default_rng(seed).standard_normal((5, 64)).astype(np.float32)
    tex = {k: torch.from_numpy(v) for k, v in ex.items()}
    got = mxfp4_gemv.reference_moe(torch.from_numpy(x), tex, (torch.from_numpy(a_e), torch.from_numpy(a_w)),
                                   2, (0, 6), mxfp4.dequant_mxfp4, chunk=2).numpy()
    want = moe_ref.reference_moe(x, ex, a_e, a_w, 2, (0, 6))
    assert moe_ref.rel_l2(got, want) < 1e-6
    assert not got[3].any()


def test_staged_pieces_keep_the_reference_signatures():
    """`bw_prep`, `BwPlan`, `bw_combine` and `bw_combine_glue` take the reference's parameters
    (mxfp4_gemv.py:2320-2346, :2349, :2440, :2449)."""
    import inspect

    names = lambda f: list(inspect.signature(f).parameters)  # noqa: E731
    assert names(mxfp4_gemv.bw_prep) == ["x", "a_expert", "a_weight", "expert_range", "plan"]
    assert names(mxfp4_gemv.bw_combine) == ["y", "a_expert", "a_weight", "expert_range", "top_k", "out"]
    assert names(mxfp4_gemv.bw_combine_glue) == ["y", "a_expert", "a_weight", "expert_range", "top_k",
                                                 "shared", "gate", "out"]
    assert names(mxfp4_gemv.BwPlan) == ["tokens", "top_k", "reduction", "local_experts", "device", "dtype",
                                        "block_t", "permute_x"]


def test_bw_plan_sizes_and_rejections():
    plan = mxfp4_gemv.BwPlan(48, 10, 4096, 512, torch.device("cpu"), torch.bfloat16)
    assert plan.block_t == 16 and plan.cursor is None and plan.xp is None
    assert plan.sorted.shape == (480,) and plan.unit.shape == (3 * plan.u_max,)
    # each live expert adds at most one partial unit beyond the full ones
    assert plan.u_max >= min(512, 480) and plan.u_max <= min(512, 480) + 480 // 16
    with pytest.raises(ValueError, match="block_t"):
        mxfp4_gemv.BwPlan(48, 10, 4096, 512, torch.device("cpu"), torch.bfloat16, block_t=32)
    x = torch.zeros(48, 4096, dtype=torch.bfloat16)
    e, w = random_routing(48, 512, 10, seed=0)
    with pytest.raises(ValueError, match="device tensors"):
        mxfp4_gemv.bw_prep(x, torch.from_numpy(e), torch.from_numpy(w), (0, 512), plan)
    out = torch.empty(48, 4096, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device tensors"):
        mxfp4_gemv.bw_combine(torch.zeros(480, 4096), torch.from_numpy(e), torch.from_numpy(w), (0, 512), 10, out)
