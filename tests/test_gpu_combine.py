"""The staged pieces at the reference's signatures: `mxfp4_gemv.bw_prep` / `BwPlan` and
`bw_combine` / `bw_combine_glue` (HIP `mtpk_moe_prep`, `mtpk_moe_combine_rows`).

Cases follow the reference's own tests (`seed_tests/test_moe_route_fused.py:101-165`): tokens 1,
7 and 48 over a 64-expert routing with the local span [16, 32), a zero-weight token, a gate read
through its own row stride, a mismatched `shared` rejected. Bars: `bw_combine` bit-identical to
the fp32 sum of the live rows in j order; `bw_combine_glue` bit-identical to `bw_combine` followed
by the three bf16 torch ops (`sigmoid`, `*`, `+`), and within the reference test's 2e-2 of the
fp32 form; dead rows of y (NaN-filled here) never read; the work list a partition of the live
assignments into units of <= 16 of one expert.
"""

import pytest
import torch

import mxfp4_gemv
from tests.moe_inputs import random_routing

pytestmark = pytest.mark.gpu

TOP_K = 10
HIDDEN = 4096
SPAN = (16, 32)


def inputs(dev, tokens, *, seed, zero_rows=(), y_dtype=torch.bfloat16):
    e, w = random_routing(tokens, 64, TOP_K, seed=seed, zero_rows=zero_rows)
    a_expert, a_weight = torch.from_numpy(e).to(dev), torch.from_numpy(w).to(dev)
    g = torch.Generator().manual_seed(seed + 1)
    y = torch.randn(tokens * TOP_K, HIDDEN, generator=g).to(y_dtype).to(dev)
    shared = torch.randn(tokens, HIDDEN, generator=g).to(torch.bfloat16).to(dev)
    gate = torch.randn(tokens, 1, generator=g).to(torch.bfloat16).to(dev)
    live = (a_expert >= SPAN[0]) & (a_expert < SPAN[1]) & (a_weight != 0)
    y[~live] = float("nan")  # dead rows must never be read
    return a_expert, a_weight, y, shared, gate, live


def live_sum(y, live, tokens):
    """fp32 sum of each token's live rows in j order (the kernel's order)."""
    yv = y.float().view(tokens, TOP_K, HIDDEN)
    lv = live.view(tokens, TOP_K)
    acc = torch.zeros(tokens, HIDDEN, device=y.device)
    for j in range(TOP_K):
        acc = torch.where(lv[:, j : j + 1], acc + yv[:, j], acc)
    return acc


@pytest.mark.parametrize("tokens", [1, 7, 48])
@pytest.mark.parametrize("y_dtype", [torch.bfloat16, torch.float32])
def test_bw_combine_sums_the_live_rows_in_order(dev, tokens, y_dtype):
    print(f"bw_combine tokens={tokens} y={y_dtype}", flush=True)
    a_expert, a_weight, y, _, _, live = inputs(dev, tokens, seed=3, zero_rows=(0,) if tokens > 1 else (),
                                               y_dtype=y_dtype)
    want = live_sum(y, live, tokens)
    for out_dtype in (torch.bfloat16, torch.float32):
        out = torch.full((tokens, HIDDEN), 7.0, dtype=out_dtype, device=dev)
        assert mxfp4_gemv.bw_combine(y, a_expert, a_weight, SPAN, TOP_K, out) is None
        assert torch.equal(out, want.to(out_dtype))
    if tokens > 1:  # the zero-weight token: exact zeros
        assert torch.equal(out[0], torch.zeros(HIDDEN, dtype=out.dtype, device=dev))


@pytest.mark.parametrize("tokens", [1, 7, 48])
def test_bw_combine_glue_matches_bw_combine_plus_glue(dev, tokens):
    print(f"bw_combine_glue tokens={tokens}", flush=True)
    a_expert, a_weight, y, shared, gate, _ = inputs(dev, tokens, seed=3, zero_rows=(0,) if tokens > 1 else ())
    unfused = torch.empty(tokens, HIDDEN, dtype=torch.bfloat16, device=dev)
    mxfp4_gemv.bw_combine(y, a_expert, a_weight, SPAN, TOP_K, unfused)
    chain = unfused + torch.sigmoid(gate) * shared  # bf16 ops, each rounded to bf16
    fused = torch.empty(tokens, HIDDEN, dtype=torch.bfloat16, device=dev)
    mxfp4_gemv.bw_combine_glue(y, a_expert, a_weight, SPAN, TOP_K, shared, gate, fused)
    assert torch.equal(fused, chain)
    want = unfused.float() + torch.sigmoid(gate.float()) * shared.float()
    err = (fused.float() - want).abs().max().item() / want.abs().max().clamp_min(1e-6).item()
    assert err < 2e-2


def test_bw_combine_glue_reads_gate_through_its_own_row_stride(dev):
    tokens = 5
    a_expert, a_weight, y, shared, _, _ = inputs(dev, tokens, seed=9)
    wide = torch.randn(tokens, 4, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16).to(dev)
    gate_view = wide[:, 3:]
    assert gate_view.stride(0) == 4
    unfused = torch.empty(tokens, HIDDEN, dtype=torch.bfloat16, device=dev)
    mxfp4_gemv.bw_combine(y, a_expert, a_weight, SPAN, TOP_K, unfused)
    fused = torch.empty(tokens, HIDDEN, dtype=torch.bfloat16, device=dev)
    mxfp4_gemv.bw_combine_glue(y, a_expert, a_weight, SPAN, TOP_K, shared, gate_view, fused)
    assert torch.equal(fused, unfused + torch.sigmoid(gate_view) * shared)


def test_bw_combine_glue_rejects_bad_shared_and_gate(dev):
    tokens = 3
    a_expert, a_weight, y, shared, gate, _ = inputs(dev, tokens, seed=1)
    out = torch.empty(tokens, HIDDEN, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="shared"):
        mxfp4_gemv.bw_combine_glue(y, a_expert, a_weight, SPAN, TOP_K, shared[:-1], gate, out)
    with pytest.raises(ValueError, match="gate"):
        mxfp4_gemv.bw_combine_glue(y, a_expert, a_weight, SPAN, TOP_K, shared,
                                   torch.zeros(2, tokens, device=dev).t(), out)
    with pytest.raises(ValueError, match="y"):
        mxfp4_gemv.bw_combine(y[:-1], a_expert, a_weight, SPAN, TOP_K, out)


@pytest.mark.parametrize("tokens", [1, 48, 192])
def test_bw_prep_partitions_the_live_assignments(dev, tokens):
    print(f"bw_prep tokens={tokens}", flush=True)
    e, w = random_routing(tokens, 64, TOP_K, seed=tokens, zero_rows=(0,) if tokens > 1 else ())
    a_expert, a_weight = torch.from_numpy(e).to(dev), torch.from_numpy(w).to(dev)
    x = torch.zeros(tokens, HIDDEN, dtype=torch.bfloat16, device=dev)
    plan = mxfp4_gemv.BwPlan(tokens, TOP_K, HIDDEN, SPAN[1] - SPAN[0], dev, torch.bfloat16)
    assert plan.block_t == 16 and plan.xp is None
    plan.sorted.fill_(-7)
    mxfp4_gemv.bw_prep(x, a_expert, a_weight, SPAN, plan)
    n = int(plan.n_units.item())
    units = plan.unit[: 3 * n].view(n, 3).cpu().tolist()
    order = plan.sorted.cpu().tolist()
    live = [a for a in range(tokens * TOP_K) if SPAN[0] <= e[a] < SPAN[1] and w[a] != 0]
    seen = []
    for ex, first, cnt in units:
        assert 1 <= cnt <= 16
        ids = order[first : first + cnt]
        assert all(e[a] - SPAN[0] == ex for a in ids)
        seen += ids
    assert sorted(seen) == live
    assert n <= plan.u_max
