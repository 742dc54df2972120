"""The `mtpk` custom ops on the device: `torch.library.opcheck` (schema, fake kernel against the
real one, autograd registration, AOT dispatch with dynamic shapes), bit-equality with the Python
wrappers they dispatch to, a HIP graph that replays all five ops, and `torch.compile`
(aot_eager backend) tracing through them as single nodes."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import graph_mtp
import mtp
import mtpk_ops
import mxfp4_gemv
import router_fused
from tests.moe_inputs import random_experts, random_routing

pytestmark = pytest.mark.gpu

E, H, I, K, T = 16, 256, 128, 4, 6
B, KD, V = 5, 3, 1000


def moe_args(dev, tokens=T):
    ex = {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev)
          for k, v in random_experts(E, H, I, seed=3).items()}
    a_e, a_w = random_routing(tokens, E, K, seed=4)
    g = torch.Generator(dev).manual_seed(5)
    x = torch.randn(tokens, H, device=dev, generator=g).to(torch.bfloat16)
    shared = torch.randn(tokens, H, device=dev, generator=g).to(torch.bfloat16)
    gate = torch.randn(tokens, 1, device=dev, generator=g).to(torch.bfloat16)
    return (x, ex["gate_up"], ex["gate_up_scale"], ex["down"], ex["down_scale"],
            torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev), K, 0, E, shared, gate)


def layer_args(dev, tokens=T):
    """A small whole layer: hidden 256, 16 experts (I = 128), shared expert 256."""
    x, gu, gus, dn, dns = moe_args(dev, tokens)[:5]
    g = torch.Generator(dev).manual_seed(11)
    rg = (torch.randn(E + 1, H, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    sgu = (torch.randn(2 * 256, H, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    sdn = (torch.randn(H, 256, device=dev, generator=g) * 0.05).to(torch.bfloat16)
    return x, rg, sgu, sdn, gu, gus, dn, dns, K, 0, E


def accept_args(dev):
    g = torch.Generator(dev).manual_seed(7)
    step = torch.randint(0, 9, (B, KD + 1), device=dev, generator=g)
    draft = torch.where(torch.rand(B, KD, device=dev, generator=g) < 0.7, step[:, :KD],
                        torch.randint(0, 9, (B, KD), device=dev, generator=g))
    active = torch.tensor([True, True, False, True, True], device=dev)
    pos = torch.randint(0, 100, (B,), device=dev, generator=g)
    budget = torch.tensor([9, 1, 5, 2, 9], device=dev)
    stops = torch.full((B, mtp.MAX_STOP_IDS), -1, dtype=torch.long, device=dev)
    stops[0, 0] = 3
    return step, draft, active, pos, budget, stops, 3


def rejection_args(dev):
    g = torch.Generator(dev).manual_seed(8)
    tl = torch.randn(B, KD + 1, V, device=dev, generator=g)
    dl = tl[:, :KD] + 0.3 * torch.randn(B, KD, V, device=dev, generator=g)
    dt = torch.randint(0, V, (B, KD), device=dev, generator=g)
    return (tl, dl.contiguous(), dt, torch.rand(B, KD, device=dev, generator=g),
            torch.rand(B, device=dev, generator=g), 0.8)


def route_args(dev):
    r = torch.randn(T, E + 1, device=dev, generator=torch.Generator(dev).manual_seed(9))
    return r.to(torch.bfloat16), E, K, torch.int32


def argmax_args(dev):
    x = torch.randn(2, 3, V, device=dev, generator=torch.Generator(dev).manual_seed(10))
    x[0, 1, 17] = x[0, 1, 400] = 1e4  # a tie: the first occurrence wins
    return (x,)


CASES = {
    "fused_moe": (torch.ops.mtpk.fused_moe.default, moe_args),
    "moe_layer": (torch.ops.mtpk.moe_layer.default, layer_args),
    "route": (torch.ops.mtpk.route.default, route_args),
    "argmax_rows": (torch.ops.mtpk.argmax_rows.default, argmax_args),
    "greedy_accept": (torch.ops.mtpk.greedy_accept.default, accept_args),
    "rejection_sample": (torch.ops.mtpk.rejection_sample.default, rejection_args),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_opcheck(dev, name):
    op, make = CASES[name]
    if name in ("fused_moe", "moe_layer"):
        mxfp4_gemv.supports({k: v for k, v in zip(("gate_up", "gate_up_scale", "down", "down_scale"),
                                                   moe_args(dev)[1:5], strict=True)})
    torch.library.opcheck(op, make(dev))


def test_ops_equal_the_wrappers(dev):
    args = moe_args(dev)
    x, gu, gus, dn, dns, ae, aw, k, lo, hi, shared, gate = args
    ex = {"gate_up": gu, "gate_up_scale": gus, "down": dn, "down_scale": dns}
    want = mxfp4_gemv.fused_moe(x, ex, (ae, aw), k, (lo, hi), shared=shared, shared_gate=gate)
    assert torch.equal(torch.ops.mtpk.fused_moe(*args), want)
    la = layer_args(dev)
    h, rg, sgu, sdn = la[:4]
    tw = torch.empty(T, K, device=dev)
    ti = torch.empty(T, K, dtype=torch.int32, device=dev)
    want = mxfp4_gemv.fused_moe_layer(h, rg, sgu, sdn, ex, K, (lo, hi), routing_out=(tw, ti))
    for a, b in zip(torch.ops.mtpk.moe_layer(*la), (want, tw, ti), strict=True):
        assert torch.equal(a, b)
    r, e, kk, dt = route_args(dev)
    for a, b in zip(torch.ops.mtpk.route(r, e, kk, dt), router_fused.route(r, e, kk, index_dtype=dt),
                    strict=True):
        assert torch.equal(a, b)
    (lg,) = argmax_args(dev)
    got = torch.ops.mtpk.argmax_rows(lg)
    assert torch.equal(got, mtp.argmax_rows(lg)) and int(got[0, 1]) == 17
    res = graph_mtp.greedy_accept(*accept_args(dev))
    fields = ("accept_len", "lengths", "packed_src", "packed_cu", "conv_idx", "keep", "bonus",
              "next_pos", "budget_left", "live", "hidden_src")
    for f, got in zip(fields, torch.ops.mtpk.greedy_accept(*accept_args(dev)), strict=True):
        assert torch.equal(got, getattr(res, f)), f
    want = graph_mtp.rejection_sample(*rejection_args(dev), with_margin=True)
    for a, b in zip(torch.ops.mtpk.rejection_sample(*rejection_args(dev)), want, strict=True):
        assert torch.equal(a, b)


def _all_ops(moe, rt, am, acc, rej):
    out = torch.ops.mtpk.fused_moe(*moe)
    w, i = torch.ops.mtpk.route(*rt)
    best = torch.ops.mtpk.argmax_rows(*am)
    a = torch.ops.mtpk.greedy_accept(*acc)
    r = torch.ops.mtpk.rejection_sample(*rej)
    return [out, w, i, best, *a, *r]


def test_graph_replays_all_ops(dev):
    """Captured once, replayed three times with other eager work and a sync between: every
    replay equals the eager result (no memset nodes, no per-call allocation in the graph)."""
    moe, rt, am, acc, rej = moe_args(dev), route_args(dev), argmax_args(dev), accept_args(dev), rejection_args(dev)
    want = [t.clone() for t in _all_ops(moe, rt, am, acc, rej)]
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        _all_ops(moe, rt, am, acc, rej)  # warm-up off the capture
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = _all_ops(moe, rt, am, acc, rej)
    for r in range(3):
        for t in outs:
            t.zero_() if t.dtype != torch.bool else t.fill_(False)
        graph.replay()
        torch.cuda.synchronize(dev)
        _ = (torch.randn(128, 128, device=dev) @ torch.randn(128, 128, device=dev)).sum().item()
        for j, (g, w) in enumerate(zip(outs, want, strict=True)):
            assert torch.equal(g, w), (r, j)


def test_compile_traces_the_ops(dev):
    moe, rt, am, acc, rej = moe_args(dev), route_args(dev), argmax_args(dev), accept_args(dev), rejection_args(dev)
    want = _all_ops(moe, rt, am, acc, rej)
    compiled = torch.compile(_all_ops, backend="aot_eager", fullgraph=True)
    for g, w in zip(compiled(moe, rt, am, acc, rej), want, strict=True):
        assert torch.equal(g, w)


def test_reference_sized_scratch_allocates_nothing_per_call(dev):
    """The reference's `[max_batch * top_k, intermediate]` scratch is too small for the kernels'
    workspace; such calls share one grow-only workspace per stream, so repeated calls leave the
    allocator's count of allocations unchanged."""
    x, gu, gus, dn, dns, ae, aw, k, lo, hi, shared, gate = moe_args(dev)
    ex = {"gate_up": gu, "gate_up_scale": gus, "down": dn, "down_scale": dns}
    small = torch.empty(T * K, I, dtype=torch.bfloat16, device=dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    want = mxfp4_gemv.fused_moe(x, ex, (ae, aw), k, (lo, hi), inter=small).clone()
    torch.cuda.synchronize(dev)
    before = torch.cuda.memory_stats(dev)["allocation.all.allocated"]
    for _ in range(5):
        mxfp4_gemv.fused_moe(x, ex, (ae, aw), k, (lo, hi), out=out, inter=small)
    torch.cuda.synchronize(dev)
    assert torch.cuda.memory_stats(dev)["allocation.all.allocated"] == before
    assert torch.equal(out, want)
