"""Routed bf16 experts on the device (`mtp_dense_moe`, `mtpk_moe_dense`) against the float64
oracle (`oracle/moe_ref.dense_moe`) and a torch fp32 reference at real dims.

The bar is the MoE's: rel-L2 <= 2e-3 against fp32 (the output is bf16). Unowned, zero-weight
and inactive assignments give exact zeros, expert shards sum to the whole, repeated launches
and graph replays are bit-identical.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import graph_mtp
import mtp
import mtp_dense_moe as dm
import verify_model as vm
from oracle import moe_ref
from tests.moe_inputs import random_routing, zipf_routing

pytestmark = pytest.mark.gpu


def _experts(e, h, i, dev, seed, std=0.05):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return {"gate_up": (torch.randn(e, 2 * i, h, generator=g) * std).to(torch.bfloat16).to(dev),
            "down": (torch.randn(e, h, i, generator=g) * std).to(torch.bfloat16).to(dev)}


def _x(t, h, dev, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(t, h, generator=g).to(torch.bfloat16).to(dev)


def _routing(a_e, a_w, t, k, dev):
    return (torch.from_numpy(a_e).view(t, k).to(dev), torch.from_numpy(a_w).view(t, k).to(dev))


def _oracle(x, ex, a_e, a_w, k, span, active=None):
    dense = {n: v.float().cpu().numpy() for n, v in ex.items()}
    return moe_ref.dense_moe(x.float().cpu().numpy(), dense, a_e, a_w, k, span, active=active)


@pytest.mark.parametrize("t,e,h,i,k", [(5, 8, 256, 256, 2), (40, 4, 512, 256, 2), (1, 16, 256, 512, 4),
                                       (33, 6, 768, 512, 3)])
def test_matches_oracle(dev, t, e, h, i, k):
    """Includes experts with more than 16 assignments (several work units) and ragged units."""
    ex = _experts(e, h, i, dev, seed=t + e)
    a_e, a_w = random_routing(t, e, k, seed=t)
    x = _x(t, h, dev, seed=1)
    got = dm.fused_moe(x, ex, _routing(a_e, a_w, t, k, dev), k, (0, e))
    assert got.dtype == torch.bfloat16 and got.shape == (t, h)
    want = _oracle(x, ex, a_e, a_w, k, (0, e))
    assert moe_ref.rel_l2(got.float().cpu().numpy(), want) <= 2e-3


def test_duplicate_expert_in_a_token(dev):
    ex = _experts(4, 256, 256, dev, seed=2)
    a_e = np.array([1, 1, 3, 0, 2, 2], dtype=np.int32)  # tokens 0 and 2 repeat an expert
    a_w = np.array([0.5, 0.5, 0.7, 0.3, 0.25, 0.75], dtype=np.float32)
    x = _x(3, 256, dev, seed=3)
    got = dm.fused_moe(x, ex, _routing(a_e, a_w, 3, 2, dev), 2, (0, 4))
    assert moe_ref.rel_l2(got.float().cpu().numpy(), _oracle(x, ex, a_e, a_w, 2, (0, 4))) <= 2e-3


def test_zero_unowned_and_inactive_give_zeros_and_shards_sum(dev):
    t, e, h, i, k = 12, 8, 256, 256, 3
    ex = _experts(e, h, i, dev, seed=4)
    a_e, a_w = random_routing(t, e, k, seed=5, zero_rows=(2, 7))
    x = _x(t, h, dev, seed=6)
    route = _routing(a_e, a_w, t, k, dev)
    full = dm.fused_moe(x, ex, route, k, (0, e))
    assert not full[[2, 7]].any()
    active = torch.ones(t, dtype=torch.bool, device=dev)
    active[[0, 5]] = False
    part = dm.fused_moe(x, ex, route, k, (0, e), active=active)
    assert not part[[0, 5]].any()
    keep = [r for r in range(t) if r not in (0, 5)]
    assert torch.equal(part[keep], full[keep])
    lo_half = dm.fused_moe(x, {n: v[: e // 2] for n, v in ex.items()}, route, k, (0, e // 2))
    hi_half = dm.fused_moe(x, {n: v[e // 2 :].contiguous() for n, v in ex.items()}, route, k, (e // 2, e))
    want = _oracle(x, ex, a_e, a_w, k, (0, e))
    both = lo_half.float() + hi_half.float()
    assert moe_ref.rel_l2(both.cpu().numpy(), want) <= 3e-3  # two bf16 roundings


@pytest.fixture(scope="module")
def real_layer():
    """512 bf16 experts at real dims, drawn on the device 64 experts at a time."""
    from tests.conftest import gpu_device

    dev = gpu_device()
    g = torch.Generator(device=dev).manual_seed(7)
    ex = {"gate_up": torch.empty(512, 2048, 4096, dtype=torch.bfloat16, device=dev),
          "down": torch.empty(512, 4096, 1024, dtype=torch.bfloat16, device=dev)}
    for name, ten in ex.items():
        for e0 in range(0, 512, 64):
            ten[e0 : e0 + 64] = torch.randn(ten[e0 : e0 + 64].shape, generator=g, device=dev) * 0.02
    yield ex
    del ex
    torch.cuda.empty_cache()


def _torch_fp32(x, ex, a_e, a_w, k):
    out = torch.zeros(x.shape[0], x.shape[1], dtype=torch.float32, device=x.device)
    a_e_t = torch.from_numpy(a_e).long().to(x.device)
    a_w_t = torch.from_numpy(a_w).to(x.device)
    tok = torch.arange(a_e_t.numel(), device=x.device) // k
    for ex_id in a_e_t[a_w_t != 0].unique().tolist():
        sel = ((a_e_t == ex_id) & (a_w_t != 0)).nonzero()[:, 0]
        gate, up = (x[tok[sel]].float() @ ex["gate_up"][ex_id].float().T).chunk(2, dim=-1)
        y = (F.silu(gate) * up) @ ex["down"][ex_id].float().T
        out.index_add_(0, tok[sel], y * a_w_t[sel, None])
    return out


@pytest.mark.parametrize("t,seed", [(48, 0), (1, 1), (192, 2)])
def test_real_dims_rel_l2(dev, real_layer, t, seed):
    """H 4096, I 1024, 512 bf16 experts (12.9 GB), top-10 with Zipf(1.1) routing and 5% zero
    weights: the MTP draft step's shape at B = 48, one token, and 192 rows."""
    a_e, a_w = zipf_routing(t, 512, 10, seed=seed, zero_frac=0.05)
    x = _x(t, 4096, dev, seed=seed + 10)
    got = dm.fused_moe(x, real_layer, _routing(a_e, a_w, t, 10, dev), 10, (0, 512))
    want = _torch_fp32(x, real_layer, a_e, a_w, 10)
    err = float((got.float() - want).norm() / want.norm())
    assert err <= 2e-3, err


def test_repeats_and_graph_replays_are_bit_identical(dev, real_layer):
    t = 48
    a_e, a_w = zipf_routing(t, 512, 10, seed=3)
    x = _x(t, 4096, dev, seed=4)
    route = _routing(a_e, a_w, t, 10, dev)
    scratch = dm.grouped_scratch(t, 10, 512, 4096, dev, intermediate=1024)
    inter = torch.empty(t * 10, 1024, dtype=torch.bfloat16, device=dev)
    out = torch.empty(t, 4096, dtype=torch.bfloat16, device=dev)
    eager = dm.grouped_moe(x, real_layer, route, 10, (0, 512), inter, out, scratch).clone()
    assert torch.equal(dm.fused_moe(x, real_layer, route, 10, (0, 512)), eager)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dm.grouped_moe(x, real_layer, route, 10, (0, 512), inter, out, scratch)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        _ = (torch.randn(128, 128, device=dev) @ torch.randn(128, 128, device=dev)).sum().item()
        assert torch.equal(out, eager)


def test_rejects_bad_inputs(dev):
    ex = _experts(4, 256, 256, dev, seed=8)
    a_e, a_w = random_routing(3, 4, 2, seed=9)
    route = _routing(a_e, a_w, 3, 2, dev)
    with pytest.raises(ValueError, match="BF16"):
        dm.fused_moe(torch.zeros(3, 256, device=dev), ex, route, 2, (0, 4))
    with pytest.raises(ValueError, match="routing"):
        dm.fused_moe(_x(3, 256, dev, 1), ex, (route[0].reshape(-1), route[1].reshape(-1)), 2, (0, 4))
    with pytest.raises(ValueError, match="expert_range"):
        dm.fused_moe(_x(3, 256, dev, 1), ex, route, 2, (0, 5))
    odd = _experts(4, 320, 256, dev, seed=8)  # H not a multiple of 256: the C check refuses
    with pytest.raises(ValueError, match="mtpk_moe_dense"):
        dm.fused_moe(_x(3, 320, dev, 1), odd, route, 2, (0, 4))


def test_config5_dims_rounds_with_dense_mtp_experts(dev) -> None:
    """The real checkpoint's layout: MXFP4 target layers, bf16 experts in the MTP layer. Rounds
    commit 1..k+1 valid ids and keep the hidden seed finite."""
    def build():
        model = vm.Model(vm.verify_cfg(), dev, torch.bfloat16, lanes=2, max_seq=96, seed=0,
                         expert_mode="bytes", moe_rows=8)
        mtp.attach(model, k=3, seed=1, expert_mode="dense")
        return model

    a = build()
    assert set(a.mtp.weights["experts"]) == {"gate_up", "down"}
    gen = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, 248320, (4 + 5 * j,), generator=gen).tolist() for j in range(2)]
    toks, pos = [], []
    for lane, p in enumerate(prompts):
        toks.append(int(a.argmax(a.prefill(lane, p)[None])[0]))
        pos.append(len(p))
    eager = graph_mtp.MTPVerifyRunner(a, capacity=2)
    for _ in range(2):
        got = eager.speculative_decode([0, 1], toks, pos)
        for j, c in enumerate(got):
            assert 1 <= len(c) <= 4 and all(0 <= x < 248320 for x in c)
            pos[j] += len(c)
            toks[j] = c[-1]
    assert torch.isfinite(a.hidden_cache.float()).all()
