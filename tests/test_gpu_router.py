"""`router_fused.route` (HIP `mtpk_route_topk`) against the oracle: the reference test shapes
(`test_router_fused.py:43-83`) with a wider row than `experts_out`, exact selection order, weights
within 1e-5, int32 == int64, planted ties, and the real shape [192, 513] in bf16."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import router_fused
from oracle import router_ref
from oracle.mxfp4_ref import bf16_round

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


@pytest.mark.parametrize("t,e,k", GOLDEN["router_shapes"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_matches_oracle(dev, t, e, k, dtype):
    rng = np.random.default_rng(t * 1000 + e * 10 + k)
    logits = (rng.standard_normal((t, e + 3)) * 4).astype(np.float32)
    if dtype == torch.bfloat16:
        logits = bf16_round(logits)
    want_w, want_i = router_ref.route(logits, e, k)
    got_w, got_i = router_fused.route(torch.from_numpy(logits).to(dev, dtype), e, k)
    assert got_i.dtype == torch.int64 and got_w.dtype == torch.float32
    assert np.array_equal(got_i.cpu().numpy(), want_i)
    # fp32 exp(l - max) / S, then p / sum(p_sel): a few ulp from the float64 weights
    assert np.abs(got_w.cpu().numpy() - want_w).max() < 1e-5
    assert (np.abs(got_w.cpu().numpy() - want_w) <= 4e-6 * want_w + 1e-12).all()
    assert np.abs(got_w.sum(-1).cpu().numpy() - 1).max() < 1e-5
    i32_w, i32_i = router_fused.route(torch.from_numpy(logits).to(dev, dtype), e, k,
                                      index_dtype=torch.int32)
    assert i32_i.dtype == torch.int32
    assert torch.equal(i32_i.long(), got_i) and torch.equal(i32_w, got_w)


def test_ties_pick_lower_index(dev):
    logits = torch.tensor([[1.0, 3.0, 3.0, 0.5, 3.0, -2.0]], device=dev)
    w, i = router_fused.route(logits, 5, 3)
    assert i.tolist() == [[1, 2, 4]]
    assert np.allclose(w.cpu().numpy(), 1 / 3, atol=1e-6)


def test_real_shape_strided_bf16(dev):
    rng = np.random.default_rng(5)
    full = bf16_round(rng.standard_normal((192, 513)).astype(np.float32))
    want_w, want_i = router_ref.route(full, 512, 10)
    t = torch.from_numpy(full).to(dev, torch.bfloat16)
    got_w, got_i = router_fused.route(t, 512, 10)
    assert np.array_equal(got_i.cpu().numpy(), want_i)
    assert np.abs(got_w.cpu().numpy() - want_w).max() < 1e-5
    assert (np.abs(got_w.cpu().numpy() - want_w) <= 4e-6 * want_w + 1e-12).all()


def test_rejects_over_cap(dev):
    with pytest.raises(ValueError, match="MAX_TOP_K"):
        router_fused.route(torch.randn(2, 8, device=dev), 8, router_fused.MAX_TOP_K + 1)
    with pytest.raises(ValueError, match="index_dtype"):
        router_fused.route(torch.randn(2, 8, device=dev), 8, 2, index_dtype=torch.int16)
