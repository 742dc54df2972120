"""Pins oracle.moe_ref: brute force on tiny shapes, and the invariants the reference tests
state for the fused MoE (`test_mxfp4_fused_gemv.py:246-347`)."""

import numpy as np
import pytest

from oracle import moe_ref
from tests.moe_inputs import random_experts, random_routing


@pytest.mark.parametrize("seed", [0, 1])
def test_matches_brute_force(seed):
    tokens, experts, hidden, inter, top_k = 2, 4, 32, 32, 2
    ex = random_experts(experts, hidden, inter, seed=seed, scale_lo=124, scale_hi=130)
    a_e, a_w = random_routing(tokens, experts, top_k, seed=seed + 10)
    x = np.random.default_rng(seed).standard_normal((tokens, hidden)).astype(np.float32)
    got = moe_ref.reference_moe(x, ex, a_e, a_w, top_k, (0, experts))
    want = moe_ref.brute_force_moe(x, ex, a_e, a_w, top_k, (0, experts))
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())


def test_swapping_gate_and_up_changes_the_answer():
    """A plausible slip (gate/up halves swapped) must not pass the oracle checks."""
    ex = random_experts(2, 32, 32, seed=3, scale_lo=124, scale_hi=130)
    a_e, a_w = random_routing(1, 2, 1, seed=4)
    x = np.random.default_rng(5).standard_normal((1, 32)).astype(np.float32)
    good = moe_ref.reference_moe(x, ex, a_e, a_w, 1, (0, 2))
    swapped = dict(ex)
    gu, gs = ex["gate_up"], ex["gate_up_scale"]
    swapped["gate_up"] = np.concatenate([gu[:, 32:], gu[:, :32]], 1)
    swapped["gate_up_scale"] = np.concatenate([gs[:, 32:], gs[:, :32]], 1)
    bad = moe_ref.reference_moe(x, swapped, a_e, a_w, 1, (0, 2))
    assert moe_ref.rel_l2(bad, good) > 1e-2


def test_zero_weight_rows_are_exact_zeros():
    ex = random_experts(8, 64, 32, seed=11)
    a_e, a_w = random_routing(4, 8, 3, seed=12, zero_rows=(0, 2))
    x = np.random.default_rng(13).standard_normal((4, 64)).astype(np.float32)
    out = moe_ref.reference_moe(x, ex, a_e, a_w, 3, (0, 8))
    assert not out[0].any() and not out[2].any() and out[1].any()


def test_shards_sum_to_the_whole():
    ex = random_experts(9, 64, 32, seed=21)
    a_e, a_w = random_routing(5, 9, 3, seed=22)
    x = np.random.default_rng(23).standard_normal((5, 64)).astype(np.float32)
    whole = moe_ref.reference_moe(x, ex, a_e, a_w, 3, (0, 9)).astype(np.float64)
    cuts = [0, 3, 6, 9]
    parts = sum(
        moe_ref.reference_moe(x, {k: v[lo:hi] for k, v in ex.items()}, a_e, a_w, 3, (lo, hi)).astype(np.float64)
        for lo, hi in zip(cuts, cuts[1:])
    )
    assert moe_ref.rel_l2(parts, whole) < 1e-6


def test_metrics():
    a = np.array([1.0, 2.0, -4.0])
    assert moe_ref.relative_error(a + np.array([0, 0, 0.4]), a) == pytest.approx(0.1)
    assert moe_ref.rel_l2(a * 1.01, a) == pytest.approx(0.01)


def _dense_experts(ex):
    from oracle.mxfp4_ref import dequant_mxfp4

    return {"gate_up": np.stack([dequant_mxfp4(ex["gate_up"][e], ex["gate_up_scale"][e])
                                 for e in range(ex["gate_up"].shape[0])]),
            "down": np.stack([dequant_mxfp4(ex["down"][e], ex["down_scale"][e])
                              for e in range(ex["down"].shape[0])])}


@pytest.mark.parametrize("seed", [0, 1])
def test_dense_moe_matches_its_brute_force(seed):
    rng = np.random.default_rng(seed)
    dense = {"gate_up": rng.standard_normal((4, 6, 8)), "down": rng.standard_normal((4, 8, 3))}
    a_e, a_w = random_routing(3, 4, 2, seed=seed + 7, zero_rows=(1,))
    x = rng.standard_normal((3, 8))
    want = moe_ref.brute_force_dense_moe(x, dense, a_e, a_w, 2, (0, 4))
    got = moe_ref.dense_moe(x, dense, a_e, a_w, 2, (0, 4))
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    assert not got[1].any()  # the zero-weight token


def test_dense_moe_equals_the_mxfp4_oracle_on_dequantised_experts():
    ex = random_experts(6, 64, 32, seed=3)
    a_e, a_w = random_routing(5, 6, 2, seed=4)
    x = np.random.default_rng(5).standard_normal((5, 64)).astype(np.float32)
    want = moe_ref.reference_moe(x, ex, a_e, a_w, 2, (0, 6))
    got = moe_ref.dense_moe(x, _dense_experts(ex), a_e, a_w, 2, (0, 6))
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())
    # a shard: experts [2, 5) only
    sub = {k: v[2:5] for k, v in _dense_experts(ex).items()}
    part = moe_ref.dense_moe(x, sub, a_e, a_w, 2, (2, 5))
    np.testing.assert_allclose(part, moe_ref.reference_moe(x, {k: v[2:5] for k, v in ex.items()},
                                                           a_e, a_w, 2, (2, 5)), rtol=1e-6, atol=1e-6)


def test_dense_moe_inactive_tokens_are_zero():
    ex = _dense_experts(random_experts(4, 32, 32, seed=8))
    a_e, a_w = random_routing(4, 4, 2, seed=9)
    x = np.random.default_rng(10).standard_normal((4, 32))
    active = np.array([True, False, True, False])
    got = moe_ref.dense_moe(x, ex, a_e, a_w, 2, (0, 4), active=active)
    full = moe_ref.dense_moe(x, ex, a_e, a_w, 2, (0, 4))
    assert not got[1].any() and not got[3].any()
    np.testing.assert_array_equal(got[[0, 2]], full[[0, 2]])
