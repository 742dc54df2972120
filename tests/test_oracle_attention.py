"""Pins `oracle/attention_ref.py` (paged causal GQA attention) on closed forms, on the CPU."""

from __future__ import annotations

import numpy as np

from oracle import attention_ref as ar


def _pools(rng, rows, kvh, hd):
    return rng.standard_normal((rows, kvh, hd)), rng.standard_normal((rows, kvh, hd))


def test_identical_keys_average_the_visible_values() -> None:
    rng = np.random.default_rng(0)
    k, v = _pools(rng, 64, 2, 8)
    k[:] = k[0:1, :, :]  # every key the same (per kv head)
    k[:, 1] = k[0, 1]
    table = np.array([[2, 1, 3]])
    q = rng.standard_normal((1, 4, 2, 8))
    out = ar.paged_attention(q, k, v, table, [5], 0.7)
    for s in range(2):
        rows = ar.physical_rows(table[0], 5 + s + 1, 16)
        for h in range(4):
            np.testing.assert_allclose(out[0, h, s], v[rows, h // 2].mean(0), rtol=1e-12, atol=1e-12)


def test_lone_position_returns_its_value_and_mask_is_causal() -> None:
    rng = np.random.default_rng(1)
    k, v = _pools(rng, 48, 1, 4)
    table = np.array([[1, 2]])
    q = rng.standard_normal((1, 2, 3, 4))
    out = ar.paged_attention(q, k, v, table, [0], 0.5)
    np.testing.assert_allclose(out[0, :, 0], np.broadcast_to(v[16, 0], (2, 4)), rtol=1e-12)
    # row 1 sees positions 0..1 only: changing position 2's key leaves it unchanged
    k2 = k.copy()
    k2[18] += 10.0
    out2 = ar.paged_attention(q, k2, v, table, [0], 0.5)
    np.testing.assert_allclose(out2[0, :, :2], out[0, :, :2], rtol=1e-12)
    assert not np.allclose(out2[0, :, 2], out[0, :, 2])


def test_dominant_key_and_block_relabelling() -> None:
    rng = np.random.default_rng(2)
    k, v = _pools(rng, 96, 2, 16)
    table = np.array([[3, 1, 5], [2, 4, 0]])
    q = rng.standard_normal((2, 2, 1, 16))
    base = [30, 20]
    # the key equal to q (largest dot product) dominates at a huge scale
    rows0 = ar.physical_rows(table[0], 31, 16)
    k[rows0[7], 0] = q[0, 0, 0] * 3.0
    out = ar.paged_attention(q, k, v, table, base, 50.0)
    np.testing.assert_allclose(out[0, 0, 0], v[rows0[7], 0], rtol=1e-9, atol=1e-9)
    # move lane 1's logical blocks to other physical blocks: same output
    perm = {2: 1, 4: 3, 0: 5}
    k2, v2 = k.copy(), v.copy()
    for old, new in perm.items():
        k2[new * 16 : new * 16 + 16] = k[old * 16 : old * 16 + 16]
        v2[new * 16 : new * 16 + 16] = v[old * 16 : old * 16 + 16]
    t2 = np.array([[3, 1, 5], [1, 3, 5]])
    out2 = ar.paged_attention(q[1:], k2, v2, t2[1:], base[1:], 50.0)
    np.testing.assert_allclose(out2[0], out[1], rtol=1e-12, atol=1e-12)
