"""Pins oracle.router_ref: brute force over k-subsets, planted ties, renormalisation."""

import itertools
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import router_ref

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def _brute(row, k):
    """The k-subset with the largest total softmax mass; among equal masses the lexicographically
    smallest index set (lowest-index tie-break)."""
    p = np.exp(row - row.max())
    p /= p.sum()
    best, best_set = -1.0, None
    for sub in itertools.combinations(range(len(row)), k):
        mass = sum(p[i] for i in sub)
        if mass > best + 1e-15:
            best, best_set = mass, sub
    return best_set, p


@pytest.mark.parametrize("seed", range(6))
def test_brute_force_small_rows(seed):
    rng = np.random.default_rng(seed)
    e, k = 7, 3
    logits = (rng.standard_normal((2, e + 2)) * 4).astype(np.float32)
    w, i = router_ref.route(logits, e, k)
    for r in range(2):
        sub, p = _brute(logits[r, :e].astype(np.float64), k)
        assert sorted(i[r].tolist()) == list(sub)
        assert np.allclose(w[r], p[i[r]] / p[list(sub)].sum(), rtol=1e-6)
        assert (np.diff(w[r]) <= 0).all()  # highest weight first


def test_ties_pick_the_lower_index():
    logits = np.array([[1.0, 3.0, 3.0, 0.5, 3.0]], np.float32)
    w, i = router_ref.route(logits, 5, 2)
    assert i[0].tolist() == [1, 2]
    assert np.allclose(w[0], [0.5, 0.5])


@pytest.mark.parametrize("t,e,k", GOLDEN["router_shapes"])
def test_reference_shapes_renormalise_and_shift_invariance(t, e, k):
    rng = np.random.default_rng(t * 1000 + e * 10 + k)
    logits = (rng.standard_normal((t, e + 3)) * 4).astype(np.float32)
    w, i = router_ref.route(logits, e, k)
    assert w.shape == (t, k) and i.shape == (t, k)
    assert np.allclose(w.sum(-1), 1.0, atol=1e-6)
    assert (i < e).all()
    w2, i2 = router_ref.route(logits + 7.0, e, k)
    assert np.array_equal(i, i2) and np.allclose(w, w2, atol=1e-6)
