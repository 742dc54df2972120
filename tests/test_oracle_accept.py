"""Pins oracle.accept_ref against the reference tests' literal vectors and its scalar forms."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import accept_ref as ar

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def test_accept_len_golden():
    g = GOLDEN["accept_len"]
    draft, sa = np.array(g["draft"]), np.array(g["step_argmax"])
    assert ar.accept_len(draft, sa).tolist() == g["want"]
    scalar = [ar.greedy_accept_length(d.tolist(), s[:3].tolist()) for d, s in zip(draft, sa)]
    assert scalar == g["want"]


def test_greedy_accept_length_golden():
    for case in GOLDEN["greedy_accept_length"]:
        assert ar.greedy_accept_length(case["draft"], case["argmax"]) == case["want"]


def test_commit_limit_golden():
    g = GOLDEN["commit_limit"]
    sa, acc = np.array(g["step_argmax"]), np.array(g["accept"])
    budget, stops = np.array(g["budget"]), np.array(g["stops"])
    assert ar.commit_limit_batched(acc, sa, budget, stops).tolist() == g["want"]
    scalar = [
        ar.commit_limit(int(acc[j]), sa[j].tolist(), int(budget[j]), [s for s in stops[j] if s >= 0])
        for j in range(len(acc))
    ]
    assert scalar == g["want"]


def test_pack_index_golden():
    g = GOLDEN["pack_index"]
    for case in g["cases"]:
        src, cu = ar.fixed_prefix_pack_index(np.array(case["lengths"]), g["width"])
        assert src.shape == (3 * g["width"],)
        assert cu.tolist() == case["cu"]
        assert src[: cu[-1]].tolist() == case["live"]
        assert ((src >= 0) & (src < 3 * g["width"])).all()


@pytest.mark.parametrize("seed", range(5))
def test_batched_forms_match_scalar_forms(seed):
    rng = np.random.default_rng(seed)
    b, k = 64, 3
    t = k + 1
    sa = rng.integers(0, 4, (b, t))
    draft = np.where(rng.random((b, k)) < 0.7, sa[:, :k], rng.integers(0, 4, (b, k)))
    budget = rng.integers(0, 6, b)
    stops = np.where(rng.random((b, 2)) < 0.3, rng.integers(0, 4, (b, 2)), -1)
    acc = ar.accept_len(draft, sa)
    lim = ar.commit_limit_batched(acc, sa, budget, stops)
    for j in range(b):
        a = ar.greedy_accept_length(draft[j].tolist(), sa[j, :k].tolist())
        assert acc[j] == a
        want = ar.commit_limit(a, sa[j].tolist(), int(budget[j]), [s for s in stops[j] if s >= 0])
        assert lim[j] == want


def test_pack_index_gathers_each_lane_prefix():
    rng = np.random.default_rng(7)
    for _ in range(20):
        b, t = rng.integers(1, 9), rng.integers(1, 5)
        lengths = rng.integers(1, t + 1, b)
        src, cu = ar.fixed_prefix_pack_index(lengths, t)
        want = [j * t + s for j in range(b) for s in range(lengths[j])]
        assert src[: cu[-1]].tolist() == want


def test_round_indices_semantics():
    sa = np.array([[5, 6, 7, 8], [5, 6, 7, 8], [1, 2, 3, 4]])
    draft = np.array([[5, 6, 7], [5, 0, 7], [1, 2, 3]])
    active = np.array([True, True, False])
    pos = np.array([10, 20, 30])
    budget = np.array([9, 9, 2])
    stops = np.array([[8, -1], [-1, -1], [-1, -1]])
    r = ar.round_indices(draft, sa, active, pos, budget, stops, conv_k1=3)
    assert r["accept_len"].tolist() == [3, 1, 1]
    assert r["lengths"].tolist() == [4, 2, 1]  # padding row clamps to 1
    assert r["bonus"].tolist() == [8, 6, 2]
    assert r["next_pos"].tolist() == [14, 22, 32]
    assert r["budget_left"].tolist() == [5, 7, 0]
    assert r["live"].tolist() == [False, True, False]  # row 0 emitted its stop id
    assert r["keep"].tolist() == [[1, 1, 1, 1], [1, 1, 0, 0], [0, 0, 0, 0]]
    assert r["conv_idx"].tolist() == [[4, 5, 6], [2, 3, 4], [1, 2, 3]]
    assert r["hidden_src"].tolist() == [3, 5, 9]
    assert r["packed_cu"].tolist() == [0, 4, 6, 7]


def test_argmax_first_and_kv_rows():
    x = np.array([[1.0, 3.0, 3.0], [-0.0, 0.0, -1.0]], np.float32)
    assert ar.argmax_first(x).tolist() == [1, 0]
    table = np.array([[5, 9, 0], [2, 3, 0]])
    rows = ar.kv_rows(np.array([14, 0]), table, 4, 16)
    assert rows.tolist() == [[94, 95, 144, 145], [32, 33, 34, 35]]


def test_forced_rows_equal_an_unforced_row_accepting_the_same_count():
    """A forced row (`graph_verify_wide.py:196-200`) accepts exactly its forced count (at most
    k) whatever its drafts, stop ids and budget say: its outputs equal those of an unforced row
    whose drafts agree with the target for exactly that many steps, with no stop id and an
    unbounded budget — except `budget_left`, charged one token (`mtp_overlap.py:62-64`).
    Unforced rows in the same batch are unchanged by the forced ones."""
    rng = np.random.default_rng(31)
    for _ in range(50):
        b, k = int(rng.integers(1, 9)), int(rng.integers(1, 5))
        t = k + 1
        sa = rng.integers(0, 6, (b, t))
        draft = rng.integers(0, 6, (b, k))
        active = rng.random(b) < 0.8
        pos = rng.integers(0, 100, b)
        budget = rng.integers(1, 8, b)
        stops = np.where(rng.random((b, 2)) < 0.5, rng.integers(0, 6, (b, 2)), -1)
        forced_n = np.where(rng.random(b) < 0.5, rng.integers(1, k + 3, b), 0)  # > k: clamped
        got = ar.round_indices(draft, sa, active, pos, budget, stops, 3, forced_n)
        plain = ar.round_indices(draft, sa, active, pos, budget, stops, 3)
        # the equivalent unforced rows: drafts = target for f steps then a mismatch
        eq_draft = draft.copy()
        for j in range(b):
            f = min(int(forced_n[j]), k)
            if f:
                eq_draft[j, :f] = sa[j, :f]
                if f < k:
                    eq_draft[j, f] = sa[j, f] + 1
        big = np.full(b, 1 << 40)
        eq = ar.round_indices(eq_draft, sa, active, pos, np.where(forced_n > 0, big, budget),
                              np.where((forced_n > 0)[:, None], -1, stops), 3)
        for j in range(b):
            ref = eq if forced_n[j] else plain
            for key in ("accept_len", "lengths", "conv_idx", "keep", "bonus", "next_pos",
                        "hidden_src"):
                assert np.array_equal(got[key][j], ref[key][j]), (key, j)
            assert got["accept_len"][j] == (min(forced_n[j], k) if forced_n[j] else plain["accept_len"][j])
            charge = 1 if forced_n[j] else plain["accept_len"][j] + 1
            assert got["budget_left"][j] == budget[j] - charge
            stopped = bool((stops[j] == got["bonus"][j]).any())
            assert got["live"][j] == ((not stopped) and got["budget_left"][j] > 0)
        # the pack map is a function of the lengths alone
        src, cu = ar.fixed_prefix_pack_index(got["lengths"], t)
        assert np.array_equal(got["packed_src"], src) and np.array_equal(got["packed_cu"], cu)
