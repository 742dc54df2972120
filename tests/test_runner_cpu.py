"""The round runner's bucket contract on the CPU engine (config 1's tiny model in fp32).

`MTPVerifyBuffers` is one bucket: row `j < n` is the round's `j`-th lane and rows `>= n` are
padding (`MTP_INTERFACE.md:17-33`, `graph_mtp.py:141-178`, `:795-874`). These tests follow the
reference's own (`seed_tests/test_graph_mtp.py:260-299`): a narrower batch pads into a larger
bucket and commits what the unpadded round commits, the filler lane comes out untouched, a
forced round's acceptance outputs follow the forced lengths, and capture validation refuses a
captured round that disagrees with the eager one (`graph_mtp.py:712-769`, `:978-1059`).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import graph_mtp
from oracle import accept_ref as ar
from tests import model_helpers as mh


def _prefilled(lanes: int, n: int, k: int = 3):
    ids = mh.prompts(n)
    model = mh.build(k=k, lanes=lanes)
    toks, pos = [], []
    for lane, p in enumerate(ids):
        toks.append(int(model.argmax(model.prefill(lane, p)[None])[0]))
        pos.append(len(p))
    return model, toks, pos


def _idle_state(model, lane: int) -> list[torch.Tensor]:
    out = [p[name][lane].clone() for p in model.pool for name in ("conv", "rec") if name in p]
    return out + [model.hidden_cache[lane].clone(), model.blocks.table[lane].clone()]


def test_buckets_and_padding_rows():
    model, toks, pos = _prefilled(4, 3)
    runner = graph_mtp.MTPVerifyRunner(model, capacity=4)
    assert runner.buckets == [1, 2, 4] and runner.bucket_for(3) == 4
    buf = runner.buffers(3)
    runner.fill(buf, [0, 1, 2], toks, pos, budgets=[5, 6, 7], stops=[[1], [], [2, 3]])
    assert buf.capacity == 4
    assert buf.active.tolist() == [True, True, True, False]
    assert buf.slot_rows.tolist() == [0, 1, 2, 3]  # the filler is the idle lane 3
    assert buf.pos[3] == 0 and buf.budget[3] == buf.t and (buf.stops[3] == -1).all()
    assert (buf.block_table[3] == graph_mtp.RESERVED_BLOCK).all()
    assert torch.equal(buf.block_table[:3], model.blocks.table[:3])
    bs = model.cfg.block_size
    want = ar.kv_rows(buf.pos.numpy(), buf.block_table.numpy(), buf.t, bs)
    assert np.array_equal(buf.write_rows.numpy(), want)
    assert torch.equal(buf.draft_hidden, model.hidden_cache[buf.slot_rows])
    with pytest.raises(ValueError, match="distinct"):
        runner.fill(buf, [0, 0, 1], toks, pos)
    with pytest.raises(ValueError, match="1..4"):
        runner.buffers(5)


def test_padded_bucket_commits_what_the_unpadded_round_commits():
    """A 3-lane round on a 4-row bucket (one padding row naming idle lane 3) and the same round
    on a 3-row bucket of an identical model: the same committed ids every round, the same lane
    state, and lane 3 (its DeltaNet state, hidden seed and block table) untouched."""
    k = 3
    a, toks, pos = _prefilled(4, 3, k)
    b, _, _ = _prefilled(4, 3, k)
    padded = graph_mtp.MTPVerifyRunner(a, buckets=[4])
    exact = graph_mtp.MTPVerifyRunner(b, buckets=[3, 4])
    idle = _idle_state(a, 3)
    lanes = [0, 1, 2]
    pa, pb = list(pos), list(pos)
    for r in range(4):
        got = padded.speculative_decode(lanes, toks, pa, budgets=[40, 40, 3 + r], stops=[[], [7], []])
        want = exact.speculative_decode(lanes, toks, pb, budgets=[40, 40, 3 + r], stops=[[], [7], []])
        assert got == want, f"round {r}"
        assert padded.bufs[4].capacity == 4 and 3 in exact.bufs
        for j, c in enumerate(got):
            pa[j] += len(c)
            pb[j] += len(c)
            toks[j] = c[-1]
    for lane in lanes:
        mh.assert_slot_state_close(a, b, lane, pa[lane], rtol=1e-5, atol=1e-6)
    for before, now in zip(idle, _idle_state(a, 3), strict=True):
        assert torch.equal(before, now)


def test_forced_round_outputs_follow_the_forced_lengths():
    """A forced round on a padded bucket: the buffers' eleven acceptance outputs equal the
    oracle's `round_indices` with the forced counts (stop ids and budgets notwithstanding), the
    forced ids were fed as drafts, and each lane commits the target's argmax after every fed
    token (`step_argmax[j, : forced + 1]`)."""
    k = 3
    model, toks, pos = _prefilled(4, 3, k)
    runner = graph_mtp.MTPVerifyRunner(model, buckets=[4])
    forced = [[5, 6], [], [9, 10, 11]]
    got = runner.speculative_decode([0, 1, 2], toks, pos, budgets=[2, 9, 1], stops=[[6], [], [10]],
                                    forced=forced)
    buf = runner.bufs[4]
    want = ar.round_indices(buf.token_matrix[:, 1:].numpy(), buf.step_argmax.numpy(),
                            buf.active.numpy(), buf.pos.numpy(), buf.budget.numpy(),
                            buf.stops.numpy(), buf.conv_k1, buf.forced_n.numpy())
    for name, w in want.items():
        assert np.array_equal(getattr(buf, name).numpy().astype(w.dtype), w), name
    assert buf.accept_len[0] == 2 and buf.accept_len[2] == 3
    assert buf.token_matrix[0, 1:3].tolist() == [5, 6] and buf.token_matrix[2, 1:].tolist() == [9, 10, 11]
    assert got[0] == buf.step_argmax[0, :3].tolist() and got[2] == buf.step_argmax[2].tolist()
    assert buf.budget_left.tolist()[:3] == [1, 9 - len(got[1]), 0]


class _Diverging(graph_mtp.GraphMTPRunner):
    """A captured round that disagrees with its eager step (its replay perturbs the argmax after
    the round), standing in for a capture that froze a host value."""

    def _capture(self, buf):
        inner = super()._capture(buf)

        def replay():
            inner()
            buf.step_argmax.add_(1)

        return replay


def test_prepare_validates_every_bucket():
    model, _, _ = _prefilled(4, 0)
    runner = graph_mtp.GraphMTPRunner(model, graph_mtp.EagerBackend(), capacity=4)
    assert runner.prepare() is True
    assert runner.validated == {1: True, 2: True, 4: True} and runner.enabled
    assert not any(model.blocks.host[lane] for lane in range(4))  # boot-only: lanes reset
    model.prefill(0, mh.prompts(1)[0])
    with pytest.raises(RuntimeError, match="boot-only"):
        runner.prepare()


def test_prepare_refuses_a_divergent_capture(monkeypatch):
    """Validation catches the divergent replay: the captured round is disabled and rounds are
    served eagerly with the right ids; under SEED_MTP_REQUIRE_GRAPH=1 prepare() raises."""
    model, _, _ = _prefilled(4, 0)
    runner = _Diverging(model, graph_mtp.EagerBackend(), capacity=4)
    assert runner.prepare() is False and not runner.enabled
    assert set(runner.validated.values()) == {False}
    ids = mh.prompts(2)
    twin, toks, pos = _prefilled(4, 2)
    for lane, p in enumerate(ids):
        model.prefill(lane, p)
    eager = graph_mtp.MTPVerifyRunner(twin, capacity=4)
    assert runner.speculative_decode([0, 1], toks, pos) == eager.speculative_decode([0, 1], toks, pos)
    assert runner.eager_rounds == 1
    monkeypatch.setenv(graph_mtp.REQUIRE_GRAPH_ENV, "1")
    other, _, _ = _prefilled(4, 0)
    with pytest.raises(RuntimeError, match="SEED_MTP_REQUIRE_GRAPH"):
        _Diverging(other, graph_mtp.EagerBackend(), capacity=4).prepare()


def test_grow_many_equals_grow_per_lane():
    """`BlockTables.grow_many` (one copy per round) hands out the same blocks into the same table
    entries as `grow` lane by lane, and refuses an over-long lane before changing anything."""
    import verify_model as vm

    a = vm.BlockTables(4, 96, 16, torch.device("cpu"), seed=3)
    b = vm.BlockTables(4, 96, 16, torch.device("cpu"), seed=3)
    for lanes, lengths in (([0, 2], [5, 40]), ([1, 2, 3], [17, 41, 0]), ([0, 3], [80, 33])):
        for lane, n in zip(lanes, lengths):
            a.grow(lane, n)
        b.grow_many(lanes, lengths)
        assert torch.equal(a.table, b.table) and a.host == b.host and a._free == b._free
    before = (b.table.clone(), [list(h) for h in b.host], list(b._free))
    with pytest.raises(ValueError, match="exceed"):
        b.grow_many([1, 2], [20, 97])
    assert torch.equal(b.table, before[0]) and b.host == before[1] and b._free == before[2]
