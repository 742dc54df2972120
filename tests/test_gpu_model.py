"""The MTP step on the GPU: draft head, verify forward and acceptance on the HIP kernels.

Config 1's model runs on the device in fp32 with the same weights as the CPU model; its
speculative rounds (`graph_mtp.MTPVerifyRunner`: MTP draft steps, wide verify, the acceptance
kernel and the commit) must reproduce plain greedy decode, and its logits must agree with the
CPU path. Config 5's layer dimensions are exercised at a few lanes and a short context.
"""

from __future__ import annotations

import pytest
import torch

import graph_mtp
import mtp
import verify_model as vm
from tests import model_helpers as mh

pytestmark = pytest.mark.gpu


def test_config1_prefill_logits_match_cpu(dev) -> None:
    ids = mh.prompts(2)
    cpu, gpu = mh.build("cpu"), mh.build(dev)
    for lane, p in enumerate(ids):
        want = cpu.prefill(lane, p)
        got = gpu.prefill(lane, p).cpu()
        torch.testing.assert_close(got, want, rtol=1e-4, atol=2e-5)
        assert int(got.argmax()) == int(want.argmax())


def test_config1_torch_moe_path_on_device(dev, monkeypatch) -> None:
    """`SEED_FUSED_MOE=0`, the reference's A/B switch: the device model takes the torch
    dequant-then-multiply MoE (`_routed_grouped`, `model.py:3170-3236`) instead of the fused
    kernels, and its logits still match the CPU model's."""
    import mxfp4_gemv

    monkeypatch.setenv("SEED_FUSED_MOE", "0")
    assert not mxfp4_gemv.available(dev)
    ids = mh.prompts(1)
    want = mh.build("cpu").prefill(0, ids[0])
    got = mh.build(dev).prefill(0, ids[0]).cpu()
    torch.testing.assert_close(got, want, rtol=1e-4, atol=2e-5)


@pytest.mark.parametrize("k", [1, 3])
def test_config1_speculative_rounds_match_greedy(dev, k: int) -> None:
    """2 prompts of 16 ids, 32 tokens: the device rounds commit the CPU greedy sequence."""
    ids = mh.prompts()
    truth = mh.greedy_truth(mh.build("cpu", k=k), ids, mh.GEN_TOKENS)
    model = mh.build(dev, k=k)
    runner = graph_mtp.MTPVerifyRunner(model, capacity=2)
    got, toks, pos = [], [], []
    for lane, p in enumerate(ids):
        base = int(model.argmax(model.prefill(lane, p)[None])[0])
        got.append([base])
        toks.append(base)
        pos.append(len(p))
    while min(len(g) for g in got) < mh.GEN_TOKENS + 1:
        committed = runner.speculative_decode([0, 1], toks, pos)
        for j, c in enumerate(committed):
            assert 1 <= len(c) <= k + 1
            got[j].extend(c)
            pos[j] += len(c)
            toks[j] = c[-1]
    for g, t in zip(got, truth, strict=True):
        assert g[: mh.GEN_TOKENS + 1] == t


@pytest.mark.parametrize("accept", [1, 2, 3])
def test_config1_forced_round_matches_sequential(dev, accept: int) -> None:
    """Forced drafts (the greedy continuation) accepted unconditionally: committed ids and all
    slot state equal `accept + 1` plain decode steps on the device."""
    k, lane = 3, 0
    ids = mh.prompts(1)
    truth = mh.greedy_truth(mh.build(dev, k=k, lanes=1), ids, k + 1)[0]
    seq = mh.build(dev, k=k, lanes=1)
    seq.prefill(lane, ids[0])
    vm.greedy_reference(seq, lane, truth[0], len(ids[0]), accept + 1)
    spec = mh.build(dev, k=k, lanes=1)
    spec.prefill(lane, ids[0])
    runner = graph_mtp.MTPVerifyRunner(spec, capacity=1)
    committed = runner.speculative_decode([lane], [truth[0]], [len(ids[0])], forced=[truth[1 : accept + 1]])
    assert committed == [truth[1 : accept + 2]]
    mh.assert_slot_state_close(spec, seq, lane, len(ids[0]) + accept + 1, rtol=1e-4, atol=1e-5)


def test_config1_runner_matches_eager_verify(dev) -> None:
    """The device round (acceptance kernel, device commit) and the eager host-accept round
    commit the same ids and leave the same state, with budgets and stop ids in play."""
    k = 3
    ids = mh.prompts(2)
    a, b = mh.build(dev, k=k), mh.build(dev, k=k)
    toks, pos = [], []
    for lane, p in enumerate(ids):
        toks.append(int(a.argmax(a.prefill(lane, p)[None])[0]))
        b.prefill(lane, p)
        pos.append(len(p))
    runner = graph_mtp.MTPVerifyRunner(a, capacity=4)
    budgets, stops = [2, 50], [[3], [7, 9]]
    for _ in range(3):
        got = runner.speculative_decode([0, 1], toks, pos, budgets, stops)
        drafts = runner.bufs[2].token_matrix[:, 1:].tolist()
        want = mtp.verify_and_commit(b, b.mtp, [0, 1], toks, drafts, pos, budgets, stops)
        assert got == want
        for j, c in enumerate(got):
            pos[j] += len(c)
            toks[j] = c[-1]
    for lane in range(2):
        mh.assert_slot_state_close(a, b, lane, pos[lane], rtol=1e-5, atol=1e-6)


def test_config5_dims_round(dev) -> None:
    """Real layer dimensions (3 DeltaNet + 1 gated GQA, 512 experts top-10, vocab 248320) at 4
    lanes: rounds commit 1..k+1 valid ids and keep every state finite."""
    k = 3
    model = vm.Model(vm.verify_cfg(), dev, torch.bfloat16, lanes=4, max_seq=96, seed=0,
                     expert_mode="bytes", moe_rows=16)
    mtp.attach(model, k=k, seed=1, expert_mode="bytes")
    gen = torch.Generator().manual_seed(9)
    toks, pos = [], []
    for lane in range(4):
        p = torch.randint(0, model.cfg.vocab, (5 + 3 * lane,), generator=gen).tolist()
        toks.append(int(model.argmax(model.prefill(lane, p)[None])[0]))
        pos.append(len(p))
    runner = graph_mtp.MTPVerifyRunner(model, capacity=4)
    for _ in range(3):
        got = runner.speculative_decode([0, 1, 2, 3], toks, pos)
        for j, c in enumerate(got):
            assert 1 <= len(c) <= k + 1
            assert all(0 <= x < model.cfg.vocab for x in c)
            pos[j] += len(c)
            toks[j] = c[-1]
    assert torch.isfinite(model.hidden_cache.float()).all()
    for ty, p in zip(model.cfg.layer_types, model.pool, strict=True):
        if ty != vm.ATTN:
            assert torch.isfinite(p["rec"]).all() and torch.isfinite(p["conv"].float()).all()


def _graph_vs_eager(dev, build, prompts, rounds):
    """Identical models, one on the eager runner and one on the captured runner: every round
    commits the same ids (replays separated by unrelated eager work and a synchronisation)."""
    a, b = build(), build()
    toks, pos = [], []
    for lane, p in enumerate(prompts):
        toks.append(int(a.argmax(a.prefill(lane, p)[None])[0]))
        b.prefill(lane, p)
        pos.append(len(p))
    lanes = list(range(len(prompts)))
    eager = graph_mtp.MTPVerifyRunner(a, capacity=len(prompts))
    graph = graph_mtp.GraphMTPRunner(b, capacity=len(prompts))
    for r in range(rounds):
        want = eager.speculative_decode(lanes, toks, pos)
        got = graph.speculative_decode(lanes, toks, pos)
        assert got == want, f"round {r}"
        torch.cuda.synchronize()
        _ = (torch.randn(256, 256, device=dev) @ torch.randn(256, 256, device=dev)).sum().item()
        for j, c in enumerate(want):
            pos[j] += len(c)
            toks[j] = c[-1]
    assert len(graph.graphs) == 1
    return a, b, pos


def test_config1_graph_runner_matches_eager(dev) -> None:
    k = 3
    a, b, pos = _graph_vs_eager(dev, lambda: mh.build(dev, k=k), mh.prompts(2), 5)
    # the library GEMMs may pick another algorithm under capture: states agree to fp32 rounding
    for lane in range(2):
        mh.assert_slot_state_close(a, b, lane, pos[lane], rtol=1e-5, atol=1e-6)


def test_config5_dims_graph_runner_matches_eager(dev) -> None:
    def build():
        model = vm.Model(vm.verify_cfg(), dev, torch.bfloat16, lanes=3, max_seq=96, seed=0,
                         expert_mode="bytes", moe_rows=16)
        mtp.attach(model, k=3, seed=1, expert_mode="bytes")
        return model

    gen = torch.Generator().manual_seed(9)
    prompts = [torch.randint(0, 248320, (4 + 5 * j,), generator=gen).tolist() for j in range(3)]
    _graph_vs_eager(dev, build, prompts, 3)


@pytest.mark.parametrize("accept", [1, 3])
def test_config1_graph_forced_round_replays(dev, accept) -> None:
    """A forced round on the captured runner replays the same graph as a normal round and
    commits the forced drafts plus one target token, like plain greedy decode."""
    k = 3
    ids = mh.prompts(2)
    truth = mh.greedy_truth(mh.build(dev, k=k), ids, 2 * (k + 1))
    spec = mh.build(dev, k=k)
    for lane, p in enumerate(ids):
        spec.prefill(lane, p)
    runner = graph_mtp.GraphMTPRunner(spec, capacity=2)
    toks = [t[0] for t in truth]
    pos = [len(p) for p in ids]
    first = runner.speculative_decode([0, 1], toks, pos)  # eager, then captured
    done = [len(c) for c in first]
    for j in range(2):
        assert first[j] == truth[j][1 : done[j] + 1]
    forced = [truth[j][done[j] + 1 : done[j] + 1 + accept] for j in range(2)]
    got = runner.speculative_decode([0, 1], [truth[j][done[j]] for j in range(2)],
                                    [pos[j] + done[j] for j in range(2)], forced=forced)
    assert len(runner.graphs) == 1
    for j in range(2):
        assert got[j] == truth[j][done[j] + 1 : done[j] + accept + 2]
    seq = mh.build(dev, k=k)
    for lane, p in enumerate(ids):
        seq.prefill(lane, p)
        vm.greedy_reference(seq, lane, truth[lane][0], len(p), done[lane] + accept + 1)
    for lane in range(2):
        mh.assert_slot_state_close(spec, seq, lane, pos[lane] + done[lane] + accept + 1,
                                   rtol=1e-4, atol=1e-5)


def _rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def test_config5_full_size_graph_rounds(dev) -> None:
    """The benchmark's round at its real size (B=48, k=3, 8192-token context, GraphMTPRunner):
    normal rounds commit 1..k+1 valid ids per lane and keep every state finite; a forced round
    (lane j accepts 1 + j % 3 drafts, replayed through the same graph) commits what accept + 1
    plain decode steps produce and leaves the same slot state, to bf16 rounding (router ties
    aside)."""
    b, k, ctx = 48, 3, 8192
    model, toks, pos = mh.c5_model(dev, b, k, ctx)
    lanes = list(range(b))
    runner = graph_mtp.GraphMTPRunner(model, capacity=b)
    for _ in range(2):
        got = runner.speculative_decode(lanes, toks, pos)
        for j, c in enumerate(got):
            assert 1 <= len(c) <= k + 1
            assert all(0 <= x < model.cfg.vocab for x in c)
            pos[j] += len(c)
            toks[j] = c[-1]
    assert torch.isfinite(model.hidden_cache.float()).all()
    for ty, p in zip(model.cfg.layer_types, model.pool, strict=True):
        for name, ten in p.items():
            assert torch.isfinite(ten.float()).all(), (ty, name)
    before = mh.snapshot(model)

    # plain decode: lane j runs accept_j + 1 greedy steps
    accept = [1 + j % 3 for j in range(b)]
    truth = [[toks[j]] for j in range(b)]
    rows = [[] for _ in range(b)]  # plain decode's logits per lane and step
    for s in range(k + 1):
        live = [j for j in lanes if accept[j] >= s]
        logits = model.decode(live, [truth[j][-1] for j in live], [pos[j] + s for j in live]).float()
        for i, j in enumerate(live):
            truth[j].append(int(logits[i].argmax()))
            rows[j].append(logits[i])
    plain = [mh.slot_state(model, j, pos[j] + accept[j] + 1) for j in lanes]

    mh.restore(model, before)
    forced = [truth[j][1 : accept[j] + 1] for j in lanes]
    got = runner.speculative_decode(lanes, toks, pos, forced=forced)
    assert len(runner.graphs) == 1
    # bf16 rounding differs between the 48-row decode and the 192-row verify forward; where it
    # reorders an exact tie among the router's top-10 logits a lane takes another expert and
    # its rows differ for real (rel-L2 ~0.1). With 4 routed layers and up to 4 rows per lane a
    # few lanes in 48 meet such a tie (7 on the seeds here); everything else agrees.
    for j in lanes:
        assert len(got[j]) == accept[j] + 1
    same = sum(x == y for j in lanes for x, y in zip(got[j], truth[j][1:], strict=False))
    total = sum(len(got[j]) for j in lanes)
    worst = []
    for j in lanes:
        spec = mh.slot_state(model, j, pos[j] + accept[j] + 1)
        worst.append(max(_rel_l2(x, y) for x, y in zip(spec, plain[j], strict=True)))
    worst_t = torch.tensor(worst)
    print(f"C5 forced round: {same}/{total} ids as plain decode; slot-state rel-L2 median "
          f"{float(worst_t.median()):.2e}, lanes above 2e-2: {int((worst_t > 2e-2).sum())}")
    assert same >= 0.9 * total
    assert float(worst_t.median()) < 1e-2
    assert int((worst_t > 2e-2).sum()) <= b // 4


# ---------------------------------------------------------------- buckets and padding rows


def _idle(model, lanes) -> list[torch.Tensor]:
    out = []
    for lane in lanes:
        out += [p[n][lane].clone() for p in model.pool for n in ("conv", "rec") if n in p]
        out += [model.hidden_cache[lane].clone(), model.blocks.table[lane].clone()]
    return out


def test_config1_padded_graph_bucket_matches_unpadded(dev) -> None:
    """A 3-lane round replayed on a captured 4-row bucket (one padding row naming idle lane 3)
    commits what the unpadded 3-row eager round of an identical model commits, round after
    round, the lanes' state agrees, and lane 3 comes out untouched
    (`seed_tests/test_graph_mtp.py:260-299`)."""
    k = 3
    ids = mh.prompts(3)
    a, b = mh.build(dev, k=k, lanes=4), mh.build(dev, k=k, lanes=4)
    toks, pos = [], []
    for lane, p in enumerate(ids):
        toks.append(int(a.argmax(a.prefill(lane, p)[None])[0]))
        b.prefill(lane, p)
        pos.append(len(p))
    idle = _idle(a, [3])
    padded = graph_mtp.GraphMTPRunner(a, buckets=[4])
    exact = graph_mtp.MTPVerifyRunner(b, buckets=[3, 4])
    lanes = [0, 1, 2]
    for r in range(4):
        got = padded.speculative_decode(lanes, toks, pos, budgets=[40, 40, 3 + r], stops=[[], [7], []])
        want = exact.speculative_decode(lanes, toks, pos, budgets=[40, 40, 3 + r], stops=[[], [7], []])
        assert got == want, f"round {r}"
        for j, c in enumerate(got):
            pos[j] += len(c)
            toks[j] = c[-1]
    assert list(padded.graphs) == [4]
    for lane in lanes:
        mh.assert_slot_state_close(a, b, lane, pos[lane], rtol=1e-5, atol=1e-6)
    for before, now in zip(idle, _idle(a, [3]), strict=True):
        assert torch.equal(before, now)


def test_graph_prepare_validates_and_refuses_a_divergent_capture(dev, monkeypatch) -> None:
    """`prepare()` captures every bucket as a HIP graph and replays a synthetic round against
    the eager step (`graph_mtp.py:712-769`); a capture whose replay diverges (here a host-side
    perturbation of the argmax after the replay) is refused: rounds then run eagerly, and under
    SEED_MTP_REQUIRE_GRAPH=1 prepare() raises."""

    class Diverging(graph_mtp.GraphMTPRunner):
        def _capture(self, buf):
            inner = super()._capture(buf)

            def replay():
                inner()
                buf.step_argmax.add_(1)

            return replay

    good = graph_mtp.GraphMTPRunner(mh.build(dev, k=3, lanes=4), capacity=4)
    assert good.prepare() is True and good.validated == {1: True, 2: True, 4: True}
    bad = Diverging(mh.build(dev, k=3, lanes=4), capacity=4)
    assert bad.prepare() is False and not bad.enabled
    ids = mh.prompts(2)
    twin = mh.build(dev, k=3, lanes=4)
    toks, pos = [], []
    for lane, p in enumerate(ids):
        toks.append(int(twin.argmax(twin.prefill(lane, p)[None])[0]))
        bad.model.prefill(lane, p)
        good.model.prefill(lane, p)
        pos.append(len(p))
    want = graph_mtp.MTPVerifyRunner(twin, capacity=4).speculative_decode([0, 1], toks, pos)
    assert bad.speculative_decode([0, 1], toks, pos) == want
    assert good.speculative_decode([0, 1], toks, pos) == want  # a validated graph replay
    monkeypatch.setenv(graph_mtp.REQUIRE_GRAPH_ENV, "1")
    with pytest.raises(RuntimeError, match="SEED_MTP_REQUIRE_GRAPH"):
        Diverging(mh.build(dev, k=3, lanes=4), capacity=4).prepare()


def test_config5_bucket48_serves_45_lanes(dev) -> None:
    """Config 5's dimensions (bf16, 512 MXFP4 experts, vocab 248320): a 48-row captured bucket
    serving 45 lanes. The three idle lanes (45..47) come out bit-identical (no K/V row, DeltaNet
    commit or hidden seed from the padding rows), and the 45 real rows' results do not depend on
    what the padding rows read: re-running the round from the same state after scrambling the
    idle lanes' state gives bit-identical ids and lane state."""
    b, k, ctx, n = 48, 3, 256, 45
    model, toks, pos = mh.c5_model(dev, b, k, ctx)
    lanes = list(range(n))
    runner = graph_mtp.GraphMTPRunner(model, buckets=[b])
    start = mh.snapshot(model)
    runner.speculative_decode(lanes, toks[:n], pos[:n])  # eager, then captured
    assert list(runner.graphs) == [b]
    mh.restore(model, start)
    idle = _idle(model, range(n, b))
    got = runner.speculative_decode(lanes, toks[:n], pos[:n])  # graph replay
    for j, c in enumerate(got):
        assert 1 <= len(c) <= k + 1 and all(0 <= x < model.cfg.vocab for x in c)
    for before, now in zip(idle, _idle(model, range(n, b)), strict=True):
        assert torch.equal(before, now)
    after = [mh.slot_state(model, j, pos[j] + len(got[j])) for j in lanes]

    mh.restore(model, start)
    g = torch.Generator(device=dev).manual_seed(77)
    for p in model.pool:
        for name in ("conv", "rec"):
            if name in p:
                p[name][n:].normal_(generator=g)
    model.hidden_cache[n:].normal_(generator=g)
    again = runner.speculative_decode(lanes, toks[:n], pos[:n])  # graph replay
    assert again == got
    for j in lanes:
        for x, y in zip(after[j], mh.slot_state(model, j, pos[j] + len(got[j])), strict=True):
            assert torch.equal(x, y), j
