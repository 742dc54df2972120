"""HIP argmax + greedy acceptance (`mtpk_argmax_rows`, `mtpk_greedy_accept`) against the
oracle: the reference tests' literal vectors, random batches (every output, bit-exact), and
config 4 at full size (target/draft bf16 [48, 4, 248320])."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import graph_mtp
from tests.model_helpers import shape_model
import mtp
from oracle import accept_ref as ar

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def dev_long(a, dev):
    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, dtype=np.int64))).to(dev)


def accept(dev, sa, draft, active, pos, budget, stops, conv_k1=3, forced_n=None):
    return graph_mtp.greedy_accept(
        dev_long(sa, dev), dev_long(draft, dev), torch.from_numpy(np.asarray(active, bool)).to(dev),
        dev_long(pos, dev), dev_long(budget, dev), dev_long(stops, dev), conv_k1,
        forced_n=None if forced_n is None else dev_long(forced_n, dev),
    )


def test_accept_len_golden(dev):
    g = GOLDEN["accept_len"]
    b = len(g["want"])
    r = accept(dev, g["step_argmax"], g["draft"], [True] * b, [0] * b, [99] * b, [[-1]] * b)
    assert r.accept_len.tolist() == g["want"]


def test_commit_limit_golden(dev):
    g = GOLDEN["commit_limit"]
    sa = np.array(g["step_argmax"])
    acc = np.array(g["accept"])
    # drafts agreeing with step_argmax exactly up to the given accept length
    draft = sa[:, :2].copy()
    for j, a in enumerate(acc):
        if a < 2:
            draft[j, a] = sa[j, a] + 1000
    r = accept(dev, sa, draft, [True] * 5, [0] * 5, g["budget"], g["stops"])
    assert r.accept_len.tolist() == g["want"]


def test_pack_index_golden(dev):
    g = GOLDEN["pack_index"]
    width = g["width"]
    for case in g["cases"]:
        lengths = np.array(case["lengths"])
        sa = np.arange(3 * width).reshape(3, width)
        draft = sa[:, : width - 1].copy()
        for j, n in enumerate(lengths):
            if n - 1 < width - 1:
                draft[j, n - 1] = -5
        r = accept(dev, sa, draft, [True] * 3, [0] * 3, [99] * 3, [[-1]] * 3)
        assert r.lengths.tolist() == case["lengths"]
        assert r.packed_cu.tolist() == case["cu"]
        src = r.packed_src.cpu().numpy()
        assert src[: case["cu"][-1]].tolist() == case["live"]
        assert ((src >= 0) & (src < 3 * width)).all()


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("b,k", [(1, 1), (7, 2), (48, 3), (1024, 3)])
def test_random_batches_every_output(dev, seed, b, k):
    rng = np.random.default_rng(seed * 100 + b + k)
    t = k + 1
    sa = rng.integers(0, 5, (b, t))
    draft = np.where(rng.random((b, k)) < 0.75, sa[:, :k], rng.integers(0, 5, (b, k)))
    active = rng.random(b) < 0.85
    pos = rng.integers(0, 8000, b)
    budget = rng.integers(0, 6, b)
    stops = np.where(rng.random((b, 8)) < 0.15, rng.integers(0, 5, (b, 8)), -1)
    want = ar.round_indices(draft, sa, active, pos, budget, stops, 3)
    r = accept(dev, sa, draft, active, pos, budget, stops, 3)
    for name, w in want.items():
        got = getattr(r, name).cpu().numpy()
        assert np.array_equal(got.astype(w.dtype), w), name


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("b,k", [(1, 1), (9, 2), (48, 3), (1024, 3)])
def test_forced_rows_every_output(dev, seed, b, k):
    """Forced feed (`forced_n > 0`): the row accepts exactly its forced drafts, stop ids and
    budget notwithstanding, and every lane-table and rollback output follows from that
    (`accept_ref.round_indices(..., forced_n)`), bit for bit; unforced rows of the same batch
    are as without forcing."""
    rng = np.random.default_rng(seed * 10 + b)
    t = k + 1
    sa = rng.integers(0, 5, (b, t))
    draft = np.where(rng.random((b, k)) < 0.6, sa[:, :k], rng.integers(0, 5, (b, k)))
    active = rng.random(b) < 0.85
    pos = rng.integers(0, 8000, b)
    budget = rng.integers(1, 6, b)
    stops = np.where(rng.random((b, 8)) < 0.2, rng.integers(0, 5, (b, 8)), -1)
    forced_n = np.where(rng.random(b) < 0.5, rng.integers(1, k + 3, b), 0)  # > k clamps to k
    want = ar.round_indices(draft, sa, active, pos, budget, stops, 3, forced_n)
    r = accept(dev, sa, draft, active, pos, budget, stops, 3, forced_n)
    for name, w in want.items():
        got = getattr(r, name).cpu().numpy()
        assert np.array_equal(got.astype(w.dtype), w), name
    plain = accept(dev, sa, draft, active, pos, budget, stops, 3, np.zeros(b, np.int64))
    free = ar.round_indices(draft, sa, active, pos, budget, stops, 3)
    for name, w in free.items():
        assert np.array_equal(getattr(plain, name).cpu().numpy().astype(w.dtype), w), name


def test_argmax_first_occurrence_and_zero_signs(dev):
    x = torch.tensor([[1.0, 3.0, 3.0, 2.0], [-0.0, 0.0, -1.0, -2.0], [-5, -4, -4, -9.0]], device=dev)
    for dt in (torch.float32, torch.bfloat16):
        assert mtp.argmax_rows(x.to(dt)).tolist() == [1, 0, 1]
    # max at the very last element of a row whose length is not a multiple of 8
    y = torch.zeros(2, 1000 * 8 + 3, device=dev, dtype=torch.bfloat16)
    y[0, -1] = 1
    y[1, 5] = 1
    y[1, 4000] = 1
    assert mtp.argmax_rows(y).tolist() == [8002, 5]


def test_config4_greedy_full_vocab(dev):
    """Config 4: target N(0,3), draft = target + N(0,1), bf16 [48, 4, 248320]; greedy drafts are
    the draft argmaxes of positions 0..k-1; outputs bit-exact against numpy."""
    B, t, V = 48, 4, 248320
    g = torch.Generator(dev).manual_seed(4)
    target = (torch.randn(B, t, V, device=dev, generator=g) * 3).to(torch.bfloat16)
    draft_logits = (target.float() + torch.randn(B, t, V, device=dev, generator=g)).to(torch.bfloat16)
    step_argmax = mtp.argmax_rows(target)
    drafts = mtp.argmax_rows(draft_logits[:, : t - 1])
    tnp = target.float().cpu().numpy()
    dnp = draft_logits.float().cpu().numpy()
    assert np.array_equal(step_argmax.cpu().numpy(), ar.argmax_first(tnp))
    assert np.array_equal(drafts.cpu().numpy(), ar.argmax_first(dnp[:, : t - 1]))
    rng = np.random.default_rng(44)
    active = rng.random(B) < 0.9
    pos = rng.integers(0, 8000, B)
    budget = rng.integers(1, 8, B)
    stops = np.full((B, 8), -1)
    stops[:, 0] = rng.integers(0, V, B)
    r = accept(dev, step_argmax.cpu().numpy(), drafts.cpu().numpy(), active, pos, budget, stops)
    want = ar.round_indices(drafts.cpu().numpy(), step_argmax.cpu().numpy(), active, pos, budget,
                            stops, 3)
    for name, w in want.items():
        assert np.array_equal(getattr(r, name).cpu().numpy().astype(w.dtype), w), name


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("b,t,v", [(1, 4, 248320), (48, 4, 248320), (3, 2, 1003), (1024, 4, 600),
                                   (5, 1, 3000), (64, 64, 40)])
def test_keys_path_finishes_the_argmax(dev, dt, b, t, v):
    """`mtpk_argmax_keys` + `mtpk_greedy_accept_keys` against numpy: the written step_argmax is
    the first-occurrence argmax (coarse logits, so ties across vocabulary chunks are common) and
    every acceptance output equals the oracle's on it."""
    g = torch.Generator(dev).manual_seed(b + t)
    logits = torch.randint(-6, 6, (b * t, v), device=dev, generator=g).to(dt)
    rng = np.random.default_rng(b * 7 + v)
    want_sa = ar.argmax_first(logits.float().cpu().numpy()).reshape(b, t)
    draft = np.where(rng.random((b, t - 1)) < 0.7, want_sa[:, : t - 1], rng.integers(0, v, (b, t - 1)))
    active = rng.random(b) < 0.9
    pos = rng.integers(0, 8000, b)
    budget = rng.integers(1, 8, b)
    stops = np.where(rng.random((b, 8)) < 0.1, rng.integers(0, v, (b, 8)), -1)
    step_argmax = torch.full((b, t), -7, dtype=torch.long, device=dev)
    r = graph_mtp.greedy_accept(
        step_argmax, dev_long(draft, dev), torch.from_numpy(active).to(dev), dev_long(pos, dev),
        dev_long(budget, dev), dev_long(stops, dev), 3, keys=mtp.argmax_keys(logits))
    assert np.array_equal(step_argmax.cpu().numpy(), want_sa)
    want = ar.round_indices(draft, want_sa, active, pos, budget, stops, 3)
    for name, w in want.items():
        assert np.array_equal(getattr(r, name).cpu().numpy().astype(w.dtype), w), name
    # the same launch with forced feed on some rows
    forced_n = np.where(rng.random(b) < 0.5, rng.integers(0, t, b), 0)
    r = graph_mtp.greedy_accept(
        step_argmax, dev_long(draft, dev), torch.from_numpy(active).to(dev), dev_long(pos, dev),
        dev_long(budget, dev), dev_long(stops, dev), 3, keys=mtp.argmax_keys(logits),
        forced_n=dev_long(forced_n, dev))
    want = ar.round_indices(draft, want_sa, active, pos, budget, stops, 3, forced_n)
    for name, w in want.items():
        assert np.array_equal(getattr(r, name).cpu().numpy().astype(w.dtype), w), name


def test_keys_path_limits(dev):
    """batch * t above 4096 verify rows is refused by the C check; a keys tensor of another
    row count by the wrapper."""
    b, t = 1024, 5
    keys = mtp.argmax_keys(torch.zeros(b * t, 16, device=dev))
    ones = torch.ones(b, dtype=torch.bool, device=dev)
    z = torch.zeros(b, dtype=torch.long, device=dev)
    stops = torch.full((b, 1), -1, dtype=torch.long, device=dev)
    draft = torch.zeros(b, t - 1, dtype=torch.long, device=dev)
    with pytest.raises(ValueError, match="mtpk_greedy_accept"):
        graph_mtp.greedy_accept(torch.zeros(b, t, dtype=torch.long, device=dev), draft, ones, z,
                                z + 1, stops, 0, keys=keys)
    with pytest.raises(ValueError, match="keys must be"):
        graph_mtp.greedy_accept(torch.zeros(2, 2, dtype=torch.long, device=dev), draft[:2, :1],
                                ones[:2], z[:2], z[:2] + 1, stops[:2], 0, keys=keys)


def test_accept_round_writes_buffers(dev):
    buf = graph_mtp.MTPVerifyBuffers(shape_model(64, 4), 8, 4, dev)
    rng = np.random.default_rng(3)
    sa = rng.integers(0, 3, (8, 4))
    buf.token_matrix[:, 1:] = dev_long(np.where(rng.random((8, 3)) < 0.7, sa[:, :3], 9), dev)
    buf.active[:6] = True
    buf.budget.fill_(9)
    graph_mtp.accept_round(buf, dev_long(sa, dev))
    want = ar.accept_len(buf.token_matrix[:, 1:].cpu().numpy(), sa)
    assert np.array_equal(buf.accept_len.cpu().numpy(), want)
    assert np.array_equal(buf.bonus.cpu().numpy(), sa[np.arange(8), want])
    torch_acc = graph_mtp._accept_len(buf.token_matrix[:, 1:], dev_long(sa, dev))
    assert torch.equal(torch_acc, buf.accept_len)
