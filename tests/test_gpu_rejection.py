"""Sampling-mode acceptance on the device (`mtpk_rejection_sample`, `mtpk_sample_rows`) against
the float64 restatement of the published method (`oracle/rejection_ref.py`).

The kernels compute in fp32, the oracle in float64, so an accept decision is compared only
where the oracle's margin `p(x) - u q(x)` is clear of rounding, and a drawn token is checked
for consistency with the oracle's cumulative weights: the kernel's index `v` must have
`cum[v-1] <= r * total <= cum[v]` up to a small tolerance and positive weight (an inverse-CDF
draw may move to a neighbour only when `r * total` sits on a boundary within rounding).
Config 4: target and draft bf16 `[48, 4, 248320]`, target N(0, 3), draft = target + N(0, 1),
T = 0.7, seeded uniforms.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import graph_mtp
import mtp
from oracle import accept_ref, rejection_ref as rj

pytestmark = pytest.mark.gpu

MARGIN_RTOL = 1e-4  # fp32 softmax over up to 248320 logits vs float64
CDF_TOL = 2e-5


def _weights(p_row: np.ndarray, q_row: np.ndarray | None) -> np.ndarray:
    if q_row is None:
        return p_row
    resid = np.maximum(p_row - q_row, 0.0)
    return resid if resid.sum() > 0 else p_row


def _token_consistent(w: np.ndarray, r: float, v: int) -> bool:
    c = np.cumsum(w)
    total = c[-1]
    x = r * total
    tol = CDF_TOL * total
    before = c[v - 1] if v > 0 else 0.0
    return w[v] > 0 and before <= x + tol and c[v] >= x - tol


def _case(b, k, vocab, dtype, seed, target_scale=3.0, noise=1.0, temperature=0.7):
    g = np.random.default_rng(seed)
    tl = (g.standard_normal((b, k + 1, vocab)) * target_scale).astype(np.float32)
    dl = tl[:, :k] + (g.standard_normal((b, k, vocab)) * noise).astype(np.float32)
    tt = torch.from_numpy(tl).to(dtype)
    dd = torch.from_numpy(dl).to(dtype)
    tl64, dl64 = tt.double().numpy(), dd.double().numpy()  # the values the kernel sees
    drafts = rj.sample_drafts(dl64, g.random((b, k)), temperature)
    ua = g.random((b, k)).astype(np.float32)
    us = g.random(b).astype(np.float32)
    return tt, dd, tl64, dl64, drafts, ua, us


def _check(dev, tt, dd, tl64, dl64, drafts, ua, us, temperature, max_skip_frac=0.05):
    b, t, _ = tt.shape
    k = t - 1
    acc, tok, emitted, margin = graph_mtp.rejection_sample(
        tt.to(dev), dd.to(dev), torch.from_numpy(drafts).to(dev), torch.from_numpy(ua).to(dev),
        torch.from_numpy(us).to(dev), temperature, with_margin=True)
    acc, tok, emitted, margin = acc.cpu().numpy(), tok.cpu().numpy(), emitted.cpu().numpy(), margin.cpu().numpy()
    want_acc, _, want_margin = rj.rejection_accept(tl64, dl64, drafts, ua.astype(np.float64),
                                                   us.astype(np.float64), temperature)
    np.testing.assert_allclose(margin, want_margin, rtol=1e-3, atol=5e-6)
    skipped = 0
    for j in range(b):
        p = rj.softmax_t(tl64[j], temperature)
        q = rj.softmax_t(dl64[j], temperature)
        x = drafts[j]
        scale = np.maximum(p[np.arange(k), x], ua[j] * q[np.arange(k), x])
        clear = np.abs(want_margin[j]) > MARGIN_RTOL * scale
        decided = int(want_acc[j])
        # every margin up to and including the deciding one must be clear of rounding
        if not clear[: min(decided + 1, k)].all():
            skipped += 1
            continue
        assert acc[j] == decided, (j, acc[j], decided)
        w = _weights(p[decided], q[decided] if decided < k else None)
        assert _token_consistent(w, float(us[j]), int(tok[j])), (j, int(tok[j]))
        assert emitted[j, :decided].tolist() == drafts[j, :decided].tolist()
        assert (emitted[j, decided:] == tok[j]).all()
    assert skipped <= max_skip_frac * b + 1
    return acc, tok, emitted


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_small_vocab_matches_oracle(dev, dtype) -> None:
    for seed, (b, k, vocab) in enumerate([(6, 3, 1000), (5, 1, 4097), (8, 2, 130), (3, 3, 8191)]):
        case = _case(b, k, vocab, dtype, seed)
        _check(dev, *case, 0.7)


def test_config4_full_vocab(dev) -> None:
    """[48, 4, 248320] bf16, T = 0.7: decisions and draws agree with the oracle."""
    case = _case(48, 3, 248320, torch.bfloat16, 11)
    acc, _, _ = _check(dev, *case, 0.7)
    assert 0 < acc.mean() < 3  # noise 1 on scale 3 logits: partial acceptance


def test_identical_distributions_accept_everything(dev) -> None:
    g = np.random.default_rng(3)
    b, k, vocab, temp = 16, 3, 5000, 0.7
    tl = torch.from_numpy((g.standard_normal((b, k + 1, vocab)) * 3).astype(np.float32)).to(torch.bfloat16)
    drafts = rj.sample_drafts(tl[:, :k].double().numpy(), g.random((b, k)), temp)
    ua = torch.from_numpy(g.random((b, k)).astype(np.float32) * 0.999)
    acc, _, _, _ = graph_mtp.rejection_sample(tl.to(dev), tl[:, :k].contiguous().to(dev),
                                              torch.from_numpy(drafts).to(dev), ua.to(dev),
                                              torch.rand(b).to(dev), temp)
    assert (acc.cpu() == k).all()


def test_near_one_hot_reduces_to_greedy(dev) -> None:
    """Sharp target and draft at a tiny temperature: rejection sampling is greedy acceptance,
    the resampled or bonus token the target argmax."""
    g = np.random.default_rng(4)
    b, k, vocab = 16, 3, 3000
    tl = (g.standard_normal((b, k + 1, vocab)) * 20).astype(np.float32)
    dl = (tl[:, :k] + g.standard_normal((b, k, vocab)) * 15).astype(np.float32)
    drafts = dl.argmax(-1)
    acc, tok, _, _ = graph_mtp.rejection_sample(
        torch.from_numpy(tl).to(dev), torch.from_numpy(dl).to(dev), torch.from_numpy(drafts).to(dev),
        torch.from_numpy(g.random((b, k)).astype(np.float32) * 0.99).to(dev),
        torch.from_numpy(g.random(b).astype(np.float32)).to(dev), 1e-3)
    sa = tl.argmax(-1)
    for j in range(b):
        want = accept_ref.greedy_accept_length(drafts[j].tolist(), sa[j, :k].tolist())
        assert int(acc[j]) == want
        assert int(tok[j]) == sa[j, want]


def test_deterministic_and_round_indices(dev) -> None:
    """Same inputs, same outputs; `rejection_accept` gives the oracle's rollback indices for
    the emitted tokens, with the budget and stop ids applied."""
    tt, dd, _, _, drafts, ua, us = _case(48, 3, 248320, torch.bfloat16, 12)
    args = (tt.to(dev), dd.to(dev), torch.from_numpy(drafts).to(dev), torch.from_numpy(ua).to(dev),
            torch.from_numpy(us).to(dev), 0.7)
    a1 = graph_mtp.rejection_sample(*args)
    a2 = graph_mtp.rejection_sample(*args)
    for x, y in zip(a1[:3], a2[:3]):
        assert torch.equal(x, y)
    g = np.random.default_rng(5)
    b = 48
    active = g.random(b) < 0.9
    pos = g.integers(0, 8000, b)
    budget = g.integers(1, 6, b)
    stops = np.full((b, 8), -1, dtype=np.int64)
    emitted = a1[2].cpu().numpy()
    stops[::5, 0] = emitted[::5, 1]
    res, em = graph_mtp.rejection_accept(
        *args[:5], 0.7, torch.from_numpy(active).to(dev), torch.from_numpy(pos).to(dev),
        torch.from_numpy(budget).to(dev), torch.from_numpy(stops).to(dev), 3)
    want = accept_ref.round_indices(drafts, em.cpu().numpy(), active, pos, budget, stops, 3)
    for name, val in want.items():
        got = getattr(res, name).cpu().numpy()
        np.testing.assert_array_equal(got.astype(val.dtype), val, err_msg=name)


def test_sample_rows_inverse_cdf(dev) -> None:
    g = np.random.default_rng(6)
    rows, vocab, temp = 64, 248320, 0.7
    lg = torch.from_numpy((g.standard_normal((rows, vocab)) * 3).astype(np.float32)).to(torch.bfloat16)
    u = g.random(rows).astype(np.float32)
    tok = mtp.sample_rows(lg.to(dev), temp, torch.from_numpy(u).to(dev)).cpu().numpy()
    l64 = lg.double().numpy()
    for j in range(rows):
        assert _token_consistent(rj.softmax_t(l64[j], temp), float(u[j]), int(tok[j])), j
    lf = torch.from_numpy((g.standard_normal((rows, 5000)) * 50).astype(np.float32))  # no ties
    sharp = mtp.sample_rows(lf.to(dev), 1e-3, torch.from_numpy(u).to(dev)).cpu()
    assert torch.equal(sharp, lf.argmax(-1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_chunk_and_masked_draft_logit(dev, dtype) -> None:
    """A whole 4096-logit chunk of -inf (and a ragged -inf tail), plus a -inf target logit on a
    drafted token: margins stay finite, no masked token is drawn, and the decisions and draws
    follow the oracle."""
    b, k, vocab = 8, 3, 3 * 4096 + 500
    tt, dd, tl64, dl64, drafts, ua, us = _case(b, k, vocab, dtype, 21)
    masked = np.r_[4096:8192, vocab - 300 : vocab]
    for ten in (tt, dd):
        ten[..., torch.from_numpy(masked)] = -float("inf")
    tl64, dl64 = tt.double().numpy(), dd.double().numpy()
    g = np.random.default_rng(22)
    drafts = rj.sample_drafts(dl64, g.random((b, k)), 0.7)
    tt[2, 0, int(drafts[2, 0])] = -float("inf")  # lane 2's first draft has p = 0
    tl64 = tt.double().numpy()
    acc, tok, emitted = _check(dev, tt, dd, tl64, dl64, drafts, ua, us, 0.7)
    assert acc[2] == 0
    assert not np.isin(tok, masked).any()


def test_sample_rows_masked_chunk(dev) -> None:
    rows, vocab = 6, 3 * 4096
    g = np.random.default_rng(23)
    logits = (g.standard_normal((rows, vocab)) * 3).astype(np.float32)
    logits[:, 4096:8192] = -np.inf
    u = g.random(rows).astype(np.float32)
    got = mtp.sample_rows(torch.from_numpy(logits).to(dev), 0.7, torch.from_numpy(u).to(dev)).cpu().numpy()
    for r in range(rows):
        p = rj.softmax_t(logits[r].astype(np.float64), 0.7)
        assert _token_consistent(p, float(u[r]), int(got[r]))
        assert not 4096 <= got[r] < 8192


@pytest.mark.parametrize("b,k,dtype", [(48, 3, torch.bfloat16), (300, 1, torch.float32),
                                       (7, 0, torch.float32), (1024, 3, torch.bfloat16)])
def test_fused_acceptance_equals_sample_then_greedy_accept(dev, b, k, dtype) -> None:
    """`rejection_accept` (one pass: the sampler's launches also write every acceptance output)
    equals `rejection_sample` followed by `greedy_accept` over the emitted tokens, bit for bit:
    inactive lanes, budgets of 0..5, stop ids on drafts and on drawn tokens, and up to 1024
    lanes (the pack's scan over several waves)."""
    vocab = 3000
    tt, dd, _, _, drafts, ua, us = _case(b, k, vocab, dtype, 40 + b + k, noise=0.7)
    g = np.random.default_rng(b + k)
    args = (tt.to(dev), dd.to(dev), torch.from_numpy(drafts).to(dev), torch.from_numpy(ua).to(dev),
            torch.from_numpy(us).to(dev), 0.7)
    _, _, emitted, _ = graph_mtp.rejection_sample(*args)
    em = emitted.cpu().numpy()
    active = torch.from_numpy(g.random(b) < 0.85).to(dev)
    pos = torch.from_numpy(g.integers(0, 8000, b)).to(dev)
    budget = torch.from_numpy(g.integers(0, 6, b)).to(dev)
    stops = np.full((b, 3), -1, dtype=np.int64)
    if k > 0:
        stops[::3, 0] = drafts[::3, 0]          # a stop on the first draft
    stops[1::4, 1] = em[1::4, min(1, k)]        # on a later column: a draft or the drawn token
    stops = torch.from_numpy(stops).to(dev)
    want = graph_mtp.greedy_accept(emitted, args[2], active, pos, budget, stops, 3)
    got, em2 = graph_mtp.rejection_accept(*args, active, pos, budget, stops, 3)
    assert torch.equal(em2, emitted)
    for name in ("accept_len", "lengths", "packed_src", "packed_cu", "conv_idx", "keep", "bonus",
                 "next_pos", "budget_left", "live", "hidden_src"):
        assert torch.equal(getattr(got, name), getattr(want, name)), name
