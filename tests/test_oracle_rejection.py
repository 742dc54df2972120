"""Pins oracle.rejection_ref by the method's own guarantees (no reference vector exists: the
reference engine never samples, `scheduler.py:1789`)."""

import itertools

import numpy as np

from oracle import accept_ref, rejection_ref as rj


def _enumerate_first_token(p_logits, q_logits, T, grid=24):
    """Distribution of the first emitted token by exact enumeration of the draft choice and a
    fine midpoint grid over both uniforms (the acceptance test and the residual sample)."""
    p = rj.softmax_t(p_logits, T)
    q = rj.softmax_t(q_logits, T)
    V = p.shape[-1]
    dist = np.zeros(V)
    us = (np.arange(grid) + 0.5) / grid
    for x in range(V):  # draft token x0 ~ q0
        for u in us:
            for r in us:
                acc, tok, _ = rj.rejection_accept(
                    p_logits[None], q_logits[None], np.array([[x, 0]]), np.array([[u, 0.0]]), np.array([r]), T
                )
                first = x if acc[0] >= 1 else tok[0]
                dist[first] += q[0, x] / grid**2
    return dist, p[0]


def test_emitted_token_follows_the_target():
    rng = np.random.default_rng(0)
    V, k, T = 3, 2, 0.7
    pl = rng.standard_normal((k + 1, V)) * 2
    ql = pl[:k] + rng.standard_normal((k, V))
    dist, p0 = _enumerate_first_token(pl, ql, T, grid=60)
    assert np.allclose(dist, p0, atol=2e-2)


def test_identical_distributions_accept_everything():
    rng = np.random.default_rng(1)
    B, k, V = 6, 3, 50
    tl = rng.standard_normal((B, k + 1, V)) * 3
    drafts = rj.sample_drafts(tl[:, :k], rng.random((B, k)), 0.7)
    acc, _, _ = rj.rejection_accept(tl, tl[:, :k], drafts, rng.random((B, k)) * 0.999, rng.random(B), 0.7)
    assert (acc == k).all()


def test_one_hot_reduces_to_greedy():
    rng = np.random.default_rng(2)
    B, k, V = 16, 3, 20
    tl = rng.standard_normal((B, k + 1, V)) * 50  # near one-hot at T=1e-3
    dl = tl[:, :k] + rng.standard_normal((B, k, V)) * 30
    drafts = dl.argmax(-1)
    acc, tok, _ = rj.rejection_accept(tl, dl, drafts, rng.random((B, k)) * 0.99, rng.random(B), 1e-3)
    step_argmax = tl.argmax(-1)
    for b in range(B):
        want = accept_ref.greedy_accept_length(drafts[b].tolist(), step_argmax[b, :k].tolist())
        assert acc[b] == want
        assert tok[b] == step_argmax[b, want]


def test_fixed_uniforms_are_deterministic():
    rng = np.random.default_rng(3)
    B, k, V = 4, 3, 40
    tl = rng.standard_normal((B, k + 1, V))
    dl = tl[:, :k] + rng.standard_normal((B, k, V))
    u, r = rng.random((B, k)), rng.random(B)
    d = rj.sample_drafts(dl, rng.random((B, k)), 0.7)
    a1 = rj.rejection_accept(tl, dl, d, u, r, 0.7)
    a2 = rj.rejection_accept(tl, dl, d, u, r, 0.7)
    for x, y in zip(a1, a2):
        assert np.array_equal(x, y)


def test_inverse_cdf():
    w = np.array([0.0, 1.0, 0.0, 3.0])
    assert [rj.sample_inverse_cdf(w, r) for r in (0.0, 0.24, 0.25, 0.99)] == [1, 1, 3, 3]
    assert list(itertools.islice((rj.sample_inverse_cdf(np.array([0, 0, 2.0]), 0.5),), 1)) == [2]


def test_masked_logits_carry_no_mass():
    """-inf logits (a masked stretch of the vocabulary) have probability 0: the oracle on the
    full vocabulary equals the oracle on the vocabulary with the stretch cut out, tokens mapped
    back; a draft token whose target logit is -inf is rejected; one whose draft logit is -inf
    (q = 0) is accepted."""
    rng = np.random.default_rng(4)
    B, k, V, T = 6, 3, 40, 0.7
    tl = rng.standard_normal((B, k + 1, V)) * 2
    dl = tl[:, :k] + rng.standard_normal((B, k, V))
    cut = np.arange(10, 22)
    tl[:, :, cut] = -np.inf
    dl[:, :, cut] = -np.inf
    keep = np.setdiff1d(np.arange(V), cut)
    drafts = rj.sample_drafts(dl, rng.random((B, k)), T)
    assert not np.isin(drafts, cut).any()
    ua, us = rng.random((B, k)), rng.random(B)
    acc, tok, margin = rj.rejection_accept(tl, dl, drafts, ua, us, T)
    remap = np.searchsorted(keep, drafts)
    acc2, tok2, margin2 = rj.rejection_accept(tl[..., keep], dl[..., keep], remap, ua, us, T)
    assert np.array_equal(acc, acc2) and np.array_equal(tok, keep[tok2])
    assert np.allclose(margin, margin2)
    assert not np.isin(tok, cut).any() and np.isfinite(margin).all()
    # draft token 0 of lane 0: target logit -inf -> p = 0 -> rejected at position 0
    t2 = tl.copy()
    t2[0, 0, drafts[0, 0]] = -np.inf
    acc3, _, m3 = rj.rejection_accept(t2, dl, drafts, ua, us, T)
    assert acc3[0] == 0 and m3[0, 0] <= 0
    # draft logit -inf on the drafted token of lane 1, position 0: q = 0 -> accepted there
    d2 = dl.copy()
    d2[1, 0, drafts[1, 0]] = -np.inf
    _, _, m4 = rj.rejection_accept(tl, d2, drafts, ua, us, T)
    assert m4[1, 0] > 0
