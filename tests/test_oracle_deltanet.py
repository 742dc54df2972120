"""Pins `oracle/deltanet_ref.py` (the gated delta rule) on closed forms, on the CPU."""

from __future__ import annotations

import numpy as np

from oracle import deltanet_ref as dn


def _unit(rng, n):
    x = rng.standard_normal(n)
    return x / np.linalg.norm(x)


def test_zero_beta_is_pure_decay() -> None:
    rng = np.random.default_rng(0)
    s = rng.standard_normal((8, 5))
    q, k, v = rng.standard_normal(8), _unit(rng, 8), rng.standard_normal(5)
    new, out = dn.delta_rule_step(s, q, k, v, -0.3, 0.0)
    np.testing.assert_allclose(new, np.exp(-0.3) * s, rtol=1e-14)
    np.testing.assert_allclose(out, (np.exp(-0.3) * s).T @ q, rtol=1e-14)


def test_full_write_then_read_returns_v() -> None:
    """g = 0, beta = 1, |k| = 1: the step stores v under key k exactly (S'^T k = v)."""
    rng = np.random.default_rng(1)
    s = rng.standard_normal((16, 7))
    k, v = _unit(rng, 16), rng.standard_normal(7)
    new, out = dn.delta_rule_step(s, k, k, v, 0.0, 1.0)
    np.testing.assert_allclose(new.T @ k, v, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(out, v, rtol=1e-12, atol=1e-12)


def test_step_matches_matrix_form() -> None:
    rng = np.random.default_rng(2)
    s = rng.standard_normal((6, 4))
    q, k, v = rng.standard_normal(6), _unit(rng, 6), rng.standard_normal(4)
    g, beta = -0.7, 0.4
    new, out = dn.delta_rule_step(s, q, k, v, g, beta)
    want = (np.eye(6) - beta * np.outer(k, k)) @ (np.exp(g) * s) + beta * np.outer(k, v)
    np.testing.assert_allclose(new, want, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(out, want.T @ q, rtol=1e-13, atol=1e-13)


def test_rows_compose_steps_and_commit_prefix() -> None:
    """Two steps equal the composed affine maps; a commit of n steps equals the verify state
    after n steps; the verify pass leaves the pool unchanged; q/k heads are shared by rep."""
    rng = np.random.default_rng(3)
    slots_total, heads, qk_heads, dk, dv, b, t = 5, 4, 2, 6, 3, 3, 3
    pool = rng.standard_normal((slots_total, heads, dk, dv))
    q = rng.standard_normal((b, t, qk_heads, dk))
    k = rng.standard_normal((b, t, qk_heads, dk))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((b, t, heads, dv))
    g = -rng.random((b, t, heads))
    beta = rng.random((b, t, heads))
    slots = [4, 0, 2]
    same, out = dn.delta_rule_rows(pool, slots, q, k, v, g, beta)
    np.testing.assert_array_equal(same, pool)
    j, h = 1, 3
    s0 = pool[slots[j], h]
    maps = []
    for st in range(2):
        kk = k[j, st, h // 2]
        a = (np.eye(dk) - beta[j, st, h] * np.outer(kk, kk)) * np.exp(g[j, st, h])
        maps.append((a, beta[j, st, h] * np.outer(kk, v[j, st, h])))
    s2 = maps[1][0] @ (maps[0][0] @ s0 + maps[0][1]) + maps[1][1]
    np.testing.assert_allclose(out[j, 1, h], s2.T @ q[j, 1, h // 2], rtol=1e-12, atol=1e-12)
    lengths = np.array([0, 2, 5])
    new, _ = dn.delta_rule_rows(pool, slots, q, k, v, g, beta, lengths)
    np.testing.assert_allclose(new[slots[1], h], s2, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(new[slots[0]], pool[slots[0]])  # length 0: untouched
    np.testing.assert_array_equal(new[1], pool[1])  # not a row's slot
    np.testing.assert_array_equal(new[3], pool[3])
