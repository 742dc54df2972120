"""Gated delta-rule recurrence of the Gated DeltaNet layers, restated in float64 numpy.
TEST INFRASTRUCTURE ONLY (see oracle/__init__).

Reference: the decode/verify recurrence `_delta_rule_verify_exact_kernel`
(`deltanet_fused.py:343-392`) and its torch form (`model.py:651-697`). Per step, for one
(row, head) with state S [dk, dv], normalised q, k [dk], v [dv], log decay g, strength beta:

    S <- exp(g) S;   S <- S + beta k (v - S^T k)^T;   out = S^T q

The verify pass runs `t` steps from the stored state and keeps every output; the commit
(`deltanet_verify_rollback`, `model.py:3907-3972`) advances the stored state by each row's
accepted prefix of `lengths[j]` steps.

Pinning (tests/test_oracle_deltanet.py): closed forms that a dropped term, a wrong sign or a
transposed operand breaks — pure decay when beta = 0; the delta rule's write-then-read
identity S'^T k = v when g = 0, beta = 1 and |k| = 1; the matrix form
(I - beta k k^T) e^g S + beta k v^T; steps composing as a product of those affine maps; and
the commit equal to the verify state after `lengths[j]` steps.
"""

from __future__ import annotations

import numpy as np


def delta_rule_step(state: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray, g: float,
                    beta: float) -> tuple[np.ndarray, np.ndarray]:
    """One step for one (row, head): returns (new state [dk, dv], out [dv]), float64."""
    s = np.asarray(state, np.float64) * np.exp(np.float64(g))
    k = np.asarray(k, np.float64)
    delta = (np.asarray(v, np.float64) - s.T @ k) * np.float64(beta)
    s = s + np.outer(k, delta)
    return s, s.T @ np.asarray(q, np.float64)


def delta_rule_rows(state: np.ndarray, slots, q: np.ndarray, k: np.ndarray, v: np.ndarray,
                    g: np.ndarray, beta: np.ndarray, lengths=None) -> tuple[np.ndarray, np.ndarray]:
    """Every row and head. `state` [slots_total, heads, dk, dv]; `q`, `k`
    [B, t, qk_heads, dk] (head h reads q/k head h // (heads // qk_heads)); `v` [B, t, heads, dv];
    `g`, `beta` [B, t, heads]. Without `lengths`: returns (the state pool unchanged, outputs
    [B, t, heads, dv]). With `lengths` [B]: row j's slot advances by min(lengths[j], t) steps;
    returns (the new pool, the outputs of the steps taken, zeros past them)."""
    pool = np.array(state, np.float64, copy=True)
    b, t = q.shape[:2]
    heads, dv = pool.shape[1], pool.shape[3]
    rep = heads // q.shape[2]
    slots = list(range(b)) if slots is None else [int(s) for s in slots]
    out = np.zeros((b, t, heads, dv))
    new = pool.copy()
    for j in range(b):
        n = t if lengths is None else int(min(max(int(lengths[j]), 0), t))
        for h in range(heads):
            s = pool[slots[j], h]
            for st in range(n):
                s, out[j, st, h] = delta_rule_step(s, q[j, st, h // rep], k[j, st, h // rep],
                                                   v[j, st, h], g[j, st, h], beta[j, st, h])
            if lengths is not None:
                new[slots[j], h] = s
    return (pool if lengths is None else new), out
