"""Speculative rejection sampling, restated in numpy (float64). TEST INFRASTRUCTURE ONLY.

The reference engine has no rejection sampling: MTP rounds run only when every lane is greedy
(`scheduler.py:1775-1793`, the `temperature <= 0` test at `:1789`; `model.py:4197-4201`). This
module therefore follows the published method, Leviathan, Kalman & Matias 2023 ("Fast Inference
from Transformers via Speculative Decoding", Algorithm 1) and Chen et al. 2023 ("Accelerating
Large Language Model Decoding with Speculative Sampling", Algorithm 2):

    p_i = softmax(target_i / T), q_i = softmax(draft_i / T)
    for i in 0..k-1: accept draft token x_i iff u_i * q_i(x_i) <= p_i(x_i)   (u_i ~ U[0,1))
    at the first rejection i: emit a sample of norm(max(0, p_i - q_i)); accepted length = i
    if all k accepted: emit a sample of p_k (the bonus); accepted length = k

Sampling from a weight vector w with a uniform r is inverse-CDF in index order: the smallest
v with cumsum(w)[v] > r * sum(w).

Pinning (tests/test_oracle_rejection.py), since no reference vector exists ("parity pinned by
invariants", no reference oracle):
- exact enumeration on a tiny vocab (V=3, k=2) over the draft's sampling and both acceptance
  draws shows the emitted first token is distributed exactly as p_0 (the method's theorem);
- p == q accepts every draft;
- one-hot p and q reduce to greedy acceptance (`oracle.accept_ref.greedy_accept_length`);
- fixed uniforms give identical outputs.
"""

from __future__ import annotations

import numpy as np


def softmax_t(logits: np.ndarray, temperature: float) -> np.ndarray:
    z = np.asarray(logits, dtype=np.float64) / temperature
    z = z - z.max(-1, keepdims=True)
    e = np.exp(z)
    return e / e.sum(-1, keepdims=True)


def sample_inverse_cdf(w: np.ndarray, r: float) -> int:
    """Smallest index v with cumsum(w)[v] > r * sum(w); the last positive index if rounding
    leaves none."""
    w = np.asarray(w, dtype=np.float64)
    c = np.cumsum(w)
    hit = np.nonzero(c > r * c[-1])[0]
    if hit.size:
        return int(hit[0])
    pos = np.nonzero(w > 0)[0]
    return int(pos[-1]) if pos.size else 0


def rejection_accept(
    target_logits: np.ndarray,
    draft_logits: np.ndarray,
    draft_tokens: np.ndarray,
    u_accept: np.ndarray,
    u_sample: np.ndarray,
    temperature: float,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """`(accept_len [B] int64, token [B] int64, ratio_margin [B, k] float64)`.

    `target_logits [B, k+1, V]`, `draft_logits [B, k, V]`, `draft_tokens [B, k]`,
    `u_accept [B, k]`, `u_sample [B]`. `token` is the resampled token at the first rejection,
    or the bonus sample when every draft was accepted. `ratio_margin[b, i]` is
    `p_i(x_i) - u_i q_i(x_i)` (>= 0 accepts), so a test can skip decisions that sit within
    floating-point noise of the boundary.
    """
    b, k1, _ = target_logits.shape
    k = k1 - 1
    acc = np.zeros(b, dtype=np.int64)
    tok = np.zeros(b, dtype=np.int64)
    margin = np.zeros((b, k), dtype=np.float64)
    for r in range(b):
        p = softmax_t(target_logits[r], temperature)
        q = softmax_t(draft_logits[r], temperature)
        a = k
        for i in range(k):
            x = int(draft_tokens[r, i])
            margin[r, i] = p[i, x] - u_accept[r, i] * q[i, x]
        for i in range(k):
            if margin[r, i] < 0:
                a = i
                break
        acc[r] = a
        if a < k:
            resid = np.maximum(p[a] - q[a], 0.0)
            tok[r] = sample_inverse_cdf(resid if resid.sum() > 0 else p[a], u_sample[r])
        else:
            tok[r] = sample_inverse_cdf(p[k], u_sample[r])
    return acc, tok, margin


def sample_drafts(draft_logits: np.ndarray, u_draft: np.ndarray, temperature: float) -> np.ndarray:
    """Draft tokens x_i ~ q_i by inverse CDF with the given uniforms `[B, k]`."""
    b, k, _ = draft_logits.shape
    out = np.zeros((b, k), dtype=np.int64)
    for r in range(b):
        q = softmax_t(draft_logits[r], temperature)
        for i in range(k):
            out[r, i] = sample_inverse_cdf(q[i], u_draft[r, i])
    return out
