"""Seeded synthetic inputs shared by the tests (numpy, host side).

Shapes follow the reference tests' fixtures: `random_experts` (`test_mxfp4_fused_gemv.py:52-77`,
bytes 0..255, scales near 2**-7), `random_routing` (`:80-96`, distinct experts per token,
weights renormalised, optional zeroed tokens), and the configs' Zipf(1.1) routing.
"""

from __future__ import annotations

import numpy as np


def random_experts(experts, hidden, inter, *, seed, scale_lo=118, scale_hi=122):
    """MXFP4 payload dict in the `load_experts` layout; scales uniform in [scale_lo, scale_hi]."""
    rng = np.random.default_rng(seed)

    def payload(rows, k):
        packed = rng.integers(0, 256, (experts, rows, k // 2), dtype=np.uint8)
        scale = rng.integers(scale_lo, scale_hi + 1, (experts, rows, k // 32), dtype=np.uint8)
        return packed, scale

    gate_up, gate_up_scale = payload(2 * inter, hidden)
    down, down_scale = payload(hidden, inter)
    return {"gate_up": gate_up, "gate_up_scale": gate_up_scale, "down": down, "down_scale": down_scale}


def random_routing(tokens, experts, top_k, *, seed, zero_rows=()):
    """`(a_expert int32 [T*k], a_weight float32 [T*k])`, distinct experts per token."""
    rng = np.random.default_rng(seed)
    picks = np.stack([rng.permutation(experts)[:top_k] for _ in range(tokens)]) if tokens else np.zeros((0, top_k), int)
    w = rng.random((tokens, top_k)).astype(np.float32)
    w = w / w.sum(-1, keepdims=True) if tokens else w
    for r in zero_rows:
        w[r] = 0.0
    return picks.astype(np.int32).reshape(-1), w.astype(np.float32).reshape(-1)


def zipf_routing(tokens, experts, top_k, *, seed, s=1.1, zero_frac=0.0):
    """Top-k without replacement from a Zipf(s) popularity over `experts` (Gumbel-top-k on
    log p), weights = softmax of N(0,1) logits over the picks; a seeded `zero_frac` of
    assignments get weight exactly 0 (the early-exit path)."""
    rng = np.random.default_rng(seed)
    logp = -s * np.log(np.arange(1, experts + 1, dtype=np.float64))
    perm = rng.permutation(experts)  # which expert id is how popular
    g = rng.gumbel(size=(tokens, experts)) + logp[None, :]
    picks = perm[np.argsort(-g, axis=1)[:, :top_k]]
    z = rng.standard_normal((tokens, top_k))
    w = np.exp(z - z.max(-1, keepdims=True))
    w = (w / w.sum(-1, keepdims=True)).astype(np.float32)
    if zero_frac > 0:
        w[rng.random(w.shape) < zero_frac] = 0.0
    return picks.astype(np.int32).reshape(-1), w.reshape(-1)


def bf16_activations(tokens, hidden, *, seed):
    """N(0,1) activations rounded to bf16 values (returned as float32)."""
    from oracle.mxfp4_ref import bf16_round

    return bf16_round(np.random.default_rng(seed).standard_normal((tokens, hidden)).astype(np.float32))
