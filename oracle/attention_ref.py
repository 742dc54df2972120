"""Causal GQA attention over a paged KV cache, restated in float64 numpy.
TEST INFRASTRUCTURE ONLY (see oracle/__init__).

Reference: `verify_attention_paged` (`model.py:1120-1205`; its torch restatement at
`model.py:1180-1205` is the spec) and the physical-row rule `block * bs + pos % bs`
(`graph_mtp.py:857-860`, `block_pool.py:38`). Query row s of lane b sits at position
`base_pos[b] + s` and attends to positions 0 .. `base_pos[b] + s`; q head h reads kv head
`h // (heads // kv_heads)`; scores are scaled by `scale` and softmax-normalised.

Pinning (tests/test_oracle_attention.py): identical keys give the mean of the visible values;
a lone visible position returns its value; a dominant key (large scale) returns that key's
value; relabelling the physical blocks (same logical rows) leaves the output unchanged; the
mask admits exactly the positions up to the row's own.
"""

from __future__ import annotations

import numpy as np


def physical_rows(table_row, n: int, block_size: int) -> np.ndarray:
    pos = np.arange(n)
    return np.asarray(table_row, np.int64)[pos // block_size] * block_size + pos % block_size


def paged_attention(q, k_pool, v_pool, block_table, base_pos, scale: float, block_size: int = 16):
    """q [B, heads, t, hd]; pools [rows, kv_heads, hd]; block_table [B, blocks]; base_pos [B].
    Returns float64 [B, heads, t, hd]."""
    q = np.asarray(q, np.float64)
    kp, vp = np.asarray(k_pool, np.float64), np.asarray(v_pool, np.float64)
    b, heads, t, hd = q.shape
    group = heads // kp.shape[1]
    out = np.zeros((b, heads, t, hd))
    for j in range(b):
        for s in range(t):
            n = int(base_pos[j]) + s + 1
            rows = physical_rows(block_table[j], n, block_size)
            for h in range(heads):
                kv = h // group
                sc = kp[rows, kv] @ q[j, h, s] * scale
                w = np.exp(sc - sc.max())
                out[j, h, s] = (w / w.sum()) @ vp[rows, kv]
    return out
