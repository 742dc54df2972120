"""Router prelude (softmax -> top-k -> renormalise) restated in numpy. TEST INFRASTRUCTURE ONLY.

Reference: `Model.moe`'s torch chain (`model.py:2840-2843`), `router_fused.route` and its
kernel (`router_fused.py:56-151`), `mtp._route` (`mtp.py:328-344`). Softmax is over the first
`experts_out` columns of a possibly wider row (the shared-expert gate rides along,
`router_fused.py:119-122`).

Selection order: descending probability; softmax is strictly increasing in the logit, so that
is descending logit, and equal logits are broken by the lower expert index (the first
occurrence, as the reference kernel's `tl.argmax` does, `router_fused.py:82-84`). Weights are
computed in float64 and returned as float32.

Pinning (tests/test_oracle_router.py): brute force over every k-subset on tiny rows (the
selected set maximises the summed probability, weights are p_i / sum p_sel), exact-tie cases
(lowest index wins), weights sum to 1, and invariance to a constant shift of the logits.
"""

from __future__ import annotations

import numpy as np


def route(logits: np.ndarray, experts_out: int, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    """`(top_w float32 [t, k], top_i int64 [t, k])`, highest weight first."""
    z = np.asarray(logits, dtype=np.float64)[:, :experts_out]
    t = z.shape[0]
    # lexsort: last key is primary. Primary -logit (descending), secondary index (ascending).
    idx = np.arange(experts_out)
    top_i = np.empty((t, top_k), dtype=np.int64)
    top_w = np.empty((t, top_k), dtype=np.float32)
    for r in range(t):
        order = np.lexsort((idx, -z[r]))[:top_k]
        m = z[r].max()
        e = np.exp(z[r] - m)
        p = e / e.sum()
        sel = p[order]
        top_i[r] = order
        top_w[r] = (sel / sel.sum()).astype(np.float32)
    return top_w, top_i


def flatten(top_w: np.ndarray, top_i: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """`(a_expert int32 [t*k], a_weight float32 [t*k])`, `a = t*k + j`
    (`model.py:3096-3100`)."""
    return top_i.reshape(-1).astype(np.int32), top_w.reshape(-1).astype(np.float32)
