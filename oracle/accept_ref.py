"""Greedy MTP acceptance, commit limit and rollback indices, restated in numpy.
TEST INFRASTRUCTURE ONLY (see oracle/__init__).

Reference functions, each restated below with its citation:
- `argmax_first`: `logits.argmax(-1)` (`graph_mtp.py:539-540`, `mtp.greedy_token`
  `mtp.py:640-658`): first index of the maximum.
- `greedy_accept_length` (`mtp.py:691-701`), `commit_limit` (`mtp.py:704-726`): host forms.
- `accept_len` (`graph_mtp.py:451-462`), `commit_limit_batched` (`graph_mtp.py:465-474`):
  batched forms.
- `fixed_prefix_pack_index` (`graph_mtp.py:440-448`).
- `round_indices`: everything the verify round derives from the accept length —
  `lengths = where(active, a + 1, 1)` (`graph_mtp.py:546-548`), the DeltaNet conv-window
  gather index (`graph_mtp.py:373-377`), the accepted-row keep mask (`graph_mtp.py:565-566`),
  the hidden-seed source row (`scatter_time_active_rows`, `mtp_dense_moe.py:322-356`,
  called at `graph_mtp.py:578-580`), the committed tokens / bonus (`graph_mtp.py:887-891`),
  the lane-table update (`mtp_overlap.py:53-71`: next token, next position, budget left,
  live), and the KV physical rows `block * bs + pos % bs` (`graph_mtp.py:857-860`,
  `block_pool.py:38` for the reserved block 0 of padding rows). With `forced_n`, the forced
  override of the wide verify (`graph_verify_wide.py:196-200`: a forced row's accept length
  is its forced count, unclamped by stops and budget) and the lane table's one-token charge
  for forced rows (`mtp_overlap.py:62-64`).

Pinning (tests/test_oracle_accept.py): the reference tests' literal vectors —
`_accept_len` -> [3, 2, 1, 0] (`test_graph_mtp.py:305-318`), `_commit_limit` -> [1, 1, 1, 0, 0]
(`test_mtp_serve.py:216-231`), `greedy_accept_length` 3/0/2 (`test_mtp.py:272-281`),
`_fixed_prefix_pack_index` three cases (`test_graph_mtp.py:321-332`) — plus scalar-vs-batched
agreement on random rows and brute-force argmax on tiny rows with planted ties. The forced
form (no reference vectors exist) is pinned by equivalence: a forced row's outputs equal an
unforced row's whose drafts agree for exactly its forced count with no stop id and an unbounded
budget, except `budget_left`, which is charged one token.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np


def argmax_first(logits: np.ndarray) -> np.ndarray:
    """Index of the first maximum along the last axis (numpy and torch agree on this)."""
    return np.asarray(logits, dtype=np.float32).argmax(-1).astype(np.int64)


def greedy_accept_length(draft_tokens: Sequence[int], step_argmax: Sequence[int]) -> int:
    """Longest prefix where `draft_tokens[i] == step_argmax[i]` (`mtp.py:691-701`)."""
    a = 0
    for d, t in zip(draft_tokens, step_argmax, strict=True):
        if d != t:
            break
        a += 1
    return a


def commit_limit(accept: int, step_argmax: Sequence[int], budget: int | None, stops) -> int:
    """`min(a, first stop index among step_argmax[:a+1], budget - 1)`, at least 0
    (`mtp.py:704-726`)."""
    limit = accept
    for s in range(accept + 1):
        if step_argmax[s] in stops:
            limit = s
            break
    if budget is not None:
        limit = min(limit, budget - 1)
    return max(limit, 0)


def accept_len(draft: np.ndarray, step_argmax: np.ndarray) -> np.ndarray:
    """Batched greedy accept length (`graph_mtp.py:451-462`)."""
    k = draft.shape[1]
    matches = draft == step_argmax[:, :k]
    mismatch_seen = np.cumsum(~matches, axis=-1) > 0
    return (~mismatch_seen).sum(-1).astype(np.int64)


def commit_limit_batched(accept, step_argmax, budget, stops) -> np.ndarray:
    """Batched commit limit (`graph_mtp.py:465-474`); `stops` padded with -1."""
    is_stop = (step_argmax[:, :, None] == stops[:, None, :]).any(-1)
    first_stop = (np.cumsum(is_stop, axis=-1) == 0).sum(-1)
    limit = np.minimum(np.minimum(accept, first_stop), budget - 1)
    return np.maximum(limit, 0).astype(np.int64)


def fixed_prefix_pack_index(lengths: np.ndarray, width: int) -> tuple[np.ndarray, np.ndarray]:
    """`(src int64 [B*width], cu int32 [B+1])` (`graph_mtp.py:440-448`)."""
    lengths = np.asarray(lengths)
    batch = lengths.shape[0]
    cu = np.zeros(batch + 1, dtype=np.int32)
    cu[1:] = np.cumsum(lengths.astype(np.int32))
    dst = np.arange(batch * width)
    lane = (dst[:, None] >= cu[1:][None, :]).sum(1)
    lane = np.minimum(lane, batch - 1)
    local = np.clip(dst - cu[lane].astype(np.int64), 0, width - 1)
    return (lane * width + local).astype(np.int64), cu


def kv_rows(pos: np.ndarray, block_table: np.ndarray, t: int, block_size: int) -> np.ndarray:
    """Physical KV rows of the round's `t` positions (`graph_mtp.py:857-860`)."""
    grid = pos[:, None] + np.arange(t)[None, :]
    block_id = np.take_along_axis(block_table.astype(np.int64), grid // block_size, axis=1)
    return block_id * block_size + grid % block_size


def round_indices(
    draft: np.ndarray,
    step_argmax: np.ndarray,
    active: np.ndarray,
    pos: np.ndarray,
    budget: np.ndarray,
    stops: np.ndarray,
    conv_k1: int,
    forced_n: np.ndarray | None = None,
) -> dict[str, np.ndarray]:
    """Every per-round output the captured verify step derives from its argmaxes.

    `draft [B, k]`, `step_argmax [B, t]` with `t = k + 1`, `active [B]` bool, `pos`/`budget`
    `[B]`, `stops [B, S]` padded with -1, `conv_k1` = conv kernel size - 1, `forced_n [B]`
    (optional) the forced draft count of each row: such a row accepts min(forced_n, k) drafts.
    """
    b, t = step_argmax.shape
    a = commit_limit_batched(accept_len(draft, step_argmax), step_argmax, budget, stops)
    forced = np.zeros(b, dtype=bool) if forced_n is None else np.asarray(forced_n) > 0
    if forced_n is not None:  # a forced row accepts min(forced, k) drafts
        a = np.where(forced, np.minimum(np.asarray(forced_n), t - 1), a).astype(np.int64)
    lengths = np.where(active, a + 1, 1).astype(np.int64)
    src, cu = fixed_prefix_pack_index(lengths, t)
    win = np.arange(conv_k1)
    conv_idx = np.minimum(lengths[:, None] + win[None, :], conv_k1 + t - 1).astype(np.int64)
    keep = active[:, None] & (np.arange(t)[None, :] <= a[:, None])
    bonus = step_argmax[np.arange(b), a]
    left = budget - np.where(forced, 1, a + 1)
    stopped = (stops == bonus[:, None]).any(1)
    return {
        "accept_len": a,
        "lengths": lengths,
        "packed_src": src,
        "packed_cu": cu,
        "conv_idx": conv_idx,
        "keep": keep,
        "bonus": bonus.astype(np.int64),
        "next_pos": (pos + a + 1).astype(np.int64),
        "budget_left": left.astype(np.int64),
        "live": (~stopped) & (left > 0),
        "hidden_src": (np.arange(b) * t + a).astype(np.int64),
    }


def committed(step_argmax: np.ndarray, accept: np.ndarray) -> list[list[int]]:
    """Committed tokens per row: `step_argmax[j, :a+1]` (`graph_mtp.py:887-891`)."""
    return [step_argmax[j, : int(accept[j]) + 1].tolist() for j in range(step_argmax.shape[0])]
