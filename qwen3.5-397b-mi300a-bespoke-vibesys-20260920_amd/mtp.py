"""MTP draft/verify/accept — the reference's `mtp` interface (`mtp.py`), acceptance half.

Host-side acceptance keeps the reference's pure functions (`greedy_accept_length`,
`commit_limit`, `mtp.py:691-726`); the device-side greedy token is the fused argmax kernel
(`mtpk_argmax_rows`), replacing `logits.float().argmax(-1, keepdim=True)` of `greedy_token`
(`mtp.py:640-658`) with a bit-identical first-occurrence argmax.
"""

from __future__ import annotations

import os
from collections.abc import Sequence

import torch

import _mtpk

MAX_STOP_IDS = 8
"""Widest per-lane stop-id set a speculative round accepts (`mtp.py:80`)."""

MTP_K_CHOICES = (1, 2, 3)
"""Draft lengths the verify buffers are sized for (`mtp.py:86-93`)."""


def _read_mtp_k() -> int:
    raw = os.environ.get("SEED_MTP_K", "3")
    try:
        k = int(raw)
    except ValueError:
        raise ValueError(f"SEED_MTP_K must be an integer in {MTP_K_CHOICES}, got {raw!r}") from None
    if k not in MTP_K_CHOICES:
        raise ValueError(f"SEED_MTP_K must be one of {MTP_K_CHOICES}, got {k}")
    return k


MTP_K = _read_mtp_k()
"""Draft tokens per round, validated at import (`mtp.py:96-111`)."""


def greedy_accept_length(draft_tokens: list[int], step_argmax: list[int]) -> int:
    """Longest prefix of `draft_tokens` equal to the target's own greedy prediction at that
    step (`step_argmax[i]` predicts `draft_tokens[i]`)."""
    a = 0
    for d, t in zip(draft_tokens, step_argmax, strict=True):
        if d != t:
            break
        a += 1
    return a


def commit_limit(accept: int, step_argmax: list[int], budget: int | None, stops: Sequence[int]) -> int:
    """`min(accept, first stop index among step_argmax[:accept+1], budget - 1)`, at least 0:
    the round commits nothing the scheduler would discard, and always at least one token."""
    limit = accept
    for s in range(accept + 1):
        if step_argmax[s] in stops:
            limit = s
            break
    if budget is not None:
        limit = min(limit, budget - 1)
    return max(limit, 0)


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """First-occurrence argmax over the last dim of a `[..., vocab]` f32/bf16 device tensor,
    int64 `[...]` (`mtpk_argmax_rows`). The last dim must have unit stride."""
    device = _mtpk.require_device(logits)
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    vocab = logits.shape[-1]
    lead = logits.shape[:-1]
    flat = logits.reshape(-1, vocab) if logits.dim() != 2 else logits
    rows = flat.shape[0]
    out = torch.empty(rows, dtype=torch.int64, device=device)
    lib = _mtpk.lib()
    partials = torch.empty(max(int(lib.mtpk_argmax_partials(rows, vocab)), 1), dtype=torch.int64,
                           device=device)
    _mtpk.check(
        lib.mtpk_argmax_rows(flat.data_ptr(), _mtpk.float_code(flat.dtype), rows, vocab,
                             flat.stride(0), partials.data_ptr(), out.data_ptr(),
                             _mtpk.stream_of(device)),
        "mtpk_argmax_rows",
    )
    return out.reshape(lead)


def greedy_token(model, normed: torch.Tensor) -> torch.Tensor:
    """`model.unembed(normed).float().argmax(-1, keepdim=True)` for `[B, hidden]` rows, `[B, 1]`
    long. On a device the argmax is the HIP kernel; the fp32 cast is not needed because the
    kernel compares bf16 logits exactly."""
    logits = model.unembed(normed)
    if logits.device.type == "cuda":
        return argmax_rows(logits)[..., None]
    return logits.float().argmax(-1, keepdim=True)
