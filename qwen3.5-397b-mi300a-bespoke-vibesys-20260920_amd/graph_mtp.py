"""Captured MTP round — the reference's `graph_mtp` interface (`graph_mtp.py`), acceptance
tail.

`_accept_len`, `_commit_limit` and `_fixed_prefix_pack_index` keep the reference's tensor-op
spellings (`graph_mtp.py:440-474`): fixed shapes, no host read. `accept_round` is what the
verify step runs on a device: one launch of `mtpk_greedy_accept` that computes the commit-limited
accept length and every index the rollback and the next round need, in place of the chain of
small torch ops of `verify_round_step` (`graph_mtp.py:541-580`) and `LaneTables.update`
(`mtp_overlap.py:53-71`).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

import _mtpk
import mtp as mtp_mod


def _fixed_prefix_pack_index(lengths: torch.Tensor, width: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Fixed-size gather map packing each lane's prefix of `lengths[j]` rows (of `width`)."""
    batch = lengths.shape[0]
    cu = torch.zeros(batch + 1, dtype=torch.int32, device=lengths.device)
    cu[1:] = lengths.to(torch.int32).cumsum(0)
    dst = torch.arange(batch * width, device=lengths.device)
    lane = (dst[:, None] >= cu[1:][None, :]).sum(dim=1).clamp(max=batch - 1)
    local = (dst - torch.gather(cu, 0, lane).to(dst.dtype)).clamp(min=0, max=width - 1)
    return lane * width + local, cu


def _accept_len(draft_tokens: torch.Tensor, step_argmax: torch.Tensor) -> torch.Tensor:
    """Batched `mtp.greedy_accept_length`: the longest agreeing prefix per row."""
    matches = draft_tokens == step_argmax[:, : draft_tokens.shape[1]]
    mismatch_seen = (~matches).cumsum(dim=-1) > 0
    return (~mismatch_seen).sum(dim=-1)


def _commit_limit(accept: torch.Tensor, step_argmax: torch.Tensor, budget: torch.Tensor,
                  stops: torch.Tensor) -> torch.Tensor:
    """Batched `mtp.commit_limit`; `stops` is `[B, S]` padded with -1."""
    is_stop = (step_argmax[:, :, None] == stops[:, None, :]).any(-1)
    first_stop = (is_stop.cumsum(dim=-1) == 0).sum(dim=-1)
    limit = torch.minimum(torch.minimum(accept, first_stop), budget - 1)
    return limit.clamp(min=0)


class MTPVerifyBuffers:
    """One bucket's static tensors for the verify + accept + rollback step
    (`graph_mtp.py:141-178`): written before each replay (`token_matrix`, `pos`, `active`,
    `block_table`, `write_rows`, `slot_rows`, `budget`, `stops`), read after it
    (`step_argmax`, `accept_len` and the rollback indices below)."""

    def __init__(self, capacity: int, t: int, hidden: int, max_blocks_per_lane: int,
                 device: torch.device, dtype: torch.dtype = torch.bfloat16,
                 conv_k1: int = 3) -> None:
        self.capacity, self.t, self.conv_k1 = capacity, t, conv_k1
        long = dict(dtype=torch.long, device=device)
        self.token_matrix = torch.zeros(capacity, t, **long)
        self.pos = torch.zeros(capacity, **long)
        self.active = torch.zeros(capacity, dtype=torch.bool, device=device)
        self.block_table = torch.zeros(capacity, max_blocks_per_lane, dtype=torch.int32,
                                       device=device)
        self.block_valid = torch.zeros(capacity, dtype=torch.int32, device=device)
        self.write_rows = torch.zeros(capacity, t, **long)
        self.slot_rows = torch.zeros(capacity, **long)
        self.draft_hidden = torch.zeros(capacity, hidden, dtype=dtype, device=device)
        self.step_argmax = torch.zeros(capacity, t, **long)
        self.accept_len = torch.zeros(capacity, **long)
        self.budget = torch.full((capacity,), t, **long)
        self.stops = torch.full((capacity, mtp_mod.MAX_STOP_IDS), -1, **long)
        # rollback / next-round indices written by `accept_round`
        self.lengths = torch.ones(capacity, **long)
        self.packed_src = torch.zeros(capacity * t, **long)
        self.packed_cu = torch.zeros(capacity + 1, dtype=torch.int32, device=device)
        self.conv_idx = torch.zeros(capacity, conv_k1, **long)
        self.keep = torch.zeros(capacity, t, dtype=torch.bool, device=device)
        self.bonus = torch.zeros(capacity, **long)
        self.next_pos = torch.zeros(capacity, **long)
        self.budget_left = torch.zeros(capacity, **long)
        self.live = torch.zeros(capacity, dtype=torch.bool, device=device)
        self.hidden_src = torch.zeros(capacity, **long)


@dataclass
class AcceptResult:
    """Outputs of one acceptance pass, all `[B]`-leading device tensors."""

    accept_len: torch.Tensor
    lengths: torch.Tensor
    packed_src: torch.Tensor
    packed_cu: torch.Tensor
    conv_idx: torch.Tensor
    keep: torch.Tensor
    bonus: torch.Tensor
    next_pos: torch.Tensor
    budget_left: torch.Tensor
    live: torch.Tensor
    hidden_src: torch.Tensor


def accept_round(buf: MTPVerifyBuffers, step_argmax: torch.Tensor | None = None) -> None:
    """Commit-limited greedy acceptance and every rollback index, into `buf`, in one launch.

    `step_argmax` defaults to `buf.step_argmax` (written by the verify forward); drafts are
    `buf.token_matrix[:, 1:]`.
    """
    sa = buf.step_argmax if step_argmax is None else step_argmax
    if sa is not buf.step_argmax:
        buf.step_argmax.copy_(sa)
    greedy_accept(
        buf.step_argmax, buf.token_matrix[:, 1:], buf.active, buf.pos, buf.budget, buf.stops,
        buf.conv_k1,
        out=AcceptResult(buf.accept_len, buf.lengths, buf.packed_src, buf.packed_cu,
                         buf.conv_idx, buf.keep, buf.bonus, buf.next_pos, buf.budget_left,
                         buf.live, buf.hidden_src),
    )


def greedy_accept(step_argmax: torch.Tensor, draft: torch.Tensor, active: torch.Tensor,
                  pos: torch.Tensor, budget: torch.Tensor, stops: torch.Tensor, conv_k1: int,
                  *, out: AcceptResult | None = None) -> AcceptResult:
    """`mtpk_greedy_accept` on device tensors: step_argmax i64 [B, t], draft i64 [B, t-1] (row
    stride free, unit column stride), active bool [B], pos/budget i64 [B], stops i64 [B, S]."""
    device = _mtpk.require_device(step_argmax, draft, active, pos, budget, stops)
    b, t = step_argmax.shape
    if draft.shape != (b, t - 1) or (t > 1 and draft.stride(1) != 1) or step_argmax.stride(1) != 1:
        raise ValueError("draft must be [B, t-1] and step_argmax [B, t], unit column stride")
    for name, ten in (("step_argmax", step_argmax), ("draft", draft), ("pos", pos),
                      ("budget", budget), ("stops", stops)):
        if ten.dtype != torch.int64:
            raise ValueError(f"{name} must be int64")
    if active.dtype != torch.bool or not stops.is_contiguous():
        raise ValueError("active must be bool and stops contiguous")
    if out is None:
        long = dict(dtype=torch.long, device=device)
        out = AcceptResult(
            torch.empty(b, **long), torch.empty(b, **long), torch.empty(b * t, **long),
            torch.empty(b + 1, dtype=torch.int32, device=device),
            torch.empty(b, conv_k1, **long), torch.empty(b, t, dtype=torch.bool, device=device),
            torch.empty(b, **long), torch.empty(b, **long), torch.empty(b, **long),
            torch.empty(b, dtype=torch.bool, device=device), torch.empty(b, **long),
        )
    _mtpk.check(
        _mtpk.lib().mtpk_greedy_accept(
            step_argmax.data_ptr(), step_argmax.stride(0), draft.data_ptr(),
            draft.stride(0) if t > 1 else 0, active.contiguous().data_ptr(),
            pos.contiguous().data_ptr(), budget.contiguous().data_ptr(), stops.data_ptr(),
            stops.shape[1], b, t, conv_k1, out.accept_len.data_ptr(), out.lengths.data_ptr(),
            out.packed_src.data_ptr(), out.packed_cu.data_ptr(),
            out.conv_idx.data_ptr() if conv_k1 > 0 else None, out.keep.data_ptr(),
            out.bonus.data_ptr(), out.next_pos.data_ptr(), out.budget_left.data_ptr(),
            out.live.data_ptr(), out.hidden_src.data_ptr(), _mtpk.stream_of(device),
        ),
        "mtpk_greedy_accept",
    )  # fmt: skip
    return out


def kv_write_rows(pos: torch.Tensor, block_table: torch.Tensor, t: int, block_size: int) -> torch.Tensor:
    """Physical KV rows `block * bs + pos % bs` of a round's t positions (`graph_mtp.py:857-860`)."""
    grid = pos[:, None] + torch.arange(t, device=pos.device)[None, :]
    block_id = torch.gather(block_table.long(), 1, (grid // block_size).long())
    return block_id * block_size + grid % block_size
