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

from collections.abc import Callable
from dataclasses import dataclass

import torch

import _mtpk
import blas_tune
import rownorm
import mtp as mtp_mod
import verify_model as vm


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


STAGE_TOKEN, STAGE_POS, STAGE_BUDGET, STAGE_SLOT, STAGE_FORCED, STAGE_ACTIVE, STAGE_IDS = range(7)
"""Columns of `MTPVerifyBuffers.staging`: token, position, budget, slot, forced count, active,
then the forced ids (k columns) and the stop ids (`MAX_STOP_IDS` columns, -1 padded)."""


class MTPVerifyBuffers:
    """One bucket's static tensors for the draft + verify + accept + rollback step
    (`graph_mtp.py:141-178`, same constructor): written before each replay (`token_matrix`,
    `pos`, `active`, `block_table`, `write_rows`, `slot_rows`, `budget`, `stops`, `forced_n`,
    `forced_ids`), read after it (`step_argmax`, `accept_len` and the rollback indices below).
    Row `j` is the round's `j`-th lane, `slot_rows[j]` its slot. The sizes come from `model`:
    its hidden width, dtype, block-table width and DeltaNet conv window."""

    def __init__(self, model, capacity: int, t: int, device: torch.device) -> None:
        hidden, dtype = model.cfg.hidden, model.dtype
        max_blocks_per_lane = model.blocks.max_blocks
        conv_k1 = model.cfg.conv_k - 1
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
        self.draft_seed = torch.zeros(capacity, hidden, dtype=dtype, device=device)  # its final norm
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
        # forced feed: row j's first forced_n[j] drafts are forced_ids[j] and are accepted
        # unconditionally (zero on every other row)
        self.forced_n = torch.zeros(capacity, **long)
        self.forced_ids = torch.zeros(capacity, max(t - 1, 1), **long)
        # index tables the fill derives for the steps: row j's positions pos + s, row major and
        # step major (draft step s reads row s), and the commit's slot (-1 on padding rows)
        self.pos_grid = torch.zeros(capacity, t, **long)
        self.pos_steps = torch.zeros(t, capacity, **long)
        self.commit_slots = torch.full((capacity,), -1, **long)
        # a round's host inputs, one row per buffer row (`STAGE_*` columns): written on the
        # host (pinned on a device), copied once, unpacked into the fields above on the device
        cols = STAGE_IDS + max(t - 1, 1) + mtp_mod.MAX_STOP_IDS
        self.staging = torch.zeros(capacity, cols, **long)
        pin = torch.device(device).type == "cuda"
        self.staging_host = torch.zeros(capacity, cols, dtype=torch.long, pin_memory=pin)
        # recorded after each staging copy (device buffers): the next round's host writes wait
        # for it before reusing the pinned rows
        self.staged = torch.cuda.Event() if pin else None


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


KEY_ROWS = 4096
"""Verify rows (B * t) up to which `greedy_accept(..., keys=)` takes the argmax keys."""


def greedy_accept(step_argmax: torch.Tensor, draft: torch.Tensor, active: torch.Tensor,
                  pos: torch.Tensor, budget: torch.Tensor, stops: torch.Tensor, conv_k1: int,
                  *, out: AcceptResult | None = None,
                  keys: tuple[torch.Tensor, int] | None = None,
                  forced_n: torch.Tensor | None = None) -> AcceptResult:
    """`mtpk_greedy_accept` on device tensors: step_argmax i64 [B, t], draft i64 [B, t-1] (row
    stride free, unit column stride), active bool [B], pos/budget i64 [B], stops i64 [B, S].
    With `keys` (`mtp.argmax_keys` of the [B * t, vocab] verify logits) the same launch first
    finishes the argmax and writes it into `step_argmax` (`mtpk_greedy_accept_keys`). With
    `forced_n` i64 [B], rows with `forced_n > 0` accept exactly their forced drafts (no stop or
    budget clamp, one token charged to the budget), and every output follows from that."""
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
    if keys is not None:
        key_t, chunks = keys
        if key_t.shape != (b * t, chunks) or not key_t.is_contiguous():
            raise ValueError(f"keys must be contiguous [{b * t}, {chunks}]")
    if forced_n is not None and (forced_n.shape != (b,) or forced_n.dtype != torch.int64
                                 or not forced_n.is_contiguous()):
        raise ValueError(f"forced_n must be a contiguous int64 [{b}] tensor")
    _mtpk.check(
        (_mtpk.lib().mtpk_greedy_accept_keys if keys is not None else _mtpk.lib().mtpk_greedy_accept)(
            *((keys[0].data_ptr(), keys[1]) if keys is not None else ()),
            step_argmax.data_ptr(), step_argmax.stride(0), draft.data_ptr(),
            draft.stride(0) if t > 1 else 0, active.contiguous().data_ptr(),
            pos.contiguous().data_ptr(), budget.contiguous().data_ptr(), stops.data_ptr(),
            stops.shape[1], _mtpk.ptr(forced_n), b, t, conv_k1, out.accept_len.data_ptr(), out.lengths.data_ptr(),
            out.packed_src.data_ptr(), out.packed_cu.data_ptr(),
            out.conv_idx.data_ptr() if conv_k1 > 0 else None, out.keep.data_ptr(),
            out.bonus.data_ptr(), out.next_pos.data_ptr(), out.budget_left.data_ptr(),
            out.live.data_ptr(), out.hidden_src.data_ptr(), _mtpk.stream_of(device),
        ),
        "mtpk_greedy_accept_keys" if keys is not None else "mtpk_greedy_accept",
    )  # fmt: skip
    return out


def kv_write_rows(pos: torch.Tensor, block_table: torch.Tensor, t: int, block_size: int) -> torch.Tensor:
    """Physical KV rows `block * bs + pos % bs` of a round's t positions (`graph_mtp.py:857-860`)."""
    grid = pos[:, None] + torch.arange(t, device=pos.device)[None, :]
    return vm.table_rows(block_table, grid, block_size)


RESERVED_BLOCK = 0
"""The block id padding rows' tables hold: never handed to a lane (`block_pool.py:38`)."""


def accept_torch(step_argmax: torch.Tensor, draft: torch.Tensor, active: torch.Tensor,
                 pos: torch.Tensor, budget: torch.Tensor, stops: torch.Tensor, conv_k1: int,
                 forced_n: torch.Tensor | None, out: AcceptResult) -> None:
    """What `greedy_accept` computes, in the reference's tensor ops, for CPU tensors (the CPU
    engine's verify tail, `graph_mtp.py:541-580`, `graph_verify_wide.py:196-200`,
    `mtp_overlap.py:53-71`); device tensors take the HIP kernel."""
    b, t = step_argmax.shape
    a = _commit_limit(_accept_len(draft, step_argmax), step_argmax, budget, stops)
    forced = torch.zeros_like(active) if forced_n is None else forced_n > 0
    if forced_n is not None:
        a = torch.where(forced, forced_n.clamp(max=t - 1), a)
    lengths = torch.where(active, a + 1, torch.ones_like(a))
    src, cu = _fixed_prefix_pack_index(lengths, t)
    win = torch.arange(conv_k1, device=a.device)
    rows = torch.arange(b, device=a.device)
    bonus = step_argmax[rows, a]
    left = budget - torch.where(forced, torch.ones_like(a), a + 1)
    stopped = (stops == bonus[:, None]).any(-1)
    for dst, val in ((out.accept_len, a), (out.lengths, lengths), (out.packed_src, src),
                     (out.packed_cu, cu), (out.conv_idx, (lengths[:, None] + win).clamp(max=conv_k1 + t - 1)),
                     (out.keep, active[:, None] & (torch.arange(t, device=a.device)[None, :] <= a[:, None])),
                     (out.bonus, bonus), (out.next_pos, pos + a + 1), (out.budget_left, left),
                     (out.live, ~stopped & (left > 0)), (out.hidden_src, rows * t + a)):
        dst.copy_(val)


# ---------------------------------------------------------------- the device round


def _draft_rows(model, m, buf: MTPVerifyBuffers) -> None:
    """`m.k` MTP draft steps over every row of `buf`, drafts written into
    `buf.token_matrix[:, 1:]` (`draft_round_step`, `graph_mtp.py:477-504`): seeded from the
    fill-time copy `buf.draft_hidden`, reading the MTP cache through `buf.block_table`. A row
    with `forced_n[j] > 0` feeds (and keeps) its forced tokens instead of its first drafts.
    Padding rows (`active` False) write no MTP cache row. No host read."""
    if buf.draft_hidden.is_cuda:  # the seed kept in the buffer: the verify's MTP cache rows reuse it
        hid = rownorm.rmsnorm(buf.draft_hidden, model.final_norm, model.cfg.eps, out=buf.draft_seed)
    else:
        hid = mtp_mod.draft_seed(model, buf.draft_hidden)
    tok = buf.token_matrix[:, :1]
    on_device = vm.kv_write_in_kernel(model)
    for s in range(m.k):
        rows = None if on_device else buf.write_rows[:, s]
        # the fed token's positions: row s of the fill's step-major table (pos + s)
        hid, tok = mtp_mod.draft_step(model, m, hid, tok, buf.pos_steps[s], rows, buf.block_table,
                                      buf.block_valid, buf.active)
        if tok.is_cuda:  # forced override and the column write in one launch
            draft_feed(tok[:, 0], buf.forced_n, buf.forced_ids[:, s], s, buf.token_matrix[:, s + 1])
        else:
            tok = torch.where((buf.forced_n > s)[:, None], buf.forced_ids[:, s : s + 1], tok)
            buf.token_matrix[:, s + 1] = tok[:, 0]
        tok = buf.token_matrix[:, s + 1 : s + 2]


def draft_feed(tok: torch.Tensor, forced_n: torch.Tensor, forced: torch.Tensor, step: int,
               out: torch.Tensor) -> None:
    """`out[j] = forced[j] if forced_n[j] > step else tok[j]` on device int64 `[B]` vectors (any
    strides): `mtpk_draft_feed`."""
    device = _mtpk.require_device(tok, forced_n, forced, out)
    b = out.shape[0]
    for name, ten in (("tok", tok), ("forced_n", forced_n), ("forced", forced), ("out", out)):
        if ten.dtype != torch.int64 or ten.shape != (b,):
            raise ValueError(f"{name} must be int64 [{b}]")
    _mtpk.check(_mtpk.lib().mtpk_draft_feed(
        tok.data_ptr(), tok.stride(0), forced_n.contiguous().data_ptr(), forced.data_ptr(),
        forced.stride(0), step, out.data_ptr(), out.stride(0), b, _mtpk.stream_of(device)),
        "mtpk_draft_feed")  # fmt: skip


def _verify_rows(model, m, buf: MTPVerifyBuffers, ctx_len: int) -> None:
    """Verify forward over every row of `buf.token_matrix`, argmax, acceptance with every
    rollback index (`mtpk_greedy_accept`, forced rows accepting their forced drafts), then the
    commit of DeltaNet state, MTP cache rows and the hidden seed to each row's accepted length
    (`verify_round_step`, `graph_mtp.py:513-582`). Reads `buf.block_table` and
    `buf.draft_hidden`; padding rows (`active` False) touch no lane state: no K/V row, no
    DeltaNet commit, no MTP cache row, no hidden seed. No host read."""
    t, b = buf.t, buf.capacity
    dev = buf.pos.device
    pos, slots, active = buf.pos, buf.slot_rows, buf.active
    res = model.forward_rows(buf.token_matrix, slots, pos, ctx_len, block_table=buf.block_table,
                             active=active, positions=buf.pos_grid, final_norm=True)
    normed = res.normed.reshape(b * t, -1)
    out = AcceptResult(buf.accept_len, buf.lengths, buf.packed_src, buf.packed_cu, buf.conv_idx,
                       buf.keep, buf.bonus, buf.next_pos, buf.budget_left, buf.live, buf.hidden_src)
    draft = buf.token_matrix[:, 1:]
    if dev.type == "cuda":
        keys = None
        if model.fused_argmax(b * t, normed):  # the LM head GEMM with the argmax in its epilogue
            model.next_tokens(normed, out=buf.step_argmax.view(-1))
        elif b * t <= KEY_ROWS:  # the accept launch finishes the argmax
            keys = mtp_mod.argmax_keys(model.unembed(normed))
        else:
            buf.step_argmax.copy_(model.argmax(model.unembed(normed)).view(b, t))
        greedy_accept(buf.step_argmax, draft, active, pos, buf.budget, buf.stops, buf.conv_k1,
                      out=out, keys=keys, forced_n=buf.forced_n)
    else:
        buf.step_argmax.copy_(model.argmax(model.unembed(normed)).view(b, t))
        accept_torch(buf.step_argmax, draft, active, pos, buf.budget, buf.stops, buf.conv_k1,
                     buf.forced_n, out)
    if dev.type == "cuda":  # the fill's commit slots: -1 on padding rows, which commit nothing
        model.commit(res, buf.commit_slots, out.lengths, conv_idx=out.conv_idx)
    else:
        model.commit(res, slots, out.lengths, conv_idx=out.conv_idx, active=active)
    grid = buf.pos_grid
    if dev.type == "cuda":
        # the final-normed previous rows: the draft's seed, then the forward's own normed rows
        # (the same kernel over the same values as `draft_seed` of the raw rows)
        previous = torch.cat([buf.draft_seed[:, None], res.normed[:, :-1]], dim=1)
        seeded = True
    else:
        previous = torch.cat([buf.draft_hidden[:, None], res.hidden[:, :-1]], dim=1)
        seeded = False
    if vm.kv_write_in_kernel(model):
        mtp_mod.cache_target_rows(model, m, buf.token_matrix, previous, grid, None, out.keep,
                                  block_table=buf.block_table, base_pos=pos, seeded=seeded)
    else:
        mtp_mod.cache_target_rows(model, m, buf.token_matrix, previous, grid, buf.write_rows, out.keep,
                                  seeded=seeded)
    if dev.type == "cuda":  # one launch: slot commit_slots[j] <- verify row hidden_src[j]
        copy_rows(res.hidden.reshape(b * t, -1), out.hidden_src, model.hidden_cache, buf.commit_slots)
    else:
        seed = res.hidden.reshape(b * t, -1)[out.hidden_src]
        # padding rows name an idle lane and write back its own seed: no row of the round writes it
        model.hidden_cache[slots] = torch.where(active[:, None], seed, model.hidden_cache[slots])


def copy_rows(src: torch.Tensor, src_idx: torch.Tensor, dst: torch.Tensor, dst_idx: torch.Tensor) -> None:
    """`dst[dst_idx[j]] = src[src_idx[j]]` on device 2-D tensors of one dtype and row width (rows
    at any stride), skipping every j whose index lies outside its table: `mtpk_copy_rows`."""
    device = _mtpk.require_device(src, src_idx, dst, dst_idx)
    n = src_idx.shape[0]
    if (src.dim() != 2 or dst.dim() != 2 or src.dtype != dst.dtype or src.shape[1] != dst.shape[1]
            or src.stride(1) != 1 or dst.stride(1) != 1):
        raise ValueError("src and dst must be 2-D of one dtype and width, rows contiguous")
    if src_idx.shape != (n,) or dst_idx.shape != (n,) or src_idx.dtype != torch.int64 \
            or dst_idx.dtype != torch.int64:
        raise ValueError("src_idx and dst_idx must be int64 vectors of one length")
    es = src.element_size()
    _mtpk.check(_mtpk.lib().mtpk_copy_rows(
        src.data_ptr(), src.shape[0], src.stride(0) * es, src_idx.contiguous().data_ptr(),
        dst.data_ptr(), dst.shape[0], dst.stride(0) * es, dst_idx.contiguous().data_ptr(), n,
        src.shape[1] * es, _mtpk.stream_of(device)), "mtpk_copy_rows")  # fmt: skip


def _ctx_bound(model) -> int:
    """Context length every captured round is sized for: the block tables' full capacity, so
    the attention's key splits do not depend on a round's positions."""
    return model.blocks.max_blocks * model.cfg.block_size


def draft_round_step(model, mtp, buf: MTPVerifyBuffers, t: int) -> Callable[[], None]:
    """The draft step to capture (`graph_mtp.py:477-504`, same arguments): `t - 1` MTP steps
    over every row of `buf`, seeded from `draft_hidden` and the base token
    (`token_matrix[:, 0]`), each step's greedy token written into `token_matrix[:, 1 + step]`;
    rows with `forced_n > 0` feed and keep `forced_ids` instead."""
    if t != buf.t or t != mtp.k + 1:
        raise ValueError(f"t={t} does not match the buffers ({buf.t}) and the MTP head (k={mtp.k})")

    def step() -> None:
        _draft_rows(model, mtp, buf)

    return step


build_draft_step = draft_round_step
"""The reference's alias for the draft entry point (`graph_mtp.py:507-510`)."""


def verify_round_step(model, mtp, buf: MTPVerifyBuffers, t: int) -> Callable[[], None]:
    """The verify step to capture (`graph_mtp.py:513-582`, same arguments): one forward over
    every row of `buf`, the argmax, commit-limited acceptance with every rollback index, and the
    commit of DeltaNet state, MTP cache rows and the hidden seed to each active row's accepted
    length."""
    if t != buf.t:
        raise ValueError(f"t={t} does not match the buffers ({buf.t})")
    ctx = _ctx_bound(model)

    def step() -> None:
        _verify_rows(model, mtp, buf, ctx)

    return step


def pad_slot_for(slots, lanes: int) -> int:
    """The lane padding rows name (`graph_decode.pad_slot_for`'s role): the lowest lane not in
    this round, so no real row of the round writes it and padding reads only idle state."""
    taken = set(int(s) for s in slots)
    for lane in range(lanes):
        if lane not in taken:
            return lane
    raise ValueError("a padded round needs a lane outside the round")


def _stage(model, buf: MTPVerifyBuffers, slots, tokens, positions, budgets, stops, forced) -> None:
    """The host half of `_fill`: checks, the lanes' KV blocks grown for t more positions, and
    the round's rows written into `buf.staging_host` and copied to `buf.staging` (one copy).
    The device waits while this runs, so the common round (no forced drafts, no stop ids, no
    lane growing a block) takes builtin checks over the lists and one numpy write per column."""
    n, t, k = len(slots), buf.t, buf.t - 1
    lanes = model.lanes
    sl = [int(x) for x in slots]
    if not 1 <= n <= buf.capacity or len(set(sl)) != n:
        raise ValueError(f"need 1..{buf.capacity} distinct slots, got {slots}")
    if min(sl) < 0 or max(sl) >= lanes:
        raise ValueError(f"slots must lie in [0, {lanes}), got {slots}")
    for name, seq in (("tokens", tokens), ("positions", positions), ("budgets", budgets),
                      ("stops", stops), ("forced", forced)):
        if seq is not None and len(seq) != n:
            raise ValueError(f"{name} has {len(seq)} entries for {n} slots")
    if stops is not None and any(len(s) > mtp_mod.MAX_STOP_IDS for s in stops):
        raise ValueError(f"at most {mtp_mod.MAX_STOP_IDS} stop ids per lane")
    vocab = model.cfg.vocab
    if min(tokens) < 0 or max(tokens) >= vocab or (
            forced and any(not 0 <= int(x) < vocab for ids in forced for x in list(ids)[:k])):
        raise ValueError(f"token ids must lie in [0, {vocab})")
    model.blocks.grow_many(sl, [p + t for p in positions])
    if buf.staged is not None:
        buf.staged.synchronize()  # the previous round's copy has left the pinned rows
    h = buf.staging_host.numpy()
    width = max(k, 1)
    h[:, STAGE_IDS : STAGE_IDS + width] = 0
    h[:, STAGE_IDS + width :] = -1
    h[:n, STAGE_TOKEN] = tokens
    h[:n, STAGE_POS] = positions
    h[:n, STAGE_BUDGET] = 1 << 40 if budgets is None else budgets
    h[:n, STAGE_SLOT] = sl
    h[:n, STAGE_ACTIVE] = 1
    h[:n, STAGE_FORCED] = 0
    if forced or stops:
        for j in range(n):
            if forced:
                ids = list(forced[j])[:k]
                h[j, STAGE_FORCED] = len(ids)
                h[j, STAGE_IDS : STAGE_IDS + len(ids)] = ids
            if stops and len(stops[j]):
                h[j, STAGE_IDS + width : STAGE_IDS + width + len(stops[j])] = list(stops[j])
    # padding rows: inactive, position 0, budget t, an idle lane as slot, no stop ids
    if n < buf.capacity:
        h[n:, STAGE_TOKEN] = 0
        h[n:, STAGE_POS] = 0
        h[n:, STAGE_BUDGET] = t
        h[n:, STAGE_SLOT] = pad_slot_for(sl, lanes)
        h[n:, STAGE_FORCED] = 0
        h[n:, STAGE_ACTIVE] = 0
    buf.staging.copy_(buf.staging_host, non_blocking=True)
    if buf.staged is not None:
        buf.staged.record()


def _unpack(model, buf: MTPVerifyBuffers) -> None:
    """The device half of `_fill`: `buf.staging` into the round's fields, and the fill-owned
    `block_table` (the reserved block on padding rows), `block_valid`, `write_rows` and
    `draft_hidden` from the model's tables. On a device this is one launch of
    `mtpk_round_fill`; CPU buffers take the same steps as tensor ops."""
    if buf.staging.is_cuda:
        round_fill(model, buf)
        return
    t, k = buf.t, buf.t - 1
    width = max(k, 1)
    st = buf.staging
    buf.token_matrix.zero_()
    buf.token_matrix[:, 0] = st[:, STAGE_TOKEN]
    buf.pos.copy_(st[:, STAGE_POS])
    buf.budget.copy_(st[:, STAGE_BUDGET])
    buf.slot_rows.copy_(st[:, STAGE_SLOT])
    buf.forced_n.copy_(st[:, STAGE_FORCED])
    buf.active.copy_(st[:, STAGE_ACTIVE] != 0)
    buf.forced_ids.copy_(st[:, STAGE_IDS : STAGE_IDS + width])
    buf.stops.copy_(st[:, STAGE_IDS + width :])
    bs = model.cfg.block_size
    buf.block_table.copy_(torch.where(buf.active[:, None], model.blocks.table[buf.slot_rows],
                                      torch.full_like(buf.block_table, RESERVED_BLOCK)))
    buf.block_valid.copy_(((buf.pos + t + bs - 1) // bs).to(torch.int32))
    buf.write_rows.copy_(kv_write_rows(buf.pos, buf.block_table, t, bs))
    buf.draft_hidden.copy_(model.hidden_cache[buf.slot_rows])
    buf.pos_grid.copy_(buf.pos[:, None] + torch.arange(t, device=buf.pos.device)[None, :])
    buf.pos_steps.copy_(buf.pos_grid.t())
    buf.commit_slots.copy_(torch.where(buf.active, buf.slot_rows, torch.full_like(buf.slot_rows, -1)))


def round_fill(model, buf: MTPVerifyBuffers) -> None:
    """`mtpk_round_fill` on device buffers: what `_unpack` computes, in one launch."""
    table, hidden = model.blocks.table, model.hidden_cache
    fields = (buf.staging, table, hidden, buf.token_matrix, buf.pos, buf.budget, buf.slot_rows,
              buf.forced_n, buf.active, buf.forced_ids, buf.stops, buf.block_table,
              buf.block_valid, buf.write_rows, buf.draft_hidden, buf.pos_grid, buf.pos_steps,
              buf.commit_slots)
    device = _mtpk.require_device(*fields)
    if not all(f.is_contiguous() for f in fields):
        raise ValueError("round fill needs contiguous buffers and model tables")
    rows, t = buf.token_matrix.shape
    lanes, max_blocks = table.shape
    if (table.dtype != torch.int32 or buf.block_table.shape != (rows, max_blocks)
            or hidden.dtype != buf.draft_hidden.dtype or hidden.shape[1:] != buf.draft_hidden.shape[1:]
            or hidden.shape[0] != lanes):
        raise ValueError("model tables do not match the round buffers")
    if (buf.pos_grid.shape != (rows, t) or buf.pos_steps.shape != (t, rows)
            or buf.commit_slots.shape != (rows,)):
        raise ValueError("the round's index tables do not match its token matrix")
    n_stops = buf.stops.shape[1]
    if buf.staging.shape != (rows, STAGE_IDS + max(t - 1, 1) + n_stops):
        raise ValueError(f"staging must be [{rows}, {STAGE_IDS + max(t - 1, 1) + n_stops}]")
    _mtpk.check(
        _mtpk.lib().mtpk_round_fill(
            buf.staging.data_ptr(), rows, t, n_stops, table.data_ptr(), lanes, max_blocks,
            model.cfg.block_size, RESERVED_BLOCK, hidden.data_ptr(),
            hidden[0].numel() * hidden.element_size(), buf.token_matrix.data_ptr(),
            buf.pos.data_ptr(), buf.budget.data_ptr(), buf.slot_rows.data_ptr(),
            buf.forced_n.data_ptr(), buf.active.data_ptr(), buf.forced_ids.data_ptr(),
            buf.stops.data_ptr(), buf.block_table.data_ptr(), buf.block_valid.data_ptr(),
            buf.write_rows.data_ptr(), buf.draft_hidden.data_ptr(), buf.pos_grid.data_ptr(),
            buf.pos_steps.data_ptr(), buf.commit_slots.data_ptr(), _mtpk.stream_of(device),
        ),
        "mtpk_round_fill",
    )


def _fill(model, mtp, buf: MTPVerifyBuffers, slots, tokens, positions, budgets, stops, forced) -> None:
    """Write one round's inputs into `buf`, padding to `buf.capacity` rows
    (`MTPVerifyRunner.fill`, `graph_mtp.py:795-874`; `MTP_INTERFACE.md:17-33`). Row `j < n` is the
    round's `j`-th lane; rows `>= n` are padding: `active` False, position 0, an idle lane as
    slot, no stop ids, budget `t`, and the reserved block in every block-table entry. Also
    writes the fill-owned `block_table`, `block_valid`, `write_rows` and `draft_hidden`."""
    _stage(model, buf, slots, tokens, positions, budgets, stops, forced)
    _unpack(model, buf)


def _committed(buf: MTPVerifyBuffers, n: int | None = None) -> list[list[int]]:
    """The first `n` rows' committed ids, `step_argmax[j, : accept + 1]`: one host read."""
    n = buf.capacity if n is None else n
    rows = torch.cat([buf.step_argmax[:n], buf.accept_len[:n, None]], dim=1).tolist()
    return [row[: row[-1] + 1] for row in rows]


def build_buckets(capacity: int) -> list[int]:
    """Round capacities a runner keeps buffers (and graphs) for: powers of two below
    `capacity`, then `capacity` (the role of `graph_decode.build_buckets`)."""
    out, b = [], 1
    while b < capacity:
        out.append(b)
        b *= 2
    return out + [capacity]


class MTPVerifyRunner:
    """Eager speculative rounds over static per-bucket buffers (`graph_mtp.MTPVerifyRunner`,
    `graph_mtp.py:622-976`): fill (padding the round to the smallest bucket that holds it),
    draft, verify + accept + commit, one host read. `capacity` (default, and at most: every lane
    of the model) bounds the batch size; `buckets` (default `build_buckets(capacity)`) are the
    round sizes buffers are kept for."""

    def __init__(self, model, mtp=None, capacity: int | None = None,
                 buckets: list[int] | None = None) -> None:
        mtp = model.mtp if mtp is None else mtp
        if mtp is None:
            raise ValueError("model has no MTP layer")
        self.model, self.mtp = model, mtp
        self.t = mtp.k + 1
        self.capacity = model.lanes if capacity is None else min(capacity, model.lanes)
        if self.capacity < 1:
            raise ValueError(f"capacity {capacity} leaves no lane")
        self.buckets = sorted(set(buckets)) if buckets else build_buckets(self.capacity)
        if self.buckets[0] < 1 or self.buckets[-1] > model.lanes:
            raise ValueError(f"buckets {self.buckets} must lie in 1..{model.lanes}")
        self.capacity = self.buckets[-1]
        self.bufs: dict[int, MTPVerifyBuffers] = {}

    def bucket_for(self, n: int) -> int:
        """The smallest bucket holding `n` rows (`graph_decode.bucket_for`)."""
        for b in self.buckets:
            if b >= n:
                return b
        raise ValueError(f"batch of {n} lanes: this runner takes 1..{self.capacity}")

    def buffers(self, n: int) -> MTPVerifyBuffers:
        """The buffers of the bucket serving an `n`-lane round."""
        if n < 1:
            raise ValueError("a round needs at least one lane")
        b = self.bucket_for(n)
        if b not in self.bufs:
            self.bufs[b] = MTPVerifyBuffers(self.model, b, self.t, self.model.device)
        return self.bufs[b]

    def fill(self, buf: MTPVerifyBuffers, slots, tokens, positions, budgets=None, stops=None,
             forced=None) -> None:
        _fill(self.model, self.mtp, buf, slots, tokens, positions, budgets, stops, forced)

    def _round(self, buf: MTPVerifyBuffers) -> None:
        draft_round_step(self.model, self.mtp, buf, self.t)()
        verify_round_step(self.model, self.mtp, buf, self.t)()

    def speculative_decode(self, slots: list[int], tokens: list[int], positions: list[int],
                           budgets=None, stops=None, forced=None) -> list[list[int]]:
        """Each slot's committed ids for one round (`Model.speculative_decode`'s contract);
        `forced` rows commit their forced drafts plus one target token."""
        buf = self.buffers(len(slots))
        self.fill(buf, slots, tokens, positions, budgets, stops, forced)
        self._round(buf)
        return _committed(buf, len(slots))


class CudaGraphBackend:
    """Captures a step as one HIP graph (`torch.cuda.CUDAGraph`) and returns its replay."""

    def capture(self, fn: Callable[[], None], device: torch.device) -> Callable[[], None]:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        return graph.replay


class EagerBackend:
    """Runs the step itself at every replay: the capture-free backend the reference's tests
    use (`EagerBackend`), which lets the runner's bucketing and validation run on the CPU."""

    def capture(self, fn: Callable[[], None], device: torch.device) -> Callable[[], None]:
        return fn


REQUIRE_GRAPH_ENV = "SEED_MTP_REQUIRE_GRAPH"
"""`=1`: a bucket that fails capture or validation raises instead of serving eager rounds
(`graph_mtp.py:112-116`)."""


class GraphMTPRunner(MTPVerifyRunner):
    """`MTPVerifyRunner` with each bucket's draft and verify steps captured as one graph
    (`GraphMTPRunner(model, backend=None)`, `graph_mtp.py:1062-1120`). A round pads to its
    bucket, writes the bucket's static buffers, replays its graph and reads the committed ids
    once; forced feed rides in the buffers, so forced rounds replay the same graph.

    `prepare()` (boot) captures every bucket and validates each capture against the eager step
    on a synthetic round (`graph_mtp.py:712-769`, `:978-1059`); a bucket that fails disables
    the captured round, and rounds then run eagerly, or, under `SEED_MTP_REQUIRE_GRAPH=1`,
    `prepare()` raises. Without `prepare()`, a bucket is captured on its first round (which
    runs eagerly) and is not validated. `backend` is the capture backend: None for HIP graphs,
    or `EagerBackend()`. `tune_blas` (None: `MTPK_BLAS_TUNE=1` in the environment) runs each
    bucket's eager round before its capture inside a `blas_tune.session`, so the round's library
    GEMMs are captured with their tuned solutions (the reference's startup tuning,
    `blas_tune.py:178-255`); it applies on a ROCm GPU only."""

    def __init__(self, model, backend=None, *, capacity: int | None = None,
                 buckets: list[int] | None = None, tune_blas: bool | None = None) -> None:
        import os

        super().__init__(model, None, capacity, buckets)
        if tune_blas is None:
            tune_blas = os.environ.get("MTPK_BLAS_TUNE", "0") == "1"
        self.tune_blas = bool(tune_blas)
        self.backend = CudaGraphBackend() if backend is None else backend
        self.graphs: dict[int, Callable[[], None]] = {}
        self.enabled = True
        self.validated: dict[int, bool] = {}
        self.eager_rounds = 0

    def forced_drafts(self) -> bool:
        """Whether rounds may carry forced feed (`graph_mtp.py:1116-1118`): always."""
        return True

    def _capture(self, buf: MTPVerifyBuffers) -> Callable[[], None]:
        """The bucket's round as one graph: the fill's device half (`_unpack`, reading the
        staged rows) and then draft + verify + accept + commit, so a round is one staging copy
        and one replay. Replaying after `fill()` unpacks the same staged rows again."""

        def step() -> None:
            _unpack(self.model, buf)
            self._round(buf)

        return self.backend.capture(step, buf.pos.device)

    def _eager_round(self, buf: MTPVerifyBuffers) -> None:
        """The bucket's round run eagerly before its capture, on a side stream on a device (so
        every lazy allocation and library handle exists before capture begins), and with
        `tune_blas` inside a tuning session (so every library GEMM shape is searched first)."""
        dev = buf.pos.device
        if dev.type != "cuda":
            self._round(buf)
            return
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            if self.tune_blas and blas_tune.available():
                with blas_tune.session(dev):
                    self._round(buf)
            else:
                self._round(buf)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize(dev)

    def _reset_lanes(self) -> None:
        for lane in range(self.model.lanes):
            self.model.reset(lane)

    def _validate(self, bucket: int, buf: MTPVerifyBuffers, replay: Callable[[], None]) -> bool:
        """One synthetic round on `bucket` fresh lanes, eager and replayed from the same state:
        committed ids and every lane's resulting state must agree bit for bit. Positions past
        the first KV block, budgets and a stop id that clamp some rows mid-accept."""
        model, t = self.model, self.t
        vocab, bs = model.cfg.vocab, model.cfg.block_size
        slots = list(range(bucket))
        tokens = [(7 * i + 3) % vocab for i in range(bucket)]
        positions = [bs + 1 + i % 3 for i in range(bucket)]
        budgets = [1 + i % t for i in range(bucket)]
        stops = [[(5 * i) % vocab] for i in range(bucket)]
        self._reset_lanes()
        grid = torch.arange(model.hidden_cache.numel(), device=model.device)
        model.hidden_cache.copy_((grid.reshape(model.hidden_cache.shape) * 0.37).sin().to(model.hidden_cache.dtype))
        before = [{k: v.clone() for k, v in p.items() if k in ("conv", "rec")} for p in model.pool]
        seed = model.hidden_cache.clone()
        self.fill(buf, slots, tokens, positions, budgets, stops)
        self._round(buf)
        want = _committed(buf, bucket)
        want_state = ([{k: v.clone() for k, v in p.items() if k in ("conv", "rec")} for p in model.pool],
                      model.hidden_cache.clone())
        for p, snap in zip(model.pool, before, strict=True):
            for k, v in snap.items():
                p[k].copy_(v)
        model.hidden_cache.copy_(seed)
        self.fill(buf, slots, tokens, positions, budgets, stops)
        replay()
        got = _committed(buf, bucket)
        ok = got == want and torch.equal(model.hidden_cache, want_state[1])
        for p, snap in zip(model.pool, want_state[0], strict=True):
            for k, v in snap.items():
                ok = ok and torch.equal(p[k], v)
        return bool(ok)

    def prepare(self) -> bool:
        """Capture and validate every bucket (the reference's boot hook, `graph_mtp.py:712-769`).
        Boot-only: every lane must be idle; all lanes are reset afterwards. Returns whether the
        captured round is enabled."""
        import os

        model = self.model
        if any(model.blocks.host[lane] for lane in range(model.lanes)):
            raise RuntimeError("prepare() is boot-only: some lanes hold KV blocks")
        self.graphs, self.validated = {}, {}
        ok = True
        try:
            for bucket in self.buckets:
                buf = self.buffers(bucket)
                # warm every lazy allocation on real rows, then capture from a clean state
                self._reset_lanes()
                self.fill(buf, list(range(bucket)), [0] * bucket, [0] * bucket)
                self._eager_round(buf)
                self._reset_lanes()
                replay = self._capture(buf)
                good = self._validate(bucket, buf, replay)
                self.validated[bucket] = good
                self.graphs[bucket] = replay
                ok = ok and good
        except Exception as exc:  # a failed capture disables the captured round, as a mismatch does
            if os.environ.get(REQUIRE_GRAPH_ENV, "0") == "1":
                raise RuntimeError(f"{REQUIRE_GRAPH_ENV}: captured MTP round failed: {exc!r}") from exc
            ok = False
        finally:
            self._reset_lanes()
        self.enabled = ok
        if not ok and os.environ.get(REQUIRE_GRAPH_ENV, "0") == "1":
            raise RuntimeError(f"{REQUIRE_GRAPH_ENV}: captured MTP round failed validation "
                               f"({self.validated})")
        return ok

    def speculative_decode(self, slots: list[int], tokens: list[int], positions: list[int],
                           budgets=None, stops=None, forced=None) -> list[list[int]]:
        if not self.enabled:
            self.eager_rounds += 1
            return super().speculative_decode(slots, tokens, positions, budgets, stops, forced)
        buf = self.buffers(len(slots))
        replay = self.graphs.get(buf.capacity)
        if replay is None:
            self.fill(buf, slots, tokens, positions, budgets, stops, forced)
            self._eager_round(buf)  # this round, run eagerly; then the bucket is captured
            self.graphs[buf.capacity] = self._capture(buf)
        else:
            _stage(self.model, buf, slots, tokens, positions, budgets, stops, forced)
            replay()  # unpacks the staged rows, then the round
        return _committed(buf, len(slots))


# ---------------------------------------------------------------- sampling-mode acceptance


def rejection_workspace(batch: int, k: int, vocab: int, device: torch.device) -> torch.Tensor:
    n = int(_mtpk.lib().mtpk_rejection_workspace_bytes(batch, k, vocab))
    return torch.empty(max(n, 1), dtype=torch.uint8, device=device)


def rejection_sample(target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_tokens: torch.Tensor,
                     u_accept: torch.Tensor, u_sample: torch.Tensor, temperature: float, *,
                     workspace: torch.Tensor | None = None,
                     with_margin: bool = False) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Speculative rejection sampling on the device (`mtpk_rejection_sample`): returns
    `(accept_len i64 [B], token i64 [B], emitted i64 [B, k+1], margin f32 [B, k] or None)`.

    `target_logits` `[B, k+1, V]` and `draft_logits` `[B, k, V]` (f32 or bf16, same dtype),
    `draft_tokens` i64 `[B, k]`, uniforms f32 `u_accept` `[B, k]` and `u_sample` `[B]`.
    `emitted` is the accepted drafts then the drawn token: fed to `greedy_accept` as the
    step argmax it gives the same accept length and every rollback index."""
    device = _mtpk.require_device(target_logits, draft_logits, draft_tokens, u_accept, u_sample)
    b, t, vocab = target_logits.shape
    k = t - 1
    if draft_logits.shape != (b, k, vocab) or draft_logits.dtype != target_logits.dtype:
        raise ValueError("draft_logits must be [B, k, V] of target_logits' dtype")
    if draft_tokens.shape != (b, k) or draft_tokens.dtype != torch.int64:
        raise ValueError("draft_tokens must be int64 [B, k]")
    if u_accept.shape != (b, k) or u_sample.shape != (b,):
        raise ValueError("u_accept must be [B, k] and u_sample [B]")
    if not temperature > 0:
        raise ValueError("rejection sampling needs temperature > 0 (greedy rounds use greedy_accept)")
    tl, dl = target_logits.contiguous(), draft_logits.contiguous()
    ua, us = u_accept.float().contiguous(), u_sample.float().contiguous()
    dt = draft_tokens.contiguous()
    ws = workspace if workspace is not None else rejection_workspace(b, k, vocab, device)
    long = dict(dtype=torch.long, device=device)
    acc, tok, emitted = torch.empty(b, **long), torch.empty(b, **long), torch.empty(b, t, **long)
    margin = torch.empty(b, max(k, 1), dtype=torch.float32, device=device) if with_margin else None
    _mtpk.check(
        _mtpk.lib().mtpk_rejection_sample(
            tl.data_ptr(), dl.data_ptr(), _mtpk.float_code(tl.dtype), b, k, vocab, dt.data_ptr(),
            ua.data_ptr(), us.data_ptr(), float(temperature), ws.data_ptr(), ws.numel(),
            acc.data_ptr(), tok.data_ptr(), emitted.data_ptr(),
            margin.data_ptr() if margin is not None else None, _mtpk.stream_of(device),
        ),
        "mtpk_rejection_sample",
    )  # fmt: skip
    return acc, tok, emitted, margin[:, :k] if margin is not None else None


def rejection_accept(target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_tokens: torch.Tensor,
                     u_accept: torch.Tensor, u_sample: torch.Tensor, temperature: float,
                     active: torch.Tensor, pos: torch.Tensor, budget: torch.Tensor, stops: torch.Tensor,
                     conv_k1: int, *, workspace: torch.Tensor | None = None,
                     out: AcceptResult | None = None) -> tuple[AcceptResult, torch.Tensor]:
    """Sampling-mode acceptance with the round's rollback indices (`mtpk_rejection_accept`):
    rejection sampling, and in the same launches what `greedy_accept` gives over the emitted
    tokens (the stop ids and the budget applied), taken from the sampler's accept length.
    Returns `(AcceptResult, emitted [B, k+1])`; committed ids are `emitted[j, :a+1]`."""
    device = _mtpk.require_device(target_logits, draft_logits, draft_tokens, u_accept, u_sample,
                                  active, pos, budget, stops)
    b, t, vocab = target_logits.shape
    k = t - 1
    if draft_logits.shape != (b, k, vocab) or draft_logits.dtype != target_logits.dtype:
        raise ValueError("draft_logits must be [B, k, V] of target_logits' dtype")
    if draft_tokens.shape != (b, k) or draft_tokens.dtype != torch.int64:
        raise ValueError("draft_tokens must be int64 [B, k]")
    if u_accept.shape != (b, k) or u_sample.shape != (b,):
        raise ValueError("u_accept must be [B, k] and u_sample [B]")
    if not temperature > 0:
        raise ValueError("rejection sampling needs temperature > 0 (greedy rounds use greedy_accept)")
    for name, ten in (("pos", pos), ("budget", budget), ("stops", stops)):
        if ten.dtype != torch.int64:
            raise ValueError(f"{name} must be int64")
    if active.dtype != torch.bool or active.shape != (b,) or stops.dim() != 2 or stops.shape[0] != b:
        raise ValueError("active must be bool [B] and stops [B, S]")
    tl, dl = target_logits.contiguous(), draft_logits.contiguous()
    ua, us = u_accept.float().contiguous(), u_sample.float().contiguous()
    dt = draft_tokens.contiguous()
    st = stops.contiguous()
    ws = workspace if workspace is not None else rejection_workspace(b, k, vocab, device)
    long = dict(dtype=torch.long, device=device)
    if out is None:
        out = AcceptResult(
            torch.empty(b, **long), torch.empty(b, **long), torch.empty(b * t, **long),
            torch.empty(b + 1, dtype=torch.int32, device=device),
            torch.empty(b, conv_k1, **long), torch.empty(b, t, dtype=torch.bool, device=device),
            torch.empty(b, **long), torch.empty(b, **long), torch.empty(b, **long),
            torch.empty(b, dtype=torch.bool, device=device), torch.empty(b, **long),
        )
    tok, emitted = torch.empty(b, **long), torch.empty(b, t, **long)
    _mtpk.check(
        _mtpk.lib().mtpk_rejection_accept(
            tl.data_ptr(), dl.data_ptr(), _mtpk.float_code(tl.dtype), b, k, vocab, dt.data_ptr(),
            ua.data_ptr(), us.data_ptr(), float(temperature), ws.data_ptr(), ws.numel(),
            active.contiguous().data_ptr(), pos.contiguous().data_ptr(), budget.contiguous().data_ptr(),
            st.data_ptr(), st.shape[1], conv_k1, out.accept_len.data_ptr(), out.lengths.data_ptr(),
            out.packed_src.data_ptr(), out.packed_cu.data_ptr(),
            out.conv_idx.data_ptr() if conv_k1 > 0 else None, out.keep.data_ptr(),
            out.bonus.data_ptr(), out.next_pos.data_ptr(), out.budget_left.data_ptr(),
            out.live.data_ptr(), out.hidden_src.data_ptr(), tok.data_ptr(), emitted.data_ptr(),
            _mtpk.stream_of(device),
        ),
        "mtpk_rejection_accept",
    )  # fmt: skip
    return out, emitted
