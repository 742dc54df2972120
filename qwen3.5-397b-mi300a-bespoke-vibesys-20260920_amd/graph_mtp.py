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
                  keys: tuple[torch.Tensor, int] | None = None) -> AcceptResult:
    """`mtpk_greedy_accept` on device tensors: step_argmax i64 [B, t], draft i64 [B, t-1] (row
    stride free, unit column stride), active bool [B], pos/budget i64 [B], stops i64 [B, S].
    With `keys` (`mtp.argmax_keys` of the [B * t, vocab] verify logits) the same launch first
    finishes the argmax and writes it into `step_argmax` (`mtpk_greedy_accept_keys`)."""
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
    _mtpk.check(
        (_mtpk.lib().mtpk_greedy_accept_keys if keys is not None else _mtpk.lib().mtpk_greedy_accept)(
            *((keys[0].data_ptr(), keys[1]) if keys is not None else ()),
            step_argmax.data_ptr(), step_argmax.stride(0), draft.data_ptr(),
            draft.stride(0) if t > 1 else 0, active.contiguous().data_ptr(),
            pos.contiguous().data_ptr(), budget.contiguous().data_ptr(), stops.data_ptr(),
            stops.shape[1], b, t, conv_k1, out.accept_len.data_ptr(), out.lengths.data_ptr(),
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
    block_id = torch.gather(block_table.long(), 1, (grid // block_size).long())
    return block_id * block_size + grid % block_size


# ---------------------------------------------------------------- the device round


def _draft_rows(model, m, buf: MTPVerifyBuffers, lanes: torch.Tensor, b: int,
                forced: torch.Tensor | None = None, forced_n: torch.Tensor | None = None) -> None:
    """`m.k` MTP draft steps for the first `b` rows of `buf` (lanes `lanes`), drafts written
    into `buf.token_matrix[:, 1:]`. Device-only, no host read. A row with `forced_n[j] > 0`
    feeds (and keeps) its forced tokens instead of its first drafts."""
    hid = mtp_mod.draft_seed(model, model.hidden_cache[lanes])
    tok = buf.token_matrix[:b, :1]
    table = model.blocks.table[lanes]
    on_device = vm.kv_write_in_kernel(model)
    for s in range(m.k):
        pos = buf.pos[:b] + s
        rows = None if on_device else model.blocks.physical_rows(lanes, pos[:, None])[:, 0]
        hid, tok = mtp_mod.draft_step(model, m, hid, tok, pos, rows, table)
        if forced is not None:
            tok = torch.where((forced_n > s)[:, None], forced[:, s : s + 1], tok)
        buf.token_matrix[:b, s + 1] = tok[:, 0]


def _verify_rows(model, m, buf: MTPVerifyBuffers, lanes: torch.Tensor, b: int, ctx_len: int,
                 forced_n: torch.Tensor | None = None) -> None:
    """Verify forward over `buf.token_matrix[:b]`, argmax, acceptance with every rollback
    index (`mtpk_greedy_accept`), then the commit of DeltaNet state, MTP cache rows and the
    cached hidden seed to each lane's accepted length. Device-only. Rows with
    `forced_n[j] > 0` accept their forced drafts unconditionally."""
    t = buf.t
    dev = buf.pos.device
    pos = buf.pos[:b]
    res = model.forward_rows(buf.token_matrix[:b], lanes, pos, ctx_len)
    logits = model.logits(res.hidden)
    keys = None
    if dev.type == "cuda" and b * t <= KEY_ROWS:  # the accept launch finishes the argmax
        keys = mtp_mod.argmax_keys(logits.reshape(b * t, -1))
    else:
        buf.step_argmax[:b] = model.argmax(logits).view(b, t)
    out = AcceptResult(buf.accept_len[:b], buf.lengths[:b], buf.packed_src[: b * t],
                       buf.packed_cu[: b + 1], buf.conv_idx[:b], buf.keep[:b], buf.bonus[:b],
                       buf.next_pos[:b], buf.budget_left[:b], buf.live[:b], buf.hidden_src[:b])
    greedy_accept(buf.step_argmax[:b], buf.token_matrix[:b, 1:], buf.active[:b], pos,
                  buf.budget[:b], buf.stops[:b], buf.conv_k1, out=out, keys=keys)
    if forced_n is not None:
        # A forced lane commits its forced tokens plus one target token; stop ids and the
        # budget do not apply to forced tokens (`graph_verify_wide.py:196-200`).
        # Rows without forced feed keep the acceptance launch's outputs as they are.
        f = (forced_n > 0) & buf.active[:b]
        a = forced_n
        length = a + 1
        win = torch.arange(buf.conv_k1, device=dev)
        keep = torch.arange(t, device=dev)[None, :] <= a[:, None]
        conv = torch.clamp(length[:, None] + win[None, :], max=buf.conv_k1 + t - 1)
        out.accept_len.copy_(torch.where(f, a, out.accept_len))
        out.lengths.copy_(torch.where(f, length, out.lengths))
        out.keep.copy_(torch.where(f[:, None], keep, out.keep))
        out.hidden_src.copy_(torch.where(f, torch.arange(b, device=dev) * t + a, out.hidden_src))
        out.conv_idx.copy_(torch.where(f[:, None], conv, out.conv_idx))
    model.commit(res, lanes, out.lengths, conv_idx=out.conv_idx)
    grid = pos[:, None] + torch.arange(t, device=dev)[None, :]
    raw_seed = model.hidden_cache[lanes]
    previous = torch.cat([raw_seed[:, None], res.hidden[:, :-1]], dim=1)
    if vm.kv_write_in_kernel(model):
        mtp_mod.cache_target_rows(model, m, buf.token_matrix[:b], previous, grid, None, out.keep,
                                  block_table=model.blocks.table[lanes], base_pos=pos)
    else:
        mtp_mod.cache_target_rows(model, m, buf.token_matrix[:b], previous, grid,
                                  model.blocks.physical_rows(lanes, grid), out.keep)
    model.hidden_cache[lanes] = res.hidden.reshape(b * t, -1)[out.hidden_src]


def _ctx_bound(model) -> int:
    """Context length every captured round is sized for: the block tables' full capacity, so
    the attention's key splits do not depend on a round's positions."""
    return model.blocks.max_blocks * model.cfg.block_size


def draft_round_step(model, mtp, buf: MTPVerifyBuffers, t: int) -> Callable[[], None]:
    """The draft step to capture (`graph_mtp.py:477-504`, same arguments): `t - 1` MTP steps
    over every row of `buf`, seeded from each row's lane (`slot_rows`) and base token
    (`token_matrix[:, 0]`), each step's greedy token written into `token_matrix[:, 1 + step]`;
    rows with `forced_n > 0` feed and keep `forced_ids` instead."""
    if t != buf.t or t != mtp.k + 1:
        raise ValueError(f"t={t} does not match the buffers ({buf.t}) and the MTP head (k={mtp.k})")

    def step() -> None:
        _draft_rows(model, mtp, buf, buf.slot_rows, buf.capacity, buf.forced_ids, buf.forced_n)

    return step


build_draft_step = draft_round_step
"""The reference's alias for the draft entry point (`graph_mtp.py:507-510`)."""


def verify_round_step(model, mtp, buf: MTPVerifyBuffers, t: int) -> Callable[[], None]:
    """The verify step to capture (`graph_mtp.py:513-582`, same arguments): one forward over
    every row of `buf`, the argmax, commit-limited acceptance with every rollback index, and the
    commit of DeltaNet state, MTP cache rows and the hidden seed to each row's accepted length."""
    if t != buf.t:
        raise ValueError(f"t={t} does not match the buffers ({buf.t})")
    ctx = _ctx_bound(model)

    def step() -> None:
        _verify_rows(model, mtp, buf, buf.slot_rows, buf.capacity, ctx, buf.forced_n)

    return step


def _fill(model, mtp, buf: MTPVerifyBuffers, slots, tokens, positions, budgets, stops, forced) -> None:
    """Write one round's inputs into `buf` (`MTPVerifyRunner.fill`, `graph_mtp.py:790-870`):
    every row is a real lane (a bucket is sized to its round), so no row is padding."""
    b, t, k = len(slots), buf.t, buf.t - 1
    if b != buf.capacity or len(set(slots)) != b:
        raise ValueError(f"need {buf.capacity} distinct slots, got {slots}")
    if stops is not None and any(len(s) > mtp_mod.MAX_STOP_IDS for s in stops):
        raise ValueError(f"at most {mtp_mod.MAX_STOP_IDS} stop ids per lane")
    for s, p in zip(slots, positions, strict=True):
        model.blocks.grow(s, p + t)
    big = 1 << 40
    rows = []
    for j, (tk, p) in enumerate(zip(tokens, positions, strict=True)):
        ids = list(forced[j])[:k] if forced else []
        st = list(stops[j]) if stops else []
        rows.append([tk, p, big if budgets is None else budgets[j], int(slots[j]), len(ids),
                     *(ids + [0] * (max(k, 1) - len(ids))), *(st + [-1] * (mtp_mod.MAX_STOP_IDS - len(st)))])
    host = torch.tensor(rows, dtype=torch.long).to(buf.pos.device)
    buf.token_matrix[:, 0] = host[:, 0]
    buf.pos.copy_(host[:, 1])
    buf.budget.copy_(host[:, 2])
    buf.slot_rows.copy_(host[:, 3])
    buf.forced_n.copy_(host[:, 4])
    buf.forced_ids.copy_(host[:, 5 : 5 + max(k, 1)])
    buf.stops.copy_(host[:, 5 + max(k, 1) :])
    buf.active.fill_(True)


def _committed(buf: MTPVerifyBuffers) -> list[list[int]]:
    """The round's committed ids, `step_argmax[j, : accept + 1]`: one host read."""
    rows = torch.cat([buf.step_argmax, buf.accept_len[:, None]], dim=1).tolist()
    return [row[: row[-1] + 1] for row in rows]


class MTPVerifyRunner:
    """Eager speculative rounds over static per-batch-size buffers (`graph_mtp.MTPVerifyRunner`,
    `graph_mtp.py:893-918`): fill, draft, verify + accept + commit, one host read. `capacity`
    (default: every lane of the model) bounds the batch size."""

    def __init__(self, model, mtp=None, capacity: int | None = None) -> None:
        mtp = model.mtp if mtp is None else mtp
        if mtp is None:
            raise ValueError("model has no MTP layer")
        self.model, self.mtp = model, mtp
        self.t = mtp.k + 1
        self.capacity = model.lanes if capacity is None else capacity
        self.bufs: dict[int, MTPVerifyBuffers] = {}

    def buffers(self, b: int) -> MTPVerifyBuffers:
        if not 1 <= b <= self.capacity:
            raise ValueError(f"batch of {b} lanes: this runner takes 1..{self.capacity}")
        if b not in self.bufs:
            self.bufs[b] = MTPVerifyBuffers(self.model, b, self.t, self.model.device)
        return self.bufs[b]

    def speculative_decode(self, slots: list[int], tokens: list[int], positions: list[int],
                           budgets=None, stops=None, forced=None) -> list[list[int]]:
        """Each slot's committed ids for one round (`Model.speculative_decode`'s contract);
        `forced` rows commit their forced drafts plus one target token."""
        buf = self.buffers(len(slots))
        _fill(self.model, self.mtp, buf, slots, tokens, positions, budgets, stops, forced)
        draft_round_step(self.model, self.mtp, buf, self.t)()
        verify_round_step(self.model, self.mtp, buf, self.t)()
        return _committed(buf)


class GraphMTPRunner(MTPVerifyRunner):
    """`MTPVerifyRunner` with each batch size's draft and verify steps captured in one HIP graph
    (`GraphMTPRunner(model, backend=None)`, `graph_mtp.py:1062-1120`). A round writes the
    bucket's static buffers, replays its graph and reads the committed ids once; forced feed
    rides in the buffers, so forced rounds replay the same graph. The first round of a batch size
    runs eagerly on the capture stream (its result is that round's) and is then captured.

    `backend` is the reference's capture-backend slot: HIP graphs through `torch.cuda.CUDAGraph`
    are the only backend here, so it must be None. `capacity` (keyword) bounds the batch size."""

    def __init__(self, model, backend=None, *, capacity: int | None = None) -> None:
        if backend is not None:
            raise ValueError("GraphMTPRunner captures HIP graphs only; backend must be None")
        super().__init__(model, None, capacity)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}

    def prepare(self) -> bool:
        """The reference's boot hook (`graph_mtp.py:1077-1081`): graphs are captured on each
        batch size's first round instead, so there is nothing to do up front."""
        return True

    def forced_drafts(self) -> bool:
        """Whether rounds may carry forced feed (`graph_mtp.py:1116-1118`): always."""
        return True

    def _round(self, buf: MTPVerifyBuffers) -> None:
        draft_round_step(self.model, self.mtp, buf, self.t)()
        verify_round_step(self.model, self.mtp, buf, self.t)()

    def speculative_decode(self, slots: list[int], tokens: list[int], positions: list[int],
                           budgets=None, stops=None, forced=None) -> list[list[int]]:
        b = len(slots)
        buf = self.buffers(b)
        _fill(self.model, self.mtp, buf, slots, tokens, positions, budgets, stops, forced)
        graph = self.graphs.get(b)
        if graph is None:
            dev = buf.pos.device
            side = torch.cuda.Stream(dev)
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self._round(buf)  # this round, run eagerly; also warms the allocator
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize(dev)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                self._round(buf)
            self.graphs[b] = graph
        else:
            graph.replay()
        return _committed(buf)


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
                     conv_k1: int) -> tuple[AcceptResult, torch.Tensor]:
    """Sampling-mode acceptance with the round's rollback indices: rejection sampling, then
    `greedy_accept` over the emitted tokens (which applies the stop ids and the budget).
    Returns `(AcceptResult, emitted [B, k+1])`; committed ids are `emitted[j, :a+1]`."""
    _, _, emitted, _ = rejection_sample(target_logits, draft_logits, draft_tokens, u_accept, u_sample,
                                        temperature)
    res = greedy_accept(emitted, draft_tokens, active, pos, budget, stops, conv_k1)
    return res, emitted
