"""MTP draft / verify / accept — the reference's `mtp` interface (`mtp.py`).

The MTP head (`MTP`, `attach`, `draft_step`, `draft`, `cache_target_rows`) is one decoder
layer fed by `fc(cat(norm(embed(token)), norm(hidden)))` (`mtp.py:191-549`); its attention
reads its own K/V pool through the target's block tables and its MoE is the same routed MXFP4
call as a target layer's. `verify_and_commit` / `speculative_decode` are the eager round
(`mtp.py:729-817`, `model.py:4183-4220`); `graph_mtp.MTPVerifyRunner` is the device round.

Host-side acceptance keeps the reference's pure functions (`greedy_accept_length`,
`commit_limit`, `mtp.py:691-726`); the device-side greedy token is the fused argmax kernel
(`mtpk_argmax_rows`), replacing `logits.float().argmax(-1, keepdim=True)` of `greedy_token`
(`mtp.py:640-658`) with a bit-identical first-occurrence argmax.
"""

from __future__ import annotations

import os
from collections.abc import Sequence
from dataclasses import dataclass

import torch

import _mtpk
import attention
import rownorm

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


def _flag(name: str) -> bool:
    return os.environ.get(name, "0") not in ("0", "", "false", "False")


def mtp_enabled() -> bool:
    """Whether speculative decoding is on: `SEED_MTP_SERVE=1` or its older alias `SEED_MTP=1`
    (`mtp.py:57-61`). Read when called, so a process (or a test) can set it after import."""
    return _flag("SEED_MTP_SERVE") or _flag("SEED_MTP")


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


def argmax_keys(logits: torch.Tensor) -> tuple[torch.Tensor, int]:
    """The first launch of `argmax_rows` alone (`mtpk_argmax_keys`): the first-occurrence
    (value, index) keys of each row's vocabulary chunks, `(keys u64-as-int64 [rows, chunks],
    chunks)` for `graph_mtp.greedy_accept(..., keys=)`, which finishes the argmax."""
    device = _mtpk.require_device(logits)
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    vocab = logits.shape[-1]
    flat = logits.reshape(-1, vocab) if logits.dim() != 2 else logits
    rows = flat.shape[0]
    lib = _mtpk.lib()
    chunks = max(int(lib.mtpk_argmax_partials(rows, vocab)) // max(rows, 1), 1)
    keys = torch.empty(rows, chunks, dtype=torch.int64, device=device)
    _mtpk.check(lib.mtpk_argmax_keys(flat.data_ptr(), _mtpk.float_code(flat.dtype), rows, vocab,
                                     flat.stride(0), keys.data_ptr(), _mtpk.stream_of(device)),
                "mtpk_argmax_keys")
    return keys, chunks


def greedy_token(model, normed: torch.Tensor) -> torch.Tensor:
    """`model.unembed(normed).float().argmax(-1, keepdim=True)` for `[B, hidden]` rows, `[B, 1]`
    long. On a device this is `model.next_tokens` (the HIP argmax compares the bf16 logits
    exactly, so the fp32 cast is not needed)."""
    if normed.device.type == "cuda":
        return model.next_tokens(normed)[..., None]
    return model.unembed(normed).float().argmax(-1, keepdim=True)


# ---------------------------------------------------------------- the MTP head


@dataclass
class MTP:
    """The MTP module and its paged KV cache (`mtp.py:114-128`). `weights` holds one decoder
    layer (`in_norm`, `post_norm`, gated attention, router, shared expert, MXFP4 experts) keyed
    like a target layer; the pool is indexed by the target's block tables."""

    k: int
    weights: dict
    fc: torch.Tensor
    pre_fc_norm_embedding: torch.Tensor
    pre_fc_norm_hidden: torch.Tensor
    norm: torch.Tensor
    pool: dict


def attach(model, k: int | None = None, seed: int = 1, expert_mode: str = "quantized") -> MTP:
    """Random-init MTP layer for `model` (the same initialisers as its target layers), stored
    as `model.mtp`. `k` defaults to `MTP_K`."""
    import verify_model as vm

    c, dev, dt = model.cfg, model.device, model.dtype
    gen = torch.Generator(device="cpu" if c.hidden < 1024 else dev).manual_seed(seed)
    w = {"in_norm": vm._normal((c.hidden,), 0.02, dt, dev, gen),
         "post_norm": vm._normal((c.hidden,), 0.02, dt, dev, gen)}
    w.update(vm.attention_weights(c, dt, dev, gen))
    w.update(vm.moe_weights(c, dt, dev, gen, expert_mode))
    shape = (model.blocks.rows, c.kv_heads, c.head_dim)
    m = MTP(
        k=MTP_K if k is None else k,
        weights=w,
        fc=vm._normal((c.hidden, 2 * c.hidden), 0.02, dt, dev, gen),
        pre_fc_norm_embedding=vm._normal((c.hidden,), 0.02, dt, dev, gen),
        pre_fc_norm_hidden=vm._normal((c.hidden,), 0.02, dt, dev, gen),
        norm=vm._normal((c.hidden,), 0.02, dt, dev, gen),
        pool={"k": torch.zeros(shape, dtype=dt, device=dev),
              "v": torch.zeros(model.blocks.rows // c.block_size, c.kv_heads, c.head_dim, c.block_size,
                               dtype=dt, device=dev)},
    )
    model.mtp = m
    return m


def load(ck, full_cfg, tp, dev, dtype: torch.dtype, max_batch: int, kv_rows: int) -> MTP | None:
    """The checkpoint's MTP module (`mtp.py:131-190`, same arguments), or None when the flag is
    off or the checkpoint has no `mtp.fc.weight`.

    `ck` is a `weights.Checkpoint`, `full_cfg` the model's `Cfg`, `dev` / `dtype` where and as
    what the dense tensors land (MXFP4 expert payloads stay uint8). The decoder layer's tensors
    are stored under the keys a target layer uses: the router rows and the shared expert's gate
    row concatenated into `router_gate`, its gate and up projections into `shared_gate_up`. The
    K pool is `[kv_rows, kv_heads, head_dim]` and the V pool the same rows transposed per block,
    `[kv_rows / block_size, kv_heads, head_dim, block_size]`, indexed by the target's block
    tables. This build runs on one GPU: `tp` is None or a plan of world size 1. `max_batch`
    sizes no scratch here (the kernels take their workspaces per call); it is checked only. The
    attention projections are stacked into one `qkv_proj` weight (`verify_model.fuse_qkv`), the
    three keys left as views of it."""
    import verify_model as vm
    import weights as wt

    if not mtp_enabled() or not ck.has("mtp.fc.weight"):
        return None
    if tp is not None and getattr(tp, "world", 1) != 1:
        raise ValueError("this build loads the MTP layer for one GPU (tp world size 1)")
    c = full_cfg
    if max_batch < 1:
        raise ValueError(f"max_batch must be positive, got {max_batch}")
    if kv_rows <= 0 or kv_rows % c.block_size:
        raise ValueError(f"kv_rows must be a positive multiple of the block size {c.block_size}")
    dev = torch.device(dev)
    qd, kd = c.heads * c.head_dim, c.kv_heads * c.head_dim

    def read(name: str, shape: tuple[int, ...]) -> torch.Tensor:
        t = ck.load(f"mtp.{name}", dev, dtype)
        if tuple(t.shape) != shape:
            raise ValueError(f"mtp.{name}: shape {tuple(t.shape)}, the config needs {shape}")
        return t

    h, si = c.hidden, c.shared_inter
    at = "layers.0.self_attn"
    mlp = "layers.0.mlp"
    w = {
        "in_norm": read("layers.0.input_layernorm.weight", (h,)),
        "post_norm": read("layers.0.post_attention_layernorm.weight", (h,)),
        "q_proj": read(f"{at}.q_proj.weight", (2 * qd, h)),  # per head: q rows, then gate rows
        "k_proj": read(f"{at}.k_proj.weight", (kd, h)),
        "v_proj": read(f"{at}.v_proj.weight", (kd, h)),
        "o_proj": read(f"{at}.o_proj.weight", (h, qd)),
        "q_norm": read(f"{at}.q_norm.weight", (c.head_dim,)),
        "k_norm": read(f"{at}.k_norm.weight", (c.head_dim,)),
        "router_gate": torch.cat([read(f"{mlp}.gate.weight", (c.experts, h)),
                                  read(f"{mlp}.shared_expert_gate.weight", (1, h))]),
        "shared_gate_up": torch.cat([read(f"{mlp}.shared_expert.gate_proj.weight", (si, h)),
                                     read(f"{mlp}.shared_expert.up_proj.weight", (si, h))]),
        "shared_down": read(f"{mlp}.shared_expert.down_proj.weight", (h, si)),
        "experts": wt.load_experts(ck, f"mtp.{mlp}", wt.Shard(0, c.experts), dev, dtype),
    }
    gu = w["experts"]["gate_up"]
    if gu.shape[:2] != (c.experts, 2 * c.inter) or w["experts"]["down"].shape[:2] != (c.experts, h):
        raise ValueError(f"mtp experts: gate_up {tuple(gu.shape)}, down "
                         f"{tuple(w['experts']['down'].shape)} do not match the config")
    vm.fuse_qkv(w)
    return MTP(
        k=MTP_K,
        weights=w,
        fc=read("fc.weight", (h, 2 * h)),
        pre_fc_norm_embedding=read("pre_fc_norm_embedding.weight", (h,)),
        pre_fc_norm_hidden=read("pre_fc_norm_hidden.weight", (h,)),
        norm=read("norm.weight", (h,)),
        pool={"k": torch.zeros(kv_rows, c.kv_heads, c.head_dim, dtype=dtype, device=dev),
              "v": torch.zeros(kv_rows // c.block_size, c.kv_heads, c.head_dim, c.block_size,
                               dtype=dtype, device=dev)},
    )


def draft_seed(model, raw_hidden: torch.Tensor) -> torch.Tensor:
    """Step 0's hidden input: the target's final-normed last hidden state (`mtp.py:433-437`,
    the default `post` seed)."""
    import verify_model as vm

    return vm.rmsnorm(raw_hidden, model.final_norm, model.cfg.eps)


def _combine_rows(model, mtp: MTP, hidden: torch.Tensor, tokens: torch.Tensor) -> torch.Tensor:
    """`fc(cat(norm(embed(tokens)), norm(hidden)))` for matching leading dims
    (`mtp.py:191-230`)."""
    import verify_model as vm

    eps = model.cfg.eps
    h = model.cfg.hidden
    if hidden.is_cuda and model.embed.is_contiguous() and hidden.is_contiguous():
        # the embedding lookup rides in the first norm, and both norms write their halves of
        # the concatenated row: two launches for gather, two norms and the cat
        x = torch.empty(*tokens.shape, 2 * h, dtype=hidden.dtype, device=hidden.device)
        rownorm.rmsnorm(model.embed, mtp.pre_fc_norm_embedding, eps, gather=tokens, out=x[..., :h])
        rownorm.rmsnorm(hidden, mtp.pre_fc_norm_hidden, eps, out=x[..., h:])
        return vm.linear(x, mtp.fc)
    emb = vm.rmsnorm(model.embed[tokens], mtp.pre_fc_norm_embedding, eps)
    hid = vm.rmsnorm(hidden, mtp.pre_fc_norm_hidden, eps)
    return vm.linear(torch.cat([emb, hid], dim=-1), mtp.fc)


def draft_step(model, mtp: MTP, hid: torch.Tensor, tok: torch.Tensor, rope_pos: torch.Tensor,
               write_rows: torch.Tensor | None, block_table: torch.Tensor,
               block_valid: torch.Tensor | None = None,
               active: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """One MTP decoder-layer step on device-resident tensors (`mtp.py:506-549`):
    `(hid [B, hidden], tok [B, 1])` -> the next pair. `rope_pos` `[B]` is the fed token's
    position, `write_rows` `[B]` its MTP pool row (None when `verify_model.kv_write_in_kernel`:
    the K/V write maps the position through the table), `block_table` `[B, blocks]` the lanes'
    tables. `active` `[B]` bool (optional) masks the step's persistent write, its MTP K/V row:
    padding rows write nothing. `block_valid` is accepted for signature compatibility (the
    attention reads the table up to its width and masks by position)."""
    import verify_model as vm

    c, w = model.cfg, mtp.weights
    x = _combine_rows(model, mtp, hid[:, None, :], tok)  # [B, 1, hidden]
    h = vm.rmsnorm(x, w["in_norm"], c.eps)
    attn = vm.gated_attention(model, w, mtp.pool, h, rope_pos,
                              None if write_rows is None else write_rows.reshape(-1, 1),
                              block_table, block_table.shape[1],
                              None if active is None else active[:, None])
    x, hm = vm.add_rmsnorm(x, attn, w["post_norm"], c.eps)
    _, normed = model.moe_add_norm(w, hm[:, 0], x[:, 0], mtp.norm)
    nxt = model.next_tokens(normed)[:, None]
    return normed, nxt


def draft(model, mtp: MTP, hidden: torch.Tensor, tokens: list[int], slots: list[int],
          positions: list[int]) -> list[list[int]]:
    """`mtp.k` greedy MTP steps from each slot's last committed token and the target's raw
    hidden state (`mtp.py:391-430`); one host read for the whole round."""
    dev = model.device
    lanes = model.lane_index(slots)
    for s, p in zip(slots, positions, strict=True):
        model.blocks.grow(s, p + mtp.k)
    hid = draft_seed(model, hidden)
    tok = torch.tensor([[t] for t in tokens], dtype=torch.long, device=dev)
    base = torch.tensor(positions, dtype=torch.long, device=dev)
    table = model.blocks.table[lanes]
    out = torch.empty(len(slots), mtp.k, dtype=torch.long, device=dev)
    for step in range(mtp.k):
        pos = base + step
        rows = model.blocks.physical_rows(lanes, pos[:, None])[:, 0]
        hid, tok = draft_step(model, mtp, hid, tok, pos, rows, table)
        out[:, step] = tok[:, 0]
    return out.tolist()


def cache_target_rows(model, mtp: MTP, tokens: torch.Tensor, raw_previous_hidden: torch.Tensor,
                      positions: torch.Tensor, write_rows: torch.Tensor | None,
                      keep: torch.Tensor | None = None, *, block_table: torch.Tensor | None = None,
                      base_pos: torch.Tensor | None = None, seeded: bool = False) -> None:
    """Write the MTP layer's canonical K/V for fed tokens from the target's hidden stream
    (`mtp.py:440-485`): token `tokens[b, s]` at `positions[b, s]` paired with the target's raw
    hidden state of the previous position. Rows with `keep` False are left as they are.
    When `verify_model.kv_write_in_kernel(model)`, `block_table` `[B, blocks]` with `base_pos`
    `[B]` (`positions[b, s] = base_pos[b] + s`) replace `write_rows`: RoPE rides on the k norm
    and one kernel writes the K/V rows through the table. `seeded`: the hidden rows given are
    already final-normed (`draft_seed` of the raw ones, e.g. the forward's own normed rows)."""
    import verify_model as vm

    c, w = model.cfg, mtp.weights
    seed = raw_previous_hidden if seeded else draft_seed(model, raw_previous_hidden)
    x = _combine_rows(model, mtp, seed, tokens)
    x = vm.rmsnorm(x, w["in_norm"], c.eps)
    lead = tokens.shape
    if vm.kv_write_in_kernel(model) and block_table is not None and base_pos is not None:
        rope = (model.cos, model.sin, positions.reshape(-1))
        if "kv_proj" in w:  # k and v from one GEMM
            kp, v = vm.split_kv(vm.linear(x, w["kv_proj"]), c.kv_heads, c.head_dim)
        else:
            kp = vm.linear(x, w["k_proj"]).view(*lead, c.kv_heads, c.head_dim)
            v = vm.linear(x, w["v_proj"]).view(*lead, c.kv_heads, c.head_dim)
        k = rownorm.rmsnorm(kp, w["k_norm"], c.eps, heads=True, rope=rope)
        attention.kv_write(mtp.pool["k"], mtp.pool["v"], k, v, block_table, base_pos, keep)
        return
    k = vm.rmsnorm(vm.linear(x, w["k_proj"]).view(*lead, c.kv_heads, c.head_dim),
                   w["k_norm"], c.eps)
    v = vm.linear(x, w["v_proj"]).view(*lead, c.kv_heads, c.head_dim)
    pos = positions.long()
    k = vm.apply_rope(k, model.cos[pos][..., None, :], model.sin[pos][..., None, :])
    rows = write_rows.reshape(-1).long()
    k = k.reshape(-1, c.kv_heads, c.head_dim)
    v = v.reshape(-1, c.kv_heads, c.head_dim)
    if keep is not None:
        live = keep.reshape(-1)
        k = torch.where(live[:, None, None], k, mtp.pool["k"][rows])
        v = torch.where(live[:, None, None], v, attention.read_v(mtp.pool["v"], rows))
    mtp.pool["k"][rows] = k
    attention.write_v(mtp.pool["v"], rows, v)


def verify_and_commit(model, mtp: MTP, slots: list[int], base_tokens: list[int],
                      draft_tokens: list[list[int]], positions: list[int],
                      budgets: Sequence[int] | None = None,
                      stops: Sequence[Sequence[int]] | None = None) -> list[list[int]]:
    """One wide verify forward over the `[B, k + 1]` fed tokens, greedy acceptance, and the
    commit of every per-slot state to the accepted length (`mtp.py:729-817`). Returns each
    slot's committed ids (accepted drafts plus the bonus token)."""
    dev = model.device
    b, k = len(slots), mtp.k
    t = k + 1
    lanes = model.lane_index(slots)
    for s, p in zip(slots, positions, strict=True):
        model.blocks.grow(s, p + t)
    ids = torch.tensor([[base_tokens[j], *draft_tokens[j]] for j in range(b)], dtype=torch.long, device=dev)
    base = torch.tensor(positions, dtype=torch.long, device=dev)
    raw_seed = model.hidden_cache[lanes]
    res = model.forward_rows(ids, lanes, base, max(positions) + t)
    step_argmax = model.argmax(model.logits(res.hidden)).reshape(b, t)
    rows = step_argmax.tolist()
    accept = [
        commit_limit(greedy_accept_length(draft_tokens[j], rows[j][:k]), rows[j],
                     None if budgets is None else budgets[j], () if stops is None else stops[j])
        for j in range(b)
    ]
    acc = torch.tensor(accept, dtype=torch.long, device=dev)
    model.commit(res, lanes, acc + 1)
    grid = base[:, None] + torch.arange(t, device=dev)[None, :]
    previous = torch.cat([raw_seed[:, None], res.hidden[:, :-1]], dim=1)
    keep = torch.arange(t, device=dev)[None, :] <= acc[:, None]
    cache_target_rows(model, mtp, ids, previous, grid, model.blocks.physical_rows(lanes, grid), keep)
    model.hidden_cache[lanes] = res.hidden[torch.arange(b, device=dev), acc]
    return [rows[j][: accept[j] + 1] for j in range(b)]


def speculative_decode(model, slots: list[int], tokens: list[int], positions: list[int],
                       budgets: Sequence[int] | None = None,
                       stops: Sequence[Sequence[int]] | None = None) -> list[list[int]]:
    """Draft then verify (`Model.speculative_decode`, `model.py:4183-4220`): each slot's
    committed ids for this round."""
    m = model.mtp
    drafts = draft(model, m, model.hidden_cache[model.lane_index(slots)], tokens, slots, positions)
    return verify_and_commit(model, m, slots, tokens, drafts, positions, budgets, stops)


def sample_rows(logits: torch.Tensor, temperature: float, u: torch.Tensor) -> torch.Tensor:
    """One inverse-CDF draw per row from `softmax(logits / T)` with uniforms `u` `[rows]`
    (`mtpk_sample_rows`), int64 `[rows]`: the draft step's sampler at temperature > 0."""
    device = _mtpk.require_device(logits, u)
    if not temperature > 0:
        raise ValueError("sample_rows needs temperature > 0")
    flat = logits.reshape(-1, logits.shape[-1]).contiguous()
    rows, vocab = flat.shape
    uu = u.reshape(-1).float().contiguous()
    if uu.numel() != rows:
        raise ValueError("u must hold one uniform per row")
    lib = _mtpk.lib()
    ws = torch.empty(max(int(lib.mtpk_sample_workspace_bytes(rows, vocab)), 1), dtype=torch.uint8, device=device)
    out = torch.empty(rows, dtype=torch.long, device=device)
    _mtpk.check(lib.mtpk_sample_rows(flat.data_ptr(), _mtpk.float_code(flat.dtype), rows, vocab,
                                     float(temperature), uu.data_ptr(), ws.data_ptr(), ws.numel(),
                                     out.data_ptr(), _mtpk.stream_of(device)), "mtpk_sample_rows")
    return out.reshape(logits.shape[:-1])
