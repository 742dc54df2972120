"""Shared builders for the MTP model tests (config 1: the tiny Qwen3.5-MoE)."""

from __future__ import annotations

import torch

import attention
import mtp
import verify_model as vm

PROMPT_LEN = 16
GEN_TOKENS = 32


def build(device: str = "cpu", k: int = 1, lanes: int = 2, max_seq: int = 96,
          mtp_experts: str = "quantized") -> vm.Model:
    """Config 1's model: same weights on every device (drawn on the CPU from fixed seeds).
    `mtp_experts="dense"` gives the MTP layer bf16 experts, as in the real checkpoint."""
    model = vm.Model(vm.tiny_cfg(), device, torch.float32, lanes=lanes, max_seq=max_seq, seed=0)
    mtp.attach(model, k=k, seed=1, expert_mode=mtp_experts)
    return model


def prompts(n: int = 2, length: int = PROMPT_LEN, seed: int = 5) -> list[list[int]]:
    gen = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vm.tiny_cfg().vocab, (length,), generator=gen).tolist() for _ in range(n)]


def greedy_truth(model: vm.Model, prompt_ids: list[list[int]], n: int) -> list[list[int]]:
    """Per lane: the first greedy token after the prompt, then `n` more by plain decode."""
    out = []
    for lane, ids in enumerate(prompt_ids):
        base = int(model.argmax(model.prefill(lane, ids)[None])[0])
        out.append([base] + vm.greedy_reference(model, lane, base, len(ids), n))
    return out


def forced_drafts(truth: list[int], accept: int, k: int, vocab: int) -> list[int]:
    """Drafts agreeing with the greedy continuation for `accept` steps, then a wrong token."""
    d = list(truth[1 : accept + 1])
    while len(d) < k:
        d.append((truth[len(d) + 1] + 7) % vocab)
    return d


def slot_state(model: vm.Model, lane: int, length: int) -> list[torch.Tensor]:
    """Everything a round commits for slot `lane`, as CPU copies: attention K/V rows of
    positions < `length` per attention layer, DeltaNet conv and recurrent state per DeltaNet
    layer, the MTP layer's K/V rows of positions < `length`, and the cached hidden state."""
    lanes = torch.tensor([lane], device=model.device)
    pos = torch.arange(length, device=model.device)[None, :]
    rows = model.blocks.physical_rows(lanes, pos).reshape(-1)
    out = []
    for ty, pool in zip(model.cfg.layer_types, model.pool, strict=True):
        if ty == vm.ATTN:  # V is kept transposed per block
            out += [pool["k"][rows], attention.read_v(pool["v"], rows)]
        else:
            out += [pool["conv"][lane], pool["rec"][lane]]
    out += [model.mtp.pool["k"][rows], attention.read_v(model.mtp.pool["v"], rows)]
    out.append(model.cached_hidden(lane))
    return [x.float().cpu() for x in out]


def assert_slot_state_close(a: vm.Model, b: vm.Model, lane: int, length: int,
                            rtol: float = 1e-5, atol: float = 1e-6) -> None:
    """DeltaNet conv/recurrent state, attention and MTP K/V of positions < `length`, and the
    cached hidden state of slot `lane` agree between two models."""
    for ta, tb in zip(slot_state(a, lane, length), slot_state(b, lane, length), strict=True):
        torch.testing.assert_close(ta, tb, rtol=rtol, atol=atol)


def snapshot(model: vm.Model) -> list[torch.Tensor]:
    """Device copies of every tensor a round writes (layer pools, MTP pool, hidden seeds)."""
    live = [t for pool in model.pool for t in pool.values()]
    live += list(model.mtp.pool.values()) + [model.hidden_cache]
    return [t.clone() for t in live]


def restore(model: vm.Model, snap: list[torch.Tensor]) -> None:
    live = [t for pool in model.pool for t in pool.values()]
    live += list(model.mtp.pool.values()) + [model.hidden_cache]
    for t, s in zip(live, snap, strict=True):
        t.copy_(s)


def c5_model(dev, b: int = 48, k: int = 3, ctx: int = 8192):
    """The config-5 round the benchmark times: real layer dimensions (3 DeltaNet + 1 gated GQA +
    the MTP layer, 512 MXFP4 experts top-10), `b` lanes, each holding `ctx - 32` positions of
    seeded random context (K/V, DeltaNet state, hidden seeds). Returns (model, tokens, positions)."""
    model, _, toks, pos = c5_model_and_runner(dev, b, k, ctx, prepare=False)
    return model, toks, pos


def c5_model_and_runner(dev, b: int = 48, k: int = 3, ctx: int = 8192, prepare: bool = True):
    """`c5_model` plus a `GraphMTPRunner` with one `b`-row bucket, captured and validated by
    `prepare()` at boot (before the context is filled) when `prepare`. Returns (model, runner,
    tokens, positions)."""
    import graph_mtp

    model = vm.Model(vm.verify_cfg(), dev, torch.bfloat16, lanes=b, max_seq=ctx + 64, seed=0,
                     expert_mode="bytes", moe_rows=b * (k + 1))
    mtp.attach(model, k=k, seed=1, expert_mode="bytes")
    runner = graph_mtp.GraphMTPRunner(model, buckets=[b])
    if prepare:
        runner.prepare()
    start = ctx - 32
    for lane in range(b):
        model.blocks.grow(lane, start)
    g = torch.Generator(device=dev).manual_seed(3)
    for ty, pool in zip(model.cfg.layer_types, model.pool, strict=True):
        if ty == vm.ATTN:
            pool["k"].normal_(generator=g)
            pool["v"].normal_(generator=g)
        else:
            pool["conv"].normal_(generator=g)
            pool["rec"].normal_(0, 0.05, generator=g)
    model.mtp.pool["k"].normal_(generator=g)
    model.mtp.pool["v"].normal_(generator=g)
    model.hidden_cache.normal_(generator=g)
    toks = torch.randint(0, model.cfg.vocab, (b,), generator=torch.Generator().manual_seed(4)).tolist()
    return model, runner, toks, [start] * b


def shape_model(hidden: int, max_blocks: int, conv_k: int = 4, dtype=None):
    """The attributes `graph_mtp.MTPVerifyBuffers(model, ...)` reads from a model (hidden width,
    dtype, block-table width, DeltaNet conv window), for tests of the acceptance tail alone."""
    import types

    return types.SimpleNamespace(cfg=types.SimpleNamespace(hidden=hidden, conv_k=conv_k),
                                 dtype=dtype or torch.bfloat16,
                                 blocks=types.SimpleNamespace(max_blocks=max_blocks))
