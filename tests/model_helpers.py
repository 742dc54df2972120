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


def assert_slot_state_close(a: vm.Model, b: vm.Model, lane: int, length: int,
                            rtol: float = 1e-5, atol: float = 1e-6) -> None:
    """DeltaNet conv/recurrent state, attention and MTP K/V of positions < `length`, and the
    cached hidden state of slot `lane` agree between two models."""
    lanes = torch.tensor([lane], device=a.device)
    pos = torch.arange(length, device=a.device)[None, :]
    rows_a = a.blocks.physical_rows(lanes, pos).reshape(-1)
    rows_b = b.blocks.physical_rows(lanes.to(b.device), pos.to(b.device)).reshape(-1)
    def kv(pool, rows):  # K rows and V rows (V is kept transposed per block)
        return pool["k"][rows], attention.read_v(pool["v"], rows)

    for ty, pa, pb in zip(a.cfg.layer_types, a.pool, b.pool, strict=True):
        if ty == vm.ATTN:
            for ta, tb in zip(kv(pa, rows_a), kv(pb, rows_b), strict=True):
                torch.testing.assert_close(ta.cpu(), tb.cpu(), rtol=rtol, atol=atol)
        else:
            for name in ("conv", "rec"):
                torch.testing.assert_close(pa[name][lane].cpu(), pb[name][lane].cpu(), rtol=rtol, atol=atol)
    for ta, tb in zip(kv(a.mtp.pool, rows_a), kv(b.mtp.pool, rows_b), strict=True):
        torch.testing.assert_close(ta.cpu(), tb.cpu(), rtol=rtol, atol=atol)
    torch.testing.assert_close(a.cached_hidden(lane).cpu(), b.cached_hidden(lane).cpu(), rtol=rtol, atol=atol)
