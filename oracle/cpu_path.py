"""The reference engine's CPU MoE path restated in torch fp32, for bench.py's `cpu_baseline` leg
only. TEST/BENCH INFRASTRUCTURE ONLY (see oracle/__init__).

Follows `Model._routed_grouped` (`model.py:3170-3236`) with `expert_weights_batch`
(`model.py:2690-2704`) and `mxfp4.dequant_mxfp4` (`mxfp4.py:32-51`): drop unowned
assignments, stable sort by expert, `unique_consecutive` counts, pad each active expert's tokens
to the busiest group (a host read of `counts.max()`), dequantise the active experts, two `bmm`
with SiLU(gate) * up between them, weighted `index_add_`. Experts are processed in chunks of
`chunk` (the dense fp32 copy of ~351 experts would be 17.6 GB). The router chain is
`softmax(fp32) -> topk -> renormalise` (`model.py:2840-2843`).

Pinning: tests/test_oracle_cpu_path.py checks it against oracle.moe_ref.reference_moe.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

_FP4 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0])  # fmt: skip


def dequant(packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    lo = _FP4[(packed & 0xF).int()]
    hi = _FP4[(packed >> 4).int()]
    v = torch.stack([lo, hi], -1).flatten(-2)
    *lead, k = v.shape
    s = torch.exp2(scale.float() - 127.0).unsqueeze(-1)
    return (v.reshape(*lead, k // 32, 32) * s).reshape(*lead, k)


def route(routing: torch.Tensor, experts_out: int, top_k: int):
    probs = routing[:, :experts_out].softmax(-1, dtype=torch.float)
    top_w, top_i = probs.topk(top_k, dim=-1)
    return top_w / top_w.sum(-1, keepdim=True), top_i


def routed_grouped(h: torch.Tensor, experts: dict, top_i: torch.Tensor, top_w: torch.Tensor,
                   expert_range: tuple[int, int], chunk: int = 16) -> torch.Tensor:
    """fp32 CPU routed-expert output `[T, hidden]` (`model.py:3170-3236`)."""
    t = h.shape[0]
    lo, hi = expert_range
    top_k = top_i.shape[1]
    flat_e, flat_w = top_i.reshape(-1), top_w.reshape(-1).float()
    flat_t = torch.arange(t).repeat_interleave(top_k)
    mine = (flat_e >= lo) & (flat_e < hi) & (flat_w != 0)
    flat_e, flat_w, flat_t = flat_e[mine] - lo, flat_w[mine], flat_t[mine]
    out = torch.zeros(t, experts["down"].shape[1], dtype=torch.float32)
    if flat_e.numel() == 0:
        return out
    order = torch.argsort(flat_e, stable=True)
    se, st, sw = flat_e[order], flat_t[order], flat_w[order]
    active, counts = torch.unique_consecutive(se, return_counts=True)
    hf = h.float()
    starts = counts.cumsum(0) - counts
    for c0 in range(0, active.numel(), chunk):
        act = active[c0 : c0 + chunk]
        cnt = counts[c0 : c0 + chunk]
        st0 = starts[c0 : c0 + chunk]
        n_act, max_count = act.numel(), int(cnt.max())
        row = torch.repeat_interleave(torch.arange(n_act), cnt)
        pos = torch.cat([torch.arange(int(c)) for c in cnt])
        sel = torch.cat([torch.arange(int(s), int(s) + int(c)) for s, c in zip(st0, cnt)])
        tok_idx = torch.zeros(n_act, max_count, dtype=torch.long)
        w_pad = torch.zeros(n_act, max_count)
        mask = torch.zeros(n_act, max_count, dtype=torch.bool)
        tok_idx[row, pos] = st[sel]
        w_pad[row, pos] = sw[sel]
        mask[row, pos] = True
        gu = dequant(experts["gate_up"][act], experts["gate_up_scale"][act])
        dn = dequant(experts["down"][act], experts["down_scale"][act])
        gate, up = torch.bmm(hf[tok_idx], gu.transpose(1, 2)).chunk(2, dim=-1)
        y = torch.bmm(F.silu(gate) * up, dn.transpose(1, 2))
        out.index_add_(0, tok_idx[mask], y[mask] * w_pad[mask, None])
    return out
