"""Routed MXFP4 MoE, dequantise-then-matmul, restated in numpy. TEST INFRASTRUCTURE ONLY.

Reference: `mxfp4_gemv.reference_moe` (`mxfp4_gemv.py:1613-1651`), which is the arithmetic of
`Model._routed_grouped` (`model.py:3170-3236`): keep the assignments that are owned
(`lo <= e < hi`) and have a nonzero weight, dequantise each kept assignment's expert, two
matmuls with SiLU(gate) * up between them, then `out[t] += w * y`. The output is rounded to the
activation dtype at the end (`mxfp4_gemv.py:1651`). Assignment `a` belongs to token
`a // top_k` (`mxfp4_gemv.py:24-40`). `gate_up` rows are `cat[gate; up]` (`model.py:791`).

Accumulation is float64, so this is the exact answer up to the final rounding; the north-star
bar (rel-L2 <= 2e-3) and the reference's own bars are measured against it.

`dense_moe` is the same arithmetic over dense bf16 experts (the MTP layer of the real
checkpoint, `mtp_dense_moe.py:359-745`).

Pinning (tests/test_oracle_moe.py):
- against a brute-force per-element triple loop on tiny shapes (no matmul, no vectorised
  dequant), so a transposed operand or a swapped gate/up half fails;
- the invariants the reference tests state: zero-weight tokens give exact zeros
  (`test_mxfp4_fused_gemv.py:293-316`), shards sum to the whole (`:261-290`), assignments
  outside `expert_range` are dropped;
- `dense_moe`: against its own element-by-element loop, and equal to `reference_moe` when its
  dense experts are the dequantised MXFP4 experts; inactive tokens give exact zeros.
"""

from __future__ import annotations

import numpy as np

from .mxfp4_ref import dequant_mxfp4, dequant_mxfp4_kernel


def silu(v: np.ndarray) -> np.ndarray:
    """x * sigmoid(x), overflow-safe in float64."""
    v = np.asarray(v, dtype=np.float64)
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-v))


def live_mask(a_expert: np.ndarray, a_weight: np.ndarray, lo: int, hi: int) -> np.ndarray:
    """Owned and nonzero weight (`mxfp4_gemv.py:1640`, `:474`)."""
    a_expert = np.asarray(a_expert)
    return (a_expert >= lo) & (a_expert < hi) & (np.asarray(a_weight) != 0)


def reference_moe(
    x: np.ndarray,
    experts: dict,
    a_expert: np.ndarray,
    a_weight: np.ndarray,
    top_k: int,
    expert_range: tuple[int, int],
    *,
    kernel_scales: bool = False,
    chunk: int = 16,
) -> np.ndarray:
    """fp64-accumulated routed MoE, returned as float32 `[T, hidden]` (not yet rounded to the
    activation dtype; callers round with `bf16_round` where the reference does).

    `experts` holds numpy `gate_up [E, 2I, H/2]`, `gate_up_scale [E, 2I, H/32]`,
    `down [E, H, I/2]`, `down_scale [E, H, I/32]` for the local experts `[lo, hi)`.
    `kernel_scales` selects the kernels' scale-0 -> +0.0 convention (`dequant_mxfp4_kernel`).
    """
    deq = dequant_mxfp4_kernel if kernel_scales else dequant_mxfp4
    lo, hi = expert_range
    x = np.asarray(x, dtype=np.float64)
    a_expert = np.asarray(a_expert).reshape(-1).astype(np.int64)
    a_weight = np.asarray(a_weight, dtype=np.float64).reshape(-1)
    hidden = experts["down"].shape[1]
    inter = experts["gate_up"].shape[1] // 2
    out = np.zeros((x.shape[0], hidden), dtype=np.float64)
    keep = np.nonzero(live_mask(a_expert, a_weight, lo, hi))[0]
    # Group by expert so each expert is dequantised once per chunk of distinct experts.
    local = a_expert[keep] - lo
    order = np.argsort(local, kind="stable")
    keep, local = keep[order], local[order]
    uniq = np.unique(local)
    for start in range(0, uniq.size, chunk):
        for e in uniq[start : start + chunk]:
            sel = keep[local == e]
            gu = deq(experts["gate_up"][e], experts["gate_up_scale"][e]).astype(np.float64)
            dn = deq(experts["down"][e], experts["down_scale"][e]).astype(np.float64)
            tok = sel // top_k
            h = x[tok] @ gu.T  # [n, 2I]
            act = silu(h[:, :inter]) * h[:, inter:]
            y = act @ dn.T  # [n, H]
            np.add.at(out, tok, y * a_weight[sel, None])
    return out.astype(np.float32)


def dense_moe(
    x: np.ndarray,
    experts: dict,
    a_expert: np.ndarray,
    a_weight: np.ndarray,
    top_k: int,
    expert_range: tuple[int, int],
    active: np.ndarray | None = None,
) -> np.ndarray:
    """The routed MoE over dense (bf16-valued) experts, fp64-accumulated, float32 `[T, H]`:
    the contract of the MTP layer's `mtp_dense_moe.fused_moe` / `grouped_moe`
    (`mtp_dense_moe.py:359-745`). `experts` holds `gate_up [E, 2I, H]` (gate rows, then up)
    and `down [E, H, I]` for the local experts `[lo, hi)`. Live assignments are owned, have a
    nonzero weight and, when `active` `[T]` is given, an active token
    (`mtp_dense_moe.py:600-610`); out[t] = sum over live j of w_j * down(silu(g) * u)."""
    lo, hi = expert_range
    x = np.asarray(x, dtype=np.float64)
    a_expert = np.asarray(a_expert).reshape(-1).astype(np.int64)
    a_weight = np.asarray(a_weight, dtype=np.float64).reshape(-1)
    if active is not None:
        a_weight = a_weight * np.repeat(np.asarray(active, dtype=bool), top_k)
    inter = experts["gate_up"].shape[1] // 2
    out = np.zeros((x.shape[0], experts["down"].shape[1]), dtype=np.float64)
    keep = np.nonzero(live_mask(a_expert, a_weight, lo, hi))[0]
    for e in np.unique(a_expert[keep] - lo):
        sel = keep[a_expert[keep] - lo == e]
        tok = sel // top_k
        h = x[tok] @ np.asarray(experts["gate_up"][e], dtype=np.float64).T
        act = silu(h[:, :inter]) * h[:, inter:]
        y = act @ np.asarray(experts["down"][e], dtype=np.float64).T
        np.add.at(out, tok, y * a_weight[sel, None])
    return out.astype(np.float32)


def brute_force_dense_moe(x, experts, a_expert, a_weight, top_k, expert_range) -> np.ndarray:
    """`dense_moe` element by element, for tiny shapes only."""
    lo, hi = expert_range
    inter = experts["gate_up"].shape[1] // 2
    out = np.zeros((x.shape[0], experts["down"].shape[1]))
    for a in range(len(a_expert)):
        e, w = int(a_expert[a]), float(a_weight[a])
        if not (lo <= e < hi) or w == 0.0:
            continue
        t, gu, dn = a // top_k, experts["gate_up"][e - lo], experts["down"][e - lo]
        act = []
        for n in range(inter):
            g = sum(float(gu[n, k]) * float(x[t, k]) for k in range(x.shape[1]))
            u = sum(float(gu[inter + n, k]) * float(x[t, k]) for k in range(x.shape[1]))
            act.append(g / (1.0 + np.exp(-g)) * u)
        for n in range(out.shape[1]):
            out[t, n] += w * sum(float(dn[n, k]) * act[k] for k in range(inter))
    return out


def brute_force_moe(x, experts, a_expert, a_weight, top_k, expert_range) -> np.ndarray:
    """Element-by-element triple loop straight from the formula, for tiny shapes only."""
    from .mxfp4_ref import FP4_VALUES, e8m0_torch

    lo, hi = expert_range
    t_count, hidden = x.shape[0], experts["down"].shape[1]
    inter = experts["gate_up"].shape[1] // 2
    kin = x.shape[1]

    def w_at(packed, scale, n, k):
        byte = int(packed[n, k // 2])
        code = (byte >> 4) if (k & 1) else (byte & 0xF)
        return float(FP4_VALUES[code]) * float(e8m0_torch(np.array(scale[n, k // 32])))

    out = np.zeros((t_count, hidden))
    for a in range(len(a_expert)):
        e, w = int(a_expert[a]), float(a_weight[a])
        if not (lo <= e < hi) or w == 0.0:
            continue
        t = a // top_k
        le = e - lo
        gq, gs = experts["gate_up"][le], experts["gate_up_scale"][le]
        dq, ds = experts["down"][le], experts["down_scale"][le]
        act = []
        for n in range(inter):
            g = sum(w_at(gq, gs, n, k) * float(x[t, k]) for k in range(kin))
            u = sum(w_at(gq, gs, inter + n, k) * float(x[t, k]) for k in range(kin))
            act.append(g / (1.0 + np.exp(-g)) * u)
        for n in range(hidden):
            out[t, n] += w * sum(w_at(dq, ds, n, k) * act[k] for k in range(inter))
    return out


def relative_error(got: np.ndarray, want: np.ndarray) -> float:
    """Max elementwise difference over the largest oracle magnitude — the reference tests'
    metric (`test_mxfp4_fused_gemv.py:110-113`)."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    scale = max(np.abs(want).max(initial=0.0), 1e-30)
    return float(np.abs(got - want).max(initial=0.0) / scale)


def rel_l2(got: np.ndarray, want: np.ndarray) -> float:
    """||got - want||_2 / ||want||_2 — the north-star MoE metric."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    den = np.linalg.norm(want)
    return float(np.linalg.norm(got - want) / max(den, 1e-300))
