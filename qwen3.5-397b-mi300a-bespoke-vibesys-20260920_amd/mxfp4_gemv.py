"""Routed-expert MXFP4 MoE — the reference's `mxfp4_gemv` interface (`mxfp4_gemv.py`) on the
gfx950 HIP kernels of `libmtpk.so`.

`fused_moe` keeps the reference signature (`mxfp4_gemv.py:1020-1032`) and contract: the
routing is the flat `(a_expert, a_weight)` of `a = t * top_k + j`, assignments outside
`expert_range` or with zero weight are dropped on the GPU, `out` is written in place and
returned, a wrong routing length or a non-contiguous input raises `ValueError`
(`mxfp4_gemv.py:1062-1072`), the launch shape depends only on `(T, top_k)` and nothing is read
back to the host, so the call is capturable.

The kernels (csrc/mtpk_moe.hip) read the packed nibbles and e8m0 scales in the `load_experts`
layout and decode them in registers with gfx950's fp4 -> bf16 converter; the products run on
bf16 MFMA with fp32 accumulation. Activations and the gated intermediate are carried as exact
sums of bf16 planes (bf16 x: one plane, intermediate hi + lo; fp32 x: three planes each), so
the result is fp32-accurate rather than bf16-rounded in the middle.

`SEED_FUSED_MOE=0` makes `available` return False: the A/B switch of the reference
(`mxfp4_gemv.py:188-198`); callers then take their torch path (`reference_moe` here).
"""

from __future__ import annotations

import os
from collections.abc import Callable
from dataclasses import dataclass

import torch

import _mtpk

BLOCK_SCALE = 32
"""Elements per e8m0 scale (OCP MXFP4 group)."""

UNIT_TOKENS = _mtpk.UNIT_TOKENS
"""Assignments per work unit: one MFMA N tile of 16 token columns."""

GROUPED_MIN_PER_EXPERT = int(os.environ.get("SEED_MOE_GROUPED_MIN", "3"))


def available(device: torch.device) -> bool:
    """True when `fused_moe` runs for tensors on `device`.

    False for CPU tensors and under `SEED_FUSED_MOE=0`. On a HIP device it loads the library
    and raises if it is missing: a device caller never falls back silently.
    """
    if os.environ.get("SEED_FUSED_MOE", "1") == "0":
        return False
    if device.type != "cuda":
        return False
    _mtpk.lib()
    return True


def perm_lut(device: torch.device) -> bool:
    """Reference knob (`mxfp4_gemv.py:154-173`) for its byte-table decode. These kernels use
    the hardware fp4 converter instead, so there is no table path to select: always False."""
    return False


def use_grouped(assignments: int, experts: int) -> bool:
    """The reference's grouped-kernel threshold (`mxfp4_gemv.py:802-820`), kept for callers
    that read it. The HIP path groups by expert at every width, so it does not branch on it."""
    return assignments >= GROUPED_MIN_PER_EXPERT * max(experts, 1)


def _validate(x, experts, routing, top_k):
    a_expert, a_weight = routing
    tokens = x.shape[0]
    assignments = tokens * top_k
    if a_expert.shape != (assignments,) or a_weight.shape != (assignments,):
        raise ValueError(
            f"routing must be two [{assignments}] tensors, got "
            f"{tuple(a_expert.shape)} and {tuple(a_weight.shape)}"
        )
    for name, tensor in (("x", x), ("a_expert", a_expert), ("a_weight", a_weight)):
        if not tensor.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    for name in ("gate_up", "gate_up_scale", "down", "down_scale"):
        if name not in experts:
            raise ValueError(f"experts[{name!r}] is missing (MXFP4 layout required)")
        if not experts[name].is_contiguous():
            raise ValueError(f"experts[{name!r}] must be contiguous")
    if top_k > _mtpk.MAX_TOP_K:
        raise ValueError(f"top_k {top_k} exceeds {_mtpk.MAX_TOP_K}")


def _workspace(device: torch.device, nbytes: int, scratch: torch.Tensor | None) -> torch.Tensor:
    if (
        scratch is not None
        and scratch.device == device
        and scratch.is_contiguous()
        and scratch.numel() * scratch.element_size() >= nbytes
        and scratch.data_ptr() % 256 == 0
    ):
        return scratch
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def fused_moe(
    x: torch.Tensor,
    experts: dict,
    routing: tuple[torch.Tensor, torch.Tensor],
    top_k: int,
    expert_range: tuple[int, int],
    *,
    out: torch.Tensor | None = None,
    inter: torch.Tensor | None = None,
    order: torch.Tensor | None = None,
    grouped: bool | None = None,
    total_experts: int | None = None,
    shared: torch.Tensor | None = None,
    shared_gate: torch.Tensor | None = None,
) -> torch.Tensor:
    """Routed-expert output `[T, hidden]` for tokens `x` `[T, hidden]`, never dequantising to HBM.

    With `shared` `[T, hidden]` and `shared_gate` `[T, 1]` (the shared-gate column of the
    router GEMM output, any row stride) the layer's shared-expert term is added in the same
    launch: `out = routed + sigmoid(shared_gate) * shared` (`model.py:2871-2872`,
    `bw_combine_glue` `mxfp4_gemv.py:2266-2312`), with the unfused ops' rounding points.

    `inter` is optional caller scratch: used as the kernels' workspace when it is at least
    `workspace_bytes(...)` bytes, contiguous and 256-byte aligned (the reference sizes it
    `[max_batch * top_k, intermediate]`; pass `moe_scratch(...)` for a reusable one).
    `order`, `grouped` and `total_experts` are accepted for signature compatibility: the work
    list groups assignments by expert at every width, so there is nothing for them to select.
    """
    _validate(x, experts, routing, top_k)
    a_expert, a_weight = routing
    lo, hi = expert_range
    device = _mtpk.require_device(x, a_expert, a_weight, experts["gate_up"])
    tokens, hidden = x.shape
    gate_up, down = experts["gate_up"], experts["down"]
    local = gate_up.shape[0]
    intermediate = gate_up.shape[1] // 2
    if hi - lo != local:
        raise ValueError(f"expert_range {expert_range} does not match {local} local experts")
    if down.shape[1] != hidden or gate_up.shape[2] * 2 != hidden:
        raise ValueError("expert payload shapes do not match x")
    if out is None:
        out = torch.empty(tokens, hidden, dtype=x.dtype, device=device)
    elif out.shape != (tokens, hidden) or out.dtype != x.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous [T, hidden] tensor of x's dtype")
    lib = _mtpk.lib()
    xcode = _mtpk.float_code(x.dtype)
    nbytes = lib.mtpk_moe_workspace_bytes(tokens, top_k, local, intermediate, hidden, xcode)
    ws = _workspace(device, nbytes, inter)
    sh_ptr = gate_ptr = None
    sh_code = gate_code = gate_stride = 0
    if shared is not None:
        if shared_gate is None or shared.shape != (tokens, hidden) or not shared.is_contiguous():
            raise ValueError("shared must be a contiguous [T, hidden] tensor, with shared_gate")
        if shared_gate.dim() != 2 or shared_gate.shape[0] != tokens:
            raise ValueError("shared_gate must be [T, 1] (any row stride)")
        sh_ptr, sh_code = shared.data_ptr(), _mtpk.float_code(shared.dtype)
        gate_ptr, gate_code, gate_stride = (shared_gate.data_ptr(), _mtpk.float_code(shared_gate.dtype),
                                            shared_gate.stride(0))
    _mtpk.check(
        lib.mtpk_fused_moe_shared(
            x.data_ptr(), xcode, tokens, hidden,
            gate_up.data_ptr(), experts["gate_up_scale"].data_ptr(),
            down.data_ptr(), experts["down_scale"].data_ptr(), local, intermediate,
            a_expert.data_ptr(), _mtpk.index_code(a_expert.dtype),
            a_weight.data_ptr(), _mtpk.float_code(a_weight.dtype),
            top_k, lo, hi, sh_ptr, sh_code, gate_ptr, gate_code, gate_stride,
            ws.data_ptr(), ws.numel() * ws.element_size(), out.data_ptr(), _mtpk.stream_of(device),
        ),
        "mtpk_fused_moe_shared",
    )  # fmt: skip
    return out


def workspace_bytes(tokens: int, top_k: int, local_experts: int, intermediate: int, hidden: int,
                    dtype: torch.dtype = torch.bfloat16) -> int:
    """Bytes of scratch `fused_moe` needs at these sizes (`mtpk_moe_workspace_bytes`)."""
    return int(
        _mtpk.lib().mtpk_moe_workspace_bytes(
            tokens, top_k, local_experts, intermediate, hidden, _mtpk.float_code(dtype)
        )
    )


def moe_scratch(max_tokens: int, top_k: int, local_experts: int, intermediate: int, hidden: int,
                device: torch.device, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """A reusable workspace for every call of up to `max_tokens` tokens (pass as `inter=`)."""
    n = workspace_bytes(max_tokens, top_k, local_experts, intermediate, hidden, dtype)
    return torch.empty(n, dtype=torch.uint8, device=device)


class MoeLayerRunner:
    """Static buffers for one routed-MoE shape `(tokens, top_k, experts, I, H)` and its kernels
    launched one by one on the current stream: prep, gate_up, down, combine, or for batches of
    at most `mtpk_moe_direct_max_tokens()` tokens the direct pair gate_up, down + combine.

    Nothing is allocated per call, so a call can be captured into a HIP graph and replayed;
    `events`, when given, is a dict whose `torch.cuda.Event` pairs are recorded around each
    kernel (`"gate_up"`, `"down"`) on the launch stream. bf16 activations only.
    """

    def __init__(self, tokens: int, top_k: int, local_experts: int, intermediate: int,
                 hidden: int, device: torch.device) -> None:
        lib = _mtpk.lib()
        self.tokens, self.top_k, self.local = tokens, top_k, local_experts
        self.inter_dim, self.hidden = intermediate, hidden
        a = tokens * top_k
        self.assignments = a
        self.u_max = int(lib.mtpk_moe_max_units(a, local_experts))
        self.sorted = torch.empty(max(a, 1), dtype=torch.int32, device=device)
        self.unit = torch.empty(max(3 * self.u_max, 3), dtype=torch.int32, device=device)
        self.n_units = torch.zeros(1, dtype=torch.int32, device=device)
        self.inter = torch.empty(2 * a * intermediate, dtype=torch.bfloat16, device=device)
        self.direct = tokens <= int(lib.mtpk_moe_direct_max_tokens())
        self.y = torch.empty(a * hidden, dtype=torch.float32, device=device)

    def run(self, x: torch.Tensor, experts: dict, a_expert: torch.Tensor, a_weight: torch.Tensor,
            expert_range: tuple[int, int], out: torch.Tensor, events: dict | None = None) -> torch.Tensor:
        lib = _mtpk.lib()
        lo, hi = expert_range
        st = _mtpk.stream_of(x.device)
        if x.dtype != torch.bfloat16 or x.shape != (self.tokens, self.hidden):
            raise ValueError("x must be bf16 [tokens, hidden] of the runner's shape")
        ec, wc = _mtpk.index_code(a_expert.dtype), _mtpk.float_code(a_weight.dtype)
        if self.direct:
            if events:
                events["gate_up"][0].record()
            _mtpk.check(lib.mtpk_moe_gate_up_direct(
                x.data_ptr(), 1, self.tokens, self.hidden, experts["gate_up"].data_ptr(),
                experts["gate_up_scale"].data_ptr(), self.local, self.inter_dim,
                a_expert.data_ptr(), ec, a_weight.data_ptr(), wc, self.top_k, lo, hi,
                self.inter.data_ptr(), 2, st), "mtpk_moe_gate_up_direct")
            if events:
                events["gate_up"][1].record()
                events["down"][0].record()
            _mtpk.check(lib.mtpk_moe_down_combine(
                self.inter.data_ptr(), 2, self.inter_dim, experts["down"].data_ptr(),
                experts["down_scale"].data_ptr(), self.local, self.hidden, a_expert.data_ptr(),
                ec, a_weight.data_ptr(), wc, self.tokens, self.top_k, lo, hi, out.data_ptr(),
                _mtpk.float_code(out.dtype), st), "mtpk_moe_down_combine")
            if events:
                events["down"][1].record()
            return out
        _mtpk.check(lib.mtpk_moe_prep(a_expert.data_ptr(), ec, a_weight.data_ptr(), wc,
                                      self.assignments, lo, hi, self.sorted.data_ptr(),
                                      self.unit.data_ptr(), self.u_max, self.n_units.data_ptr(), st),
                    "mtpk_moe_prep")
        if events:
            events["gate_up"][0].record()
        _mtpk.check(lib.mtpk_moe_gate_up(
            x.data_ptr(), 1, self.tokens, self.hidden, experts["gate_up"].data_ptr(),
            experts["gate_up_scale"].data_ptr(), self.local, self.inter_dim,
            self.sorted.data_ptr(), self.unit.data_ptr(), self.n_units.data_ptr(), self.u_max,
            self.top_k, self.inter.data_ptr(), 2, self.assignments, st), "mtpk_moe_gate_up")
        if events:
            events["gate_up"][1].record()
            events["down"][0].record()
        _mtpk.check(lib.mtpk_moe_down(
            self.inter.data_ptr(), 2, self.assignments, self.inter_dim, experts["down"].data_ptr(),
            experts["down_scale"].data_ptr(), self.local, self.hidden, self.sorted.data_ptr(),
            self.unit.data_ptr(), self.n_units.data_ptr(), self.u_max, self.y.data_ptr(), st),
            "mtpk_moe_down")
        if events:
            events["down"][1].record()
        _mtpk.check(lib.mtpk_moe_combine(
            self.y.data_ptr(), a_expert.data_ptr(), ec, a_weight.data_ptr(), wc, self.tokens,
            self.top_k, self.hidden, lo, hi, out.data_ptr(), _mtpk.float_code(out.dtype), st),
            "mtpk_moe_combine")
        return out


# ---------------------------------------------------------------- staged pieces


@dataclass
class BwPlan:
    """Work list of one MoE call (`mxfp4_gemv.BwPlan`'s role): expert-grouped assignment ids,
    units `(local expert, first position, count <= 16)` and their device-side count."""

    sorted: torch.Tensor
    unit: torch.Tensor
    n_units: torch.Tensor
    u_max: int


def bw_prep(a_expert: torch.Tensor, a_weight: torch.Tensor, expert_range: tuple[int, int]) -> BwPlan:
    """Counting sort of live assignments by local expert (`mtpk_moe_prep`); no host sync."""
    device = _mtpk.require_device(a_expert, a_weight)
    lo, hi = expert_range
    a = a_expert.numel()
    lib = _mtpk.lib()
    u_max = int(lib.mtpk_moe_max_units(a, hi - lo))
    sorted_ = torch.full((max(a, 1),), -1, dtype=torch.int32, device=device)
    unit = torch.zeros(max(3 * u_max, 3), dtype=torch.int32, device=device)
    n_units = torch.zeros(1, dtype=torch.int32, device=device)
    _mtpk.check(
        lib.mtpk_moe_prep(
            a_expert.data_ptr(), _mtpk.index_code(a_expert.dtype),
            a_weight.data_ptr(), _mtpk.float_code(a_weight.dtype),
            a, lo, hi, sorted_.data_ptr(), unit.data_ptr(), u_max, n_units.data_ptr(),
            _mtpk.stream_of(device),
        ),
        "mtpk_moe_prep",
    )  # fmt: skip
    return BwPlan(sorted_, unit, n_units, u_max)


def bw_combine(y: torch.Tensor, routing: tuple[torch.Tensor, torch.Tensor], top_k: int,
               expert_range: tuple[int, int], out: torch.Tensor) -> torch.Tensor:
    """`out[t] = sum_j w[t, j] * y[t*top_k + j]` over live assignments, fixed j order."""
    a_expert, a_weight = routing
    device = _mtpk.require_device(y, a_expert, a_weight, out)
    lo, hi = expert_range
    tokens, hidden = out.shape
    _mtpk.check(
        _mtpk.lib().mtpk_moe_combine(
            y.data_ptr(), a_expert.data_ptr(), _mtpk.index_code(a_expert.dtype),
            a_weight.data_ptr(), _mtpk.float_code(a_weight.dtype), tokens, top_k, hidden,
            lo, hi, out.data_ptr(), _mtpk.float_code(out.dtype), _mtpk.stream_of(device),
        ),
        "mtpk_moe_combine",
    )  # fmt: skip
    return out


def expert_sorted_order(a_expert: torch.Tensor) -> torch.Tensor:
    """`argsort(a_expert, stable=True)` as int32 (`mxfp4_gemv.py:874-887`)."""
    return torch.argsort(a_expert, stable=True).to(torch.int32)


def fused_expert_order(a_expert: torch.Tensor, num_experts: int, *, cursor=None) -> torch.Tensor:
    """Expert-grouping permutation from the HIP counting sort: set-identical to
    `expert_sorted_order` per expert (`mxfp4_gemv.py:990-1017`)."""
    ones = torch.ones(a_expert.numel(), dtype=torch.float32, device=a_expert.device)
    return bw_prep(a_expert, ones, (0, num_experts)).sorted[: a_expert.numel()]


def grouped_block_count(assignments: int, experts: int, block_m: int) -> int:
    """Upper bound on `align_blocks`' blocks (`mxfp4_gemv.py:734-742`)."""
    return -(-assignments // block_m) + experts + 1


def align_blocks(a_expert: torch.Tensor, a_weight: torch.Tensor, expert_range: tuple[int, int],
                 block_m: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-expert `block_m` blocks with a fixed-shape result (`mxfp4_gemv.py:745-800`):
    `slot_assign[b*block_m + i]` = assignment id or -1, `block_expert[b]` = local expert or the
    sentinel `experts` for dropped assignments. Torch ops, no host sync."""
    lo, hi = expert_range
    experts = hi - lo
    n = a_expert.numel()
    device = a_expert.device
    live = (a_expert >= lo) & (a_expert < hi) & (a_weight != 0)
    bucket = torch.where(live, a_expert.to(torch.long) - lo, experts)
    counts = torch.zeros(experts + 1, dtype=torch.long, device=device)
    counts.scatter_add_(0, bucket, torch.ones_like(bucket))
    blocks = -(-counts // block_m)
    block_start = blocks.cumsum(0) - blocks
    order = torch.argsort(bucket, stable=True)
    sorted_bucket = bucket[order]
    first = counts.cumsum(0) - counts
    rank = torch.arange(n, device=device) - first[sorted_bucket]
    slot = block_start[sorted_bucket] * block_m + rank
    n_blocks = grouped_block_count(n, experts, block_m)
    slot_assign = torch.full((n_blocks * block_m,), -1, dtype=torch.int32, device=device)
    slot_assign.scatter_(0, slot, order.to(torch.int32))
    marks = torch.full((n_blocks + 1,), -1, dtype=torch.long, device=device)
    marks.scatter_reduce_(0, block_start.clamp(max=n_blocks), torch.arange(experts + 1, device=device),
                          reduce="amax")
    block_expert = marks.cummax(0).values[:n_blocks].to(torch.int32)
    return slot_assign, block_expert


def reference_moe(
    x: torch.Tensor,
    experts: dict,
    routing: tuple[torch.Tensor, torch.Tensor],
    top_k: int,
    expert_range: tuple[int, int],
    dequant: Callable[[torch.Tensor, torch.Tensor, torch.dtype], torch.Tensor],
    compute_dtype: torch.dtype | None = None,
    chunk: int = 16,
) -> torch.Tensor:
    """Dequantise-then-`bmm`, the slow readable spelling (`mxfp4_gemv.py:1613-1651`): the torch
    path selected by `SEED_FUSED_MOE=0` and the arithmetic `fused_moe` reformulates."""
    a_expert, a_weight = routing
    lo, hi = expert_range
    dt = compute_dtype or x.dtype
    keep = ((a_expert >= lo) & (a_expert < hi) & (a_weight != 0)).nonzero(as_tuple=True)[0]
    out = torch.zeros(x.shape[0], experts["down"].shape[1], dtype=dt, device=x.device)
    for start in range(0, keep.numel(), chunk):
        part = keep[start : start + chunk]
        local = (a_expert[part] - lo).to(torch.long)
        token = (part // top_k).to(torch.long)
        gate_up_w = dequant(experts["gate_up"][local], experts["gate_up_scale"][local], dt)
        down_w = dequant(experts["down"][local], experts["down_scale"][local], dt)
        gate, up = torch.bmm(x.to(dt)[token][:, None], gate_up_w.transpose(1, 2).contiguous()).chunk(2, -1)
        y = torch.bmm(torch.nn.functional.silu(gate) * up, down_w.transpose(1, 2).contiguous())[:, 0]
        out.index_add_(0, token, y * a_weight[part, None].to(dt))
    return out.to(x.dtype)
