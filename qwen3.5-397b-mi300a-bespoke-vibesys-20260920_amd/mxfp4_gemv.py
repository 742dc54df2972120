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

import functools

import os
from collections.abc import Callable

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


_SCALE_CHECK_ATTR = "_mtpk_decode_exact"
"""Attribute `supports` sets on the two scale tensors it checked: True when the in-register
decode reproduces them, False when it refused them. It lives and dies with those tensor objects,
so a freed address that a later tensor reuses inherits nothing, and a copy is checked anew."""


def bw_scales_ok(experts: dict) -> bool:
    """Precondition of the in-register decode (interface of `mxfp4_gemv.py:1761-1776`): no
    32-element block with e8m0 scale 255 holds a nonzero-magnitude code.

    The hardware fp4 converter the kernels decode with reproduces the pinned decode bit for bit
    at every other scale (byte 0 as +-0.0 through the code mask, 1..254 as they are). At 255,
    the OCP NaN scale, it returns NaN where the pinned decode gives +-inf for nonzero codes
    (zero codes are NaN in both). One device scan of the scales (the packed bytes are read only
    under scale 255) and one host sync: call at load time, never inside graph capture.
    """
    lib = _mtpk.lib()
    device = _mtpk.require_device(experts["gate_up"], experts["down"])
    bad = torch.zeros(2, dtype=torch.int32, device=device)
    st = _mtpk.stream_of(device)
    for i, (w, s) in enumerate((("gate_up", "gate_up_scale"), ("down", "down_scale"))):
        packed, scale = experts[w], experts[s]
        if not (packed.is_contiguous() and scale.is_contiguous()) or packed.numel() != 16 * scale.numel():
            raise ValueError(f"experts[{w!r}] / [{s!r}] are not a contiguous MXFP4 pair")
        _mtpk.check(lib.mtpk_scale_scan(packed.data_ptr(), scale.data_ptr(), scale.numel(),
                                        bad[i:].data_ptr(), st), "mtpk_scale_scan")
    return not bool(bad.any().item())


def supports(experts: dict) -> bool:
    """Load-time check that `fused_moe` computes these experts exactly (the role of
    `moe_hip.supports`, `moe_hip.py:204-215`): contiguous MXFP4 payloads of matching shapes
    and `bw_scales_ok`. The verdict is kept on the two scale tensors, and `fused_moe` /
    `fused_moe_layer` then raise `ValueError` for refused ones instead of decoding them.
    `weights.load_experts` runs it for every MXFP4 shard it loads onto a device, and the first
    `fused_moe` call that meets scale tensors with no verdict runs it then (outside graph
    capture; a captured call on unchecked tensors cannot sync and is not checked). One host sync."""
    gu, gus, dn, dns = (experts[k] for k in ("gate_up", "gate_up_scale", "down", "down_scale"))
    shapes = (
        gu.dim() == 3 and dn.dim() == 3 and gu.shape[1] % 2 == 0
        and gus.shape == (*gu.shape[:2], gu.shape[2] * 2 // BLOCK_SCALE)
        and dns.shape == (*dn.shape[:2], dn.shape[2] * 2 // BLOCK_SCALE)
        and dn.shape[0] == gu.shape[0] and dn.shape[1] == gu.shape[2] * 2
        and dn.shape[2] * 2 == gu.shape[1] // 2
        and all(t.is_contiguous() for t in (gu, gus, dn, dns))
    )  # fmt: skip
    ok = bool(shapes and bw_scales_ok(experts))
    setattr(gus, _SCALE_CHECK_ATTR, ok)
    setattr(dns, _SCALE_CHECK_ATTR, ok)
    return ok


def require_supported(experts: dict, what: str) -> None:
    """`supports(experts)`, raising `ValueError` (naming `what`) on a refusal: the boot-time
    form for loaders, so a checkpoint the kernels cannot decode exactly fails at load rather
    than at its first MoE call."""
    if not supports(experts):
        raise ValueError(
            f"{what}: the MXFP4 experts fail supports(): a 32-element block with e8m0 scale 255 "
            "holds a nonzero code (or the payloads are not contiguous MXFP4 pairs of matching "
            "shapes), which the fused kernels cannot decode exactly; SEED_FUSED_MOE=0 selects "
            "the torch dequant path"
        )


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
    gus, dns = experts["gate_up_scale"], experts["down_scale"]
    verdict = (getattr(gus, _SCALE_CHECK_ATTR, None), getattr(dns, _SCALE_CHECK_ATTR, None))
    if None in verdict and x.device.type == "cuda" and not torch.cuda.is_current_stream_capturing():
        # scale tensors no loader checked (a copy, a hand-built dict): scanned once, here
        supports(experts)
        verdict = (getattr(gus, _SCALE_CHECK_ATTR), getattr(dns, _SCALE_CHECK_ATTR))
    if False in verdict:
        raise ValueError("these experts failed supports(): a block with e8m0 scale 255 holds a "
                         "nonzero code, which the in-register decode cannot reproduce")


_SHARED_WS: dict[tuple[torch.device, int], torch.Tensor] = {}
"""Grow-only workspace per (device, stream) for calls whose `inter` cannot hold the kernels'
scratch (the reference's `[max_batch * top_k, intermediate]` buffer is smaller than the
intermediate planes plus the fp32 partials). Calls on one stream run in order, so they share it;
a call under graph capture allocates its own instead, which the graph keeps."""


def _workspace(device: torch.device, nbytes: int, scratch: torch.Tensor | None) -> torch.Tensor:
    if (
        scratch is not None
        and scratch.device == device
        and scratch.is_contiguous()
        and scratch.numel() * scratch.element_size() >= nbytes
        and scratch.data_ptr() % 256 == 0
    ):
        return scratch
    if torch.cuda.is_current_stream_capturing():
        # a captured call owns its scratch (allocated once, from the graph's pool)
        return torch.empty(nbytes, dtype=torch.uint8, device=device)
    key = (device, _mtpk.stream_of(device))
    ws = _SHARED_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        # 1 MiB granules, so a slowly growing batch does not reallocate on every call
        ws = torch.empty(-(-max(nbytes, 1) // (1 << 20)) << 20, dtype=torch.uint8, device=device)
        _SHARED_WS[key] = ws
    return ws


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
    `workspace_bytes(...)` bytes, contiguous and 256-byte aligned (`moe_scratch(...)` makes one).
    A smaller one, such as the reference's `[max_batch * top_k, intermediate]`, or none, takes a
    grow-only workspace kept per (device, stream): no allocation once it has reached the
    largest size used. Under graph capture the call allocates its own, once, for the graph.
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


def layer_workspace_bytes(tokens: int, hidden: int, router_rows: int, shared_inter: int, top_k: int,
                          local_experts: int, intermediate: int) -> int:
    """Bytes of scratch `fused_moe_layer` needs at these sizes (`mtpk_moe_layer_workspace_bytes`)."""
    return int(_mtpk.lib().mtpk_moe_layer_workspace_bytes(tokens, hidden, router_rows, shared_inter,
                                                          top_k, local_experts, intermediate))


def layer_fits(h: torch.Tensor, router_gate: torch.Tensor, shared_gate_up: torch.Tensor,
               shared_down: torch.Tensor, experts: dict, top_k: int,
               expert_range: tuple[int, int]) -> bool:
    """Whether `fused_moe_layer` takes these operands (else the caller runs the separate ops):
    contiguous bf16 activations and dense weights, contiguous MXFP4 experts, and every check of
    `mtpk_moe_layer` itself (`mtpk_moe_layer_supported`: 1..256 rows, hidden and the shared
    expert's width multiples of 256, top_k <= experts <= 1024, 16-byte aligned operands, 32-bit
    weight offsets, the 4-wave GEMM tiles of its co-launches). No launch, no host sync."""
    if not (h.dim() == 2 and 1 <= h.shape[0] <= 256 and "gate_up_scale" in experts
            and "down_scale" in experts):
        return False
    dense = (h, router_gate, shared_gate_up, shared_down)
    if any(t.dtype != torch.bfloat16 or t.dim() != 2 or not t.is_contiguous() for t in dense):
        return False
    names = ("gate_up", "gate_up_scale", "down", "down_scale")
    if any(experts[k].dim() != 3 or not experts[k].is_contiguous() for k in names):
        return False
    gate_up, down = experts["gate_up"], experts["down"]
    hidden, shared_inter = h.shape[1], shared_down.shape[1]
    if (router_gate.shape[1] != hidden or shared_gate_up.shape != (2 * shared_inter, hidden)
            or shared_down.shape[0] != hidden or down.shape[1] != hidden
            or gate_up.shape[2] * 2 != hidden):
        return False
    lo, hi = expert_range
    return bool(_mtpk.lib().mtpk_moe_layer_supported(
        h.data_ptr(), h.shape[0], hidden, router_gate.data_ptr(), router_gate.shape[0],
        shared_gate_up.data_ptr(), shared_down.data_ptr(), shared_inter, gate_up.data_ptr(),
        experts["gate_up_scale"].data_ptr(), down.data_ptr(), experts["down_scale"].data_ptr(),
        gate_up.shape[0], gate_up.shape[1] // 2, top_k, lo, hi))


def fused_moe_layer(
    h: torch.Tensor,
    router_gate: torch.Tensor,
    shared_gate_up: torch.Tensor,
    shared_down: torch.Tensor,
    experts: dict,
    top_k: int,
    expert_range: tuple[int, int],
    *,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    routing_out: tuple[torch.Tensor, torch.Tensor] | None = None,
    add_norm: tuple[torch.Tensor, torch.Tensor, float] | None = None,
):
    """The whole MoE layer of `Model.moe` (`model.py:2800-2873`) for bf16 rows `h` `[T, hidden]`:
    router GEMM (`router_gate` = the experts' router rows, then the shared gate's row, as
    `fuse_moe_dense` concatenates them, `model.py:913-928`), softmax top-k renormalised
    (`router_fused.route`), the routed MXFP4 experts, the shared expert's SwiGLU
    (`shared_gate_up` = [gate; up], `shared_down`), and `routed + sigmoid(gate) * shared`.

    The router and the shared expert run inside the routed layer's launches (`mtpk_moe_layer`):
    one launch for the router and shared gate/up GEMM tiles, one for the top-k and the shared
    SiLU product, then the routed launches with the shared down projection's tiles beside the
    first and its gated term in the last. Each piece computes the same values as its stand-alone
    launch (`dense.linear`, `dense.silu_linear`, `router_fused.route`, `fused_moe(shared=)`).

    `routing_out` = (top_w f32 [T, top_k], top_i int32 [T, top_k]) receives the routing when
    given. `workspace` is optional scratch of `layer_workspace_bytes(...)` bytes; without it the
    call takes the grow-only per-stream workspace `fused_moe` uses.

    `add_norm = (x, w, eps)` fuses the next norm's residual form into the last launch and
    returns `(x + out, rmsnorm(x + out, w, eps))` instead of `out`, both bf16 `[T, hidden]` and
    bit-identical to `rownorm.add_rmsnorm(x, out, w, eps)` (`mtpk_moe_layer_add_norm`; only
    for more than `direct_max_tokens()` rows and hidden 2048 or 4096, see `add_norm_supported`).
    """
    lo, hi = expert_range
    if h.dtype != torch.bfloat16 or h.dim() != 2 or not h.is_contiguous():
        raise ValueError("h must be a contiguous bf16 [T, hidden] tensor")
    for name, t in (("router_gate", router_gate), ("shared_gate_up", shared_gate_up),
                    ("shared_down", shared_down)):
        if t.dtype != torch.bfloat16 or t.dim() != 2 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bf16 matrix")
    _validate(h, experts, (torch.empty(h.shape[0] * top_k, dtype=torch.int32, device=h.device),
                           torch.empty(h.shape[0] * top_k, dtype=torch.float32, device=h.device)), top_k)
    device = _mtpk.require_device(h, router_gate, shared_gate_up, shared_down, experts["gate_up"])
    tokens, hidden = h.shape
    gate_up, down = experts["gate_up"], experts["down"]
    local, intermediate = gate_up.shape[0], gate_up.shape[1] // 2
    router_rows = router_gate.shape[0]
    shared_inter = shared_down.shape[1]
    if (router_gate.shape[1] != hidden or shared_gate_up.shape != (2 * shared_inter, hidden)
            or shared_down.shape[0] != hidden):
        raise ValueError("router / shared expert shapes do not match h")
    if hi - lo != local or down.shape[1] != hidden or gate_up.shape[2] * 2 != hidden:
        raise ValueError("expert payload shapes do not match h and expert_range")
    if out is None:
        out = torch.empty(tokens, hidden, dtype=h.dtype, device=device)
    elif out.shape != (tokens, hidden) or out.dtype != h.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous bf16 [T, hidden] tensor")
    tw_ptr = ti_ptr = None
    if routing_out is not None:
        tw, ti = routing_out
        if (tw.dtype != torch.float32 or ti.dtype != torch.int32 or tw.shape != (tokens, top_k)
                or ti.shape != (tokens, top_k) or not (tw.is_contiguous() and ti.is_contiguous())):
            raise ValueError("routing_out must be contiguous (f32, int32) [T, top_k] tensors")
        tw_ptr, ti_ptr = tw.data_ptr(), ti.data_ptr()
    lib = _mtpk.lib()
    nbytes = lib.mtpk_moe_layer_workspace_bytes(tokens, hidden, router_rows, shared_inter, top_k,
                                                local, intermediate)
    if nbytes <= 0:
        raise ValueError("unsupported fused_moe_layer sizes (tokens 1..256)")
    ws = _workspace(device, nbytes, workspace)
    if add_norm is not None:
        x, w_norm, eps = add_norm
        if not add_norm_supported(tokens, hidden):
            raise ValueError(f"add_norm takes more than {direct_max_tokens()} rows and hidden "
                             "2048 or 4096")
        if (x.shape != (tokens, hidden) or x.dtype != torch.bfloat16 or not x.is_contiguous()
                or w_norm.shape != (hidden,) or w_norm.dtype != torch.bfloat16
                or not w_norm.is_contiguous()):
            raise ValueError("add_norm needs contiguous bf16 x [T, hidden] and w [hidden]")
        total = torch.empty(tokens, hidden, dtype=h.dtype, device=device)
        normed = torch.empty_like(total)
        _mtpk.check(
            lib.mtpk_moe_layer_add_norm(
                h.data_ptr(), tokens, hidden, router_gate.data_ptr(), router_rows,
                shared_gate_up.data_ptr(), shared_down.data_ptr(), shared_inter,
                gate_up.data_ptr(), experts["gate_up_scale"].data_ptr(),
                down.data_ptr(), experts["down_scale"].data_ptr(), local, intermediate,
                top_k, lo, hi, tw_ptr, ti_ptr, ws.data_ptr(), ws.numel() * ws.element_size(),
                x.data_ptr(), w_norm.data_ptr(), float(eps), total.data_ptr(), normed.data_ptr(),
                _mtpk.stream_of(device),
            ),
            "mtpk_moe_layer_add_norm",
        )  # fmt: skip
        return total, normed
    _mtpk.check(
        lib.mtpk_moe_layer(
            h.data_ptr(), tokens, hidden, router_gate.data_ptr(), router_rows,
            shared_gate_up.data_ptr(), shared_down.data_ptr(), shared_inter,
            gate_up.data_ptr(), experts["gate_up_scale"].data_ptr(),
            down.data_ptr(), experts["down_scale"].data_ptr(), local, intermediate,
            top_k, lo, hi, tw_ptr, ti_ptr, ws.data_ptr(), ws.numel() * ws.element_size(),
            out.data_ptr(), _mtpk.stream_of(device),
        ),
        "mtpk_moe_layer",
    )  # fmt: skip
    return out


@functools.lru_cache(maxsize=None)
def direct_max_tokens() -> int:
    """Rows up to which the MoE layer takes the direct path (`mtpk_moe_direct_max_tokens`)."""
    return int(_mtpk.lib().mtpk_moe_direct_max_tokens())


def add_norm_supported(tokens: int, hidden: int) -> bool:
    """Whether `fused_moe_layer(..., add_norm=)` takes these sizes (the work-unit path)."""
    return tokens > direct_max_tokens() and hidden in (2048, 4096)


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


class BwPlan:
    """Device work list of one staged MoE call (`mxfp4_gemv.BwPlan`, mxfp4_gemv.py:2320-2346):
    `sorted` i32 [tokens * top_k] (live assignment ids grouped by local expert), `unit` i32
    [3 * u_max] of (local expert, first position in `sorted`, count <= block_t) and the
    device-side `n_units` i32 [1]. Every shape is a Python int, so a captured graph replays with
    the same buffers; `bw_prep` rewrites all of them, and none needs zeroing.

    `block_t` must be 16 (`UNIT_TOKENS`: one MFMA N tile per unit). `u_max` is the library's
    own bound (`mtpk_moe_max_units`). `cursor` and `xp` are None: the counting sort keeps its
    counters in LDS, and these kernels read x in its own K order, so there is no permuted
    activation copy to make (`permute_x` is accepted for the caller's sake and changes nothing).
    `reduction` and `dtype` are x's width and dtype, checked by `bw_prep`."""

    def __init__(self, tokens: int, top_k: int, reduction: int, local_experts: int,
                 device: torch.device, dtype: torch.dtype, *, block_t: int = UNIT_TOKENS,
                 permute_x: bool = True) -> None:
        if block_t != UNIT_TOKENS:
            raise ValueError(f"BwPlan: block_t must be {UNIT_TOKENS} (tokens per work unit), got {block_t}")
        if tokens < 0 or top_k <= 0 or local_experts <= 0:
            raise ValueError(f"BwPlan: bad sizes tokens={tokens} top_k={top_k} local_experts={local_experts}")
        assignments = tokens * top_k
        self.tokens, self.top_k, self.reduction, self.dtype = tokens, top_k, reduction, dtype
        self.local_experts, self.block_t = local_experts, block_t
        self.u_max = int(_mtpk.lib().mtpk_moe_max_units(assignments, local_experts))
        self.cursor = None
        self.sorted = torch.empty(max(assignments, 1), dtype=torch.int32, device=device)
        self.unit = torch.empty(max(3 * self.u_max, 3), dtype=torch.int32, device=device)
        self.n_units = torch.empty(1, dtype=torch.int32, device=device)
        self.xp = None


def bw_prep(x: torch.Tensor, a_expert: torch.Tensor, a_weight: torch.Tensor,
            expert_range: tuple[int, int], plan: BwPlan) -> None:
    """Routing work list into `plan` (`mxfp4_gemv.bw_prep`, mxfp4_gemv.py:2349-2376): one
    counting-sort launch (`mtpk_moe_prep`) over the live assignments (expert in `expert_range`
    and weight != 0); no host sync."""
    device = _mtpk.require_device(x, a_expert, a_weight, plan.sorted)
    lo, hi = expert_range
    a = a_expert.numel()
    if x.dim() != 2 or x.shape != (plan.tokens, plan.reduction) or x.dtype != plan.dtype:
        raise ValueError(f"bw_prep: x {tuple(x.shape)} {x.dtype} does not match the plan "
                         f"({plan.tokens}, {plan.reduction}) {plan.dtype}")
    if a != plan.tokens * plan.top_k or a_weight.numel() != a:
        raise ValueError(f"bw_prep: routing has {a} / {a_weight.numel()} entries, the plan "
                         f"{plan.tokens * plan.top_k}")
    if not 0 <= hi - lo <= plan.local_experts:
        raise ValueError(f"bw_prep: expert_range {expert_range} spans more than the plan's "
                         f"{plan.local_experts} local experts")
    _mtpk.check(
        _mtpk.lib().mtpk_moe_prep(
            a_expert.data_ptr(), _mtpk.index_code(a_expert.dtype),
            a_weight.data_ptr(), _mtpk.float_code(a_weight.dtype),
            a, lo, hi, plan.sorted.data_ptr(), plan.unit.data_ptr(), plan.u_max,
            plan.n_units.data_ptr(), _mtpk.stream_of(device),
        ),
        "mtpk_moe_prep",
    )  # fmt: skip


def _combine_rows(y, a_expert, a_weight, expert_range, top_k, out, shared, gate, what) -> None:
    lo, hi = expert_range
    tokens, hidden = out.shape
    device = _mtpk.require_device(y, a_expert, a_weight, out)
    if y.shape != (tokens * top_k, hidden) or not y.is_contiguous() or not out.is_contiguous():
        raise ValueError(f"{what}: y must be a contiguous [{tokens * top_k}, {hidden}] tensor and "
                         f"out contiguous, got y {tuple(y.shape)}")
    if a_expert.numel() != tokens * top_k or a_weight.numel() != tokens * top_k:
        raise ValueError(f"{what}: routing must have {tokens * top_k} entries")
    sp, sd, gp, gd, gs = None, _mtpk.F32, None, _mtpk.F32, 0
    if shared is not None:
        _mtpk.require_device(shared, gate)
        sp, sd = shared.data_ptr(), _mtpk.float_code(shared.dtype)
        gp, gd, gs = gate.data_ptr(), _mtpk.float_code(gate.dtype), gate.stride(0)
    _mtpk.check(
        _mtpk.lib().mtpk_moe_combine_rows(
            y.data_ptr(), _mtpk.float_code(y.dtype), a_expert.data_ptr(),
            _mtpk.index_code(a_expert.dtype), a_weight.data_ptr(), _mtpk.float_code(a_weight.dtype),
            tokens, top_k, hidden, lo, hi, sp, sd, gp, gd, gs, out.data_ptr(),
            _mtpk.float_code(out.dtype), _mtpk.stream_of(device),
        ),
        "mtpk_moe_combine_rows",
    )  # fmt: skip


def bw_combine(y: torch.Tensor, a_expert: torch.Tensor, a_weight: torch.Tensor,
               expert_range: tuple[int, int], top_k: int, out: torch.Tensor) -> None:
    """`out[t] = sum_j y[t*top_k + j]` over t's live assignments, in j order, in fp32
    (`mxfp4_gemv.bw_combine`, mxfp4_gemv.py:2440-2446): y's rows already carry the routing
    weight, and dead rows are never read (no zero fill needed). One launch
    (`mtpk_moe_combine_rows`); y f32 or bf16, out f32 or bf16."""
    _combine_rows(y, a_expert, a_weight, expert_range, top_k, out, None, None, "bw_combine")


def bw_combine_glue(y: torch.Tensor, a_expert: torch.Tensor, a_weight: torch.Tensor,
                    expert_range: tuple[int, int], top_k: int, shared: torch.Tensor,
                    gate: torch.Tensor, out: torch.Tensor) -> None:
    """`bw_combine` plus the shared expert's term in the same launch
    (`mxfp4_gemv.bw_combine_glue`, mxfp4_gemv.py:2449-2488): `out[t] = routed_sum +
    sigmoid(gate[t, 0]) * shared[t]`, with the routed sum, the sigmoid and the product each
    rounded to `out`'s dtype before the add, as `bw_combine` followed by the three torch ops
    rounds them. `gate` is `[tokens, >= 1]` with unit column stride; only column 0 is read,
    through its own row stride (a view into the router GEMM output)."""
    tokens, hidden = out.shape
    if shared.shape != (tokens, hidden) or not shared.is_contiguous():
        raise ValueError(f"bw_combine_glue: shared must be a contiguous [{tokens}, {hidden}] tensor, "
                         f"got shape {tuple(shared.shape)}")
    if gate.dim() != 2 or gate.shape[0] != tokens or gate.stride(1) != 1:
        raise ValueError(f"bw_combine_glue: gate must have {tokens} rows and unit column stride, "
                         f"got shape {tuple(gate.shape)}, stride {gate.stride()}")
    _combine_rows(y, a_expert, a_weight, expert_range, top_k, out, shared, gate, "bw_combine_glue")


def expert_sorted_order(a_expert: torch.Tensor) -> torch.Tensor:
    """`argsort(a_expert, stable=True)` as int32 (`mxfp4_gemv.py:874-887`)."""
    return torch.argsort(a_expert, stable=True).to(torch.int32)


def fused_expert_order(a_expert: torch.Tensor, num_experts: int, *, cursor=None) -> torch.Tensor:
    """Expert-grouping permutation from the HIP counting sort: set-identical to
    `expert_sorted_order` per expert (`mxfp4_gemv.py:990-1017`)."""
    a = a_expert.numel()
    ones = torch.ones(a, dtype=torch.float32, device=a_expert.device)
    x = torch.empty(a, 1, dtype=torch.bfloat16, device=a_expert.device)
    plan = BwPlan(a, 1, 1, num_experts, a_expert.device, torch.bfloat16)
    bw_prep(x, a_expert, ones, (0, num_experts), plan)
    return plan.sorted[:a]


def grouped_block_count(assignments: int, experts: int, block_m: int) -> int:
    """Upper bound on `align_blocks`' blocks (`mxfp4_gemv.py:734-742`)."""
    return -(-assignments // block_m) + experts + 1


def align_blocks(a_expert: torch.Tensor, a_weight: torch.Tensor, expert_range: tuple[int, int],
                 block_m: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-expert `block_m` blocks with a fixed-shape result (interface of
    `mxfp4_gemv.py:745-800`): `slot_assign[b*block_m + i]` = assignment id or -1,
    `block_expert[b]` = local expert, or the sentinel `experts` for the bucket of dropped
    assignments and for the unused blocks past the last one. Torch ops, no host sync.

    Bucket `experts` collects the dropped assignments. An assignment's row in its bucket is the
    number of earlier assignments of that bucket (a running count over the one-hot bucket
    matrix), its slot is that row past the bucket's first block, and block b belongs to the
    bucket whose block range contains it (a binary search over the buckets' block ends).
    """
    lo, hi = expert_range
    experts = hi - lo
    n = a_expert.numel()
    device = a_expert.device
    e = a_expert.to(torch.long) - lo
    bucket = torch.where((e >= 0) & (e < experts) & (a_weight != 0), e, experts)
    onehot = torch.nn.functional.one_hot(bucket, experts + 1).to(torch.int32)
    seen = onehot.cumsum(0)  # seen[a, b]: assignments 0..a that fall in bucket b
    row = seen.gather(1, bucket[:, None])[:, 0].to(torch.long) - 1
    count = seen[-1].to(torch.long) if n else torch.zeros(experts + 1, dtype=torch.long, device=device)
    block_end = (-(-count // block_m)).cumsum(0)  # one past each bucket's last block
    slot = (block_end - (-(-count // block_m)))[bucket] * block_m + row
    n_blocks = grouped_block_count(n, experts, block_m)
    slot_assign = torch.full((n_blocks * block_m,), -1, dtype=torch.int32, device=device)
    slot_assign[slot] = torch.arange(n, dtype=torch.int32, device=device)
    blocks = torch.arange(n_blocks, dtype=torch.long, device=device)
    owner = torch.searchsorted(block_end, blocks, right=True).clamp(max=experts)
    return slot_assign, owner.to(torch.int32)


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
    """Dequantise-then-multiply in `compute_dtype` (interface of `mxfp4_gemv.py:1613-1651`): the
    torch path selected by `SEED_FUSED_MOE=0` and the arithmetic `fused_moe` reformulates.

    Every distinct live expert is dequantised once, at most `chunk` experts at a time, and its
    assignments' token rows go through `x @ gate_upᵀ`, `silu(gate) * up`, `@ downᵀ` and the
    routing weight together; the weighted rows are added into the output per token.
    """
    a_expert, a_weight = routing
    lo, hi = expert_range
    dt = compute_dtype or x.dtype
    e = a_expert.to(torch.long) - lo
    live = (e >= 0) & (e < hi - lo) & (a_weight != 0)
    out = torch.zeros(x.shape[0], experts["down"].shape[1], dtype=dt, device=x.device)
    ids = torch.arange(a_expert.numel(), device=x.device)
    used = torch.unique(e[live])
    xs = x.to(dt)
    for g in range(0, used.numel(), chunk):
        group = used[g : g + chunk]
        w1 = dequant(experts["gate_up"][group], experts["gate_up_scale"][group], dt)
        w2 = dequant(experts["down"][group], experts["down_scale"][group], dt)
        for i, ex in enumerate(group.tolist()):
            mine = ids[live & (e == ex)]
            rows = xs[mine // top_k]
            gate, up = (rows @ w1[i].t()).chunk(2, -1)
            y = (torch.nn.functional.silu(gate) * up) @ w2[i].t()
            out.index_add_(0, mine // top_k, y * a_weight[mine, None].to(dt))
    return out.to(x.dtype)
