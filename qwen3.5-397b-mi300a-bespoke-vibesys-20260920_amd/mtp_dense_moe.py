"""Routed bf16 experts of the MTP draft layer on the device (`mtpk_moe_dense`).

The real checkpoint's MTP layer stores dense bf16 experts (`gate_up` `[E, 2I, H]`, `down`
`[E, H, I]`, as `weights.load_experts` stacks them) while the target layers' are MXFP4. The
kernels read each touched expert once per 16 of its assignments and use the routed expert id
only as a base address, so the resident `[E, ...]` tensors are never gathered: the contract of
the reference's `mtp_dense_moe.fused_moe` / `grouped_moe` (`mtp_dense_moe.py:359-745`). The
launch grid depends only on the sizes (graph capturable); assignments outside `expert_range`,
with weight 0 or of an inactive token contribute nothing, and the combine sums a token's
assignments in j order without atomics.

Device tensors only; a device call raises if the HIP library is missing.
"""

from __future__ import annotations

import torch

import _mtpk


def available(h: torch.Tensor, experts: dict) -> bool:
    """Whether the kernels take this input and resident expert layout (`mtp_dense_moe.py:42-54`)."""
    ok = (h.device.type == "cuda" and h.dtype == torch.bfloat16 and set(experts) == {"gate_up", "down"}
          and experts["gate_up"].dtype == torch.bfloat16 and experts["down"].dtype == torch.bfloat16
          and h.is_contiguous() and experts["gate_up"].is_contiguous() and experts["down"].is_contiguous())
    if ok:
        _mtpk.lib()
    return ok


def scratch_bytes(max_tokens: int, top_k: int, intermediate: int, hidden: int) -> int:
    """Bytes of the caller's two bf16 buffers, `inter_scratch` `[max_tokens * top_k, I]` and
    `out_scratch` `[max_tokens, H]` (`mtp_dense_moe.py:57-59`)."""
    return 2 * (max_tokens * top_k * intermediate + max_tokens * hidden)


def workspace_bytes(tokens: int, top_k: int, local_experts: int, intermediate: int, hidden: int) -> int:
    """Device workspace of one call: work list, the two intermediate planes, the f32 rows."""
    return int(_mtpk.lib().mtpk_moe_dense_workspace_bytes(tokens, top_k, local_experts,
                                                           intermediate, hidden))


def grouped_scratch(max_tokens: int, top_k: int, local_experts: int, hidden: int,
                    device: torch.device, intermediate: int | None = None) -> dict:
    """Address-stable scratch for `grouped_moe` (`mtp_dense_moe.py:629-639`). `intermediate`
    sizes the workspace now; without it the workspace is allocated by the first call (which
    then must not be under graph capture)."""
    s = {"max_tokens": max_tokens, "top_k": top_k, "local_experts": local_experts, "hidden": hidden,
         "workspace": None}
    if intermediate is not None:
        s["workspace"] = torch.empty(workspace_bytes(max_tokens, top_k, local_experts, intermediate,
                                                     hidden), dtype=torch.uint8, device=device)
    return s


def _check(h, experts, routing, top_k, inter_scratch, out_scratch, active):
    if not available(h, experts):
        raise ValueError("mtp_dense_moe requires contiguous BF16 CUDA inputs and dense experts")
    expert, weight = routing
    tokens, hidden = h.shape
    intermediate = experts["gate_up"].shape[1] // 2
    if expert.shape != (tokens, top_k) or weight.shape != (tokens, top_k):
        raise ValueError(f"routing must be [{tokens}, {top_k}], got {tuple(expert.shape)}, "
                         f"{tuple(weight.shape)}")
    if not (expert.is_contiguous() and weight.is_contiguous()):
        raise ValueError("routing tensors must be contiguous")
    if experts["gate_up"].shape[2] != hidden:
        raise ValueError("gate_up reduction dimension does not match h")
    if experts["down"].shape[1:] != (hidden, intermediate):
        raise ValueError("down expert shape does not match hidden/intermediate")
    if inter_scratch is not None and (inter_scratch.shape[0] < tokens * top_k
                                      or inter_scratch.shape[1] != intermediate):
        raise ValueError("MTP expert intermediate scratch is too small")
    if out_scratch is not None and (out_scratch.shape[0] < tokens or out_scratch.shape[1] != hidden
                                    or out_scratch.dtype != torch.bfloat16
                                    or not out_scratch.is_contiguous()):
        raise ValueError("MTP expert output scratch is too small")
    if active is not None and (active.shape != (tokens,) or active.dtype != torch.bool):
        raise ValueError(f"active must be bool [{tokens}]")


def _run(h, experts, routing, top_k, expert_range, out, workspace, active) -> torch.Tensor:
    expert, weight = routing
    tokens, hidden = h.shape
    local = experts["gate_up"].shape[0]
    intermediate = experts["gate_up"].shape[1] // 2
    lo, hi = expert_range
    if hi - lo != local:
        raise ValueError(f"expert_range {expert_range} does not match {local} local experts")
    if active is not None:  # an inactive token's assignments get weight 0: dropped by the prep
        weight = weight * active[:, None].to(weight.dtype)
    device = h.device
    lib = _mtpk.lib()
    nbytes = int(lib.mtpk_moe_dense_workspace_bytes(tokens, top_k, local, intermediate, hidden))
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(nbytes, dtype=torch.uint8, device=device)
    _mtpk.check(
        lib.mtpk_moe_dense(
            h.data_ptr(), tokens, hidden, experts["gate_up"].data_ptr(), experts["down"].data_ptr(),
            local, intermediate, expert.data_ptr(), _mtpk.index_code(expert.dtype),
            weight.data_ptr(), _mtpk.float_code(weight.dtype), top_k, lo, hi,
            workspace.data_ptr(), workspace.numel(), out.data_ptr(), _mtpk.stream_of(device),
        ),
        "mtpk_moe_dense",
    )  # fmt: skip
    return out


def fused_moe(h: torch.Tensor, experts: dict, routing: tuple[torch.Tensor, torch.Tensor], top_k: int,
              expert_range: tuple[int, int], inter_scratch: torch.Tensor | None = None,
              out_scratch: torch.Tensor | None = None,
              active: torch.Tensor | None = None) -> torch.Tensor:
    """Routed output `[T, H]` bf16 (`mtp_dense_moe.py:359-426`). `routing` = (global expert ids
    `[T, top_k]`, normalised weights `[T, top_k]`); `active` bool `[T]` zeroes inactive tokens.
    Written into `out_scratch[:T]` when given. `inter_scratch` is checked for the reference's
    shape and otherwise unused: the intermediate lives in the workspace, as two planes."""
    _check(h, experts, routing, top_k, inter_scratch, out_scratch, active)
    tokens, hidden = h.shape
    out = out_scratch[:tokens] if out_scratch is not None else \
        torch.empty(tokens, hidden, dtype=torch.bfloat16, device=h.device)
    return _run(h, experts, routing, top_k, expert_range, out, None, active)


def grouped_moe(h: torch.Tensor, experts: dict, routing: tuple[torch.Tensor, torch.Tensor], top_k: int,
                expert_range: tuple[int, int], inter_scratch: torch.Tensor, out_scratch: torch.Tensor,
                scratch: dict, active: torch.Tensor | None = None) -> torch.Tensor:
    """`fused_moe`'s contract with caller-owned scratch (`mtp_dense_moe.py:642-745`): `scratch`
    from `grouped_scratch` with `max_tokens >= T`."""
    _check(h, experts, routing, top_k, inter_scratch, out_scratch, active)
    tokens = h.shape[0]
    if scratch["max_tokens"] < tokens or scratch["top_k"] != top_k:
        raise ValueError("grouped scratch is too small")
    if scratch["workspace"] is None:
        if torch.cuda.is_current_stream_capturing():
            raise ValueError("grouped_scratch needs intermediate= to be used under graph capture")
        scratch["workspace"] = torch.empty(
            workspace_bytes(scratch["max_tokens"], top_k, scratch["local_experts"],
                            experts["gate_up"].shape[1] // 2, scratch["hidden"]),
            dtype=torch.uint8, device=h.device)
    return _run(h, experts, routing, top_k, expert_range, out_scratch[:tokens], scratch["workspace"], active)
