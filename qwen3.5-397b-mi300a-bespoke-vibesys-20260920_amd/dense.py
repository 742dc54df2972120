"""bf16 linears of a few token rows on the device (`mtpk_gemm_bf16`).

`linear(x, w)` is `F.linear(x, w)` for `x` `[..., K]` with at most 256 rows; `silu_linear` is
the shared expert's gate_up with its `silu(gate) * up` (`swiglu_mlp`, `model.py:638-649`) in the
same launch; `argmax_linear` the LM head with its first-occurrence argmax
(`greedy_token`, `mtp.py:640-658`) in the same launch, so the logits never reach memory.
`fits(x, w)` says whether the kernel takes the shapes; callers use `F.linear` otherwise.
"""

from __future__ import annotations

import torch

import _mtpk

MAX_ROWS = 256
STORE, SILU, ARGMAX = 0, 1, 2


def fits(x: torch.Tensor, w: torch.Tensor) -> bool:
    """bf16 device tensors, at most 256 rows, K a multiple of 256, contiguous rows."""
    if x.device.type != "cuda" or x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        return False
    rows = x.numel() // x.shape[-1] if x.dim() else 0
    k = x.shape[-1]
    return (0 < rows <= MAX_ROWS and k % 256 == 0 and w.dim() == 2 and w.shape[1] == k
            and w.is_contiguous() and w.shape[0] * k * 2 < (1 << 31))


def _run(x: torch.Tensor, w: torch.Tensor, epilogue: int, out: torch.Tensor) -> torch.Tensor:
    x2 = x.reshape(-1, x.shape[-1])
    if not x2.is_contiguous():
        x2 = x2.contiguous()
    m, k = x2.shape
    n = w.shape[0]
    lib = _mtpk.lib()
    nbytes = int(lib.mtpk_gemm_workspace_bytes(m, n, k, epilogue))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    odt = _mtpk.float_code(out.dtype) if out.dtype != torch.int64 else 0
    _mtpk.check(lib.mtpk_gemm_bf16(x2.data_ptr(), m, k, w.data_ptr(), n, epilogue, out.data_ptr(), odt,
                                   ws.data_ptr(), nbytes, _mtpk.stream_of(x.device)), "mtpk_gemm_bf16")
    return out


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """`x @ w.T` in bf16 (fp32 accumulation), x's leading shape."""
    out = torch.empty(*x.shape[:-1], w.shape[0], dtype=x.dtype, device=x.device)
    return _run(x, w, STORE, out)


def silu_linear(x: torch.Tensor, w_gate_up: torch.Tensor) -> torch.Tensor:
    """`silu(x @ g.T) * (x @ u.T)` for `w_gate_up = cat([g; u])` `[2 I, K]`: `[..., I]`."""
    out = torch.empty(*x.shape[:-1], w_gate_up.shape[0] // 2, dtype=x.dtype, device=x.device)
    return _run(x, w_gate_up, SILU, out)


def argmax_linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """First-occurrence argmax over the bf16 values of `x @ w.T`: int64 `[...]`, into `out`
    (contiguous int64 of x's leading shape) when given."""
    if out is None:
        out = torch.empty(x.shape[:-1], dtype=torch.int64, device=x.device)
    elif out.dtype != torch.int64 or out.shape != x.shape[:-1] or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous int64 {tuple(x.shape[:-1])} tensor")
    return _run(x, w, ARGMAX, out)
