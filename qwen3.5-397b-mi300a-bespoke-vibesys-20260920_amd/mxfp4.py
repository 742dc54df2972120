"""OCP MXFP4 dequantisation (e2m1 values, e8m0 scale per 32) — the reference's `mxfp4` module
interface (`mxfp4.py:1-51`).

A weight of logical shape [..., K] is uint8 [..., K/2] (two codes per byte, low nibble = even
element) plus uint8 e8m0 scales [..., K/32]. Device tensors are dequantised by the HIP kernel
(`mtpk_dequant_mxfp4`, exact fp32); CPU tensors by the torch table lookup below, which is what
the reference's CPU engine runs.

Scale byte 0: the device kernel uses the MoE kernels' convention, +0.0
(`mxfp4_gemv.py:372-382`), where torch's `exp2(0 - 127)` gives 2**-127; the two differ below
1e-37 and never move a bf16 result.
"""

from __future__ import annotations

import torch

import _mtpk

BLOCK = 32

_FP4_VALUES = (
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
)  # fmt: skip
"""e2m1 code -> value; bit 3 is the sign."""


def dequant_mxfp4(packed: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Dense [..., K] tensor in `dtype` for packed [..., K/2] and scale [..., K/32]."""
    if packed.shape[:-1] != scale.shape[:-1] or packed.shape[-1] * 2 != scale.shape[-1] * BLOCK:
        raise ValueError(f"packed {tuple(packed.shape)} and scale {tuple(scale.shape)} disagree")
    if packed.device.type == "cuda":
        return _dequant_device(packed, scale).to(dtype)
    return dequant_torch(packed, scale, dtype)


def dequant_torch(packed: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """The reference's torch table lookup (`mxfp4.py:32-51`) on `packed`'s own device: the
    CPU engine's dequant, and on a device the decode of the `SEED_FUSED_MOE=0` torch path
    (scale byte 0 gives 2**-127, 255 gives +-inf / NaN, as torch's exp2 does)."""
    if packed.shape[:-1] != scale.shape[:-1] or packed.shape[-1] * 2 != scale.shape[-1] * BLOCK:
        raise ValueError(f"packed {tuple(packed.shape)} and scale {tuple(scale.shape)} disagree")
    lut = torch.tensor(_FP4_VALUES, dtype=torch.float32, device=packed.device)
    lo = lut[(packed & 0xF).int()]
    hi = lut[(packed >> 4).int()]
    values = torch.stack([lo, hi], dim=-1).flatten(-2)
    *lead, k = values.shape
    scales = torch.exp2(scale.float() - 127.0).unsqueeze(-1)
    return (values.reshape(*lead, k // BLOCK, BLOCK) * scales).reshape(*lead, k).to(dtype)


def _dequant_device(packed: torch.Tensor, scale: torch.Tensor, mode: int = 0) -> torch.Tensor:
    _mtpk.require_device(packed, scale)
    k = packed.shape[-1] * 2
    rows = packed.numel() // packed.shape[-1] if packed.numel() else 0
    out = torch.empty(*packed.shape[:-1], k, dtype=torch.float32, device=packed.device)
    p, s = packed.contiguous(), scale.contiguous()
    _mtpk.check(
        _mtpk.lib().mtpk_dequant_mxfp4(
            p.data_ptr(), s.data_ptr(), rows, k, mode, out.data_ptr(), _mtpk.stream_of(p.device)
        ),
        "mtpk_dequant_mxfp4",
    )
    return out


def dequant_in_kernel(packed: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """fp32 view of the MoE kernels' own in-register decode (hardware fp4 -> bf16 convert with
    the block scale folded in). Equal to the exact dequant bit for bit for scale bytes 0..254
    (byte 0 as +-0.0); byte 255 gives NaN for every code. A test probe, not a serving op."""
    return _dequant_device(packed, scale, mode=1)


_FP4_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def quantize_mxfp4(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """OCP MX quantisation of a float `[..., K]` tensor to `(packed u8 [..., K/2], e8m0 scale
    u8 [..., K/32])`, on `w`'s device.

    Per block of 32 the shared exponent is `floor(log2(amax)) - 2` (e2m1's largest exponent),
    so the block maximum lands in [4, 8) and saturates at 6; each element takes the nearest
    e2m1 magnitude (ties to the smaller one) and its sign. An all-zero block gets scale byte 127
    and zero codes. This is how the random expert payloads of the small models are made.
    """
    *lead, k = w.shape
    if k % BLOCK:
        raise ValueError(f"last dim {k} is not a multiple of {BLOCK}")
    blocks = w.float().reshape(*lead, k // BLOCK, BLOCK)
    amax = blocks.abs().amax(-1)
    exp = torch.where(amax > 0, torch.floor(torch.log2(amax.clamp_min(2.0 ** -126))) - 2,
                      torch.zeros_like(amax)).clamp(-127, 127)
    mags = torch.tensor(_FP4_MAGNITUDES, device=w.device)
    scaled = blocks.abs() / torch.exp2(exp)[..., None]
    code = (scaled[..., None] - mags).abs().argmin(-1)
    code = code + 8 * ((blocks < 0) & (code > 0))
    code = code.reshape(*lead, k).to(torch.uint8)
    packed = code[..., 0::2] | (code[..., 1::2] << 4)
    return packed.contiguous(), (exp + 127).to(torch.uint8).contiguous()
