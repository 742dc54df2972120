"""MXFP4 (OCP e2m1 + e8m0) restated in numpy. TEST INFRASTRUCTURE ONLY (see oracle/__init__).

Reference: `mxfp4.py:10-51` (the torch dequant), `mxfp4_gemv.py:372-382` (the kernels' e8m0
decode, which pins scale byte 0 to +0.0), `seed_tests/test_seed_parity.py:43-54` (the tests'
quantiser, used for the config-1 model).

Pinning (each check lives in tests/test_oracle_mxfp4.py):
- `FP4_VALUES`: the OCP table; checked against the closed form 2**(e-1)*(1+m/2) / m/2 per code
  and against the reference test's hand vector (`test_seed_parity.py:117-130`).
- `dequant_mxfp4`: hand vector above; exhaustive 256 bytes at scale 127
  (`test_mxfp4_fused_gemv.py:208-228`); scale 0 -> 2**-127 and 255 -> inf as torch.exp2 gives.
- `dequant_mxfp4_kernel`: identical to `dequant_mxfp4` for scales 1..254 (checked), and the
  pinned +0.0 scale at byte 0.
- `quantize_mxfp4`: round trip dequant(quantize(w)) == recon, and recon within half a code
  step of w.
"""

from __future__ import annotations

import numpy as np

BLOCK = 32
"""Elements per e8m0 scale (`mxfp4.py:10`)."""

FP4_VALUES = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)
"""e2m1 code -> value; bit 3 is the sign (`mxfp4.py:12-29`)."""


def fp4_closed_form(code: int) -> float:
    """e2m1 from its fields: [s][e1 e0][m]; e=0 -> m*0.5 else 2**(e-1)*(1+m/2)."""
    s, e, m = (code >> 3) & 1, (code >> 1) & 3, code & 1
    mag = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1.0 + m / 2.0)
    return -mag if s else mag


def e8m0_torch(scale: np.ndarray) -> np.ndarray:
    """`torch.exp2(scale.float() - 127)` (`mxfp4.py:47-49`): 0 -> 2**-127, 255 -> +inf."""
    return np.ldexp(np.float32(1.0), scale.astype(np.int32) - 127).astype(np.float32)


def e8m0_kernel(scale: np.ndarray) -> np.ndarray:
    """The kernels' e8m0 (`mxfp4_gemv.py:372-382`): byte into the fp32 exponent field, so
    0 -> +0.0, 1..254 -> 2**(s-127), 255 -> +inf."""
    bits = scale.astype(np.uint32) << np.uint32(23)
    return bits.view(np.float32)


def _unpack(packed: np.ndarray) -> np.ndarray:
    """Low nibble = even element, high nibble = odd element (`mxfp4.py:42-44`)."""
    lo = FP4_VALUES[packed & 0xF]
    hi = FP4_VALUES[packed >> 4]
    return np.stack([lo, hi], axis=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)


def _apply(values: np.ndarray, scales: np.ndarray) -> np.ndarray:
    lead, k = values.shape[:-1], values.shape[-1]
    blocks = values.reshape(*lead, k // BLOCK, BLOCK)
    with np.errstate(invalid="ignore", over="ignore"):
        out = blocks * scales[..., None]
    return out.reshape(*lead, k).astype(np.float32)


def dequant_mxfp4(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Dense fp32 `[..., K]` from packed `[..., K/2]` and e8m0 `[..., K/32]`, torch semantics
    (`mxfp4.py:32-51`). fp32 products of a 2-significant-bit value and a power of two are
    exact, so this is the mathematically exact dequant for every scale byte 1..254."""
    packed = np.asarray(packed, dtype=np.uint8)
    scale = np.asarray(scale, dtype=np.uint8)
    return _apply(_unpack(packed), e8m0_torch(scale))


def dequant_mxfp4_kernel(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """As `dequant_mxfp4`, with the kernels' pinned scale byte 0 -> +0.0 (values become
    +-0.0, sign from the code) instead of torch's 2**-127."""
    packed = np.asarray(packed, dtype=np.uint8)
    scale = np.asarray(scale, dtype=np.uint8)
    return _apply(_unpack(packed), e8m0_kernel(scale))


def quantize_mxfp4(w: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """The reference tests' quantiser (`test_seed_parity.py:43-54`) in numpy: per 32-block
    exponent `floor(log2(amax)) - 2` so the block max maps to <= 6, nearest fp4 magnitude
    (first on a tie, as `argmin` picks), sign from the input. Returns (packed, scale, recon)."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    blocks = w.reshape(n, k // BLOCK, BLOCK)
    amax = np.maximum(np.abs(blocks).max(-1), np.float32(1e-30))
    exp = np.floor(np.log2(amax)) - 2
    sc = np.exp2(exp).astype(np.float32)[..., None]
    mags = np.abs(blocks) / sc
    pos = FP4_VALUES[:8]
    code = np.abs(mags[..., None] - pos).argmin(-1) + 8 * (blocks < 0)
    recon = np.concatenate([pos, -pos])[code] * sc
    code = code.reshape(n, k).astype(np.uint8)
    packed = (code[:, 0::2] | (code[:, 1::2] << 4)).astype(np.uint8)
    scale = (exp + 127).reshape(n, k // BLOCK).astype(np.uint8)
    return packed, scale, recon.reshape(n, k).astype(np.float32)


def bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 -> fp32, round to nearest even (NaN kept NaN)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(a)
    out[nan] = a[nan]
    return out


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern (uint16), RNE."""
    return (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> fp32 values."""
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)
