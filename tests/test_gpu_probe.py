"""gfx950 building blocks against the oracle: the MFMA 16x16x32 bf16 lane layout the MoE
kernels assume, and the MXFP4 decode (exact fp32 path and the kernels' in-register
hardware-convert path, each over every byte and every scale), and the load-time scale check."""

import numpy as np
import pytest
import torch

import _mtpk
import mxfp4
from oracle import mxfp4_ref as mx

pytestmark = pytest.mark.gpu


def test_mfma_16x16x32_lane_layout(dev):
    rng = np.random.default_rng(0)
    A = rng.integers(-4, 5, (16, 32)).astype(np.float32)
    B = rng.integers(-4, 5, (32, 16)).astype(np.float32)
    a_l = np.zeros((64, 8), np.float32)
    b_l = np.zeros((64, 8), np.float32)
    for lane in range(64):
        g, c = lane // 16, lane % 16
        a_l[lane] = A[c, 8 * g : 8 * g + 8]
        b_l[lane] = B[8 * g : 8 * g + 8, c]
    to_bf16 = lambda a: torch.from_numpy(mx.bf16_bits(a).view(np.int16)).to(dev)  # noqa: E731
    d = torch.zeros(64, 4, dtype=torch.float32, device=dev)
    ta, tb = to_bf16(a_l), to_bf16(b_l)
    _mtpk.check(_mtpk.lib().mtpk_probe_mfma_16x16x32(ta.data_ptr(), tb.data_ptr(), d.data_ptr(), None),
                "probe")
    torch.cuda.synchronize()
    d = d.cpu().numpy()
    want = A @ B
    got = np.zeros((16, 16), np.float32)
    for lane in range(64):
        for i in range(4):
            got[4 * (lane // 16) + i, lane % 16] = d[lane, i]
    assert np.array_equal(got, want)


def _all_bytes_all_scales():
    packed = np.tile(np.arange(256, dtype=np.uint8).reshape(16, 16), (256, 1))  # [4096, 16]
    scale = np.repeat(np.arange(256, dtype=np.uint8), 16)[:, None]  # one scale per row
    return packed, scale


def test_exact_dequant_every_byte_every_scale(dev):
    packed, scale = _all_bytes_all_scales()
    got = mxfp4.dequant_mxfp4(torch.from_numpy(packed).to(dev), torch.from_numpy(scale).to(dev),
                              torch.float32).cpu().numpy()
    want = mx.dequant_mxfp4_kernel(packed, scale)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))  # bits, incl. -0.0


def test_in_kernel_decode_every_byte_every_scale(dev):
    """`decode8`, the decode every MoE kernel runs, against the pinned decode: bit for bit
    (signed zeros included) at scale bytes 0..254, byte 0 giving +-0.0; at 255 (the OCP NaN
    scale) the hardware convert gives NaN for every code, which `supports` refuses at load."""
    packed, scale = _all_bytes_all_scales()
    got = mxfp4.dequant_in_kernel(torch.from_numpy(packed).to(dev),
                                  torch.from_numpy(scale).to(dev)).cpu().numpy()
    want = mx.dequant_mxfp4_kernel(packed, scale)
    rows = scale[:, 0] <= 254
    g, w = got[rows], want[rows]
    assert np.array_equal(np.isnan(g), np.isnan(w))
    fin = ~np.isnan(w)
    assert np.array_equal(g[fin].view(np.uint32), w[fin].view(np.uint32))
    for s_byte in (0, 1, 253, 254):  # the edges named explicitly: +-0.0, subnormal, overflow
        r = slice(16 * s_byte, 16 * s_byte + 16)
        assert np.array_equal(got[r].view(np.uint32), want[r].view(np.uint32)), s_byte
    assert np.isnan(got[16 * 255 :]).all()


def _payload_with_scale(dev, byte, codes_zero):
    rng = np.random.default_rng(byte)
    E, H, I = 2, 64, 32
    ex = {
        "gate_up": rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8),
        "gate_up_scale": rng.integers(118, 123, (E, 2 * I, H // 32), dtype=np.uint8),
        "down": rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8),
        "down_scale": rng.integers(118, 123, (E, H, I // 32), dtype=np.uint8),
    }
    ex["down_scale"][1, 5, 0] = byte
    if codes_zero:
        ex["down"][1, 5, :16] &= 0x88  # only signed zeros in that block
    return {k: torch.from_numpy(v).to(dev) for k, v in ex.items()}


def test_supports_refuses_scale_255_over_nonzero_codes(dev):
    import mxfp4_gemv

    x = torch.randn(3, 64, device=dev).to(torch.bfloat16)
    routing = (torch.tensor([0, 1, 1, 0, 0, 1], dtype=torch.int32, device=dev),
               torch.full((6,), 0.5, device=dev))
    for byte, zero, ok in ((255, False, False), (255, True, True), (0, False, True), (1, False, True)):
        ex = _payload_with_scale(dev, byte, zero)
        assert mxfp4_gemv.bw_scales_ok(ex) is ok
        assert mxfp4_gemv.supports(ex) is ok
        if ok:
            mxfp4_gemv.fused_moe(x, ex, routing, 2, (0, 2))
        else:
            with pytest.raises(ValueError, match="supports"):
                mxfp4_gemv.fused_moe(x, ex, routing, 2, (0, 2))
            # the verdict belongs to the refused tensors, not their addresses: a copy that no
            # one checked is scanned by its first call and refused the same way
            fresh = {k: v.clone() for k, v in ex.items()}
            with pytest.raises(ValueError, match="supports"):
                mxfp4_gemv.fused_moe(x, fresh, routing, 2, (0, 2))
            del fresh
        del ex
