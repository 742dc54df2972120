"""gfx950 building blocks against the oracle: the MFMA 16x16x32 bf16 lane layout the MoE
kernels assume, and the MXFP4 decode (exact fp32 path over every byte and scale; the kernels'
in-register hardware-convert path over every byte and scales 2..252)."""

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


def test_in_kernel_decode_every_byte_scales_2_to_252(dev):
    packed, scale = _all_bytes_all_scales()
    got = mxfp4.dequant_in_kernel(torch.from_numpy(packed).to(dev),
                                  torch.from_numpy(scale).to(dev)).cpu().numpy()
    want = mx.dequant_mxfp4_kernel(packed, scale)
    rows = (scale[:, 0] >= 2) & (scale[:, 0] <= 252)
    g, w = got[rows], want[rows]
    # bf16 holds every fp4 * 2^(s-127) exactly in this range; zeros compared by value
    assert np.array_equal(g, w)
    nz = w != 0
    assert np.array_equal(np.signbit(g[nz]), np.signbit(w[nz]))
