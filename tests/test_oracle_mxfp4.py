"""Pins oracle.mxfp4_ref against the reference tests' vectors and the OCP closed form."""

import json
from pathlib import Path

import numpy as np

from oracle import mxfp4_ref as mx

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def test_fp4_table_matches_closed_form():
    for code in range(16):
        want = mx.fp4_closed_form(code)
        got = float(mx.FP4_VALUES[code])
        assert got == want and np.signbit(got) == bool(code & 8)


def test_hand_vector_from_reference_tests():
    g = GOLDEN["mxfp4_hand"]
    packed = np.zeros(g["packed_len"], dtype=np.uint8)
    packed[:3] = g["packed_prefix"]
    out = mx.dequant_mxfp4(packed, np.array([128], np.uint8))
    assert out.shape == (32,)
    assert out[:6].tolist() == g["scale_128_first6"]
    assert np.signbit(out[5])  # code 8 is -0.0
    assert np.abs(out[6:]).sum() == 0
    half = mx.dequant_mxfp4(packed, np.array([125], np.uint8))
    assert half[3] == g["scale_125_index3"]


def test_every_byte_at_unit_scale_is_the_table():
    packed = np.arange(256, dtype=np.uint8).reshape(8, 32)
    out = mx.dequant_mxfp4(packed, np.full((8, 2), 127, np.uint8)).reshape(-1)
    for b in range(256):
        assert out[2 * b] == mx.fp4_closed_form(b & 15)
        assert out[2 * b + 1] == mx.fp4_closed_form(b >> 4)
        assert np.signbit(out[2 * b]) == bool(b & 8)


def test_scale_conventions():
    packed = np.full((1, 16), 0x72, np.uint8)  # codes 2 (1.0) and 7 (6.0)
    for s in range(1, 255):
        v = mx.dequant_mxfp4(packed, np.array([[s]], np.uint8))[0]
        assert v[0] == np.float32(2.0 ** (s - 127)) and v[1] == np.float32(6.0 * 2.0 ** (s - 127))
    torch_zero = mx.dequant_mxfp4(packed, np.array([[0]], np.uint8))[0]
    assert torch_zero[0] == np.float32(2.0**-127)  # torch.exp2(-127): a subnormal, not zero
    kern_zero = mx.dequant_mxfp4_kernel(packed, np.array([[0]], np.uint8))[0]
    assert kern_zero[0] == 0.0 and not np.signbit(kern_zero[0])
    inf = mx.dequant_mxfp4(packed, np.array([[255]], np.uint8))[0]
    assert np.isinf(inf[0]) and inf[0] > 0
    nan = mx.dequant_mxfp4(np.zeros((1, 16), np.uint8), np.array([[255]], np.uint8))[0]
    assert np.isnan(nan).all()  # 0 * inf


def test_kernel_and_torch_conventions_agree_off_zero():
    rng = np.random.default_rng(0)
    packed = rng.integers(0, 256, (37, 32), dtype=np.uint8)
    scale = rng.integers(1, 255, (37, 2), dtype=np.uint8)
    a, b = mx.dequant_mxfp4(packed, scale), mx.dequant_mxfp4_kernel(packed, scale)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_quantizer_round_trip():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((4, 64)).astype(np.float32)
    packed, scale, recon = mx.quantize_mxfp4(w)
    assert np.array_equal(mx.dequant_mxfp4(packed, scale), recon)
    # nearest code: the error is at most half the widest gap of the e2m1 grid (2.0) at scale
    step = np.exp2(scale.astype(np.float64) - 127).repeat(32, axis=1)
    assert (np.abs(recon - w) <= step + 1e-6).all()


def test_bf16_rounding_helpers():
    vals = np.array([1.0, 1.00390625, 1.01171875, -3.5, 65504.0, 1e-30], np.float32)
    r = mx.bf16_round(vals)
    # 1 + 2^-8 is a tie between 1.0 and 1 + 2^-7: round to even keeps 1.0
    assert r[1] == 1.0
    assert r[2] == np.float32(1.015625)  # 1 + 3*2^-8 ties to the even 1 + 2^-6
    assert r[3] == -3.5
    assert np.array_equal(mx.bf16_from_bits(mx.bf16_bits(vals)), r)
