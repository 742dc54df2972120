"""Skinny bf16 GEMM (`dense.linear` / `silu_linear` / `argmax_linear` -> `mtpk_gemm_bf16`)
against fp32 torch matmuls of the same bf16 inputs, at the MTP draft step's shapes (B = 48),
decode shapes (M <= 4) and ragged N (the router's 512 + 1 columns); split-K and single-split
paths both run. bf16 outputs are within one bf16 step of the fp32 product; the argmax is
bit-exact against the argmax of the kernel's own bf16 logits."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import dense

pytestmark = pytest.mark.gpu


def _inputs(dev, m, k, n, seed):
    g = torch.Generator(dev).manual_seed(seed)
    x = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    return x, w


def _close(got, want):
    err = (got.float() - want).abs()
    tol = 2 ** -7 * want.abs() + 1e-3 * want.abs().max()
    assert bool((err <= tol).all()), float((err - tol).max())


@pytest.mark.parametrize("m,k,n", [(48, 8192, 4096), (48, 4096, 16384), (48, 4096, 512), (1, 4096, 513),
                                   (4, 1024, 4096), (64, 256, 64), (17, 512, 100), (33, 4096, 20608),
                                   (40, 512, 70000), (64, 256, 66000),  # 8-wave tiles, ragged N
                                   # row groups of 64 (ragged last group, split K, 8-wave tiles)
                                   (192, 4096, 20608), (192, 8192, 4096), (100, 1024, 513),
                                   (256, 256, 66000), (130, 4096, 512),
                                   # the wide form: one group of up to 12 token tiles, 256-row tiles
                                   (192, 4096, 248320), (100, 1024, 140000), (65, 512, 131100),
                                   # ... and of 4 token tiles (17..64 rows, padded) on 512-row tiles
                                   (17, 256, 131100), (48, 4096, 140001), (64, 1024, 131072)])
def test_linear_matches_fp32(dev, m, k, n):
    x, w = _inputs(dev, m, k, n, m + n)
    assert dense.fits(x, w)
    got = dense.linear(x, w)
    assert got.shape == (m, n) and got.dtype == torch.bfloat16
    _close(got, x.float() @ w.float().T)


@pytest.mark.parametrize("m,k,inter", [(48, 4096, 1024), (1, 4096, 1024), (5, 1024, 48), (48, 256, 65552),
                                       (192, 4096, 1024), (77, 512, 96)])
def test_silu_linear_matches_swiglu(dev, m, k, inter):
    x, w = _inputs(dev, m, k, 2 * inter, 7 + m)
    got = dense.silu_linear(x, w)
    y = x.float() @ w.float().T
    want = F.silu(y[:, :inter]) * y[:, inter:]
    _close(got, want)


@pytest.mark.parametrize("m,n", [(48, 248320), (1, 248320), (7, 1000), (192, 248320), (70, 5000),
                                 (100, 248320), (150, 140001), (17, 248320), (64, 131073), (33, 140001)])
def test_argmax_linear_is_the_argmax_of_its_bf16_logits(dev, m, n):
    x, w = _inputs(dev, m, 4096, n, 3 + m)
    idx = dense.argmax_linear(x, w)
    logits = dense.linear(x, w)
    assert torch.equal(idx, logits.float().argmax(-1))  # first occurrence on ties, like argmax
    # and the fp32 product's argmax wherever its top two are clearly apart
    ref = x.float() @ w.float().T
    top = ref.topk(2, dim=-1).values
    clear = (top[:, 0] - top[:, 1]) > 1e-2 * top[:, 0].abs()
    assert torch.equal(idx[clear], ref.argmax(-1)[clear])


def test_argmax_linear_into_a_given_tensor(dev):
    """`out=` receives the same ids (a round buffer's step_argmax rows, written in place)."""
    x, w = _inputs(dev, 192, 4096, 248320, 9)
    out = torch.full((192,), -5, dtype=torch.int64, device=dev)
    assert dense.argmax_linear(x, w, out) is out
    assert torch.equal(out, dense.argmax_linear(x, w))
    with pytest.raises(ValueError):
        dense.argmax_linear(x, w, torch.empty(191, dtype=torch.int64, device=dev))


def test_ties_pick_the_lowest_column(dev):
    x = torch.ones(3, 256, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(640, 256, dtype=torch.bfloat16, device=dev)
    w[[70, 300, 600]] = 1.0  # equal maxima in three tiles
    assert dense.argmax_linear(x, w).tolist() == [70, 70, 70]


def test_rejects_unsupported(dev):
    x, w = _inputs(dev, 4, 300, 64, 1)
    assert not dense.fits(x, w)  # K not a multiple of 256
    x, w = _inputs(dev, 257, 256, 64, 1)
    assert not dense.fits(x, w)  # more than 256 rows
    with pytest.raises(ValueError):
        dense.linear(x, w)
