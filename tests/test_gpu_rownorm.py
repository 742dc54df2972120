"""Row-norm kernel (`mtpk_rownorm`) against the torch spelling of each norm, in fp32 on the
device: Qwen RMSNorm (with residual and RoPE forms), the DeltaNet gated norm and L2 norm, at
config 5's and config 1's shapes, on head slices read in place."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import rownorm
import verify_model as vm

pytestmark = pytest.mark.gpu


def ref_rms(x, w, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)) * (1.0 + w.float())


def close(got, want, dtype):
    if dtype == torch.bfloat16:  # within one bf16 step of the fp32 value
        torch.testing.assert_close(got.float(), want.float(), rtol=2 ** -7, atol=1e-6)
    else:
        torch.testing.assert_close(got.float(), want.float(), rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("rows,dim", [(192, 4096), (48, 4096), (5, 64), (7, 8192), (33, 256)])
def test_rmsnorm_rows(dev, dtype, rows, dim):
    g = torch.Generator(dev).manual_seed(rows + dim)
    x = (torch.randn(rows, dim, device=dev, generator=g) * 3).to(dtype)
    w = (torch.randn(dim, device=dev, generator=g) * 0.02).to(dtype)
    got = rownorm.rmsnorm(x, w, 1e-6)
    assert got.dtype == dtype and got.shape == x.shape
    close(got, ref_rms(x, w, 1e-6), dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_add_rmsnorm_writes_the_sum_in_x_dtype(dev, dtype):
    g = torch.Generator(dev).manual_seed(3)
    x = torch.randn(2, 96, 4096, device=dev, generator=g).to(dtype)
    r = torch.randn(2, 96, 4096, device=dev, generator=g).to(dtype)
    w = (torch.randn(4096, device=dev, generator=g) * 0.02).to(dtype)
    s, y = rownorm.add_rmsnorm(x, r, w, 1e-6)
    assert torch.equal(s, x + r)  # the same rounding as torch's add
    close(y, ref_rms(x + r, w, 1e-6), dtype)


@pytest.mark.parametrize("dtype,heads,hd,rot", [(torch.bfloat16, 32, 256, 64), (torch.float32, 4, 16, 4),
                                                (torch.bfloat16, 2, 128, 32), (torch.float32, 2, 64, 8)])
def test_head_slices_with_rope(dev, dtype, heads, hd, rot):
    """q is the first half of each head of a [B, t, heads, 2 hd] projection, read in place;
    RoPE rotates the stored (output-dtype) norm, as apply_rope does."""
    b, t = 3, 4
    g = torch.Generator(dev).manual_seed(heads * hd + rot)
    qg = torch.randn(b, t, heads, 2 * hd, device=dev, generator=g).to(dtype)
    q = qg[..., :hd]
    w = (torch.randn(hd, device=dev, generator=g) * 0.02).to(dtype)
    pos = torch.randint(0, 500, (b, t), device=dev, generator=g)
    inv = 1.0 / (10000.0 ** (torch.arange(0, rot, 2, device=dev).float() / rot))
    ang = torch.arange(512, device=dev).float()[:, None] * inv[None, :]
    cos, sin = torch.cat((ang, ang), -1).cos(), torch.cat((ang, ang), -1).sin()
    got = rownorm.rmsnorm(q, w, 1e-6, heads=True, rope=(cos, sin, pos.reshape(-1)))
    normed = ref_rms(q, w, 1e-6).to(dtype)
    want = vm.apply_rope(normed, cos[pos][:, :, None], sin[pos][:, :, None])
    close(got, want, dtype)
    # no rope: plain per-head norm of the strided slice
    close(rownorm.rmsnorm(q, w, 1e-6, heads=True), ref_rms(q, w, 1e-6), dtype)


@pytest.mark.parametrize("t", [4, 1])
def test_gated_norm_and_l2(dev, t):
    """DeltaNet's output norm (gate read from a slice of the input projection) and q/k L2. At
    t = 1 the gate view's size-1 dim has a stride other than the row pitch."""
    b, vh, vd = 4, 64, 128
    g = torch.Generator(dev).manual_seed(9)
    x = torch.randn(b, t, vh, vd, device=dev, generator=g)
    proj = torch.randn(b, t, 3 * vh * vd, device=dev, generator=g).to(torch.bfloat16)
    z = proj[..., vh * vd : 2 * vh * vd].reshape(b, t, vh, vd)
    w = torch.randn(vd, device=dev, generator=g).to(torch.bfloat16)
    got = rownorm.gated_rmsnorm(x, z, w, 1e-6, torch.bfloat16)
    y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    want = y * F.silu(z.float())
    close(got, want, torch.bfloat16)
    q = torch.randn(b, t, 16, 128, device=dev, generator=g)
    want = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * 128 ** -0.5
    close(rownorm.l2norm(q, 1e-6, 128 ** -0.5), want, torch.float32)


@pytest.mark.parametrize("dtype,dim", [(torch.bfloat16, 4096), (torch.float32, 64)])
def test_gathered_rows_into_halves_of_one_row(dev, dtype, dim):
    """The MTP head's input row: `rmsnorm(table[ids])` and `rmsnorm(hidden)` written straight
    into the two halves of one concatenated row (the embedding lookup fused, ids read through
    their strides) equal `cat([rmsnorm(table[ids]), rmsnorm(hidden)])` bit for bit, and an id
    outside the table reads its nearest row."""
    g = torch.Generator(dev).manual_seed(dim)
    table = torch.randn(50, dim, device=dev, generator=g).to(dtype)
    hidden = torch.randn(6, 1, dim, device=dev, generator=g).to(dtype)
    w1 = (torch.randn(dim, device=dev, generator=g) * 0.02).to(dtype)
    w2 = (torch.randn(dim, device=dev, generator=g) * 0.02).to(dtype)
    matrix = torch.randint(0, 50, (6, 4), device=dev, generator=g)
    ids = matrix[:, 2:3]  # a column of a token matrix: row stride 4
    x = torch.full((6, 1, 2 * dim), float("nan"), device=dev, dtype=dtype)
    rownorm.rmsnorm(table, w1, 1e-6, gather=ids, out=x[..., :dim])
    rownorm.rmsnorm(hidden, w2, 1e-6, out=x[..., dim:])
    want = torch.cat([rownorm.rmsnorm(table[ids.reshape(-1)].reshape(6, 1, dim), w1, 1e-6),
                      rownorm.rmsnorm(hidden, w2, 1e-6)], dim=-1)
    assert torch.equal(x, want)
    close(x[..., :dim], ref_rms(table[ids.reshape(-1)].reshape(6, 1, dim), w1, 1e-6), dtype)
    bad = torch.tensor([[-3], [7], [50], [10 ** 9]], device=dev)
    got = rownorm.rmsnorm(table, w1, 1e-6, gather=bad)
    near = torch.tensor([0, 7, 49, 49], device=dev)
    assert torch.equal(got, rownorm.rmsnorm(table[near], w1, 1e-6).reshape(4, 1, dim))


def test_rejects_unsupported_layouts(dev):
    x = torch.randn(4, 100, device=dev)
    with pytest.raises(ValueError):
        rownorm.rmsnorm(x, torch.zeros(100, device=dev), 1e-6)  # dim not a multiple of 8
    y = torch.randn(64, 4, device=dev).t()
    with pytest.raises(ValueError):
        rownorm.rmsnorm(y, torch.zeros(64, device=dev), 1e-6)  # last dim not contiguous
