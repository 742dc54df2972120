"""The HIP gated delta rule (`deltanet.delta_rule` -> `mtpk_delta_rule`) against the float64
oracle (`oracle/deltanet_ref.py`): verify mode (every step's output, the state pool left
bit-identical) and commit mode (each row's slot advanced in place by its accepted prefix,
other slots untouched), at config 1's and config 5's head dimensions. fp32 kernel vs float64
oracle: rtol 1e-4 / atol 1e-5 on outputs and states (t <= 4 steps of 16..128-term dots)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import deltanet
from oracle import deltanet_ref as dn

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-4, 1e-5


def _case(seed, slots_total, heads, qk_heads, dk, dv, b, t):
    rng = np.random.default_rng(seed)
    pool = (rng.standard_normal((slots_total, heads, dk, dv)) * 0.1).astype(np.float32)
    q = rng.standard_normal((b, t, qk_heads, dk)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * np.sqrt(dk)
    k = rng.standard_normal((b, t, qk_heads, dk)).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((b, t, heads, dv)).astype(np.float32)
    g = (-rng.random((b, t, heads)) * 0.5).astype(np.float32)
    beta = rng.random((b, t, heads)).astype(np.float32)
    slots = rng.permutation(slots_total)[:b]
    return pool, slots, q, k, v, g, beta


def _dev(dev, *arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in arrays]


SHAPES = [
    # slots_total, heads, qk_heads, dk, dv, rows, t
    (5, 4, 2, 16, 16, 3, 4),  # config 1's DeltaNet heads
    (6, 3, 3, 32, 96, 4, 2),  # ragged dv (lanes past dv idle)
    (4, 2, 1, 64, 64, 2, 1),
    (9, 8, 2, 128, 128, 6, 3),  # config 5's head dims
]


@pytest.mark.parametrize("shape", SHAPES)
def test_verify_outputs_and_state_untouched(dev, shape) -> None:
    pool, slots, q, k, v, g, beta = _case(sum(shape), *shape)
    want_pool, want = dn.delta_rule_rows(pool, slots, q, k, v, g, beta)
    tp, ts, tq, tk, tv, tg, tb = _dev(dev, pool, slots.astype(np.int64), q, k, v, g, beta)
    out = deltanet.delta_rule(tp, ts, tq, tk, tv, tg, tb)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=RTOL, atol=ATOL)
    assert torch.equal(tp.cpu(), torch.from_numpy(pool))


@pytest.mark.parametrize("shape", SHAPES)
def test_commit_advances_each_slot_by_its_prefix(dev, shape) -> None:
    pool, slots, q, k, v, g, beta = _case(100 + sum(shape), *shape)
    b, t = q.shape[:2]
    lengths = np.arange(b) % (t + 2) - (1 if b > 2 else 0)  # includes -1 (clamped to 0) and > t
    want_pool, _ = dn.delta_rule_rows(pool, slots, q, k, v, g, beta, lengths)
    tp, ts, tq, tk, tv, tg, tb, tl = _dev(dev, pool, slots.astype(np.int64), q, k, v, g, beta,
                                          lengths.astype(np.int64))
    assert deltanet.delta_rule(tp, ts, tq, tk, tv, tg, tb, tl, want_out=False) is None
    got = tp.cpu().numpy()
    np.testing.assert_allclose(got, want_pool, rtol=RTOL, atol=ATOL)
    for sl in range(pool.shape[0]):
        j = np.nonzero(slots == sl)[0]
        if len(j) == 0 or min(max(lengths[j[0]], 0), t) == 0:
            np.testing.assert_array_equal(got[sl], pool[sl])  # bit-identical: not advanced


def test_commit_then_verify_equals_longer_verify(dev) -> None:
    """Committing n steps and verifying the rest from the new state gives the outputs of one
    verify over all steps (the round's split into verify + commit is exact in structure)."""
    pool, slots, q, k, v, g, beta = _case(7, 4, 4, 2, 128, 128, 3, 4)
    tp, ts, tq, tk, tv, tg, tb = _dev(dev, pool, slots.astype(np.int64), q, k, v, g, beta)
    full = deltanet.delta_rule(tp, ts, tq, tk, tv, tg, tb).cpu().numpy()
    n = 2
    lengths = torch.full((3,), n, dtype=torch.int64, device=dev)
    deltanet.delta_rule(tp, ts, tq[:, :n].contiguous(), tk[:, :n].contiguous(), tv[:, :n].contiguous(),
                        tg[:, :n].contiguous(), tb[:, :n].contiguous(), lengths, want_out=False)
    rest = deltanet.delta_rule(tp, ts, tq[:, n:].contiguous(), tk[:, n:].contiguous(),
                               tv[:, n:].contiguous(), tg[:, n:].contiguous(), tb[:, n:].contiguous())
    np.testing.assert_allclose(rest.cpu().numpy(), full[:, n:], rtol=RTOL, atol=ATOL)


def test_config5_batch_matches_oracle(dev) -> None:
    """Config 5: 48 rows x 64 heads of 128 x 128 over a 48-slot pool, t = 4 (2 rows checked
    against the oracle in full, every row's commit against the verify pass's own steps)."""
    pool, slots, q, k, v, g, beta = _case(11, 48, 64, 16, 128, 128, 48, 4)
    tp, ts, tq, tk, tv, tg, tb = _dev(dev, pool, slots.astype(np.int64), q, k, v, g, beta)
    out = deltanet.delta_rule(tp, ts, tq, tk, tv, tg, tb).cpu().numpy()
    pick = [0, 47]
    _, want = dn.delta_rule_rows(pool, slots[pick], q[pick], k[pick], v[pick], g[pick], beta[pick])
    np.testing.assert_allclose(out[pick], want, rtol=RTOL, atol=ATOL)
    lengths = torch.from_numpy(np.arange(48) % 5).to(dev)
    deltanet.delta_rule(tp, ts, tq, tk, tv, tg, tb, lengths, want_out=False)
    again = deltanet.delta_rule(tp, ts, tq[:, :1].contiguous(), tk[:, :1].contiguous(),
                                tv[:, :1].contiguous(), tg[:, :1].contiguous(), tb[:, :1].contiguous())
    assert torch.isfinite(again).all()


def test_config5_heads_out_of_range_slots_and_unit_lengths(dev) -> None:
    """The k_dim = 128 form (16-byte state loads, quarter-row lanes): rows whose slot lies
    outside the pool get zero outputs and touch no state; commit lengths of 0, 1 and t advance
    each valid slot by exactly that prefix."""
    pool, slots, q, k, v, g, beta = _case(21, 6, 4, 2, 128, 128, 4, 3)
    bad = np.array([slots[0], 6, slots[2], -2], np.int64)
    ok = [0, 2]
    _, want = dn.delta_rule_rows(pool, bad[ok], q[ok], k[ok], v[ok], g[ok], beta[ok])
    tp, ts, tq, tk, tv, tg, tb = _dev(dev, pool, bad, q, k, v, g, beta)
    out = deltanet.delta_rule(tp, ts, tq, tk, tv, tg, tb).cpu().numpy()
    np.testing.assert_allclose(out[ok], want, rtol=RTOL, atol=ATOL)
    assert not out[[1, 3]].any()
    assert torch.equal(tp.cpu(), torch.from_numpy(pool))
    lengths = np.array([1, 3, 3, 0], np.int64)
    want_pool, _ = dn.delta_rule_rows(pool, bad[ok], q[ok], k[ok], v[ok], g[ok], beta[ok], lengths[ok])
    deltanet.delta_rule(tp, ts, tq, tk, tv, tg, tb, torch.from_numpy(lengths).to(dev), want_out=False)
    np.testing.assert_allclose(tp.cpu().numpy(), want_pool, rtol=RTOL, atol=ATOL)
    others = [sl for sl in range(6) if sl not in bad[ok]]
    assert torch.equal(tp.cpu()[others], torch.from_numpy(pool)[others])


@pytest.mark.parametrize("shape", [(9, 8, 2, 128, 128, 6, 3), (5, 4, 2, 16, 16, 3, 4)])
def test_one_launch_commit_equals_the_two(dev, shape) -> None:
    """`deltanet.commit` (`mtpk_deltanet_commit`: the state and the conv window in one launch at
    k_dim 128, the two launches otherwise) leaves both pools exactly as `delta_rule(...,
    lengths)` followed by `conv_commit` does, padding rows (slot -1) included."""
    pool, slots, q, k, v, g, beta = _case(40 + sum(shape), *shape)
    b, t = q.shape[:2]
    slots = slots.astype(np.int64)
    slots[-1] = -1  # a padding row
    lengths = (np.arange(b) % (t + 1)).astype(np.int64)
    gen = torch.Generator().manual_seed(3)
    c, k1, n_conv = 40, 3, pool.shape[0]
    proj = torch.randn(b, t, c + 8, generator=gen).to(torch.bfloat16).to(dev)
    conv = torch.randn(n_conv, c, k1, generator=gen).to(torch.bfloat16).to(dev)
    idx = (torch.from_numpy(lengths)[:, None] + torch.arange(k1)).clamp(max=k1 + t - 1).to(dev)
    tp, ts, tq, tk, tv, tg, tb, tl = _dev(dev, pool, slots, q, k, v, g, beta, lengths)
    want_p, want_c = tp.clone(), conv.clone()
    deltanet.delta_rule(want_p, ts, tq, tk, tv, tg, tb, tl, want_out=False)
    deltanet.conv_commit(want_c, ts, proj, idx, c)
    deltanet.commit(tp, conv, ts, tq, tk, tv, tg, tb, tl, proj, idx, c)
    assert torch.equal(tp, want_p)
    assert torch.equal(conv, want_c)


def test_rejects_bad_shapes(dev) -> None:
    pool, slots, q, k, v, g, beta = _case(3, 4, 2, 1, 16, 16, 2, 2)
    tp, ts, tq, tk, tv, tg, tb = _dev(dev, pool, slots.astype(np.int64), q, k, v, g, beta)
    with pytest.raises(ValueError):
        deltanet.delta_rule(tp, ts, tq[..., :8].contiguous(), tk[..., :8].contiguous(), tv, tg, tb)
    with pytest.raises(ValueError):
        deltanet.delta_rule(tp, ts, tq, tk, tv[:, :1].contiguous(), tg, tb)
    with pytest.raises(ValueError):
        deltanet.delta_rule(tp, ts[:1], tq, tk, tv, tg, tb)
    with pytest.raises(ValueError):
        deltanet.delta_rule(tp.double(), ts, tq, tk, tv, tg, tb)


# ---------------------------------------------------------------- verify-row preparation


def _torch_prep(proj, conv_state, slots, conv_w, a_log, dt_bias, kh, kd, vh, vd):
    """The torch chain `deltanet.prep` replaces (verify_model's CPU form of deltanet_verify)."""
    import torch.nn.functional as F

    import verify_model as vm

    b, t, _ = proj.shape
    c = 2 * kh * kd + vh * vd
    qkv, z, b_raw, a_raw = proj.split([c, vh * vd, vh, vh], dim=-1)
    window = torch.cat([conv_state[slots], qkv.transpose(1, 2)], dim=-1)
    mixed = vm.causal_conv_rows(window, conv_w, t).to(proj.dtype).transpose(1, 2)
    q = mixed[..., : kh * kd].reshape(b, t, kh, kd).float()
    k = mixed[..., kh * kd : 2 * kh * kd].reshape(b, t, kh, kd).float()
    v = mixed[..., 2 * kh * kd :].reshape(b, t, vh, vd).float()
    q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6) * kd ** -0.5
    k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    beta = torch.sigmoid(b_raw.float())
    g = -a_log.float().exp() * F.softplus(a_raw.float() + dt_bias.float())
    return q, k, v, g, beta


@pytest.mark.parametrize("dtype,b,t,kh,kd,vh,vd,slots_total", [
    (torch.bfloat16, 48, 4, 16, 128, 64, 128, 50),  # config 5's DeltaNet at 192 verify rows
    (torch.float32, 2, 4, 2, 16, 4, 16, 3),         # config 1
    (torch.bfloat16, 3, 1, 2, 256, 4, 192, 4),      # one step, wide heads
])
def test_prep_matches_the_torch_chain(dev, dtype, b, t, kh, kd, vh, vd, slots_total) -> None:
    g = torch.Generator(device="cpu").manual_seed(b + t)
    c = 2 * kh * kd + vh * vd
    width = c + vh * vd + 2 * vh + 8  # padded rows: the kernel takes a row stride
    proj = (torch.randn(b, t, width, generator=g) * 2).to(dtype).to(dev)[..., : width - 8]
    conv_state = torch.randn(slots_total, c, 3, generator=g).to(dtype).to(dev)
    conv_w = (torch.randn(c, 4, generator=g) * 0.3).to(dtype).to(dev)
    a_log = torch.log(torch.rand(vh, generator=g) * 15 + 1).to(dev)
    dt_bias = torch.rand(vh, generator=g).to(dev)
    slots = torch.randperm(slots_total, generator=g)[:b].to(dev)
    got = deltanet.prep(proj, conv_state, slots, conv_w, a_log, dt_bias, kh, kd, vh, vd)
    want = _torch_prep(proj, conv_state, slots, conv_w, a_log, dt_bias, kh, kd, vh, vd)
    for name, x, y in zip(("q", "k", "v", "g", "beta"), got, want, strict=True):
        assert x.shape == y.shape and x.dtype == torch.float32, name
        if dtype == torch.bfloat16 and name in ("q", "k", "v"):
            # a conv output may round to the neighbouring bf16 value (the sums are the same, the
            # exp inside SiLU is not): every element within one bf16 step, and elements beyond
            # fp32 rounding (the norm's sum order) rare
            assert torch.allclose(x, y, rtol=2 ** -7, atol=1e-6), name
            far = (x - y).abs() > 1e-5 * y.abs() + 1e-7
            assert float(far.float().mean()) < 1e-3, name
        else:
            torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-6, msg=name)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_conv_commit_matches_the_gather(dev, dtype) -> None:
    b, t, c, k1, slots_total = 5, 4, 300, 3, 7
    g = torch.Generator(device="cpu").manual_seed(11)
    proj = torch.randn(b, t, c + 20, generator=g).to(dtype).to(dev)
    conv = torch.randn(slots_total, c, k1, generator=g).to(dtype).to(dev)
    slots = torch.tensor([6, 0, 3, 2, 5], device=dev)
    lengths = torch.tensor([1, 4, 2, 3, 1], device=dev)
    idx = (lengths[:, None] + torch.arange(k1, device=dev)[None, :]).clamp(max=k1 + t - 1)
    window = torch.cat([conv[slots], proj[..., :c].transpose(1, 2)], dim=-1)
    want = conv.clone()
    want[slots] = torch.gather(window, 2, idx[:, None, :].expand(-1, c, -1))
    deltanet.conv_commit(conv, slots, proj, idx, c)
    assert torch.equal(conv, want)  # untouched slots 1 and 4 included


def test_out_of_range_slots_touch_no_state(dev) -> None:
    """Rows whose slot id lies outside the pool: the delta rule gives zero outputs and leaves
    every slot as it was (verify and commit), the commit's window update skips them, and the
    prep reads a zero window for them; the in-range rows are unaffected."""
    pool, slots, q, k, v, g, beta = _case(3, 5, 4, 2, 16, 16, 3, 4)
    bad = np.array([slots[0], 5, -1], np.int64)  # row 0 valid, rows 1-2 outside [0, 5)
    want_pool, want = dn.delta_rule_rows(pool, bad[:1], q[:1], k[:1], v[:1], g[:1], beta[:1])
    tp, ts, tq, tk, tv, tg, tb = _dev(dev, pool, bad, q, k, v, g, beta)
    out = deltanet.delta_rule(tp, ts, tq, tk, tv, tg, tb).cpu().numpy()
    np.testing.assert_allclose(out[:1], want, rtol=RTOL, atol=ATOL)
    assert not out[1:].any()
    assert torch.equal(tp.cpu(), torch.from_numpy(pool))
    lengths = torch.tensor([2, 4, 4], device=dev)
    deltanet.delta_rule(tp, ts, tq, tk, tv, tg, tb, lengths, want_out=False)
    want_pool, _ = dn.delta_rule_rows(pool, bad[:1], q[:1], k[:1], v[:1], g[:1], beta[:1], np.array([2]))
    np.testing.assert_allclose(tp.cpu().numpy(), want_pool, rtol=RTOL, atol=ATOL)
    others = [s for s in range(5) if s != bad[0]]
    assert torch.equal(tp.cpu()[others], torch.from_numpy(pool)[others])

    b, t, c, k1 = 3, 4, 96, 3
    gen = torch.Generator(device="cpu").manual_seed(5)
    proj = torch.randn(b, t, c + 8, generator=gen).to(dev)
    conv = torch.randn(4, c, k1, generator=gen).to(dev)
    sl = torch.tensor([2, 4, -3], device=dev)
    idx = torch.full((b, k1), 1, device=dev) + torch.arange(k1, device=dev)
    want_conv = conv.clone()
    want_conv[2] = torch.cat([conv[2], proj[0, :, :c].T], -1)[:, 1 : 1 + k1]
    deltanet.conv_commit(conv, sl, proj, idx, c)
    assert torch.equal(conv, want_conv)

    kh, kd, vh, vd = 1, 16, 2, 32
    cc = 2 * kh * kd + vh * vd
    proj = torch.randn(b, t, cc + vh * vd + 2 * vh, generator=gen).to(dev)
    conv = torch.randn(4, cc, k1, generator=gen).to(dev)
    w = (torch.randn(cc, k1 + 1, generator=gen) * 0.3).to(dev)
    a_log, dt_bias = torch.rand(vh).to(dev), torch.rand(vh).to(dev)
    got = deltanet.prep(proj, conv, sl, w, a_log, dt_bias, kh, kd, vh, vd)
    zeroed = torch.cat([conv, torch.zeros(1, cc, k1, device=dev)])
    sl_z = torch.tensor([2, 4, 4], device=dev)  # the two bad rows read slot 4: all zeros
    want = _torch_prep(proj, zeroed, sl_z, w, a_log, dt_bias, kh, kd, vh, vd)
    for x, y in zip(got, want, strict=True):
        torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-6)
