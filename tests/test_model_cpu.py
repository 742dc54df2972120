"""Config 1 (CPU plumbing): the tiny Qwen3.5-MoE through greedy MTP decode, and the layer
math of the verify forward pinned against independent spellings.

The end-to-end requirement is the reference's own invariant: under greedy decoding a
speculative round commits exactly what plain decode steps commit, whatever the draft predicts
(`seed_tests/test_mtp.py:488-513`), and after a round accepting `a` drafts every piece of
per-slot state equals the sequential model's (`seed_tests/test_mtp.py:287-351`).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import attention
import mtp
import verify_model as vm
from tests import model_helpers as mh


@pytest.mark.parametrize("k,mtp_experts", [(1, "quantized"), (3, "quantized"), (3, "dense")])
def test_speculative_decode_matches_greedy(k: int, mtp_experts: str) -> None:
    """2 prompts of 16 ids, 32 generated tokens (config 1 is k = 1); with "dense" the MTP
    layer's experts are bf16, as in the real checkpoint."""
    ids = mh.prompts()
    truth = mh.greedy_truth(mh.build(k=k), ids, mh.GEN_TOKENS)
    spec = mh.build(k=k, mtp_experts=mtp_experts)
    got, toks, pos = [], [], []
    for lane, p in enumerate(ids):
        base = int(spec.argmax(spec.prefill(lane, p)[None])[0])
        got.append([base])
        toks.append(base)
        pos.append(len(p))
    while min(len(g) for g in got) < mh.GEN_TOKENS + 1:
        committed = mtp.speculative_decode(spec, [0, 1], toks, pos)
        for j, c in enumerate(committed):
            assert 1 <= len(c) <= k + 1
            got[j].extend(c)
            pos[j] += len(c)
            toks[j] = c[-1]
    for g, t in zip(got, truth, strict=True):
        assert g[: mh.GEN_TOKENS + 1] == t


@pytest.mark.parametrize("accept", [0, 1, 2, 3])
def test_verify_and_commit_matches_sequential(accept: int) -> None:
    """Force acceptance to exactly `accept` of k = 3 drafts; the committed ids and all slot
    state (DeltaNet conv/recurrent, attention K/V, MTP K/V, hidden seed) must equal plain
    decode's, and the next draft and decode step must agree."""
    k, lane = 3, 0
    ids = mh.prompts(1)
    truth = mh.greedy_truth(mh.build(k=k, lanes=1), ids, k + 1)[0]

    seq = mh.build(k=k, lanes=1)
    seq.prefill(lane, ids[0])
    committed_seq = vm.greedy_reference(seq, lane, truth[0], len(ids[0]), accept + 1)
    assert committed_seq == truth[1 : accept + 2]

    spec = mh.build(k=k, lanes=1)
    spec.prefill(lane, ids[0])
    drafts = mh.forced_drafts(truth, accept, k, spec.cfg.vocab)
    committed = mtp.verify_and_commit(spec, spec.mtp, [lane], [truth[0]], [drafts], [len(ids[0])])
    assert committed == [truth[1 : accept + 2]]

    next_pos = len(ids[0]) + accept + 1
    mh.assert_slot_state_close(spec, seq, lane, next_pos)
    last = committed[0][-1]
    assert mtp.draft(spec, spec.mtp, spec.cached_hidden(lane), [last], [lane], [next_pos]) == mtp.draft(
        seq, seq.mtp, seq.cached_hidden(lane), [last], [lane], [next_pos])
    torch.testing.assert_close(spec.decode([lane], [last], [next_pos]), seq.decode([lane], [last], [next_pos]),
                               rtol=1e-5, atol=1e-6)


def test_budget_and_stop_clamp_the_commit() -> None:
    """A stop id or a budget inside the accepted run ends the commit there
    (`commit_limit`, `mtp.py:704-726`)."""
    k, lane = 3, 0
    ids = mh.prompts(1)
    truth = mh.greedy_truth(mh.build(k=k, lanes=1), ids, k + 1)[0]
    drafts = truth[1 : k + 1]  # all k accepted
    model = mh.build(k=k, lanes=1)
    model.prefill(lane, ids[0])
    assert mtp.verify_and_commit(model, model.mtp, [lane], [truth[0]], [drafts], [len(ids[0])],
                                 budgets=[2]) == [truth[1:3]]
    model = mh.build(k=k, lanes=1)
    model.prefill(lane, ids[0])
    assert mtp.verify_and_commit(model, model.mtp, [lane], [truth[0]], [drafts], [len(ids[0])],
                                 stops=[[truth[2]]]) == [truth[1:3]]


# ---------------------------------------------------------------- layer math


def test_delta_rule_step_matches_matrix_form() -> None:
    """`S' = (I - beta k k^T) e^g S + beta k v^T`, `out = S'^T q`, per head in float64."""
    gen = torch.Generator().manual_seed(0)
    b, h, dk, dv = 2, 3, 5, 4
    state = torch.randn(b, h, dk, dv, generator=gen)
    q, k = torch.randn(b, h, dk, generator=gen), F.normalize(torch.randn(b, h, dk, generator=gen), dim=-1)
    v = torch.randn(b, h, dv, generator=gen)
    g, beta = -torch.rand(b, h, generator=gen), torch.rand(b, h, generator=gen)
    new, out = vm.delta_rule_step(state, q, k, v, g, beta)
    for i in range(b):
        for j in range(h):
            s = state[i, j].double().numpy()
            kk, qq, vv = k[i, j].double().numpy(), q[i, j].double().numpy(), v[i, j].double().numpy()
            bb, gg = float(beta[i, j]), float(g[i, j])
            want = (np.eye(dk) - bb * np.outer(kk, kk)) @ (np.exp(gg) * s) + bb * np.outer(kk, vv)
            np.testing.assert_allclose(new[i, j].numpy(), want, rtol=1e-5, atol=1e-6)
            np.testing.assert_allclose(out[i, j].numpy(), want.T @ qq, rtol=1e-5, atol=1e-6)
    assert torch.equal(state, state.clone())  # input untouched (new tensor returned)


def test_causal_conv_matches_conv1d() -> None:
    gen = torch.Generator().manual_seed(1)
    b, c, k1, t = 2, 6, 3, 5
    window = torch.randn(b, c, k1 + t, generator=gen)
    weight = torch.randn(c, k1 + 1, generator=gen)
    want = F.silu(F.conv1d(window, weight[:, None, :], groups=c))
    torch.testing.assert_close(vm.causal_conv_rows(window, weight, t), want, rtol=1e-5, atol=1e-6)


def test_paged_attention_matches_dense_per_lane() -> None:
    """Paged rows through a shuffled block table == dense causal softmax attention per lane
    and head (brute force)."""
    gen = torch.Generator().manual_seed(2)
    bs, lanes, heads, kvh, hd, t = 4, 2, 4, 2, 8, 3
    tables = vm.BlockTables(lanes, 32, bs, torch.device("cpu"), seed=3)
    base = [9, 5]
    for j, p in enumerate(base):
        tables.grow(j, p + t)
    k_pool = torch.randn(tables.rows, kvh, hd, generator=gen)
    v_pool = torch.randn(tables.rows, kvh, hd, generator=gen)
    q = torch.randn(lanes, heads, t, hd, generator=gen)
    v_cache = attention.v_blocks(v_pool, bs)
    assert torch.equal(attention.v_rows(v_cache), v_pool)
    got = vm.paged_attention(q, k_pool, v_cache, tables.table, torch.tensor(base), tables.max_blocks, bs, 0.3)
    for j, p in enumerate(base):
        rows = tables.physical_rows(torch.tensor([j]), torch.arange(p + t)[None])[0]
        for hh in range(heads):
            kv = hh // (heads // kvh)
            for s in range(t):
                n = p + s + 1
                sc = (k_pool[rows[:n], kv] @ q[j, hh, s]) * 0.3
                want = sc.softmax(-1) @ v_pool[rows[:n], kv]
                torch.testing.assert_close(got[j, hh, s], want, rtol=1e-5, atol=1e-6)


def test_block_tables_partition_and_padding() -> None:
    tables = vm.BlockTables(3, 40, 16, torch.device("cpu"), seed=0)
    tables.grow(0, 33)
    tables.grow(1, 1)
    tables.grow(0, 20)  # idempotent below the held length
    owned = tables.host[0] + tables.host[1]
    assert len(tables.host[0]) == 3 and len(tables.host[1]) == 1
    assert len(set(owned)) == len(owned) and 0 not in owned
    assert tables.table[2].tolist() == [0] * tables.max_blocks  # unused entries -> block 0
    rows = tables.physical_rows(torch.tensor([0]), torch.arange(33)[None])[0]
    assert len(set(rows.tolist())) == 33
    with pytest.raises(ValueError):
        tables.grow(2, 3 * 16 + 1)


def test_rope_is_a_rotation_of_the_leading_channels() -> None:
    """Norm-preserving on the rotated pairs, identity on the rest, identity at position 0."""
    cfg = vm.tiny_cfg()
    cos, sin = vm.rope_table(cfg, 8, torch.device("cpu"))
    x = torch.randn(8, 2, cfg.head_dim)
    y = vm.apply_rope(x, cos[:, None], sin[:, None])
    r = cfg.rot_dim
    torch.testing.assert_close(y[..., r:], x[..., r:])
    torch.testing.assert_close(y[0], x[0])
    h = r // 2
    pair_x = x[..., :h] ** 2 + x[..., h:r] ** 2
    pair_y = y[..., :h] ** 2 + y[..., h:r] ** 2
    torch.testing.assert_close(pair_y, pair_x, rtol=1e-5, atol=1e-6)


def test_quantize_mxfp4_round_trips_grid_values() -> None:
    """Values already on the e2m1 grid times a power of two come back exactly."""
    import mxfp4

    gen = torch.Generator().manual_seed(4)
    mags = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    code = torch.randint(0, 8, (4, 64), generator=gen)
    sign = torch.where(torch.rand(4, 64, generator=gen) < 0.5, -1.0, 1.0)
    w = mags[code] * sign
    w[:, 0::32] = 6.0  # every block's max is 6, so the block exponent is 0
    exps = torch.tensor([-3.0, 0.0, 2.0, 5.0])[:, None]
    w = w * torch.exp2(exps)
    packed, scale = mxfp4.quantize_mxfp4(w)
    torch.testing.assert_close(mxfp4.dequant_mxfp4(packed, scale, torch.float32), w, rtol=0, atol=0)
    assert scale[:, 0].tolist() == [124, 127, 129, 132]


def test_dense_expert_moe_matches_the_oracle() -> None:
    """The CPU form of the routed bf16 experts (the MTP layer of the real checkpoint) against
    the float64 restatement of the same contract."""
    from oracle import moe_ref

    model = mh.build(k=1, mtp_experts="dense")
    ex = model.mtp.weights["experts"]
    c = model.cfg
    gen = torch.Generator().manual_seed(3)
    h = torch.randn(5, c.hidden, generator=gen)
    top_w, top_i = torch.rand(5, c.top_k, generator=gen).softmax(-1), torch.stack(
        [torch.randperm(c.experts, generator=gen)[: c.top_k] for _ in range(5)])
    got = model._dense_moe(ex, h, top_i, top_w)
    dense = {k: v.float().numpy() for k, v in ex.items()}
    want = moe_ref.dense_moe(h.numpy(), dense, top_i.numpy(), top_w.numpy(), c.top_k, (0, c.experts))
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-4, atol=1e-5 * np.abs(want).max())
