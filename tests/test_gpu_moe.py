"""The HIP routed MXFP4 MoE (`mxfp4_gemv.fused_moe` -> `mtpk_fused_moe`) against the fp64 CPU
oracle and, at full width, a torch fp32 reference built on the bit-exact device dequant.

Bars: fp32 activations at the reference's small shapes, max-abs/max < 1e-5 (the reference's
own bar, `test_mxfp4_fused_gemv.py:246-258`); bf16 activations, rel-L2 <= 2e-3 (north star);
zero-weight / unowned assignments exact zeros; repeat launches bit-identical.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import mxfp4
import mxfp4_gemv
from oracle import moe_ref
from oracle.mxfp4_ref import bf16_round
from tests.moe_inputs import random_experts, random_routing, zipf_routing

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())
SMALL = GOLDEN["moe_small_shapes"]


def to_dev(ex, dev):
    return {k: torch.from_numpy(np.ascontiguousarray(v)).to(dev) for k, v in ex.items()}


def run(x, dex, a_e, a_w, top_k, span, dev, **kw):
    return mxfp4_gemv.fused_moe(
        x, dex, (torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev)), top_k, span, **kw
    )


@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k", SMALL)
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_small_fp32_matches_oracle(dev, tokens, experts, hidden, inter, top_k, seed):
    ex = random_experts(experts, hidden, inter, seed=seed)
    a_e, a_w = random_routing(tokens, experts, top_k, seed=seed + 100)
    x = np.random.default_rng(seed).standard_normal((tokens, hidden)).astype(np.float32)
    want = moe_ref.reference_moe(x, ex, a_e, a_w, top_k, (0, experts))
    got = run(torch.from_numpy(x).to(dev), to_dev(ex, dev), a_e, a_w, top_k, (0, experts), dev)
    assert got.dtype == torch.float32 and got.shape == (tokens, hidden)
    assert moe_ref.relative_error(got.cpu().numpy(), want) < 1e-5


@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k", SMALL)
def test_small_bf16_matches_oracle(dev, tokens, experts, hidden, inter, top_k):
    ex = random_experts(experts, hidden, inter, seed=5)
    a_e, a_w = random_routing(tokens, experts, top_k, seed=6)
    x = bf16_round(np.random.default_rng(7).standard_normal((tokens, hidden)).astype(np.float32))
    want = bf16_round(moe_ref.reference_moe(x, ex, a_e, a_w, top_k, (0, experts)))
    got = run(torch.from_numpy(x).to(dev, torch.bfloat16), to_dev(ex, dev), a_e, a_w, top_k,
              (0, experts), dev)
    assert got.dtype == torch.bfloat16
    assert moe_ref.rel_l2(got.float().cpu().numpy(), want) <= 2e-3


# Many assignments per expert: hot experts span several 16-token work units (each unit
# streams the expert's weights for its own rows), on the LDS kernels (bf16 x, K and inter
# multiples of 512) and the register kernels (fp32 x, other widths). Zipf routing puts unit
# counts of 1..8 in one launch, with ragged last units.
MANY = [
    (128, 8, 256, 96, 6, "zipf", np.float32),
    (160, 40, 256, 64, 4, "zipf", np.float32),
    (96, 12, 512, 512, 8, "uniform", "bf16"),
    (160, 40, 512, 512, 4, "zipf", "bf16"),
    (64, 24, 1024, 1024, 10, "zipf", "bf16"),
    # the LDS kernels at three and four 512-K chunks (K = 1536 and 2048), with 4-wave
    # (80 tokens) and 8-wave (160, 200) gate_up workgroups
    (80, 40, 1536, 1024, 10, "zipf", "bf16"),
    (160, 24, 1536, 1024, 8, "zipf", "bf16"),
    (200, 32, 2048, 1024, 6, "uniform", "bf16"),
]


@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k,routing,x_dtype", MANY)
def test_many_units_per_expert_match_oracle(dev, tokens, experts, hidden, inter, top_k, routing, x_dtype):
    ex = random_experts(experts, hidden, inter, seed=tokens + experts)
    if routing == "zipf":
        a_e, a_w = zipf_routing(tokens, experts, top_k, seed=experts, zero_frac=0.05)
    else:
        a_e, a_w = random_routing(tokens, experts, top_k, seed=experts)
    x = np.random.default_rng(tokens).standard_normal((tokens, hidden)).astype(np.float32)
    if x_dtype == "bf16":
        x = bf16_round(x)
        xt = torch.from_numpy(x).to(dev, torch.bfloat16)
    else:
        xt = torch.from_numpy(x).to(dev)
    want = moe_ref.reference_moe(x, ex, a_e, a_w, top_k, (0, experts))
    got = run(xt, to_dev(ex, dev), a_e, a_w, top_k, (0, experts), dev).float().cpu().numpy()
    if x_dtype == "bf16":
        assert moe_ref.rel_l2(got, bf16_round(want)) <= 2e-3
    else:
        assert moe_ref.relative_error(got, want) < 1e-5
    zero_tok = (a_w.reshape(tokens, top_k) == 0).all(1)
    assert not got[zero_tok].any()


@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k", SMALL)
def test_drops_unowned_experts_and_shards_sum(dev, tokens, experts, hidden, inter, top_k):
    ex = random_experts(experts, hidden, inter, seed=7)
    a_e, a_w = random_routing(tokens, experts, top_k, seed=8)
    x = np.random.default_rng(9).standard_normal((tokens, hidden)).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)
    cuts = [0, experts // 3, 2 * experts // 3, experts]
    parts = []
    for lo, hi in zip(cuts, cuts[1:]):
        if hi == lo:
            continue
        local = {k: v[lo:hi] for k, v in ex.items()}
        got = run(xd, to_dev(local, dev), a_e, a_w, top_k, (lo, hi), dev).cpu().numpy()
        want = moe_ref.reference_moe(x, local, a_e, a_w, top_k, (lo, hi))
        assert moe_ref.relative_error(got, want) < 1e-5 or not want.any()
        parts.append(got.astype(np.float64))
    whole = run(xd, to_dev(ex, dev), a_e, a_w, top_k, (0, experts), dev).cpu().numpy()
    assert moe_ref.relative_error(sum(parts), whole) < 1e-5


@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k", SMALL[1:])
def test_zero_weight_rows_are_exact_zeros(dev, tokens, experts, hidden, inter, top_k):
    ex = random_experts(experts, hidden, inter, seed=11)
    a_e, a_w = random_routing(tokens, experts, top_k, seed=12, zero_rows=(0,))
    x = np.random.default_rng(13).standard_normal((tokens, hidden)).astype(np.float32)
    got = run(torch.from_numpy(x).to(dev), to_dev(ex, dev), a_e, a_w, top_k, (0, experts), dev)
    got = got.cpu().numpy()
    assert not got[0].any()
    want = moe_ref.reference_moe(x, ex, a_e, a_w, top_k, (0, experts))
    assert moe_ref.relative_error(got[1:], want[1:]) < 1e-5


def test_no_live_assignment_gives_zeros(dev):
    ex = random_experts(8, 64, 32, seed=1)
    a_e, a_w = random_routing(3, 8, 2, seed=2)
    x = torch.randn(3, 64, device=dev)
    got = run(x, to_dev({k: v[:4] for k, v in ex.items()}, dev), a_e + 100, a_w, 2, (0, 4), dev)
    assert torch.count_nonzero(got) == 0


@pytest.mark.parametrize("tokens,experts,hidden,inter,top_k", SMALL)
def test_deterministic_and_honors_out_and_scratch(dev, tokens, experts, hidden, inter, top_k):
    ex = to_dev(random_experts(experts, hidden, inter, seed=31), dev)
    a_e, a_w = random_routing(tokens, experts, top_k, seed=32)
    x = torch.randn(tokens, hidden, device=dev, generator=torch.Generator(dev).manual_seed(33))
    first = run(x, ex, a_e, a_w, top_k, (0, experts), dev).clone()
    second = run(x, ex, a_e, a_w, top_k, (0, experts), dev)
    assert torch.equal(first, second)
    out = torch.full((tokens, hidden), float("nan"), device=dev)
    scratch = mxfp4_gemv.moe_scratch(tokens, top_k, experts, inter, hidden, dev, torch.float32)
    scratch.fill_(0xFF)  # NaN-poisoned workspace must not leak into the result
    got = run(x, ex, a_e, a_w, top_k, (0, experts), dev, out=out, inter=scratch)
    assert got.data_ptr() == out.data_ptr()
    assert torch.equal(out, first)


def test_rejects_bad_routing_and_strided_input(dev):
    ex = to_dev(random_experts(4, 64, 32, seed=51), dev)
    a_e, a_w = random_routing(2, 4, 3, seed=52)
    with pytest.raises(ValueError, match="routing must be"):
        run(torch.randn(3, 64, device=dev), ex, a_e, a_w, 3, (0, 4), dev)
    with pytest.raises(ValueError, match="x must be contiguous"):
        run(torch.randn(2, 128, device=dev)[:, ::2], ex, a_e, a_w, 3, (0, 4), dev)


# ---------------------------------------------------------------- real dimensions

H, I, E, TOP_K = 4096, 1024, 512, 10


@pytest.fixture(scope="module")
def real_layer():
    """One layer at real dims on the device: 3.4 GB of MXFP4, config-2/3 byte and scale
    distributions (bytes 0..255, scales 118..130)."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    dev = torch.device("cuda:0")
    g = torch.Generator(dev).manual_seed(60)
    ex = {
        "gate_up": torch.randint(0, 256, (E, 2 * I, H // 2), dtype=torch.uint8, device=dev, generator=g),
        "gate_up_scale": torch.randint(118, 131, (E, 2 * I, H // 32), dtype=torch.uint8, device=dev, generator=g),
        "down": torch.randint(0, 256, (E, H, I // 2), dtype=torch.uint8, device=dev, generator=g),
        "down_scale": torch.randint(118, 131, (E, H, I // 32), dtype=torch.uint8, device=dev, generator=g),
    }
    yield ex
    del ex
    torch.cuda.empty_cache()


def torch_fp32_reference(x, ex, a_e, a_w, top_k):
    """fp32 dequant (bit-exact device kernel) + fp32 matmuls, grouped by expert, on device."""
    dev = x.device
    out = torch.zeros(x.shape[0], H, dtype=torch.float64, device=dev)
    live = (a_w != 0).nonzero().flatten()
    experts = a_e[live].unique()
    xf = x.float()
    for e in experts.tolist():
        sel = live[a_e[live] == e]
        tok = sel // top_k
        gu = mxfp4.dequant_mxfp4(ex["gate_up"][e], ex["gate_up_scale"][e], torch.float32)
        dn = mxfp4.dequant_mxfp4(ex["down"][e], ex["down_scale"][e], torch.float32)
        h = (xf[tok].double() @ gu.double().T)
        act = torch.nn.functional.silu(h[:, :I]) * h[:, I:]
        y = act @ dn.double().T
        out.index_add_(0, tok, y * a_w[sel, None].double())
    return out.float()


@pytest.mark.parametrize("tokens,seed", [(1, 0), (32, 1), (192, 2)])
def test_real_dims_rel_l2(real_layer, tokens, seed):
    dev = torch.device("cuda:0")
    print(f"real-dims MoE M={tokens}", flush=True)
    if tokens == 1:
        a_e, a_w = random_routing(1, E, TOP_K, seed=seed + 300)
    else:
        a_e, a_w = zipf_routing(tokens, E, TOP_K, seed=seed + 300, zero_frac=0.05)
    x = torch.randn(tokens, H, device=dev, generator=torch.Generator(dev).manual_seed(seed)).to(torch.bfloat16)
    ae, aw = torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev)
    got = mxfp4_gemv.fused_moe(x, real_layer, (ae, aw), TOP_K, (0, E)).float()
    ref = torch_fp32_reference(x, real_layer, ae.long(), aw, TOP_K)
    ref_b = ref.to(torch.bfloat16).float()
    err = (torch.linalg.norm(got - ref_b) / torch.linalg.norm(ref_b)).item()
    print(f"  rel-L2 vs fp32 reference = {err:.3e}", flush=True)
    assert err <= 2e-3
    zero_tok = (aw.view(tokens, TOP_K) == 0).all(1)
    assert torch.count_nonzero(got[zero_tok]) == 0
    # fp64 numpy oracle on a few tokens (their experts copied to the host)
    pick = list(range(min(tokens, 3)))
    sel = np.concatenate([np.arange(t * TOP_K, (t + 1) * TOP_K) for t in pick])
    used = np.unique(a_e[sel])
    sub = {k: v[torch.from_numpy(used).to(dev).long()].cpu().numpy() for k, v in real_layer.items()}
    remap = {int(e): i for i, e in enumerate(used)}
    sub_e = np.array([remap[int(e)] for e in a_e[sel]], np.int32)
    xs = x[pick].float().cpu().numpy()
    want = bf16_round(moe_ref.reference_moe(xs, sub, sub_e, a_w[sel], TOP_K, (0, len(used))))
    err64 = moe_ref.rel_l2(got[pick].cpu().numpy(), want)
    print(f"  rel-L2 vs fp64 oracle (tokens {pick}) = {err64:.3e}", flush=True)
    assert err64 <= 2e-3


@pytest.mark.parametrize("tokens", [1, 192])
def test_real_dims_edge_scale_blocks(real_layer, tokens):
    """Live experts whose gate_up and down rows carry scale-0 (pinned +-0.0) and scale-1
    (subnormal products) blocks, on the direct path (1 token) and the LDS unit path (192),
    against the fp64 oracle with the kernels' scale convention and the fp32 device reference
    (exact dequant). The payload is restored afterwards."""
    dev = torch.device("cuda:0")
    print(f"edge-scale MoE M={tokens}", flush=True)
    a_e, a_w = zipf_routing(tokens, E, TOP_K, seed=tokens + 500, zero_frac=0.05)
    used = torch.from_numpy(np.unique(a_e)).to(dev).long()
    saved = {k: real_layer[k][used].clone() for k in ("gate_up_scale", "down_scale")}
    try:
        for k in saved:
            s = real_layer[k][used]
            flat = s.view(-1)
            flat[0::7] = 0
            flat[3::11] = 1
            real_layer[k][used] = s
        x = torch.randn(tokens, H, device=dev, generator=torch.Generator(dev).manual_seed(tokens)).to(torch.bfloat16)
        ae, aw = torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev)
        got = mxfp4_gemv.fused_moe(x, real_layer, (ae, aw), TOP_K, (0, E)).float()
        ref_b = torch_fp32_reference(x, real_layer, ae.long(), aw, TOP_K).to(torch.bfloat16).float()
        err = (torch.linalg.norm(got - ref_b) / torch.linalg.norm(ref_b)).item()
        print(f"  rel-L2 vs fp32 reference = {err:.3e}", flush=True)
        assert err <= 2e-3
        pick = list(range(min(tokens, 2)))
        sel = np.concatenate([np.arange(t * TOP_K, (t + 1) * TOP_K) for t in pick])
        sub_ids = np.unique(a_e[sel])
        sub = {k: v[torch.from_numpy(sub_ids).to(dev).long()].cpu().numpy() for k, v in real_layer.items()}
        remap = {int(e): i for i, e in enumerate(sub_ids)}
        sub_e = np.array([remap[int(e)] for e in a_e[sel]], np.int32)
        want = bf16_round(moe_ref.reference_moe(x[pick].float().cpu().numpy(), sub, sub_e, a_w[sel],
                                                TOP_K, (0, len(sub_ids)), kernel_scales=True))
        err64 = moe_ref.rel_l2(got[pick].cpu().numpy(), want)
        print(f"  rel-L2 vs fp64 oracle = {err64:.3e}", flush=True)
        assert err64 <= 2e-3
    finally:
        for k, v in saved.items():
            real_layer[k][used] = v


@pytest.mark.parametrize("tokens", [1, 7, 48, 192])
def test_real_dims_pile_up(real_layer, tokens):
    """Every token routed to the same ten experts (the reference's `pile_up` case,
    `test_moe_hip.py:198-222`): at 192 tokens each expert carries twelve 16-token units in one
    launch, all reading the same weights. Against the fp32 device reference, and the direct
    path (1 token) and unit path must agree with it alike."""
    dev = torch.device("cuda:0")
    print(f"pile-up MoE M={tokens}", flush=True)
    rng = np.random.default_rng(tokens + 900)
    hot = rng.permutation(E)[:TOP_K].astype(np.int32)
    a_e = np.tile(hot, tokens)
    a_w = rng.random((tokens, TOP_K)).astype(np.float32)
    a_w = (a_w / a_w.sum(-1, keepdims=True)).reshape(-1)
    x = torch.randn(tokens, H, device=dev, generator=torch.Generator(dev).manual_seed(tokens + 900)).to(torch.bfloat16)
    ae, aw = torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev)
    got = mxfp4_gemv.fused_moe(x, real_layer, (ae, aw), TOP_K, (0, E)).float()
    ref_b = torch_fp32_reference(x, real_layer, ae.long(), aw, TOP_K).to(torch.bfloat16).float()
    err = (torch.linalg.norm(got - ref_b) / torch.linalg.norm(ref_b)).item()
    print(f"  rel-L2 vs fp32 reference = {err:.3e}", flush=True)
    assert err <= 2e-3
    # a token's output does not depend on which other tokens share its units
    one = mxfp4_gemv.fused_moe(x[-1:], real_layer, (ae[:TOP_K], aw[-TOP_K:]), TOP_K, (0, E)).float()
    err1 = (torch.linalg.norm(got[-1:] - one) / torch.linalg.norm(one)).item()
    assert err1 <= 2e-3


@pytest.mark.parametrize("tokens", [3, 48])
def test_real_dims_fp32_activations(real_layer, tokens):
    """fp32 x at real dims (split into three bf16 planes, 3-plane intermediate): the direct path
    (3 tokens) and the unit path, against the fp32 device reference without bf16 rounding."""
    dev = torch.device("cuda:0")
    print(f"real-dims MoE fp32 x M={tokens}", flush=True)
    a_e, a_w = zipf_routing(tokens, E, TOP_K, seed=tokens + 700, zero_frac=0.05)
    x = torch.randn(tokens, H, device=dev, generator=torch.Generator(dev).manual_seed(tokens + 700))
    ae, aw = torch.from_numpy(a_e).to(dev).long(), torch.from_numpy(a_w).to(dev)
    got = mxfp4_gemv.fused_moe(x, real_layer, (ae, aw), TOP_K, (0, E))
    assert got.dtype == torch.float32
    ref = torch_fp32_reference(x, real_layer, ae, aw, TOP_K)
    err = (torch.linalg.norm(got - ref) / torch.linalg.norm(ref)).item()
    print(f"  rel-L2 vs fp32 reference = {err:.3e}", flush=True)
    assert err <= 1e-5


def test_real_dims_expert_shards_sum_to_the_whole(real_layer):
    """Expert-parallel sharding at real dims (192 rows, int64 routing, fp32 x so that the shard
    outputs carry no bf16 rounding): the outputs of the four 128-expert shards (each dropping the
    other shards' assignments on the device) sum to the unsharded layer, and each matches its
    own fp32 reference."""
    dev = torch.device("cuda:0")
    a_e, a_w = zipf_routing(192, E, TOP_K, seed=801, zero_frac=0.05)
    x = torch.randn(192, H, device=dev, generator=torch.Generator(dev).manual_seed(801))
    ae, aw = torch.from_numpy(a_e).to(dev).long(), torch.from_numpy(a_w).to(dev)
    whole = mxfp4_gemv.fused_moe(x, real_layer, (ae, aw), TOP_K, (0, E)).double()
    parts = torch.zeros_like(whole)
    for lo in range(0, E, 128):
        local = {k: v[lo:lo + 128] for k, v in real_layer.items()}
        got = mxfp4_gemv.fused_moe(x, local, (ae, aw), TOP_K, (lo, lo + 128)).double()
        own = (ae >= lo) & (ae < lo + 128)
        ref = torch_fp32_reference(x, real_layer, ae, aw * own, TOP_K).double()
        err = (torch.linalg.norm(got - ref) / torch.linalg.norm(ref)).item()
        assert err <= 1e-5
        parts += got
    err = (torch.linalg.norm(parts - whole) / torch.linalg.norm(whole)).item()
    print(f"  rel-L2 of the shard sum vs the whole = {err:.3e}", flush=True)
    assert err <= 1e-5


def test_real_dims_repeat_is_bit_identical(real_layer):
    dev = torch.device("cuda:0")
    a_e, a_w = zipf_routing(192, E, TOP_K, seed=9, zero_frac=0.05)
    x = torch.randn(192, H, device=dev).to(torch.bfloat16)
    r = (torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev))
    a = mxfp4_gemv.fused_moe(x, real_layer, r, TOP_K, (0, E)).clone()
    b = mxfp4_gemv.fused_moe(x, real_layer, r, TOP_K, (0, E))
    assert torch.equal(a, b)


@pytest.mark.parametrize("tokens", [1, 4, 48, 192])
def test_shared_term_in_the_combine_equals_the_unfused_ops(real_layer, tokens):
    """`fused_moe(..., shared=, shared_gate=)` (direct path at <= 4 tokens, combine kernel
    above) is bit-identical to `routed + sigmoid(gate) * shared` as separate bf16 torch ops."""
    dev = torch.device("cuda:0")
    a_e, a_w = zipf_routing(tokens, E, TOP_K, seed=tokens, zero_frac=0.05)
    g = torch.Generator(dev).manual_seed(tokens)
    x = torch.randn(tokens, H, device=dev, generator=g).to(torch.bfloat16)
    routing = torch.randn(tokens, E + 1, device=dev, generator=g).to(torch.bfloat16)
    shared = (torch.randn(tokens, H, device=dev, generator=g) * 100).to(torch.bfloat16)
    ae, aw = torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev)
    routed = mxfp4_gemv.fused_moe(x, real_layer, (ae, aw), TOP_K, (0, E))
    want = routed + torch.sigmoid(routing[:, E:]) * shared
    got = mxfp4_gemv.fused_moe(x, real_layer, (ae, aw), TOP_K, (0, E), shared=shared,
                               shared_gate=routing[:, E:])
    assert torch.equal(got, want)


def test_shared_term_fp32(dev):
    ex = to_dev(random_experts(8, 64, 32, seed=70), dev)
    a_e, a_w = random_routing(6, 8, 2, seed=71)
    x = torch.randn(6, 64, device=dev)
    gate = torch.randn(6, 3, device=dev)[:, 1:2]  # a column view with row stride 3
    shared = torch.randn(6, 64, device=dev)
    routed = run(x, ex, a_e, a_w, 2, (0, 8), dev)
    got = run(x, ex, a_e, a_w, 2, (0, 8), dev, shared=shared, shared_gate=gate)
    torch.testing.assert_close(got, routed + torch.sigmoid(gate) * shared, rtol=1e-6, atol=1e-6)
