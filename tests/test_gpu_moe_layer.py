"""The whole MoE layer in the routed layer's launches (`mxfp4_gemv.fused_moe_layer` ->
`mtpk_moe_layer`): router GEMM + softmax top-k + routed MXFP4 experts + gated shared expert.

Bars: bit-identical to the same pieces launched one by one on the device (`dense.linear`,
`router_fused.route`, `dense.silu_linear`, `fused_moe(shared=, shared_gate=)`), routing
included, on the direct path (<= 4 tokens) and the unit path; rel-L2 <= 2e-3 against a float64
reference of the whole layer (torch on the device, exact dequant); bit-identical repeats and
graph replays.
"""

import pytest
import torch

import dense
import mxfp4_gemv
import router_fused
import rownorm
from tests.test_gpu_moe import H, I, E, TOP_K, real_layer, torch_fp32_reference  # noqa: F401

pytestmark = pytest.mark.gpu

SHARED_I = 1024


@pytest.fixture(scope="module")
def dense_layer():
    """The router (512 expert rows + the shared gate's row) and the shared expert, bf16."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    dev = torch.device("cuda:0")
    g = torch.Generator(dev).manual_seed(71)
    return {
        "router_gate": (torch.randn(E + 1, H, device=dev, generator=g) * 0.02).to(torch.bfloat16),
        "shared_gate_up": (torch.randn(2 * SHARED_I, H, device=dev, generator=g) * 0.02).to(torch.bfloat16),
        "shared_down": (torch.randn(H, SHARED_I, device=dev, generator=g) * 0.02).to(torch.bfloat16),
    }


def unfused(h, dl, experts):
    """The same layer as one device launch per piece."""
    routing = dense.linear(h, dl["router_gate"])
    top_w, top_i = router_fused.route(routing, E, TOP_K, index_dtype=torch.int32)
    shared = dense.linear(dense.silu_linear(h, dl["shared_gate_up"]), dl["shared_down"])
    out = mxfp4_gemv.fused_moe(h, experts, (top_i.reshape(-1), top_w.reshape(-1)), TOP_K, (0, E),
                               shared=shared, shared_gate=routing[:, E:])
    return out, top_w, top_i


def fused(h, dl, experts):
    t = h.shape[0]
    tw = torch.empty(t, TOP_K, dtype=torch.float32, device=h.device)
    ti = torch.empty(t, TOP_K, dtype=torch.int32, device=h.device)
    out = mxfp4_gemv.fused_moe_layer(h, dl["router_gate"], dl["shared_gate_up"], dl["shared_down"],
                                     experts, TOP_K, (0, E), routing_out=(tw, ti))
    return out, tw, ti


@pytest.mark.parametrize("tokens", [1, 3, 4, 5, 32, 48, 65, 192, 256])
def test_fused_layer_equals_the_unfused_launches(real_layer, dense_layer, tokens):
    dev = torch.device("cuda:0")
    print(f"fused MoE layer M={tokens}", flush=True)
    h = torch.randn(tokens, H, device=dev, generator=torch.Generator(dev).manual_seed(tokens)).to(torch.bfloat16)
    want, w_w, w_i = unfused(h, dense_layer, real_layer)
    got, g_w, g_i = fused(h, dense_layer, real_layer)
    assert torch.equal(g_i, w_i)
    assert torch.equal(g_w, w_w)
    assert torch.equal(got, want)


@pytest.mark.parametrize("tokens", [5, 48, 192, 256])
def test_fused_add_norm_equals_the_layer_then_the_residual_norm(real_layer, dense_layer, tokens):
    """`fused_moe_layer(add_norm=(x, w, eps))` (the combine, the residual add and the next
    RMSNorm in the layer's last launch) returns `rownorm.add_rmsnorm(x, fused_moe_layer(h), w,
    eps)` bit for bit, and the same routing."""
    dev = torch.device("cuda:0")
    print(f"fused MoE layer + add_norm M={tokens}", flush=True)
    g = torch.Generator(dev).manual_seed(300 + tokens)
    h = torch.randn(tokens, H, device=dev, generator=g).to(torch.bfloat16)
    x = (torch.randn(tokens, H, device=dev, generator=g) * 4).to(torch.bfloat16)
    w = (torch.randn(H, device=dev, generator=g) * 0.1).to(torch.bfloat16)
    out, tw, ti = fused(h, dense_layer, real_layer)
    want_s, want_n = rownorm.add_rmsnorm(x, out, w, 1e-6)
    tw2 = torch.empty_like(tw)
    ti2 = torch.empty_like(ti)
    got_s, got_n = mxfp4_gemv.fused_moe_layer(h, dense_layer["router_gate"], dense_layer["shared_gate_up"],
                                              dense_layer["shared_down"], real_layer, TOP_K, (0, E),
                                              routing_out=(tw2, ti2), add_norm=(x, w, 1e-6))
    assert torch.equal(ti2, ti) and torch.equal(tw2, tw)
    assert torch.equal(got_s, want_s)
    assert torch.equal(got_n, want_n)


def test_fused_add_norm_refuses_the_direct_path(real_layer, dense_layer):
    """At most `direct_max_tokens()` rows the layer's down launch writes its output itself: the
    fused form is refused (callers take the layer and then the row norm)."""
    dev = torch.device("cuda:0")
    n = mxfp4_gemv.direct_max_tokens()
    assert not mxfp4_gemv.add_norm_supported(n, H) and mxfp4_gemv.add_norm_supported(n + 1, H)
    h = torch.randn(n, H, device=dev).to(torch.bfloat16)
    with pytest.raises(ValueError):
        mxfp4_gemv.fused_moe_layer(h, dense_layer["router_gate"], dense_layer["shared_gate_up"],
                                   dense_layer["shared_down"], real_layer, TOP_K, (0, E),
                                   add_norm=(h, torch.zeros(H, dtype=torch.bfloat16, device=dev), 1e-6))


def layer_reference(h, dl, experts, top_i, top_w):
    """float64 reference of the layer given its routing: the router's bf16 logits, the routed
    experts from the exact dequant, the shared SwiGLU, out = routed + sigmoid(gate) * shared."""
    hf = h.double()
    routing = (hf @ dl["router_gate"].double().T).to(torch.bfloat16).double()
    routed = torch_fp32_reference(h, experts, top_i.reshape(-1).long(), top_w.reshape(-1), TOP_K).double()
    gu = hf @ dl["shared_gate_up"].double().T
    act = torch.nn.functional.silu(gu[:, :SHARED_I]) * gu[:, SHARED_I:]
    shared = act @ dl["shared_down"].double().T
    return routing, routed + torch.sigmoid(routing[:, E:]) * shared


@pytest.mark.parametrize("tokens", [1, 48])
def test_fused_layer_matches_the_fp64_reference(real_layer, dense_layer, tokens):
    dev = torch.device("cuda:0")
    print(f"fused MoE layer vs fp64 M={tokens}", flush=True)
    h = torch.randn(tokens, H, device=dev, generator=torch.Generator(dev).manual_seed(100 + tokens)).to(torch.bfloat16)
    got, tw, ti = fused(h, dense_layer, real_layer)
    routing, ref = layer_reference(h, dense_layer, real_layer, ti, tw)
    # the selected experts are the top-k of the bf16 router logits (continuous logits: no ties)
    want_i = routing[:, :E].topk(TOP_K, dim=-1).indices
    assert torch.equal(ti.long().sort(-1).values, want_i.sort(-1).values)
    p = torch.softmax(routing[:, :E], dim=-1).gather(1, ti.long())
    assert torch.allclose(tw.double(), p / p.sum(-1, keepdim=True), rtol=0, atol=1e-5)
    ref_b = ref.to(torch.bfloat16).double()
    err = (torch.linalg.norm(got.double() - ref_b) / torch.linalg.norm(ref_b)).item()
    print(f"  rel-L2 vs fp64 reference = {err:.3e}", flush=True)
    assert err <= 2e-3


def test_fused_layer_repeat_and_graph_replay_are_bit_identical(real_layer, dense_layer):
    dev = torch.device("cuda:0")
    outs = {}
    for tokens in (2, 48):
        h = torch.randn(tokens, H, device=dev, generator=torch.Generator(dev).manual_seed(7)).to(torch.bfloat16)
        ws = torch.empty(mxfp4_gemv.layer_workspace_bytes(tokens, H, E + 1, SHARED_I, TOP_K, E, I),
                         dtype=torch.uint8, device=dev)
        out = torch.empty(tokens, H, dtype=torch.bfloat16, device=dev)
        call = lambda: mxfp4_gemv.fused_moe_layer(  # noqa: E731
            h, dense_layer["router_gate"], dense_layer["shared_gate_up"], dense_layer["shared_down"],
            real_layer, TOP_K, (0, E), out=out, workspace=ws)
        eager = call().clone()
        assert torch.equal(call(), eager)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            call()
        for _ in range(3):
            out.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            mxfp4_gemv.fused_moe(h, real_layer, (torch.zeros(tokens * TOP_K, dtype=torch.int32, device=dev),
                                                  torch.ones(tokens * TOP_K, device=dev)), TOP_K, (0, E))
        outs[tokens] = eager
    assert outs[2].shape == (2, H) and outs[48].shape == (48, H)


def test_fused_layer_rejects_bad_shapes(real_layer, dense_layer):
    dev = torch.device("cuda:0")
    h = torch.randn(3, H, device=dev).to(torch.bfloat16)
    with pytest.raises(ValueError):
        mxfp4_gemv.fused_moe_layer(h.float(), dense_layer["router_gate"], dense_layer["shared_gate_up"],
                                   dense_layer["shared_down"], real_layer, TOP_K, (0, E))
    with pytest.raises(ValueError):
        mxfp4_gemv.fused_moe_layer(h, dense_layer["router_gate"][:, :2048], dense_layer["shared_gate_up"],
                                   dense_layer["shared_down"], real_layer, TOP_K, (0, E))
    big = torch.randn(257, H, device=dev).to(torch.bfloat16)
    with pytest.raises(ValueError):
        mxfp4_gemv.fused_moe_layer(big, dense_layer["router_gate"], dense_layer["shared_gate_up"],
                                   dense_layer["shared_down"], real_layer, TOP_K, (0, E))
