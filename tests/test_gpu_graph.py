"""The MoE layer, router and acceptance captured in one HIP graph: every replay (with eager work
and synchronisations between replays) matches the eager result bit for bit."""

import numpy as np
import pytest
import torch

import graph_mtp
from tests.model_helpers import shape_model
import mxfp4_gemv
import router_fused
from tests.moe_inputs import random_experts

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(dev):
    T, E, H, I, K = 48, 64, 512, 256, 10
    ex = {k: torch.from_numpy(v).to(dev) for k, v in random_experts(E, H, I, seed=3).items()}
    g = torch.Generator(dev).manual_seed(0)
    x = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E + 1, device=dev, generator=g).to(torch.bfloat16)
    runner = mxfp4_gemv.MoeLayerRunner(T, K, E, I, H, dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    buf = graph_mtp.MTPVerifyBuffers(shape_model(H, 4), 12, 4, dev)
    buf.active[:10] = True
    buf.budget.fill_(9)

    def step():
        w, i = router_fused.route(logits, E, K, index_dtype=torch.int32)
        a_w = w.reshape(-1)
        a_w.view(T, K)[::7] = 0.0  # a few inactive rows
        runner.run(x, ex, i.reshape(-1), a_w, (0, E), out)
        sa = out.float().reshape(12, 4, H).argmax(-1)
        buf.token_matrix[:, 1:].copy_(sa[:, :3])
        graph_mtp.accept_round(buf, sa)

    step()
    torch.cuda.synchronize()
    want_out, want_acc = out.clone(), buf.accept_len.clone()
    want_src = buf.packed_src.clone()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # warm the allocator on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        step()
    for r in range(4):
        out.fill_(float("nan"))
        buf.accept_len.fill_(-1)
        buf.packed_src.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_out), f"replay {r}"
        assert torch.equal(buf.accept_len, want_acc), f"replay {r}"
        assert torch.equal(buf.packed_src, want_src), f"replay {r}"
        _ = (x.float() @ x.float().T).sum().item()  # unrelated eager work between replays
    assert np.isfinite(want_out.float().cpu().numpy()).all()
