"""The `mtpk` custom ops without a GPU: registered schemas, fake kernels giving the output
shapes and dtypes (FakeTensor mode and a `make_fx` trace that keeps each op as one node), and no
CPU kernel (a CPU call fails in the dispatcher instead of computing anything)."""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

import mtp
import mtpk_ops  # noqa: F401  (registers the ops)

OPS = ("fused_moe", "moe_layer", "route", "argmax_rows", "greedy_accept", "rejection_sample")


def test_schemas():
    s = {n: str(getattr(torch.ops.mtpk, n).default._schema) for n in OPS}
    assert s["fused_moe"].startswith("mtpk::fused_moe(Tensor x, Tensor gate_up, Tensor gate_up_scale, "
                                     "Tensor down, Tensor down_scale, Tensor a_expert, Tensor a_weight")
    assert "Tensor? shared=None, Tensor? shared_gate=None) -> Tensor" in s["fused_moe"]
    assert s["route"].endswith("-> (Tensor, Tensor)")
    assert s["moe_layer"].endswith("SymInt expert_hi) -> (Tensor, Tensor, Tensor)")
    assert s["greedy_accept"].count("Tensor,") == 10
    assert s["rejection_sample"].endswith("float temperature) -> (Tensor, Tensor, Tensor, Tensor)")


def test_fake_kernels():
    b, t, v, h, e, k = 5, 4, 1000, 256, 16, 4
    with FakeTensorMode():
        out = torch.ops.mtpk.fused_moe(
            torch.empty(6, h, dtype=torch.bfloat16), torch.empty(e, 256, h // 2, dtype=torch.uint8),
            torch.empty(e, 256, h // 32, dtype=torch.uint8), torch.empty(e, h, 64, dtype=torch.uint8),
            torch.empty(e, h, 4, dtype=torch.uint8), torch.empty(6 * k, dtype=torch.int32),
            torch.empty(6 * k), k, 0, e)
        assert out.shape == (6, h) and out.dtype == torch.bfloat16
        lo, lw, li = torch.ops.mtpk.moe_layer(
            torch.empty(6, h, dtype=torch.bfloat16), torch.empty(e + 1, h, dtype=torch.bfloat16),
            torch.empty(512, h, dtype=torch.bfloat16), torch.empty(h, 256, dtype=torch.bfloat16),
            torch.empty(e, 256, h // 2, dtype=torch.uint8), torch.empty(e, 256, h // 32, dtype=torch.uint8),
            torch.empty(e, h, 64, dtype=torch.uint8), torch.empty(e, h, 4, dtype=torch.uint8), k, 0, e)
        assert (lo.shape, lo.dtype, lw.shape, li.dtype) == ((6, h), torch.bfloat16, (6, k), torch.int32)
        w, i = torch.ops.mtpk.route(torch.empty(6, e + 1, dtype=torch.bfloat16), e, k, torch.int32)
        assert (w.shape, w.dtype, i.shape, i.dtype) == ((6, k), torch.float32, (6, k), torch.int32)
        am = torch.ops.mtpk.argmax_rows(torch.empty(2, 3, v))
        assert am.shape == (2, 3) and am.dtype == torch.int64
        acc = torch.ops.mtpk.greedy_accept(
            torch.empty(b, t, dtype=torch.long), torch.empty(b, t - 1, dtype=torch.long),
            torch.empty(b, dtype=torch.bool), torch.empty(b, dtype=torch.long),
            torch.empty(b, dtype=torch.long), torch.empty(b, mtp.MAX_STOP_IDS, dtype=torch.long), 3)
        assert [tuple(x.shape) for x in acc] == [(b,), (b,), (b * t,), (b + 1,), (b, 3), (b, t), (b,),
                                                 (b,), (b,), (b,), (b,)]
        assert acc[3].dtype == torch.int32 and acc[5].dtype == torch.bool and acc[9].dtype == torch.bool
        rej = torch.ops.mtpk.rejection_sample(torch.empty(b, t, v), torch.empty(b, t - 1, v),
                                              torch.empty(b, t - 1, dtype=torch.long),
                                              torch.empty(b, t - 1), torch.empty(b), 0.7)
        assert [tuple(x.shape) for x in rej] == [(b,), (b,), (b, t), (b, t - 1)]


def test_trace_keeps_each_op_whole():
    def f(logits, routing):
        w, i = torch.ops.mtpk.route(routing, 16, 4, torch.int64)
        return torch.ops.mtpk.argmax_rows(logits) + i.sum(-1)

    gm = make_fx(f, tracing_mode="fake")(torch.empty(6, 500), torch.empty(6, 17))
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert "mtpk.route.default" in targets and "mtpk.argmax_rows.default" in targets


def test_no_cpu_kernel():
    with pytest.raises(NotImplementedError):
        torch.ops.mtpk.argmax_rows(torch.zeros(2, 5))
