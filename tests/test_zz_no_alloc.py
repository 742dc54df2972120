"""`mtpk_fused_moe_static`, the MoE entry point that allocates nothing (its scratch is the
library's static device buffer), against `mtpk_fused_moe_shared` with a caller workspace, through
the C ABI: bit-identical outputs on consecutive calls that shrink (192 rows on the wide path, then
32, then 1 on the direct path, the buffer holding the previous call's contents each time), with
the shared term, with fp32 activations, and a call too large for the buffer refused before any
launch."""

import numpy as np
import pytest
import torch

import _mtpk
import mxfp4_gemv
from tests.moe_inputs import random_experts, random_routing, zipf_routing

pytestmark = pytest.mark.gpu

H, I, E, TOP_K = 4096, 1024, 64, 10


def _static(x, ex, ae, aw, top_k, shared=None, gate=None):
    out = torch.empty_like(x)
    rc = _mtpk.lib().mtpk_fused_moe_static(
        x.data_ptr(), _mtpk.float_code(x.dtype), x.shape[0], x.shape[1],
        ex["gate_up"].data_ptr(), ex["gate_up_scale"].data_ptr(), ex["down"].data_ptr(),
        ex["down_scale"].data_ptr(), ex["down"].shape[0], ex["gate_up"].shape[1] // 2,
        ae.data_ptr(), _mtpk.index_code(ae.dtype), aw.data_ptr(), _mtpk.float_code(aw.dtype),
        top_k, 0, ex["down"].shape[0], _mtpk.ptr(shared), _mtpk.float_code(shared.dtype) if shared is not None else 0,
        _mtpk.ptr(gate), _mtpk.float_code(gate.dtype) if gate is not None else 0,
        gate.stride(0) if gate is not None else 0, out.data_ptr(), _mtpk.stream_of(x.device))  # fmt: skip
    _mtpk.check(rc, "mtpk_fused_moe_static")
    return out


@pytest.fixture(scope="module")
def layer():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    dev = torch.device("cuda:0")
    g = torch.Generator(dev).manual_seed(5)
    ex = {
        "gate_up": torch.randint(0, 256, (E, 2 * I, H // 2), dtype=torch.uint8, device=dev, generator=g),
        "gate_up_scale": torch.randint(118, 131, (E, 2 * I, H // 32), dtype=torch.uint8, device=dev, generator=g),
        "down": torch.randint(0, 256, (E, H, I // 2), dtype=torch.uint8, device=dev, generator=g),
        "down_scale": torch.randint(118, 131, (E, H, I // 32), dtype=torch.uint8, device=dev, generator=g),
    }  # fmt: skip
    yield ex
    del ex
    torch.cuda.empty_cache()


def test_static_scratch_matches_the_workspace_entry_point(layer):
    dev = torch.device("cuda:0")
    for tokens in (192, 32, 1):
        print(f"static-scratch MoE M={tokens}", flush=True)
        a_e, a_w = zipf_routing(tokens, E, TOP_K, seed=tokens, zero_frac=0.05)
        ae, aw = torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev)
        x = torch.randn(tokens, H, device=dev, generator=torch.Generator(dev).manual_seed(tokens))
        x = x.to(torch.bfloat16)
        want = mxfp4_gemv.fused_moe(x, layer, (ae, aw), TOP_K, (0, E))
        got = _static(x, layer, ae, aw, TOP_K)
        torch.cuda.synchronize()
        assert torch.equal(got, want), tokens
        gate = torch.randn(tokens, 3, device=dev).to(torch.bfloat16)[:, 1:2]
        shared = torch.randn(tokens, H, device=dev).to(torch.bfloat16)
        want_s = mxfp4_gemv.fused_moe(x, layer, (ae, aw), TOP_K, (0, E), shared=shared, shared_gate=gate)
        assert torch.equal(_static(x, layer, ae, aw, TOP_K, shared, gate), want_s), tokens


def test_static_scratch_fp32_small_shapes():
    dev = torch.device("cuda:0")
    ex = {k: torch.from_numpy(v).to(dev) for k, v in random_experts(8, 256, 128, seed=3).items()}
    for tokens in (40, 3):
        a_e, a_w = random_routing(tokens, 8, 3, seed=tokens)
        ae, aw = torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev)
        x = torch.randn(tokens, 256, device=dev)
        want = mxfp4_gemv.fused_moe(x, ex, (ae, aw), 3, (0, 8))
        assert torch.equal(_static(x, ex, ae, aw, 3), want), tokens


def test_static_scratch_refuses_an_oversized_call(layer):
    dev = torch.device("cuda:0")
    tokens = 400  # the workspace of 400 rows at these dims exceeds the static buffer
    need = _mtpk.lib().mtpk_moe_workspace_bytes(tokens, TOP_K, E, I, H, _mtpk.BF16)
    assert need > _mtpk.MOE_STATIC_SCRATCH
    a_e, a_w = random_routing(tokens, E, TOP_K, seed=1)
    ae, aw = torch.from_numpy(a_e).to(dev), torch.from_numpy(a_w).to(dev)
    x = torch.zeros(tokens, H, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="static buffer"):
        _static(x, layer, ae, aw, TOP_K)
