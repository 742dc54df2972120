"""The torch-fp32 CPU restatement used as bench.py's cpu_baseline agrees with the fp64 oracle."""

import numpy as np
import torch

from oracle import cpu_path, moe_ref, router_ref
from tests.moe_inputs import random_experts


def test_routed_grouped_matches_oracle():
    rng = np.random.default_rng(0)
    T, E, H, I, K = 6, 9, 64, 32, 3
    ex = random_experts(E, H, I, seed=1, scale_lo=120, scale_hi=128)
    logits = rng.standard_normal((T, E + 1)).astype(np.float32)
    tw, ti = cpu_path.route(torch.from_numpy(logits), E, K)
    ow, oi = router_ref.route(logits, E, K)
    assert np.array_equal(ti.numpy(), oi) and np.allclose(tw.numpy(), ow, atol=1e-6)
    tw[1] = 0.0  # an inactive token
    x = rng.standard_normal((T, H)).astype(np.float32)
    tex = {k: torch.from_numpy(v) for k, v in ex.items()}
    for span in [(0, E), (3, 7)]:
        sub = {k: v[span[0] : span[1]] for k, v in tex.items()}
        got = cpu_path.routed_grouped(torch.from_numpy(x), sub, ti, tw, span, chunk=2).numpy()
        want = moe_ref.reference_moe(x, {k: v.numpy() for k, v in sub.items()},
                                     ti.reshape(-1).numpy(), tw.reshape(-1).numpy(), K, span)
        assert moe_ref.rel_l2(got, want) < 1e-5
        assert not got[1].any()
