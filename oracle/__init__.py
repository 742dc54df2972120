"""CPU oracle for the MTP speculative-decode hot path. TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, what the reference engine computes on the path this
repository accelerates: MXFP4 dequantisation, the routed MXFP4 MoE (dequantise then matmul),
the router's softmax/top-k/renormalise chain, greedy acceptance with its commit limit and
rollback indices, and speculative rejection sampling. Each function cites the reference
`file:line` it follows.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import it, and
only as the checker (or, for `cpu_baseline`, as the timed CPU restatement). The product path in
the package never imports it: it runs the HIP library or raises.

Parity status per function (how each is pinned) is listed in each module's header.
"""
