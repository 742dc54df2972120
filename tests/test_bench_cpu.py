"""bench.py's host-side pieces that need no GPU: the roofline traffic figure read from the
committed rocprofv3 PMC summary, and the routing draw's live-expert count."""

import numpy as np

import bench


def test_profiled_traffic_reads_the_pmc_table():
    # the M = 192 gate_up row of the PMC section: fetched + written GB, both copy-calibrated
    t = bench.profiled_traffic("mtpk::" + bench.gate_up_kernel(192))
    assert t is not None
    alg = 300 * bench.EXPERT_BYTES * 2 / 3  # gate_up is 2/3 of an expert's bytes
    # a plausible launch: more than the bytes of 300 live experts' gate_up, less than 3 GB
    assert alg < t < 3e9
    # a kernel with no PMC row (the trace tables above the section do not count)
    assert bench.profiled_traffic("mtpk::k_moe_prep_gemm<4>") is None
    assert bench.profiled_traffic("mtpk::no_such_kernel") is None


def test_zipf_routing_shape_and_live_experts():
    a_e, a_w = bench.zipf_routing(192, seed=19200)
    assert a_e.shape == (192 * bench.TOP_K,) and a_w.shape == a_e.shape
    # top-k picks of one token are distinct experts
    assert all(np.unique(r).size == bench.TOP_K for r in a_e.reshape(192, bench.TOP_K))
    d = bench.d_live(a_e, a_w)
    assert 250 < d <= bench.E


def test_cpu_threads_follow_the_process_allotment(monkeypatch):
    import os

    import bench

    monkeypatch.setenv("OMP_NUM_THREADS", "3")
    assert bench.cpu_threads() == min(3, os.cpu_count())
    monkeypatch.setenv("OMP_NUM_THREADS", "100000")
    assert bench.cpu_threads() == os.cpu_count()
    monkeypatch.delenv("OMP_NUM_THREADS")
    assert bench.cpu_threads() == os.cpu_count()
