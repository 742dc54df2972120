"""`blas_tune`'s host logic: the tuned-shape table read from TunableOp's results, the routing
it drives in `verify_model.linear`, and the runner's opt-in switch."""

from __future__ import annotations

import torch

import blas_tune
import graph_mtp
import verify_model as vm
from tests import model_helpers as mh


def test_refresh_keeps_tuned_bf16_linear_shapes(monkeypatch) -> None:
    rows = [
        ("Validator", "PT_VERSION", "2.10.0", 0.0),
        ("GemmTunableOp_BFloat16_TN", "tn_4096_192_8192_ld_8192_8192_4096", "Gemm_Rocblas_618588", 0.029),
        ("GemmTunableOp_BFloat16_TN", "tn_1024_192_4096_ld_4096_4096_1024", "Default", 0.013),
        ("GemmTunableOp_float_TN", "tn_64_8_32_ld_32_32_64", "Gemm_Hipblaslt_7", 0.002),
        ("GemmTunableOp_BFloat16_TN", "tn_bad", "Gemm_Rocblas_1", 0.1),
    ]
    monkeypatch.setattr(torch.cuda.tunable, "get_results", lambda: rows)
    try:
        blas_tune._refresh()
        assert blas_tune.tuned_shapes() == {(192, 4096, 8192)}
        assert blas_tune.tuned(192, 4096, 8192) and not blas_tune.tuned(192, 1024, 4096)
        assert blas_tune.prefers_library(192, 4096, 8192)
        assert not blas_tune.prefers_library(48, 4096, 8192)
    finally:
        blas_tune._tuned.clear()
    assert not blas_tune.prefers_library(192, 4096, 8192)


def test_wide_rows_rule_follows_the_table() -> None:
    w = torch.empty(4096, 8192, dtype=torch.bfloat16)
    assert vm._dense_wide_rows(192, w) and not vm._dense_wide_rows(48, w)
    blas_tune._tuned.add((192, 4096, 8192))
    try:
        assert not vm._dense_wide_rows(192, w)
        assert vm._dense_wide_rows(128, w)  # another row count keeps the skinny GEMM
        assert vm._dense_wide_rows(192, torch.empty(4096, 1024, dtype=torch.bfloat16))
    finally:
        blas_tune._tuned.clear()


def test_runner_switch_reads_the_environment(monkeypatch) -> None:
    model = mh.build("cpu", k=3, lanes=2)
    monkeypatch.delenv("MTPK_BLAS_TUNE", raising=False)
    assert not graph_mtp.GraphMTPRunner(model, graph_mtp.EagerBackend(), capacity=2).tune_blas
    monkeypatch.setenv("MTPK_BLAS_TUNE", "1")
    assert graph_mtp.GraphMTPRunner(model, graph_mtp.EagerBackend(), capacity=2).tune_blas
    assert not graph_mtp.GraphMTPRunner(model, graph_mtp.EagerBackend(), capacity=2,
                                        tune_blas=False).tune_blas
    assert not blas_tune.available()  # no GPU here: a tuning runner runs its rounds untuned
    runner = graph_mtp.GraphMTPRunner(model, graph_mtp.EagerBackend(), capacity=2, tune_blas=True)
    assert runner.prepare() is True
