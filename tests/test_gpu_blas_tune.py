"""Library GEMM tuning for the captured round (`blas_tune`, the reference's startup TunableOp
search, `blas_tune.py:178-255`): a session searches the shapes it meets, leaves tuning off and
the lookup on, and the round routes a tuned K = 8192 projection back to the library; a runner
that tunes in its warm-up round still validates its capture against the eager round."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import blas_tune
import graph_mtp
import verify_model as vm
from tests import model_helpers as mh

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _untuned(monkeypatch, tmp_path):
    monkeypatch.setenv("MTPK_BLAS_TUNE_DIR", str(tmp_path))
    blas_tune.reset()
    yield
    blas_tune.reset()


def test_session_tunes_the_wide_projection_and_routes_it(dev) -> None:
    g = torch.Generator(dev).manual_seed(2)
    w = (torch.randn(4096, 8192, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(192, 8192, device=dev, generator=g).to(torch.bfloat16)
    want = x.float() @ w.float().t()
    assert vm._dense_wide_rows(192, w)  # untuned: the skinny GEMM's row groups
    with blas_tune.session(dev):
        assert blas_tune.prefers_library(192, 4096, 8192)
        assert not vm._dense_wide_rows(192, w)
        F.linear(x, w)
    assert not torch.cuda.tunable.tuning_is_enabled() and torch.cuda.tunable.is_enabled()
    tuned = blas_tune.tuned(192, 4096, 8192)
    assert (192, 4096, 8192) in blas_tune.tuned_shapes() or not tuned
    assert vm._dense_wide_rows(192, w) == (not tuned)
    got = vm.linear(x, w)  # the tuned solution (or the skinny GEMM if the default won)
    torch.testing.assert_close(got.float(), want, rtol=2e-2, atol=2e-2)
    again = vm.linear(x, w)
    assert torch.equal(got, again)  # no search after the session: the same solution each call


def test_runner_tunes_in_its_warm_up_round_and_validates(dev) -> None:
    runner = graph_mtp.GraphMTPRunner(mh.build(dev, k=3, lanes=4), capacity=4, tune_blas=True)
    assert runner.prepare() is True and runner.validated == {1: True, 2: True, 4: True}
    assert not torch.cuda.tunable.tuning_is_enabled()
    ids = mh.prompts(2)
    twin = mh.build(dev, k=3, lanes=4)
    toks, pos = [], []
    for lane, p in enumerate(ids):
        toks.append(int(twin.argmax(twin.prefill(lane, p)[None])[0]))
        runner.model.prefill(lane, p)
        pos.append(len(p))
    want = graph_mtp.MTPVerifyRunner(twin, capacity=4).speculative_decode([0, 1], toks, pos)
    assert runner.speculative_decode([0, 1], toks, pos) == want
