"""Per-shape library GEMM selection for the round's dense projections (PyTorch TunableOp).

The reference tunes its decode GEMMs at startup (`blas_tune.py:1-48`, `tune` at `:178-255`):
TunableOp times every hipBLASLt / rocBLAS solution of a shape the first time it is called and
keeps the fastest, instead of the library's default heuristic. Here the tuned shapes are
exactly the ones a captured round multiplies: `session()` wraps the runner's eager warm-up round
(`GraphMTPRunner(tune_blas=True)`), so every library GEMM of the round is timed once, with its
real operands and strides, before the round is captured; tuning is then switched off for good
and only the lookup stays on (a graph must not capture a search).

Measured on MI355X at the round's shapes (bf16, graph replay over rotating weight copies):
[192, 8192] x [4096, 8192]^T 58.9 us default, 46 us on the skinny GEMM's row groups, 34.5 us
tuned; [192, 4096] x [17408, 4096]^T 54.0 -> 49.2 us; [48, 4096] x [17408, 4096]^T 39.0 ->
37.3 us. `prefers_library` routes a shape the tuned library serves faster than the skinny GEMM
back to `F.linear` (`verify_model.linear`); on the C5 round (B = 48, k = 3) tuning plus that
routing took 7.87-7.90 ms to 7.82-7.83 ms.

Results live in TunableOp's in-process table and in its results file, which TunableOp writes
when the process exits: `$MTPK_BLAS_TUNE_DIR` (default `~/.cache/mtpk`), one file per GPU
architecture and device ordinal, read back by the next session so later starts skip the search.
TunableOp rejects a file written under other library versions (its validator lines).
"""

from __future__ import annotations

import contextlib
import os
import tempfile
from pathlib import Path

import torch

MAX_TUNING_MS = 30
"""Milliseconds TunableOp may spend timing the candidates of one shape."""

_active = False
_tuned: set[tuple[int, int, int]] = set()


def available() -> bool:
    """TunableOp reaches hipBLASLt / rocBLAS only on a ROCm build with a visible GPU."""
    return torch.version.hip is not None and torch.cuda.is_available()


def results_file(device: torch.device) -> Path:
    """`<dir>/tunableop_<arch>_%d.csv`; `%d` is TunableOp's device-ordinal slot. Falls back to
    the temp directory when the cache directory cannot be created."""
    root = Path(os.environ.get("MTPK_BLAS_TUNE_DIR", Path.home() / ".cache" / "mtpk"))
    try:
        root.mkdir(parents=True, exist_ok=True)
    except OSError:
        root = Path(tempfile.gettempdir())
    arch = torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]
    return root / f"tunableop_{arch}_%d.csv"


def _refresh() -> None:
    """Rebuild the tuned-shape set from TunableOp's table: bf16 `F.linear` GEMMs ("TN": x
    [M, K] by w [N, K]^T, keyed `tn_<N>_<M>_<K>_...`) whose selected solution is not the
    library default."""
    _tuned.clear()
    for op, params, solution, *_ in torch.cuda.tunable.get_results():
        if not op.startswith("GemmTunableOp_BFloat16_TN") or solution == "Default":
            continue
        parts = params.split("_")
        try:
            n, m, k = int(parts[1]), int(parts[2]), int(parts[3])
        except (IndexError, ValueError):
            continue
        _tuned.add((m, n, k))


@contextlib.contextmanager
def session(device: torch.device, max_tuning_ms: int = MAX_TUNING_MS):
    """Within: TunableOp on with tuning on, so each library GEMM shape met is searched once (a
    shape already in the table or its file is not). After: tuning off, lookup left on for the
    rest of the process, and the tuned-shape set refreshed. Raises off ROCm or without a GPU."""
    global _active
    if not available():
        raise RuntimeError("blas_tune.session needs a ROCm GPU (TunableOp)")
    tun = torch.cuda.tunable
    path = results_file(device)
    tun.set_filename(str(path), True)
    tun.enable(True)
    tun.set_max_tuning_duration(max_tuning_ms)
    if Path(tun.get_filename()).exists():
        tun.read_file()
    tun.tuning_enable(True)
    _active = True
    try:
        yield
        torch.cuda.synchronize(device)
    finally:
        tun.tuning_enable(False)
        _active = False
        _refresh()


def tuned(m: int, n: int, k: int) -> bool:
    """Whether `F.linear` of [m, k] by [n, k] has a tuned (non-default) library solution."""
    return (m, n, k) in _tuned


def tuned_shapes() -> set[tuple[int, int, int]]:
    """The (m, n, k) of every tuned `F.linear` shape so far."""
    return set(_tuned)


def prefers_library(m: int, n: int, k: int) -> bool:
    """Whether `F.linear` should take this shape from the library: during a session (so the
    shape gets searched) and afterwards when it was tuned."""
    return _active or tuned(m, n, k)


def reset() -> None:
    """TunableOp off for the process (every GEMM back on the library's default heuristic) and
    the tuned-shape set cleared, so `prefers_library` holds nowhere again."""
    if available():
        torch.cuda.tunable.tuning_enable(False)
        torch.cuda.tunable.enable(False)
    _tuned.clear()
