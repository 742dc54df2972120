"""Builds `libmtpk.so` (gfx950) in this directory with hipcc, one object per translation unit.

`python build_lib.py` or `build_lib.build()`; `__graft_entry__.build()` calls it. Rebuilds every
time it is called (the build is the compile check), in parallel across translation units.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
INCLUDE = HERE.parent / "include"
LIB = HERE / "libmtpk.so"
OBJ_DIR = HERE / "_build"
ARCH = os.environ.get("MTPK_ARCH", "gfx950")
SOURCES = ["mtpk_runtime.hip", "mtpk_moe.hip", "mtpk_router.hip", "mtpk_accept.hip", "mtpk_deltanet.hip",
           "mtpk_rejection.hip", "mtpk_attention.hip", "mtpk_norm.hip", "mtpk_gemm.hip",
           "mtpk_moe_dense.hip", "mtpk_probe.hip", "mtpk_round.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # no packed-fp32 VALU forms in the code object: some have given wrong results on this part
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    return str(path) if path.exists() else "hipcc"


def _compile(src: str) -> Path:
    obj = OBJ_DIR / (Path(src).stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(7, len(SOURCES))) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
