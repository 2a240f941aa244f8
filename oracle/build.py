"""Build the oracle's C restatement into ``oracle/_build/liboracle.so``.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Contraction is disabled so
that the C statements round exactly as written (explicit fmaf where fused).

The reference's own native code for this path (src/koemi/cuda_kernels/**/*.cu
with ATen/CUB/pybind11 and nvcc) cannot be compiled in this image, so there is
no oracle/_ref build; the oracle is pinned by the reference's tests instead.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SOURCE = ORACLE_DIR / "koemi_oracle.c"
BUILD_DIR = ORACLE_DIR / "_build"
LIBRARY = BUILD_DIR / "liboracle.so"


def build(verbose: bool = False) -> Path:
    compiler = shutil.which("gcc") or "cc"
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [compiler, "-O3", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
           str(SOURCE), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    tmp.replace(LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
