"""Compile the gfx950 HIP kernels into ``_lib/libkoemi_hip.so``.

The library is built ahead of time, in-tree, with ``hipcc`` (it cross-compiles
for gfx950 without a GPU). Nothing is compiled at import or call time: the
operator fronts load the prebuilt library and raise if it is missing.

Run ``python -m koemi_amd._build`` (with ``koemi-5hom_amd`` on ``sys.path``) or
call :func:`build_library`.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR.parent / "csrc"
BUILD_DIR = PACKAGE_DIR.parent / "_build"
LIBRARY_DIR = PACKAGE_DIR / "_lib"
LIBRARY_PATH = LIBRARY_DIR / "libkoemi_hip.so"
INCLUDE_DIR = PACKAGE_DIR.parent.parent / "include"
ROCM_LIB = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "lib"

SOURCES = (
    "abi.hip",
    "affine_scan.hip",
    "rmsnorm_silu.hip",
    "surprise.hip",
    "moe_route.hip",
    "moe_permute.hip",
    "moe_grouped_mlp.hip",
    "moe_combine.hip",
    "memory.hip",
    "salient_read.hip",
    "gates.hip",
    "blas.hip",
    "assoc_memory.hip",
    "herm_glue.hip",
    "linear_rows.hip",
    "gated_projection.hip",
    "stream_probe.hip",
    "refine.hip",
)

ARCH = "gfx950"

# Packed fp32 VALU ops (v_pk_{add,mul,fma}_f32) are disabled for every kernel:
# the compiler otherwise forms them from ordinary float code.
HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    # Code object v5: loadable by the ROCm 7.0 HIP runtime that PyTorch bundles
    # (the library binds to that runtime instance, so torch's streams are valid here).
    "-mcode-object-version=5",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
)


def hipcc_path() -> str:
    candidate = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(candidate).exists():
        raise RuntimeError("hipcc was not found; the gfx950 kernels cannot be built")
    return candidate


def _compile(source: Path, obj: Path, verbose: bool) -> None:
    cmd = [hipcc_path(), *HIPCC_FLAGS, "-I", str(INCLUDE_DIR), "-c", str(source), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stdout}\n{result.stderr}")
    noise = [
        line
        for line in result.stderr.splitlines()
        if line.strip() and "is not a recognized feature for this target" not in line
    ]
    if noise and verbose:
        print("\n".join(noise), flush=True)


def build_library(*, verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every kernel source and link the shared library; returns its path."""

    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIBRARY_DIR.mkdir(parents=True, exist_ok=True)
    sources = [SOURCE_DIR / name for name in SOURCES]
    missing = [str(path) for path in sources if not path.is_file()]
    if missing:
        raise RuntimeError(f"missing kernel sources: {missing}")
    objects = [BUILD_DIR / (path.stem + ".o") for path in sources]
    workers = jobs or min(len(sources), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda pair: _compile(pair[0], pair[1], verbose), zip(sources, objects)))
    tmp = LIBRARY_PATH.with_suffix(".so.tmp")
    # rocBLAS (the salient read's plain GEMMs): linked by soname librocblas.so.5, which
    # resolves at run time to the rocBLAS PyTorch has loaded, on PyTorch's HIP runtime.
    cmd = [hipcc_path(), f"--offload-arch={ARCH}", "-mcode-object-version=5", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objects), f"-L{ROCM_LIB}", "-lrocblas"]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking libkoemi_hip.so failed:\n{result.stdout}\n{result.stderr}")
    os.replace(tmp, LIBRARY_PATH)
    return LIBRARY_PATH


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
