"""Kernel-library status and loading, mirroring ``cuda_kernels/loader.py``.

The reference JIT-compiles each front with ``torch.utils.cpp_extension`` into
a content-addressed cache (loader.py:139-221). This build compiles every
gfx950 kernel ahead of time into one C-ABI library (``_build.py``); loading
checks the GPU runtime and the library's ABI version and never compiles.
The public names, exception classes and the ABI attribute
(``KOEMI_CUDA_ABI_VERSION = 1``) are kept so callers of the reference loader
keep working.
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import torch

from koemi_amd import _native

__all__ = [
    "CUDA_EXTENSION_ABI_VERSION",
    "CudaExtensionLoadError",
    "CudaExtensionUnavailableError",
    "CudaExtensionValidationError",
    "CudaToolchainStatus",
    "cuda_extension_available",
    "detect_cuda_toolchain",
]

CUDA_EXTENSION_ABI_VERSION = _native.ABI_VERSION


class CudaExtensionUnavailableError(RuntimeError):
    """Raised when the GPU runtime or the kernel library is not available."""


class CudaExtensionValidationError(ValueError):
    """Raised when an operator call violates its contract."""


class CudaExtensionLoadError(RuntimeError):
    """Raised when the kernel library cannot be loaded or has a wrong ABI."""


@dataclass(frozen=True)
class CudaToolchainStatus:
    """Snapshot of the GPU runtime and the prebuilt kernel library."""

    runtime_available: bool
    torch_hip_version: str | None
    library_path: Path
    library_built: bool
    reason: str

    @property
    def compiler_available(self) -> bool:
        # Kept for the reference's attribute name: here it means "kernels are built".
        return self.library_built

    @property
    def ready(self) -> bool:
        return self.runtime_available and self.library_built


def detect_cuda_toolchain() -> CudaToolchainStatus:
    """Inspect the ROCm runtime seen by torch and the prebuilt gfx950 library."""

    runtime_available = bool(torch.cuda.is_available())
    hip_version = torch.version.hip
    built = _native.library_built()
    missing: list[str] = []
    if not runtime_available:
        missing.append("torch.cuda.is_available() is False")
    if hip_version is None:
        missing.append("the installed PyTorch has no ROCm build")
    if not built:
        missing.append(f"the kernel library {_native.library_path()} is not built")
    reason = "GPU runtime and gfx950 kernel library are available" if not missing else "; ".join(missing)
    return CudaToolchainStatus(
        runtime_available=runtime_available,
        torch_hip_version=hip_version,
        library_path=Path(_native.library_path()),
        library_built=built,
        reason=reason,
    )


def cuda_extension_available() -> bool:
    """Return whether this process can execute the gfx950 kernels."""

    return detect_cuda_toolchain().ready


def require_library() -> None:
    """Load the kernel library or raise the loader's typed errors."""

    status = detect_cuda_toolchain()
    if not status.ready:
        raise CudaExtensionUnavailableError(f"GPU kernel library is unavailable: {status.reason}.")
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise CudaExtensionLoadError(str(error)) from error
