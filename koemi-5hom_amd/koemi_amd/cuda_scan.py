"""Chunked scan front ``cuda_affine_scan`` on the gfx950 HIP kernel.

Mirrors ``src/koemi/model/cuda_scan.py`` of the reference (same signature,
``chunk_size`` contract, diagnostics dataclass, exceptions and messages). The
reference runs a Hillis-Steele scan per ``chunk_size`` segment in PyTorch and
carries the last state into the next segment (cuda_scan.py:203-239). Here the
whole sequence runs through ``koemi_affine_scan_forward``, which carries the
exact state across its internal 64-step chunks in registers; the result is
the same recurrence for every ``chunk_size``, which is validated and reported
in ``CudaScanDiagnostics.chunk_count`` as in the reference.
"""

from __future__ import annotations

from dataclasses import dataclass
from time import perf_counter

import torch
from torch import Tensor

from koemi_amd.dense import _DenseAffineScanFunction, native_cuda_available

__all__ = [
    "CudaScanDiagnostics",
    "CudaScanUnavailableError",
    "CudaScanValidationError",
    "cuda_affine_scan",
    "diagnose_cuda_affine_scan",
]

_SUPPORTED_CUDA_DTYPES: tuple[torch.dtype, ...] = (
    torch.float16,
    torch.bfloat16,
    torch.float32,
    torch.float64,
)


class CudaScanUnavailableError(RuntimeError):
    """Raised when the scan cannot run because no GPU (or no kernel library) is available."""


class CudaScanValidationError(ValueError):
    """Raised when scan tensors or options violate the scan contract."""


@dataclass(frozen=True)
class CudaScanDiagnostics:
    """Result and measurements returned by the scan diagnostic API."""

    states: Tensor
    elapsed_seconds: float
    token_count: int
    chunk_count: int


def cuda_affine_scan(
    retention: Tensor,
    increment: Tensor,
    initial: Tensor | None = None,
    *,
    chunk_size: int | None = None,
) -> Tensor:
    """Run the affine scan on GPU tensors only (reference cuda_scan.py:79-102).

    ``retention`` may broadcast over the state dimensions and ``initial`` has
    shape ``[batch, ...]`` (zeros when omitted). Returns states with the shape,
    device and dtype of ``increment``; never moves tensors or falls back to CPU.
    """

    sequence_length, _, _ = _validate_inputs(retention, increment, initial, chunk_size)
    return _run_scan(retention, increment, initial, sequence_length)


def diagnose_cuda_affine_scan(
    retention: Tensor,
    increment: Tensor,
    initial: Tensor | None = None,
    *,
    chunk_size: int | None = None,
) -> CudaScanDiagnostics:
    """Run the scan and report synchronized elapsed time and work counts
    (reference cuda_scan.py:105-131)."""

    sequence_length, chunk_count, device = _validate_inputs(retention, increment, initial, chunk_size)
    torch.cuda.synchronize(device)
    started_at = perf_counter()
    states = _run_scan(retention, increment, initial, sequence_length)
    torch.cuda.synchronize(device)
    elapsed_seconds = perf_counter() - started_at
    return CudaScanDiagnostics(
        states=states,
        elapsed_seconds=elapsed_seconds,
        token_count=retention.shape[0] * sequence_length,
        chunk_count=chunk_count,
    )


def _validate_inputs(
    retention: Tensor,
    increment: Tensor,
    initial: Tensor | None,
    chunk_size: int | None,
) -> tuple[int, int, torch.device]:
    for name, value in (("retention", retention), ("increment", increment), ("initial", initial)):
        if value is not None and not isinstance(value, Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
    if retention.ndim < 2 or increment.ndim < 2:
        raise CudaScanValidationError("retention and increment must have at least two dimensions")
    if retention.ndim != increment.ndim:
        raise CudaScanValidationError("retention and increment must have the same rank")
    if retention.shape[:2] != increment.shape[:2]:
        raise CudaScanValidationError("retention and increment must have the same batch and sequence dimensions")
    try:
        broadcast_shape = torch.broadcast_shapes(retention.shape, increment.shape)
    except RuntimeError as error:
        raise CudaScanValidationError("retention must broadcast to increment's shape") from error
    if broadcast_shape != increment.shape:
        raise CudaScanValidationError("retention must broadcast to increment's shape")

    tensor_values = (retention, increment) if initial is None else (retention, increment, initial)
    tensor_dtypes = {value.dtype for value in tensor_values}
    unsupported_dtypes = tensor_dtypes.difference(_SUPPORTED_CUDA_DTYPES)
    if unsupported_dtypes:
        names = ", ".join(str(dtype) for dtype in sorted(unsupported_dtypes, key=str))
        raise CudaScanValidationError(f"unsupported scan dtype(s): {names}")
    if len(tensor_dtypes) != 1:
        raise CudaScanValidationError("retention, increment and initial must have the same dtype")

    if initial is not None:
        expected_initial_shape = (increment.shape[0],) + tuple(increment.shape[2:])
        if initial.shape != expected_initial_shape:
            raise CudaScanValidationError(
                f"initial must have shape {expected_initial_shape}, got {tuple(initial.shape)}"
            )

    if chunk_size is not None and (isinstance(chunk_size, bool) or not isinstance(chunk_size, int)):
        raise CudaScanValidationError("chunk_size must be a positive integer or None")
    if chunk_size is not None and chunk_size < 1:
        raise CudaScanValidationError("chunk_size must be a positive integer or None")

    if not torch.cuda.is_available():
        raise CudaScanUnavailableError("GPU affine scan is unavailable: torch.cuda.is_available() is False")

    non_cuda_tensors = [value for value in tensor_values if value.device.type != "cuda"]
    if non_cuda_tensors:
        devices = ", ".join(str(value.device) for value in non_cuda_tensors)
        raise CudaScanValidationError(f"all scan tensors must be on CUDA; found {devices}")
    scan_devices = {value.device for value in tensor_values}
    if len(scan_devices) != 1:
        devices = ", ".join(sorted(str(device) for device in scan_devices))
        raise CudaScanValidationError(f"all scan tensors must use one CUDA device; found {devices}")
    if not native_cuda_available():
        raise CudaScanUnavailableError("GPU affine scan is unavailable: the gfx950 kernel library is not built")

    sequence_length = increment.shape[1]
    resolved_chunk_size = sequence_length if chunk_size is None else min(chunk_size, sequence_length)
    chunk_count = 0 if sequence_length == 0 else (sequence_length + resolved_chunk_size - 1) // resolved_chunk_size
    return sequence_length, chunk_count, increment.device


def _run_scan(retention: Tensor, increment: Tensor, initial: Tensor | None, sequence_length: int) -> Tensor:
    if sequence_length == 0:
        return increment.new_empty(increment.shape)
    if initial is None:
        initial = increment.new_zeros((increment.shape[0],) + tuple(increment.shape[2:]))
    return _DenseAffineScanFunction.apply(retention, increment.contiguous(), initial.contiguous())
