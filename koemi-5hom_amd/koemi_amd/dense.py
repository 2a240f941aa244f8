"""Dense affine scan front: ``dense_affine_scan`` on the gfx950 HIP kernel.

Mirrors ``src/koemi/cuda_kernels/dense/affine_scan.py`` of the reference:
same signature, exception classes, validation order and message substrings,
and the same autograd contract (first-order gradients for retention, increment
and initial; broadcast retention gradients reduced back to the input shape).
The computation runs in ``csrc/affine_scan.hip`` through
``koemi_affine_scan_forward`` / ``koemi_affine_scan_backward``. There is no CPU
fallback: CPU tensors are rejected before any native call.
"""

from __future__ import annotations

import torch
from torch import Tensor

from koemi_amd import _native

__all__ = [
    "DenseCudaBuildError",
    "DenseCudaUnavailableError",
    "DenseCudaValidationError",
    "dense_affine_scan",
    "native_cuda_available",
]

_SUPPORTED_CUDA_DTYPES: tuple[torch.dtype, ...] = (
    torch.float16,
    torch.bfloat16,
    torch.float32,
    torch.float64,
)


class DenseCudaUnavailableError(RuntimeError):
    """Raised when the native dense kernel cannot run in the current process."""


class DenseCudaBuildError(DenseCudaUnavailableError):
    """Raised when the prebuilt gfx950 kernel library is missing or cannot be loaded."""


class DenseCudaValidationError(ValueError):
    """Raised when tensors violate the native dense affine-scan contract."""


def native_cuda_available() -> bool:
    """Return whether a ROCm device and the prebuilt gfx950 library are available.

    The reference checks ``torch.version.cuda`` and ``CUDA_HOME``
    (affine_scan.py:45-48), which are both unset on ROCm; this build checks the
    HIP runtime and its own prebuilt library instead.
    """

    return bool(torch.cuda.is_available() and torch.version.hip and _native.library_built())


def dense_affine_scan(
    retention: Tensor,
    increment: Tensor,
    initial: Tensor | None = None,
) -> Tensor:
    """Run the native affine scan with first-order autograd support.

    ``retention`` and ``increment`` have shape ``[batch, sequence, ...]`` and
    ``retention`` may broadcast over state dimensions. ``initial`` has shape
    ``[batch, ...]``; omitted initial state is zero. All tensors must share one
    device and dtype (float16, bfloat16, float32 or float64; accumulation is
    fp32, fp64 for float64). Reference: dense/affine_scan.py:51-82.
    """

    _validate_inputs(retention, increment, initial)
    if not native_cuda_available():
        raise DenseCudaUnavailableError(
            "native dense scan requires torch ROCm support, a GPU device, and the built gfx950 library"
        )
    normalized_initial = initial
    if normalized_initial is None:
        normalized_initial = increment.new_zeros((increment.shape[0],) + tuple(increment.shape[2:]))
    return _DenseAffineScanFunction.apply(retention, increment.contiguous(), normalized_initial.contiguous())


class _DenseAffineScanFunction(torch.autograd.Function):
    @staticmethod
    def forward(context, retention: Tensor, increment: Tensor, initial: Tensor) -> Tensor:  # type: ignore[override]
        normalized_retention = _normalize_retention(retention, increment)
        states = scan_forward(normalized_retention, increment, initial)
        context.save_for_backward(normalized_retention, initial, states)
        context.retention_shape = retention.shape
        return states

    @staticmethod
    def backward(context, gradient_states: Tensor):  # type: ignore[override]
        retention, initial, states = context.saved_tensors
        gradient_retention, gradient_increment, gradient_initial = scan_backward(
            retention, initial, states, gradient_states.contiguous()
        )
        return _reduce_to_shape(gradient_retention, context.retention_shape), gradient_increment, gradient_initial


def _geometry(increment: Tensor) -> tuple[int, int, int]:
    batch, sequence = int(increment.shape[0]), int(increment.shape[1])
    features = increment.numel() // (batch * sequence) if batch * sequence else 0
    return batch, sequence, features


def _load() -> None:
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise DenseCudaBuildError(f"failed to load the native dense scan library: {error}") from error


def scan_forward(retention: Tensor, increment: Tensor, initial: Tensor) -> Tensor:
    """Native forward on already normalized contiguous tensors (no autograd)."""

    _load()
    states = torch.empty_like(increment)
    if increment.numel() == 0:
        return states
    batch, sequence, features = _geometry(increment)
    broadcast = retention.numel() == batch * sequence
    with torch.cuda.device(increment.device):
        _native.call(
            "koemi_affine_scan_forward",
            retention.data_ptr(),
            increment.data_ptr(),
            initial.data_ptr(),
            states.data_ptr(),
            batch,
            sequence,
            features,
            int(broadcast),
            _native.dtype_code(increment.dtype),
            _native.stream_of(increment.device),
        )
    return states


def scan_backward(
    retention: Tensor, initial: Tensor, states: Tensor, gradient_states: Tensor
) -> tuple[Tensor, Tensor, Tensor]:
    """Native reverse-time adjoint; gradient_retention has the full state shape."""

    _load()
    gradient_retention = torch.empty_like(states)
    gradient_increment = torch.empty_like(states)
    gradient_initial = torch.zeros_like(initial)
    if states.numel() == 0:
        return gradient_retention, gradient_increment, gradient_initial
    batch, sequence, features = _geometry(states)
    broadcast = retention.numel() == batch * sequence
    with torch.cuda.device(states.device):
        _native.call(
            "koemi_affine_scan_backward",
            retention.data_ptr(),
            initial.data_ptr(),
            states.data_ptr(),
            gradient_states.data_ptr(),
            gradient_retention.data_ptr(),
            gradient_increment.data_ptr(),
            gradient_initial.data_ptr(),
            batch,
            sequence,
            features,
            int(broadcast),
            _native.dtype_code(states.dtype),
            _native.stream_of(states.device),
        )
    return gradient_retention, gradient_increment, gradient_initial


def _validate_inputs(retention: Tensor, increment: Tensor, initial: Tensor | None) -> None:
    """Contract checks in the reference order (dense/affine_scan.py:146-217)."""

    _validate_tensor("retention", retention)
    _validate_tensor("increment", increment)
    if initial is not None:
        _validate_tensor("initial", initial)

    if retention.ndim < 2 or increment.ndim < 2:
        raise DenseCudaValidationError("retention and increment must have at least two dimensions")
    if retention.ndim != increment.ndim:
        raise DenseCudaValidationError("retention and increment must have the same rank")
    if retention.shape[:2] != increment.shape[:2]:
        raise DenseCudaValidationError("retention and increment must have the same batch and sequence dimensions")
    try:
        broadcast_shape = torch.broadcast_shapes(retention.shape, increment.shape)
    except RuntimeError as error:
        raise DenseCudaValidationError("retention must broadcast to increment's shape") from error
    if broadcast_shape != increment.shape:
        raise DenseCudaValidationError("retention must broadcast to increment's shape")

    tensor_values = (retention, increment) if initial is None else (retention, increment, initial)
    tensor_dtypes = {value.dtype for value in tensor_values}
    unsupported_dtypes = tensor_dtypes.difference(_SUPPORTED_CUDA_DTYPES)
    if unsupported_dtypes:
        names = ", ".join(sorted(str(dtype) for dtype in unsupported_dtypes))
        raise DenseCudaValidationError(f"unsupported CUDA dtype(s): {names}")
    if len(tensor_dtypes) != 1:
        raise DenseCudaValidationError("retention, increment and initial must have the same dtype")

    if initial is not None:
        expected_initial_shape = (increment.shape[0],) + tuple(increment.shape[2:])
        if initial.shape != expected_initial_shape:
            raise DenseCudaValidationError(
                f"initial must have shape {expected_initial_shape}, got {tuple(initial.shape)}"
            )

    if not torch.cuda.is_available():
        raise DenseCudaUnavailableError("native dense CUDA scan is unavailable: torch.cuda.is_available() is False")
    scan_tensors = tensor_values
    non_cuda_tensors = [value for value in scan_tensors if value.device.type != "cuda"]
    if non_cuda_tensors:
        devices = ", ".join(str(value.device) for value in non_cuda_tensors)
        raise DenseCudaValidationError(f"all dense scan tensors must be on CUDA; found {devices}")
    scan_devices = {value.device for value in scan_tensors}
    if len(scan_devices) != 1:
        devices = ", ".join(sorted(str(device) for device in scan_devices))
        raise DenseCudaValidationError(f"all dense scan tensors must use one CUDA device; found {devices}")


def _validate_tensor(name: str, value: Tensor) -> None:
    if not isinstance(value, Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")


def _normalize_retention(retention: Tensor, increment: Tensor) -> Tensor:
    """Full-shape or per-(batch, position) retention stays as is; partial
    broadcasts are expanded (dense/affine_scan.py:225-230)."""

    if retention.shape == increment.shape:
        return retention.contiguous()
    if all(dimension == 1 for dimension in retention.shape[2:]):
        return retention.contiguous()
    return retention.expand_as(increment).contiguous()


def _reduce_to_shape(gradient: Tensor, target_shape: torch.Size) -> Tensor:
    """Sum a full-shape gradient back to a broadcast retention shape
    (dense/affine_scan.py:233-255)."""

    if gradient.shape == target_shape:
        return gradient
    if len(target_shape) > gradient.ndim:
        raise DenseCudaValidationError(
            f"native gradient rank {gradient.ndim} is smaller than target rank {len(target_shape)}"
        )
    reduced = gradient
    while reduced.ndim > len(target_shape):
        reduced = reduced.sum(dim=-1)
    for dimension in range(reduced.ndim - 1, 1, -1):
        if target_shape[dimension] == 1 and reduced.shape[dimension] != 1:
            reduced = reduced.sum(dim=dimension, keepdim=True)
        elif target_shape[dimension] != reduced.shape[dimension]:
            raise DenseCudaValidationError(
                f"native gradient dimension {dimension} has shape {reduced.shape[dimension]}, "
                f"expected {target_shape[dimension]}"
            )
    if reduced.shape != target_shape:
        raise DenseCudaValidationError(
            f"native gradient shape {tuple(reduced.shape)} does not match {tuple(target_shape)}"
        )
    return reduced
