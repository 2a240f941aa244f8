"""Fused RMSNorm-SiLU front: ``fused_rmsnorm_silu`` on the gfx950 HIP kernel.

Mirrors ``src/koemi/cuda_kernels/core/rmsnorm_silu.py`` (front, autograd,
validation order and messages) and the native op surface of
``core/rmsnorm_silu.cpp:73-77``: ``load_core_extension()`` returns an object
exposing ``KOEMI_CUDA_ABI_VERSION``, ``rmsnorm_silu_forward(x, w, eps) ->
[y, inverse_rms]`` and ``rmsnorm_silu_backward(g, x, w, inverse_rms, eps) ->
[dx, dw]``, implemented over ``koemi_rmsnorm_silu_forward`` / ``_backward``.
"""

from __future__ import annotations

import math
from typing import Any

import torch
from torch import Tensor

from koemi_amd import _native
from koemi_amd.loader import (
    CUDA_EXTENSION_ABI_VERSION,
    CudaExtensionValidationError,
    require_library,
)

__all__ = ["fused_rmsnorm_silu", "load_core_extension", "rmsnorm_silu_forward", "rmsnorm_silu_backward"]

_SUPPORTED_DTYPES = frozenset({torch.float16, torch.bfloat16, torch.float32})


def rmsnorm_silu_forward(input_tensor: Tensor, weight: Tensor, eps: float) -> list[Tensor]:
    """Native forward: returns ``[silu(x * inv * w), inv]`` with fp32 ``inv`` of shape [rows]."""

    _check_native_inputs(input_tensor, weight, eps)
    output = torch.empty_like(input_tensor)
    inverse_rms = torch.empty((input_tensor.shape[0],), device=input_tensor.device, dtype=torch.float32)
    if input_tensor.shape[0] == 0:
        return [output, inverse_rms]
    with torch.cuda.device(input_tensor.device):
        _native.call(
            "koemi_rmsnorm_silu_forward",
            input_tensor.data_ptr(),
            weight.data_ptr(),
            output.data_ptr(),
            inverse_rms.data_ptr(),
            input_tensor.shape[0],
            input_tensor.shape[1],
            float(eps),
            _native.dtype_code(input_tensor.dtype),
            _native.stream_of(input_tensor.device),
        )
    return [output, inverse_rms]


def rmsnorm_silu_backward(
    gradient_output: Tensor, input_tensor: Tensor, weight: Tensor, inverse_rms: Tensor, eps: float
) -> list[Tensor]:
    """Native backward: returns ``[dx, dw]``; dw is reduced without atomics."""

    _check_native_inputs(input_tensor, weight, eps)
    if gradient_output.shape != input_tensor.shape or gradient_output.dtype != input_tensor.dtype:
        raise RuntimeError("gradient_output must match input shape and dtype")
    if inverse_rms.dtype != torch.float32 or inverse_rms.shape != (input_tensor.shape[0],):
        raise RuntimeError("inverse_rms must be a float32 tensor of shape [rows]")
    gradient_output = gradient_output.contiguous()
    rows, hidden = input_tensor.shape
    gradient_input = torch.empty_like(input_tensor)
    gradient_weight = torch.empty_like(weight)
    workspace_bytes = _native.query("koemi_rmsnorm_silu_backward_workspace_bytes", rows, hidden)
    workspace = torch.empty((max(workspace_bytes, 1),), device=input_tensor.device, dtype=torch.uint8)
    with torch.cuda.device(input_tensor.device):
        _native.call(
            "koemi_rmsnorm_silu_backward",
            gradient_output.data_ptr(),
            input_tensor.data_ptr(),
            weight.data_ptr(),
            inverse_rms.data_ptr(),
            gradient_input.data_ptr(),
            gradient_weight.data_ptr(),
            rows,
            hidden,
            _native.dtype_code(input_tensor.dtype),
            workspace.data_ptr(),
            workspace_bytes,
            _native.stream_of(input_tensor.device),
        )
    return [gradient_input, gradient_weight]


class _CoreExtension:
    """Object with the attributes of the reference's pybind core module."""

    KOEMI_CUDA_ABI_VERSION = CUDA_EXTENSION_ABI_VERSION
    rmsnorm_silu_forward = staticmethod(rmsnorm_silu_forward)
    rmsnorm_silu_backward = staticmethod(rmsnorm_silu_backward)


_CORE_EXTENSION = _CoreExtension()


def load_core_extension(*, device: torch.device | str | int | None = None, verbose: bool = False) -> Any:
    """Load the prebuilt kernel library (reference core/rmsnorm_silu.py:31-34).

    ``device`` and ``verbose`` are accepted for signature compatibility; the
    gfx950 code object serves every device of this architecture.
    """

    del device, verbose
    require_library()
    return _CORE_EXTENSION


def fused_rmsnorm_silu(input_tensor: Tensor, weight: Tensor, eps: float = 1e-6) -> Tensor:
    """Apply RMSNorm and SiLU in one kernel with an autograd backward
    (reference core/rmsnorm_silu.py:37-42)."""

    _validate_inputs(input_tensor, weight, eps)
    extension = load_core_extension(device=input_tensor.device)
    return _FusedRMSNormSiLU.apply(input_tensor, weight, float(eps), extension)


class _FusedRMSNormSiLU(torch.autograd.Function):
    @staticmethod
    def forward(context, input_tensor: Tensor, weight: Tensor, eps: float, extension: Any) -> Tensor:  # type: ignore[override]
        output, inverse_rms = extension.rmsnorm_silu_forward(input_tensor, weight, eps)
        context.save_for_backward(input_tensor, weight, inverse_rms)
        context.eps = eps
        context.extension = extension
        return output

    @staticmethod
    def backward(context, gradient_output: Tensor):  # type: ignore[override]
        input_tensor, weight, inverse_rms = context.saved_tensors
        gradient_input, gradient_weight = context.extension.rmsnorm_silu_backward(
            gradient_output.contiguous(), input_tensor, weight, inverse_rms, context.eps
        )
        return gradient_input, gradient_weight, None, None


def _check_native_inputs(input_tensor: Tensor, weight: Tensor, eps: float) -> None:
    """Checks of the native entry (rmsnorm_silu.cpp:20-35), raised as RuntimeError."""

    if input_tensor.device.type != "cuda" or weight.device.type != "cuda":
        raise RuntimeError("input must be a CUDA tensor")
    if input_tensor.dim() != 2 or weight.dim() != 1 or weight.shape[0] != input_tensor.shape[1]:
        raise RuntimeError("input must have shape [rows, hidden] and weight shape [hidden]")
    if input_tensor.shape[1] <= 0:
        raise RuntimeError("input hidden dimension must be positive")
    if not input_tensor.is_contiguous() or not weight.is_contiguous():
        raise RuntimeError("input must be contiguous")
    if input_tensor.dtype not in _SUPPORTED_DTYPES or weight.dtype != input_tensor.dtype:
        raise RuntimeError("input and weight must have the same dtype (float16, bfloat16 or float32)")
    if not (math.isfinite(float(eps)) and float(eps) > 0.0):
        raise RuntimeError("eps must be finite and positive")


def _validate_inputs(input_tensor: Tensor, weight: Tensor, eps: float) -> None:
    """Front checks in the reference order (core/rmsnorm_silu.py:74-100)."""

    if not isinstance(input_tensor, Tensor):
        raise TypeError("input_tensor must be a torch.Tensor")
    if not isinstance(weight, Tensor):
        raise TypeError("weight must be a torch.Tensor")
    if input_tensor.ndim != 2:
        raise CudaExtensionValidationError("input_tensor must have shape [rows, hidden]")
    if input_tensor.shape[1] == 0:
        raise CudaExtensionValidationError("input_tensor hidden dimension must be positive")
    if weight.ndim != 1 or weight.shape[0] != input_tensor.shape[1]:
        raise CudaExtensionValidationError(
            f"weight must have shape {(input_tensor.shape[1],)}, got {tuple(weight.shape)}"
        )
    if input_tensor.dtype not in _SUPPORTED_DTYPES or weight.dtype not in _SUPPORTED_DTYPES:
        raise CudaExtensionValidationError("input_tensor and weight must use float16, bfloat16 or float32")
    if input_tensor.dtype != weight.dtype:
        raise CudaExtensionValidationError("input_tensor and weight must have the same dtype")
    if input_tensor.device != weight.device:
        raise CudaExtensionValidationError("input_tensor and weight must use the same device")
    if input_tensor.device.type != "cuda":
        raise CudaExtensionValidationError(f"input_tensor must be on CUDA, got {input_tensor.device}")
    if not input_tensor.is_contiguous() or not weight.is_contiguous():
        raise CudaExtensionValidationError("input_tensor and weight must be contiguous")
    if isinstance(eps, bool) or not isinstance(eps, (float, int)) or not math.isfinite(float(eps)):
        raise CudaExtensionValidationError("eps must be a finite positive number")
    if float(eps) <= 0.0:
        raise CudaExtensionValidationError("eps must be a finite positive number")
