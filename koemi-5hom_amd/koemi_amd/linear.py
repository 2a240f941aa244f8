"""Projections of a few rows (decode steps) on the ``koemi_linear_rows`` kernel.

The HERM block's ``nn.Linear`` layers (reference model/network.py:296-441,
model/memory.py) run as library GEMMs for a window of many rows. For a decode
step's few rows ``linear_rows`` streams the bf16 weights once in one kernel,
rounds fp32 inputs to bf16 in registers (the cast of bf16 autocast) and takes
the fusion layer's input as its pieces without concatenating them. There is
no torch fallback.
"""

from __future__ import annotations

import torch
from torch import Tensor

from koemi_amd import _native
from koemi_amd.dense import DenseCudaUnavailableError, DenseCudaValidationError

__all__ = ["MAX_ROWS", "linear_rows"]

MAX_ROWS = 64  # rows up to which the kernel beats a library GEMM (one pass over the weights)


def linear_rows(pieces: list[Tensor] | tuple[Tensor, ...], weight: Tensor, bias: Tensor | None) -> Tensor:
    """``cat(pieces, -1) @ weight.T + bias`` in fp32 for bf16 ``weight``
    ``[N, K]``. ``pieces``: one to four tensors ``[..., K / len(pieces)]`` of
    one dtype (float32 or bfloat16) and leading shape; ``bias`` fp32 ``[N]``
    or None. Returns ``[..., N]`` fp32."""

    if not 1 <= len(pieces) <= 4:
        raise DenseCudaValidationError("linear_rows takes one to four input pieces")
    first = pieces[0]
    for t in (*pieces, weight) + ((bias,) if bias is not None else ()):
        if not isinstance(t, Tensor) or t.device.type != "cuda" or t.device != first.device:
            raise DenseCudaValidationError("linear_rows tensors must be CUDA tensors on one device")
    if first.dtype not in (torch.float32, torch.bfloat16) or any(
            p.dtype != first.dtype or p.shape != first.shape for p in pieces):
        raise DenseCudaValidationError("linear_rows pieces must share one shape and a float32 or bfloat16 dtype")
    width = first.shape[-1]
    if weight.dtype != torch.bfloat16 or weight.ndim != 2 or weight.shape[1] != width * len(pieces):
        raise DenseCudaValidationError("weight must be bfloat16 [out_features, sum of the piece widths]")
    if bias is not None and (bias.dtype != torch.float32 or bias.shape != (weight.shape[0],)):
        raise DenseCudaValidationError("bias must be float32 [out_features]")
    if width % 64 != 0 or (len(pieces) > 1 and width % 1024 != 0):
        raise DenseCudaValidationError("linear_rows needs piece widths that are multiples of 64 "
                                       "(of 1024 for several pieces)")
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise DenseCudaUnavailableError(str(error)) from error
    flat = [p.reshape(-1, width).contiguous() for p in pieces]
    rows = flat[0].shape[0]
    out = torch.empty((rows, weight.shape[0]), device=first.device, dtype=torch.float32)
    if rows:
        ptrs = [_native.ptr(p) for p in flat] + [None] * (4 - len(flat))
        _native.call("koemi_linear_rows", *ptrs, len(flat), width, _native.dtype_code(first.dtype),
                     _native.ptr(weight.contiguous()), _native.ptr(bias.contiguous()) if bias is not None else None,
                     _native.ptr(out), rows, weight.shape[0], _native.stream_of(first.device))
    return out.view(*first.shape[:-1], weight.shape[0])
