"""Bounded recurrent state on the GPU: gates and the working-state scan.

Fronts for ``BoundedRecurrentState.gates`` (reference model/memory.py:14-30)
and the first steps of the HERM window (network.py:306-310: gates, masking of
invalid positions, affine scan from the carried working state). The gates run
``koemi_recurrent_gates`` (two rocBLAS products with fp32 accumulation and one
HIP epilogue kernel); the fp32 window scan runs ``koemi_recurrent_scan``, the
same products followed by one HIP kernel that forms the gates in registers
inside the affine scan; other dtypes run the gates and then the dense
affine-scan kernel. There is no torch fallback. Inference only (no autograd
through the gates).
"""

from __future__ import annotations

import torch
from torch import Tensor

from koemi_amd import _native
from koemi_amd.dense import DenseCudaUnavailableError, DenseCudaValidationError, dense_affine_scan

__all__ = ["GatedScanTimeoutError", "check_gated_scan_status", "gated_scan", "recurrent_gates", "recurrent_scan"]

# koemi_gated_projection_scan: spin_limit bit that stops tiles publishing their
# transfers (include/koemi_hip.h KOEMI_GP_WITHHOLD_TRANSFERS), so the host can
# drive the bounded waits to their timeout in a test.
GP_WITHHOLD_TRANSFERS = 0x80000000


class GatedScanTimeoutError(RuntimeError):
    """A tile of ``gated_projection_scan`` gave up waiting for an earlier
    tile's transfer: its states (and what was computed from them) are NaN."""


def check_gated_scan_status(status: Tensor) -> None:
    """Raise ``GatedScanTimeoutError`` when the device status word that
    ``gated_projection_scan`` (``status=``) reports into is set. Reads it to the
    host, so it waits for the work queued before it on the current stream."""

    if int(status.reshape(-1)[0].item()) != 0:
        raise GatedScanTimeoutError("gated projection scan: a tile timed out waiting for an earlier tile's carry; "
                                    "its states are NaN")

_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def recurrent_gates(
    input_state: Tensor,
    retention_weight: Tensor,
    retention_bias: Tensor,
    candidate_weight: Tensor,
    candidate_bias: Tensor,
    valid_mask: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """(retention, increment) of ``BoundedRecurrentState.gates`` (memory.py:14-30).

    ``input_state`` ``[..., D]``; the weights ``[D, D]`` and biases ``[D]`` of
    ``retention_projection`` and ``candidate_projection`` (``nn.Linear``
    layout: out x in). ``retention = 2^-8 + (1 - 2^-7) * sigmoid(u W_r^T + b_r)``,
    ``increment = (1 - retention) * tanh(u W_c^T + b_c)``. With ``valid_mask``
    (``input_state.shape[:-1]``, bool) invalid positions get retention 1 and
    increment 0, as network.py:307-309 applies them. Outputs in the input
    dtype; products accumulate in fp32.
    """

    _check_gate_arguments(input_state, retention_weight, retention_bias, candidate_weight, candidate_bias, valid_mask)
    width = input_state.shape[-1]
    device = input_state.device
    rows = input_state.numel() // width if width else 0
    retention = torch.empty(input_state.shape, device=device, dtype=input_state.dtype)
    increment = torch.empty_like(retention)
    if rows == 0:
        return retention, increment
    workspace = torch.empty(_native.query("koemi_recurrent_gates_workspace_bytes", rows, width), dtype=torch.uint8,
                            device=device)
    u = input_state.contiguous()
    params = [t.contiguous() for t in (retention_weight, retention_bias, candidate_weight, candidate_bias)]
    mask = valid_mask.contiguous() if valid_mask is not None else None
    _native.call(
        "koemi_recurrent_gates",
        _native.ptr(u),
        *(_native.ptr(t) for t in params),
        _native.ptr(mask) if mask is not None else None,
        _native.ptr(retention),
        _native.ptr(increment),
        rows,
        width,
        _native.dtype_code(input_state.dtype),
        _native.ptr(workspace),
        workspace.numel(),
        _native.stream_of(device),
    )
    return retention, increment


def _check_gate_arguments(input_state, retention_weight, retention_bias, candidate_weight, candidate_bias,
                          valid_mask) -> None:
    tensors = {
        "input_state": input_state,
        "retention_weight": retention_weight,
        "retention_bias": retention_bias,
        "candidate_weight": candidate_weight,
        "candidate_bias": candidate_bias,
    }
    if valid_mask is not None:
        tensors["valid_mask"] = valid_mask
    for name, tensor in tensors.items():
        if not isinstance(tensor, Tensor):
            raise DenseCudaValidationError(f"{name} must be a torch.Tensor")
        if tensor.device.type != "cuda":
            raise DenseCudaValidationError(f"{name} must be on CUDA")
    if len({t.device for t in tensors.values()}) != 1:
        raise DenseCudaValidationError("recurrent gate tensors must be on the same CUDA device")
    if input_state.ndim < 1:
        raise DenseCudaValidationError("input_state must have a trailing feature dimension")
    width = input_state.shape[-1]
    for name in ("retention_weight", "candidate_weight"):
        if tensors[name].shape != (width, width):
            raise DenseCudaValidationError(f"{name} must have shape [{width}, {width}]")
    for name in ("retention_bias", "candidate_bias"):
        if tensors[name].shape != (width,):
            raise DenseCudaValidationError(f"{name} must have shape [{width}]")
    if input_state.dtype not in _SUPPORTED_DTYPES:
        raise DenseCudaValidationError("unsupported dtype for the recurrent gates (float16, bfloat16, float32)")
    if any(t.dtype != input_state.dtype for n, t in tensors.items() if n != "valid_mask"):
        raise DenseCudaValidationError("input_state and the gate parameters must have the same dtype")
    if valid_mask is not None and (valid_mask.dtype != torch.bool or valid_mask.shape != input_state.shape[:-1]):
        raise DenseCudaValidationError("valid_mask must be a bool tensor of shape input_state.shape[:-1]")
    if width % 4 != 0:
        raise DenseCudaValidationError("the feature width must be a multiple of 4")
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise DenseCudaUnavailableError(str(error)) from error


def recurrent_scan(
    input_state: Tensor,
    retention_weight: Tensor,
    retention_bias: Tensor,
    candidate_weight: Tensor,
    candidate_bias: Tensor,
    valid_mask: Tensor,
    initial: Tensor | None = None,
) -> Tensor:
    """Working states of one window (network.py:306-310).

    ``input_state`` ``[B, L, D]``, ``valid_mask`` ``[B, L]``, ``initial``
    ``[B, D]`` (zeros when omitted): gates with invalid positions masked to
    (1, 0), then ``h_t = a_t h_{t-1} + b_t`` from ``initial``.
    """

    if not isinstance(input_state, Tensor) or input_state.ndim != 3:
        raise DenseCudaValidationError("input_state must be a [batch, length, width] tensor")
    if input_state.dtype != torch.float32:
        retention, increment = recurrent_gates(input_state, retention_weight, retention_bias, candidate_weight,
                                               candidate_bias, valid_mask)
        return dense_affine_scan(retention, increment, initial)
    _check_gate_arguments(input_state, retention_weight, retention_bias, candidate_weight, candidate_bias, valid_mask)
    batch, length, width = input_state.shape
    device = input_state.device
    if initial is None:
        initial = torch.zeros((batch, width), device=device, dtype=torch.float32)
    elif not isinstance(initial, Tensor) or initial.shape != (batch, width) or initial.dtype != torch.float32 \
            or initial.device != device:
        raise DenseCudaValidationError("initial must be a float32 [batch, width] tensor on the input's device")
    states = torch.empty((batch, length, width), device=device, dtype=torch.float32)
    if states.numel() == 0:
        return states
    workspace = torch.empty(_native.query("koemi_recurrent_gates_workspace_bytes", batch * length, width),
                            dtype=torch.uint8, device=device)
    u = input_state.contiguous()
    params = [t.contiguous() for t in (retention_weight, retention_bias, candidate_weight, candidate_bias)]
    mask = valid_mask.contiguous() if valid_mask is not None else None
    h0 = initial.contiguous()
    _native.call(
        "koemi_recurrent_scan",
        _native.ptr(u),
        *(_native.ptr(t) for t in params),
        _native.ptr(mask) if mask is not None else None,
        _native.ptr(h0),
        _native.ptr(states),
        batch,
        length,
        width,
        _native.ptr(workspace),
        workspace.numel(),
        _native.stream_of(device),
    )
    return states


def gated_scan(preactivations: Tensor, valid_mask: Tensor | None, initial: Tensor, *, width: int,
               retention_offset: int = 0, candidate_offset: int | None = None,
               with_bf16: bool = False, two_phase: bool = True, retention_bias: Tensor | None = None,
               candidate_bias: Tensor | None = None, out_bf16: Tensor | None = None,
               out: Tensor | None = None) -> Tensor | tuple[Tensor, Tensor]:
    """Working states of one window from precomputed gate pre-activations.

    ``preactivations`` ``[B, L, C]`` fp32 or bf16 (last dimension contiguous) holds
    ``u W_r^T + b_r`` in columns ``retention_offset .. + width`` and
    ``u W_c^T + b_c`` in ``candidate_offset .. + width`` (default: right
    after the retention columns), as one stacked projection produces them.
    The gates of memory.py:22-26, the masking of network.py:307-309 and the
    scan of network.py:310 from ``initial`` ``[B, width]`` run in one kernel
    (``koemi_gated_scan``). Returns ``[B, L, width]`` fp32, and with
    ``with_bf16`` also its bf16 copy (written by the same kernel) for a
    following bf16 GEMM. ``retention_bias`` and ``candidate_bias`` (fp32
    ``[width]``, None: none) are added to the pre-activations inside the
    kernel. ``out_bf16`` (with ``with_bf16``): a bf16 ``[B, L, width]`` view
    with contiguous columns and evenly spaced rows (a column block of a wider
    matrix) that receives the bf16 copy. With ``two_phase`` the kernel gets the workspace of
    its two-phase form, which it takes when the batch's columns alone would
    leave the chip short of workgroups (a few long rows); the result is the
    same to the bit either way. ``out``: a contiguous fp32 ``[B, L, width]``
    tensor that receives the states (a graph's static state), not
    overlapping the inputs.
    """

    if candidate_offset is None:
        candidate_offset = retention_offset + width
    if (not isinstance(preactivations, Tensor) or preactivations.ndim != 3
            or preactivations.dtype not in (torch.float32, torch.bfloat16)):
        raise DenseCudaValidationError("preactivations must be a float32 or bfloat16 [batch, length, columns] tensor")
    if preactivations.device.type != "cuda":
        raise DenseCudaValidationError("preactivations must be on CUDA")
    batch, length, columns = preactivations.shape
    if min(retention_offset, candidate_offset) < 0 or max(retention_offset, candidate_offset) + width > columns:
        raise DenseCudaValidationError("the gate columns must lie inside the pre-activation rows")
    if not isinstance(initial, Tensor) or initial.shape != (batch, width) or initial.dtype != torch.float32 \
            or initial.device != preactivations.device:
        raise DenseCudaValidationError("initial must be a float32 [batch, width] tensor on the same device")
    if valid_mask is not None and (valid_mask.dtype != torch.bool or valid_mask.shape != (batch, length)
                                   or valid_mask.device != preactivations.device):
        raise DenseCudaValidationError("valid_mask must be a bool [batch, length] tensor on the same device")
    for bias in (retention_bias, candidate_bias):
        if bias is not None and (not isinstance(bias, Tensor) or bias.shape != (width,) or bias.dtype != torch.float32
                                 or bias.device != preactivations.device or not bias.is_contiguous()):
            raise DenseCudaValidationError("gate biases must be contiguous float32 [width] tensors on the same device")
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise DenseCudaUnavailableError(str(error)) from error
    z = preactivations.contiguous()
    if out is not None and (out.shape != (batch, length, width) or out.dtype != torch.float32
                            or not out.is_contiguous() or out.device != z.device):
        raise DenseCudaValidationError("out must be a contiguous float32 [batch, length, width] tensor")
    states = out if out is not None else torch.empty((batch, length, width), device=z.device, dtype=torch.float32)
    states16 = None
    if with_bf16:
        states16 = out_bf16 if out_bf16 is not None else torch.empty(states.shape, device=z.device,
                                                                     dtype=torch.bfloat16)
        if (states16.shape != states.shape or states16.dtype != torch.bfloat16 or states16.stride(2) != 1
                or states16.stride(0) != length * states16.stride(1)):
            raise DenseCudaValidationError("out_bf16 must be a bf16 [batch, length, width] view with evenly spaced rows")
    if states.numel():
        mask = valid_mask.contiguous() if valid_mask is not None else None
        need = _native.query("koemi_gated_scan_workspace_bytes", batch, length, width) if two_phase else 0
        workspace = torch.empty(need, device=z.device, dtype=torch.uint8) if need else None
        _native.call(
            "koemi_gated_scan",
            _native.ptr(z), _native.dtype_code(z.dtype), columns, retention_offset, candidate_offset,
            _native.ptr(retention_bias),
            _native.ptr(candidate_bias),
            _native.ptr(mask) if mask is not None else None,
            _native.ptr(initial.contiguous()), _native.ptr(states), _native.ptr(states16),
            states16.stride(1) if states16 is not None else 0,
            batch, length, width, _native.ptr(workspace), need, _native.stream_of(z.device),
        )
    return (states, states16) if with_bf16 else states


def gated_projection_fits(inputs: Tensor, weight: Tensor) -> bool:
    """Whether ``gated_projection_scan`` takes these shapes: bf16 ``inputs``
    ``[B, L, K]`` and stacked ``weight`` ``[2 width, K]`` with L a multiple of
    256, width of 128 and K of 64."""

    return (inputs.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and inputs.ndim == 3
            and weight.ndim == 2 and weight.shape[1] == inputs.shape[2] and inputs.shape[1] % 256 == 0
            and (weight.shape[0] // 2) % 128 == 0 and weight.shape[0] % 2 == 0 and inputs.shape[2] % 64 == 0)


def gated_projection_scan(inputs: Tensor, weight: Tensor, bias: Tensor | None, valid_mask: Tensor | None,
                          initial: Tensor, *, with_bf16: bool = False, out_bf16: Tensor | None = None,
                          final_out: Tensor | None = None, status: Tensor | None = None,
                          spin_limit: int = 0) -> Tensor | tuple[Tensor, Tensor]:
    """The gates of model/memory.py:14-30 with their two projections, the
    masking of network.py:307-309 and the scan of network.py:310, for a bf16
    window under autocast, in one kernel (``koemi_gated_projection_scan``):
    ``inputs`` ``[B, L, K]`` bf16, ``weight`` ``[2 width, K]`` bf16 (W_r
    stacked over W_c), ``bias`` ``[2 width]`` bf16 (b_r then b_c) or None,
    ``valid_mask`` ``[B, L]`` bool or None, ``initial`` ``[B, width]`` fp32.
    Returns the states ``[B, L, width]`` fp32 and, with ``with_bf16``, their
    bf16 copy (into ``out_bf16`` when given: a bf16 ``[B, L, width]`` view with
    contiguous columns and evenly spaced rows). ``final_out`` (a contiguous
    fp32 ``[B, width]`` tensor, or None) receives the last position's states
    as well (the carried state). Shapes outside ``gated_projection_fits``
    raise; the projection's results are rounded to bf16 after the bias (the
    autocast GEMM's output) before the gates.

    Each tile's wait for the tiles before it is bounded (``spin_limit`` polls,
    0 = the kernel's default). A wait that runs out makes that tile's states
    NaN and is reported: with ``status`` (an int32 device tensor of one
    element the caller zeroed) the kernel sets it to 1 and nothing syncs — the
    caller checks it later with ``check_gated_scan_status``, which is how a
    captured graph uses this; without it the front reads a status word of its
    own after the launch (a host sync) and raises ``GatedScanTimeoutError``.
    Under graph capture ``status`` is required."""

    if not gated_projection_fits(inputs, weight):
        raise DenseCudaValidationError("gated_projection_scan needs bf16 inputs [B, L, K] and weight [2 width, K] "
                                       "with L % 256 == 0, width % 128 == 0 and K % 64 == 0")
    if inputs.device.type != "cuda" or weight.device != inputs.device:
        raise DenseCudaValidationError("inputs and weight must be on the same CUDA device")
    batch, length, k = inputs.shape
    width = weight.shape[0] // 2
    if not isinstance(initial, Tensor) or initial.shape != (batch, width) or initial.dtype != torch.float32 \
            or initial.device != inputs.device:
        raise DenseCudaValidationError("initial must be a float32 [batch, width] tensor on the same device")
    if valid_mask is not None and (valid_mask.dtype != torch.bool or valid_mask.shape != (batch, length)
                                   or valid_mask.device != inputs.device):
        raise DenseCudaValidationError("valid_mask must be a bool [batch, length] tensor on the same device")
    if bias is not None and (bias.shape != (2 * width,) or bias.dtype != torch.bfloat16 or bias.device != inputs.device):
        raise DenseCudaValidationError("bias must be a bf16 [2 width] tensor on the same device")
    if status is not None and (status.dtype != torch.int32 or status.numel() != 1 or status.device != inputs.device
                               or not status.is_contiguous()):
        raise DenseCudaValidationError("status must be a contiguous int32 tensor of one element on the same device")
    if not 0 <= int(spin_limit) <= 0xFFFFFFFF:
        raise DenseCudaValidationError("spin_limit must fit in 32 bits")
    own_status = status is None
    if own_status and torch.cuda.is_current_stream_capturing():
        raise DenseCudaValidationError("gated_projection_scan under graph capture needs status= (checked after replay)")
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise DenseCudaUnavailableError(str(error)) from error
    x = inputs.contiguous()
    w = weight.contiguous()
    states = torch.empty((batch, length, width), device=x.device, dtype=torch.float32)
    states16 = None
    if with_bf16:
        states16 = out_bf16 if out_bf16 is not None else torch.empty(states.shape, device=x.device,
                                                                     dtype=torch.bfloat16)
        if (states16.shape != states.shape or states16.dtype != torch.bfloat16 or states16.stride(2) != 1
                or states16.stride(0) != length * states16.stride(1)):
            raise DenseCudaValidationError("out_bf16 must be a bf16 [batch, length, width] view with evenly spaced rows")
    if final_out is not None and (final_out.shape != (batch, width) or final_out.dtype != torch.float32
                                  or not final_out.is_contiguous() or final_out.device != inputs.device):
        raise DenseCudaValidationError("final_out must be a contiguous float32 [batch, width] tensor")
    if states.numel():
        need = _native.query("koemi_gated_projection_scan_workspace_bytes", batch, length, width)
        workspace = torch.empty(need, device=x.device, dtype=torch.uint8)
        if own_status:
            status = torch.zeros(1, device=x.device, dtype=torch.int32)
        mask = valid_mask.contiguous() if valid_mask is not None else None
        _native.call(
            "koemi_gated_projection_scan",
            _native.ptr(x), _native.ptr(w), _native.ptr(bias.contiguous()) if bias is not None else None,
            _native.ptr(mask) if mask is not None else None, _native.ptr(initial.contiguous()), _native.ptr(states),
            _native.ptr(states16), states16.stride(1) if states16 is not None else 0, _native.ptr(final_out),
            batch, length, width, k,
            _native.ptr(workspace), need, _native.ptr(status), int(spin_limit), _native.stream_of(x.device),
        )
        if own_status:
            check_gated_scan_status(status)
    return (states, states16) if with_bf16 else states
