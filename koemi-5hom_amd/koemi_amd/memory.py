"""Salient (exact-recall) and local memory on the GPU: ring reads and ring update.

Fronts for ``LocalKeyValueMemory.read_salient_window`` (reference
model/memory.py:405-429: each query attends to the carried ring entries and to
the window's admitted entries at earlier positions) and
``LocalKeyValueMemory.salient_tail`` (memory.py:431-455: the carried ring
entries followed by the window's entries, the latest ``capacity`` admitted
ones kept in time order, invalid slots zeroed). They run ``koemi_salient_read``
and ``koemi_salient_tail``; there is no torch fallback. ``read_local_window``
is the local memory's sliding-window read (memory.py:332-383) on the same
kernels (``koemi_local_read``).
"""

from __future__ import annotations

import torch
from torch import Tensor

from koemi_amd import _native
from koemi_amd.think import CudaThinkUnavailableError, CudaThinkValidationError

__all__ = ["local_novelty", "read_local_window", "read_salient_window", "salient_tail"]

_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_MAX_CAPACITY = 4096


def read_salient_window(
    carried_keys: Tensor,
    carried_values: Tensor,
    carried_valid: Tensor,
    keys: Tensor,
    values: Tensor,
    admission_mask: Tensor,
    queries: Tensor,
    *,
    out: Tensor | None = None,
) -> Tensor:
    """Salient read of one window (reference model/memory.py:405-429).

    ``carried_*``: ``[B, S, D]``, ``[B, S, D]``, ``[B, S]`` bool (the ring);
    window ``keys``/``values`` ``[B, L, D]``, ``admission_mask`` ``[B, L]`` bool and
    ``queries`` ``[B, L, D]``. Query t attends, with scores ``key . query /
    sqrt(D)``, to the valid carried entries and to the admitted window entries
    at positions before t; rows with no such entry read zeros. Returns
    ``[B, L, D]`` in the queries' dtype (fp32 accumulation). With ``out`` (a
    float32 or bfloat16 ``[B, L, D]`` view with contiguous columns and evenly
    spaced rows, e.g. a column block of a wider matrix) the read is written
    there, by one kernel where ``koemi_memory_read_into`` takes the shape, and
    ``out`` is returned; that kernel also takes fp32 queries with bfloat16
    ``keys``/``values`` viewed in place (contiguous columns, evenly spaced
    rows, e.g. column blocks of the block's key/value projection), widened
    exactly.
    """

    return _masked_read(
        "read_salient_window", "admission_mask", carried_keys, carried_values, carried_valid, keys, values,
        admission_mask, queries, 0, out,
    )


def read_local_window(
    carried_keys: Tensor,
    carried_values: Tensor,
    carried_valid: Tensor,
    keys: Tensor,
    values: Tensor,
    valid_mask: Tensor,
    queries: Tensor,
    *,
    window: int,
    out: Tensor | None = None,
) -> Tensor:
    """Local-memory read of one window: the value output of
    ``LocalKeyValueMemory.read_window`` (reference model/memory.py:332-362).

    Same layouts as ``read_salient_window`` with the window's ``valid_mask`` in
    place of the admission mask; query t attends to the valid entries among
    the ``window`` positions strictly before its own entry in
    ``[carried ; window entries]`` (``sliding_window_mask``, memory.py:364-383).
    The novelty output of the reference method is not computed (the refine
    path that reads it is off under the default ``no_refine`` ablation).
    ``out`` as for ``read_salient_window``.
    """

    if isinstance(window, bool) or not isinstance(window, int) or window < 1:
        raise CudaThinkValidationError("window must be a positive integer")
    return _masked_read(
        "read_local_window", "valid_mask", carried_keys, carried_values, carried_valid, keys, values, valid_mask,
        queries, window, out,
    )


def local_novelty(carried_keys: Tensor, carried_valid: Tensor, keys: Tensor, valid_mask: Tensor, queries: Tensor, *,
                  window: int) -> Tensor:
    """The novelty output of ``LocalKeyValueMemory.read_window`` (reference
    model/memory.py:354-361) on ``koemi_local_novelty``: per query, 1 minus the
    largest cosine similarity with a key of its sliding window (the slots
    ``read_local_window`` attends to), clamped to [0, 1]; 1 with no eligible
    slot. ``carried_keys`` fp32 [B, C, D] with ``carried_valid`` [B, C] bool;
    ``keys`` [B, L, D] fp32 or bf16 (evenly spaced rows, e.g. a column block
    of the block's projection) with ``valid_mask`` [B, L] bool; ``queries``
    fp32 [B, L, D] (evenly spaced rows). Returns [B, L] fp32."""

    if isinstance(window, bool) or not isinstance(window, int) or window < 1:
        raise CudaThinkValidationError("window must be a positive integer")
    batch, length, width = queries.shape
    cap = carried_keys.shape[1]
    if carried_keys.shape != (batch, cap, width) or carried_keys.dtype != torch.float32:
        raise CudaThinkValidationError("carried_keys must be float32 [batch, capacity, width]")
    if carried_valid.shape != (batch, cap) or valid_mask.shape != (batch, length):
        raise CudaThinkValidationError("carried_valid and valid_mask must match the keys")
    if queries.dtype != torch.float32:
        raise CudaThinkValidationError("queries must be float32")
    key_stride = _row_stride(keys, (batch, length, width), "keys")
    query_stride = _row_stride(queries, (batch, length, width), "queries")
    novelty = torch.empty((batch, length), device=queries.device, dtype=torch.float32)
    ck, cv, vm = carried_keys.contiguous(), carried_valid.contiguous(), valid_mask.contiguous()
    _native.call("koemi_local_novelty", _native.ptr(ck), _native.ptr(cv), _native.ptr(keys),
                 _native.dtype_code(keys.dtype), key_stride, _native.ptr(vm), _native.ptr(queries), query_stride,
                 _native.ptr(novelty), batch, cap, length, width, window, _native.stream_of(queries.device))
    return novelty


def _row_stride(out: Tensor, shape: tuple[int, int, int], name: str = "out", any_dtype: bool = False) -> int:
    """Row stride of a view [batch, length, width] whose rows are evenly
    spaced with contiguous columns (a column block of a wider matrix)."""

    if not isinstance(out, Tensor) or tuple(out.shape) != shape or (
            not any_dtype and out.dtype not in (torch.float32, torch.bfloat16)):
        raise CudaThinkValidationError(f"{name} must be a float32 or bfloat16 tensor of shape {list(shape)}")
    if out.stride(2) != 1 or out.stride(0) != shape[1] * out.stride(1) or out.stride(1) % 4:
        raise CudaThinkValidationError(f"{name} must have contiguous columns and evenly spaced rows (stride % 4 == 0)")
    return out.stride(1)


def _fused_read_fits(carried: int, length: int, width: int, window: int) -> bool:
    """Shapes koemi_memory_read_into takes (the one-launch fused read): at
    most 152 candidate slots per 32 queries (local: 64)."""

    if width % 8:
        return False
    if window > 0:
        return carried <= 64 and window + 31 <= 64
    return carried <= 152 and carried + length - 1 <= 152


def _masked_read(
    front: str,
    mask_name: str,
    carried_keys: Tensor,
    carried_values: Tensor,
    carried_valid: Tensor,
    keys: Tensor,
    values: Tensor,
    mask: Tensor,
    queries: Tensor,
    window: int,
    out: Tensor | None = None,
) -> Tensor:
    tensors = {
        "carried_keys": carried_keys,
        "carried_values": carried_values,
        "carried_valid": carried_valid,
        "keys": keys,
        "values": values,
        mask_name: mask,
        "queries": queries,
    }
    for name, tensor in tensors.items():
        if not isinstance(tensor, Tensor):
            raise CudaThinkValidationError(f"{name} must be a torch.Tensor")
        if tensor.device.type != "cuda":
            raise CudaThinkValidationError(f"{name} must be on CUDA")
    if len({t.device for t in tensors.values()}) != 1:
        raise CudaThinkValidationError(f"{front} tensors must be on the same CUDA device")
    if queries.ndim != 3 or keys.shape != queries.shape or values.shape != queries.shape:
        raise CudaThinkValidationError("keys, values and queries must have the same shape [batch, length, width]")
    batch, length, width = queries.shape
    if carried_keys.ndim != 3 or carried_values.shape != carried_keys.shape:
        raise CudaThinkValidationError("carried keys and values must have the same shape [batch, carried, width]")
    if carried_keys.shape[0] != batch or carried_keys.shape[2] != width:
        raise CudaThinkValidationError("carried entries must match the window's batch and width")
    carried = carried_keys.shape[1]
    if carried_valid.shape != (batch, carried) or mask.shape != (batch, length):
        raise CudaThinkValidationError(f"carried_valid and {mask_name} must be [batch, carried] and [batch, length]")
    if carried_valid.dtype != torch.bool or mask.dtype != torch.bool:
        raise CudaThinkValidationError(f"carried_valid and {mask_name} must be torch.bool")
    if queries.dtype not in _SUPPORTED_DTYPES:
        raise CudaThinkValidationError("queries must be float32, float16 or bfloat16")
    # bf16 window entries read in place by the fused fp32 read
    in_place = (keys.dtype == torch.bfloat16 and queries.dtype == torch.float32 and out is not None
                and _fused_read_fits(carried_keys.shape[1], length, width, window)
                and keys.stride(1) % 8 == 0 and keys.data_ptr() % 16 == 0)
    widen = keys.dtype == torch.bfloat16 and queries.dtype == torch.float32 and not in_place
    if any(t.dtype != queries.dtype for t in (carried_keys, carried_values)) or values.dtype != keys.dtype or (
            keys.dtype != queries.dtype and not (keys.dtype == torch.bfloat16 and queries.dtype == torch.float32)):
        raise CudaThinkValidationError("keys, values, queries and the carried entries must share a dtype "
                                       "(or bfloat16 keys and values with fp32 queries)")
    if widen:  # bf16 entries for a read that cannot take them in place: widened (exactly) first
        keys, values = keys.float(), values.float()
    key_stride = width
    if in_place:
        key_stride = _row_stride(keys, (batch, length, width), "keys", any_dtype=True)
        if _row_stride(values, (batch, length, width), "values", any_dtype=True) != key_stride:
            raise CudaThinkValidationError("keys and values must have the same row stride")
    if width < 1:
        raise CudaThinkValidationError("width must be positive")
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise CudaThinkUnavailableError(str(error)) from error

    device = queries.device
    if out is not None:
        stride = _row_stride(out, (batch, length, width))
        if batch == 0 or length == 0:
            return out
        if queries.dtype == torch.float32 and _fused_read_fits(carried, length, width, window):
            ck, cv, cvalid, fl, qs = (t.contiguous() for t in (carried_keys, carried_values, carried_valid, mask,
                                                               queries))
            if not in_place:
                keys, values = keys.contiguous(), values.contiguous()
            ptr = lambda t: _native.ptr(t) if t.numel() else None
            _native.call("koemi_memory_read_into", ptr(ck), ptr(cv), ptr(cvalid), ptr(keys), ptr(values),
                         _native.dtype_code(keys.dtype), key_stride, ptr(fl), ptr(qs), _native.ptr(out),
                         _native.dtype_code(out.dtype), stride, batch, carried, length, width, window,
                         _native.stream_of(device))
        else:
            out.copy_(_masked_read(front, mask_name, carried_keys, carried_values, carried_valid, keys, values, mask,
                                   queries, window))
        return out
    out = torch.empty_like(queries, memory_format=torch.contiguous_format)
    if batch == 0 or length == 0:
        return out
    dtype = _native.dtype_code(queries.dtype)
    workspace = torch.empty(
        _native.query("koemi_salient_read_workspace_bytes", batch, carried, length, width, dtype),
        dtype=torch.uint8,
        device=device,
    )
    contiguous = [t.contiguous() for t in (carried_keys, carried_values, carried_valid, keys, values, mask, queries)]
    pointers = [_native.ptr(t) if t.numel() else None for t in contiguous]
    sizes = (batch, carried, length, width) + ((window,) if window else ())
    _native.call(
        "koemi_local_read" if window else "koemi_salient_read",
        *pointers,
        _native.ptr(out),
        *sizes,
        dtype,
        _native.ptr(workspace),
        workspace.numel(),
        _native.stream_of(device),
    )
    return out


def salient_tail(
    carried_keys: Tensor,
    carried_values: Tensor,
    carried_valid: Tensor,
    keys: Tensor,
    values: Tensor,
    admission_mask: Tensor,
    capacity: int,
    *,
    out: tuple[Tensor, Tensor, Tensor] | None = None,
) -> tuple[Tensor, Tensor, Tensor]:
    """Ring update of the salient memory (reference model/memory.py:431-455).

    ``carried_*``: ``[B, S, D]``, ``[B, S, D]``, ``[B, S]`` bool; window
    ``keys``/``values`` ``[B, L, D]`` and ``admission_mask`` ``[B, L]`` bool.
    Returns ``(keys, values, valid)`` of ``[B, min(S + L, capacity), ...]``.
    When ``S + L <= capacity`` they are the concatenations unchanged. Otherwise
    they hold the latest valid entries (and, when fewer than ``capacity`` are
    valid, the latest invalid ones as filler) in ascending time order, with the
    keys and values of invalid slots zeroed. The reference ranks entries with
    ``torch.topk`` over ``valid ? t : -1``, whose choice among tied invalid
    entries is unspecified; this front fixes it to the latest ones. ``out``
    (build-side): contiguous buffers of those shapes that receive the result
    (a graph's static state), not overlapping the inputs.
    """

    tensors = {
        "carried_keys": carried_keys,
        "carried_values": carried_values,
        "carried_valid": carried_valid,
        "keys": keys,
        "values": values,
        "admission_mask": admission_mask,
    }
    for name, tensor in tensors.items():
        if not isinstance(tensor, Tensor):
            raise CudaThinkValidationError(f"{name} must be a torch.Tensor")
        if tensor.device.type != "cuda":
            raise CudaThinkValidationError(f"{name} must be on CUDA")
    if len({t.device for t in tensors.values()}) != 1:
        raise CudaThinkValidationError("salient_tail tensors must be on the same CUDA device")
    if isinstance(capacity, bool) or not isinstance(capacity, int) or capacity < 1:
        raise CudaThinkValidationError("capacity must be a positive integer")
    if capacity > _MAX_CAPACITY:
        raise CudaThinkValidationError(f"capacity must not exceed {_MAX_CAPACITY}")
    if keys.ndim != 3 or values.shape != keys.shape:
        raise CudaThinkValidationError("keys and values must have the same shape [batch, length, width]")
    batch, length, width = keys.shape
    if carried_keys.ndim != 3 or carried_values.shape != carried_keys.shape:
        raise CudaThinkValidationError("carried keys and values must have the same shape [batch, carried, width]")
    if carried_keys.shape[0] != batch or carried_keys.shape[2] != width:
        raise CudaThinkValidationError("carried entries must match the window's batch and width")
    carried = carried_keys.shape[1]
    if carried_valid.shape != (batch, carried) or admission_mask.shape != (batch, length):
        raise CudaThinkValidationError("carried_valid and admission_mask must be [batch, carried] and [batch, length]")
    if carried_valid.dtype != torch.bool or admission_mask.dtype != torch.bool:
        raise CudaThinkValidationError("carried_valid and admission_mask must be torch.bool")
    if keys.dtype not in _SUPPORTED_DTYPES:
        raise CudaThinkValidationError("keys must be float32, float16 or bfloat16")
    if any(t.dtype != keys.dtype for t in (values, carried_keys, carried_values)):
        raise CudaThinkValidationError("keys, values and the carried entries must share a dtype")
    if width < 1:
        raise CudaThinkValidationError("width must be positive")
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise CudaThinkUnavailableError(str(error)) from error

    device = keys.device
    slots = min(carried + length, capacity)
    if out is not None:
        out_keys, out_values, out_valid = out
        if (out_keys.shape != (batch, slots, width) or out_values.shape != out_keys.shape
                or out_valid.shape != (batch, slots) or out_keys.dtype != keys.dtype
                or out_values.dtype != keys.dtype or out_valid.dtype != torch.bool
                or not all(t.is_contiguous() for t in out)):
            raise CudaThinkValidationError("out must be contiguous [batch, slots, width] keys and values and "
                                           "[batch, slots] bool flags")
    else:
        out_keys = torch.empty((batch, slots, width), device=device, dtype=keys.dtype)
        out_values = torch.empty_like(out_keys)
        out_valid = torch.empty((batch, slots), device=device, dtype=torch.bool)
    if batch == 0 or slots == 0:
        return out_keys, out_values, out_valid
    contiguous = [t.contiguous() for t in (carried_keys, carried_values, carried_valid, keys, values, admission_mask)]
    _native.call(
        "koemi_salient_tail",
        *(_native.ptr(t) if t.numel() else None for t in contiguous),
        _native.ptr(out_keys),
        _native.ptr(out_values),
        _native.ptr(out_valid),
        batch,
        carried,
        length,
        width,
        capacity,
        _native.dtype_code(keys.dtype),
        _native.stream_of(device),
    )
    return out_keys, out_values, out_valid
