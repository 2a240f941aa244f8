"""ctypes binding of the C ABI declared in ``include/koemi_hip.h``.

The operator fronts pass ``tensor.data_ptr()`` values, element counts and the
current HIP stream of the tensors' device to the prebuilt ``libkoemi_hip.so``.
Loading never compiles anything; a missing library raises
:class:`NativeLibraryUnavailableError` so that no operator can silently fall
back to another implementation.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_double, c_float, c_int, c_int64, c_size_t, c_uint32, c_void_p
from typing import Any

import torch

from koemi_amd._build import LIBRARY_PATH

ABI_VERSION = 1

# koemi_dtype codes
F32, F16, BF16, F64, I32, I64, BOOL = range(7)
_DTYPE_CODES = {
    torch.float32: F32,
    torch.float16: F16,
    torch.bfloat16: BF16,
    torch.float64: F64,
    torch.int32: I32,
    torch.int64: I64,
    torch.bool: BOOL,
}

# koemi_status codes
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_LAUNCH = range(4)


class NativeLibraryUnavailableError(RuntimeError):
    """Raised when libkoemi_hip.so is missing or exports an unexpected ABI."""


class NativeCallError(RuntimeError):
    """Raised when a C ABI entry point returns a non-zero status."""

    def __init__(self, function: str, status: int, message: str) -> None:
        super().__init__(f"{function} failed (status {status}): {message}")
        self.function = function
        self.status = status
        self.message = message


_P = c_void_p
_SIGNATURES: dict[str, tuple[Any, tuple[Any, ...]]] = {
    "koemi_abi_version": (c_int, ()),
    "koemi_last_error": (ctypes.c_char_p, ()),
    "koemi_affine_scan_forward": (c_int, (_P, _P, _P, _P, c_int64, c_int64, c_int64, c_int, c_int, _P)),
    "koemi_affine_scan_backward": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int, c_int, _P),
    ),
    "koemi_rmsnorm_silu_forward": (c_int, (_P, _P, _P, _P, c_int64, c_int64, c_double, c_int, _P)),
    "koemi_rmsnorm_silu_backward_workspace_bytes": (c_size_t, (c_int64, c_int64)),
    "koemi_rmsnorm_silu_backward": (
        c_int,
        (_P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int, _P, c_size_t, _P),
    ),
    "koemi_surprise_rows_forward": (c_int, (_P, _P, _P, _P, _P, c_int64, c_int64, c_float, c_int, _P)),
    "koemi_surprise_rows_backward": (
        c_int,
        (_P, _P, _P, _P, _P, _P, c_int64, c_int64, c_float, c_int, _P),
    ),
    "koemi_admission_threshold": (c_int, (_P, _P, _P, c_int64, c_float, c_int, _P)),
    "koemi_admission_quantile_workspace_bytes": (c_size_t, (c_int64,)),
    "koemi_admission_quantile": (c_int, (_P, _P, _P, _P, c_int64, c_float, _P, c_size_t, _P)),
    "koemi_admission_quantile_noalloc": (c_int, (_P, _P, _P, _P, c_int64, c_float, _P)),
    "koemi_moe_route_hash": (c_int, (_P, _P, _P, c_int, _P, _P, c_int64, c_int64, c_int64, _P)),
    "koemi_moe_route_modulo": (c_int, (_P, _P, c_int, _P, c_int64, c_int64, c_int64, _P)),
    "koemi_moe_route_learned": (c_int, (_P, _P, _P, _P, c_int64, c_int64, c_int64, _P)),
    "koemi_moe_route_learned_stats_workspace_bytes": (c_size_t, (c_int64, c_int64)),
    "koemi_moe_route_learned_stats": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_moe_router_balance_loss": (c_int, (_P, _P, _P, c_int64, _P, _P)),
    "koemi_stream_read": (c_int, (_P, c_int64, c_int, c_int, c_int64, _P, _P)),
    "koemi_herm_sample_tokens": (c_int, (_P, c_int64, c_int64, c_int64, c_int64, c_float, c_int64, _P, _P, _P, _P)),
    "koemi_moe_check_assignments": (c_int, (_P, c_int, _P, _P, c_int64, c_int64, c_int64, _P)),
    "koemi_moe_expert_counts": (c_int, (_P, c_int, _P, _P, c_int64, c_int64, c_int64, _P)),
    "koemi_salient_tail": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, c_int, _P),
    ),
    "koemi_window_rings": (
        c_int,
        (_P, _P, _P, _P, _P, c_int, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64,
         c_int64, c_int64, c_int, c_int, _P),
    ),
    "koemi_recurrent_gates_workspace_bytes": (c_size_t, (c_int64, c_int64)),
    "koemi_recurrent_gates": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int, _P, c_size_t, _P),
    ),
    "koemi_recurrent_scan": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_gated_scan_workspace_bytes": (c_size_t, (c_int64, c_int64, c_int64)),
    "koemi_gated_scan": (
        c_int,
        (_P, c_int, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, c_size_t,
         _P),
    ),
    "koemi_gated_projection_scan_workspace_bytes": (c_size_t, (c_int64, c_int64, c_int64)),
    "koemi_gated_projection_scan": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, c_int64, _P, c_int64, c_int64, c_int64, c_int64, _P, c_size_t, _P, c_uint32,
         _P),
    ),
    "koemi_linear_rows": (
        c_int,
        (_P, _P, _P, _P, c_int, c_int64, c_int, _P, _P, _P, c_int64, c_int64, _P),
    ),
    "koemi_linear_rows_gated": (
        c_int,
        (_P, c_int, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P),
    ),
    "koemi_linear_rows_split": (
        c_int,
        (_P, _P, _P, _P, c_int, c_int64, c_int, _P, _P, _P, c_int64, c_int64, c_int, _P),
    ),
    "koemi_linear_rows_batched": (
        c_int,
        (_P, c_int, _P, _P, _P, c_int, c_int64, c_int64, c_int64, _P),
    ),
    "koemi_salient_read_workspace_bytes": (c_size_t, (c_int64, c_int64, c_int64, c_int64, c_int)),
    "koemi_salient_read": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_size_t, _P),
    ),
    "koemi_assoc_scan_read_workspace_bytes": (c_size_t, (c_int64, c_int64, c_int64, c_int64)),
    "koemi_assoc_scan_read": (
        c_int,
        (_P, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, c_int, c_int64, _P, _P,
         c_int64, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_assoc_scan_read_windows_workspace_bytes": (c_size_t, (c_int64, c_int64, c_int64, c_int64, c_int64)),
    "koemi_assoc_scan_read_windows": (
        c_int,
        (_P, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, c_int, c_int64, _P, _P,
         c_int64, c_int64, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_assoc_refine_scan_read_workspace_bytes": (c_size_t, (c_int64, c_int64, c_int64, c_int64)),
    "koemi_assoc_refine_scan_read": (
        c_int,
        (_P, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, c_float, _P, c_int, c_int64, _P,
         _P, _P, c_int, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_assoc_refine_scan_read_windows_workspace_bytes": (c_size_t, (c_int64, c_int64, c_int64, c_int64, c_int64)),
    "koemi_assoc_refine_scan_read_windows": (
        c_int,
        (_P, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, c_float, _P, c_int, c_int64, _P,
         _P, _P, c_int, c_int64, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_local_novelty": (
        c_int,
        (_P, _P, _P, c_int, c_int64, _P, _P, c_int64, _P, c_int64, c_int64, c_int64, c_int64, c_int64, _P),
    ),
    "koemi_herm_refine_gate": (
        c_int,
        (_P, c_int64, _P, c_int64, _P, c_int64, _P, c_int, c_int64, _P, c_int, _P, c_int, _P, c_int, c_int64, c_int64,
         c_int64, _P),
    ),
    "koemi_memory_read_into": (
        c_int,
        (_P, _P, _P, _P, _P, c_int, c_int64, _P, _P, _P, c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
         _P),
    ),
    "koemi_herm_surprise_shifted": (
        c_int, (_P, _P, _P, _P, _P, _P, _P, c_float, c_int64, c_int64, c_int64, c_float, _P),
    ),
    "koemi_herm_surprise_layers": (
        c_int, (_P, _P, _P, _P, _P, _P, c_float, c_int, c_int64, c_int64, c_float, _P),
    ),
    "koemi_herm_rmsnorm": (c_int, (_P, c_int, _P, c_int, _P, _P, _P, _P, c_int64, c_int64, c_float, _P)),
    "koemi_herm_rmsnorm_parts": (c_int, (_P, c_int, _P, c_int, _P, _P, _P, c_int64, c_int64, c_float, _P)),
    "koemi_herm_concat_bf16": (c_int, (_P, _P, _P, _P, c_int, c_int64, c_int64, _P, _P)),
    "koemi_read_step_pair": (
        c_int,
        (_P, _P, _P, c_int64, c_int64, _P, _P, _P, c_int64, _P, _P, _P, c_int64, c_int64, _P),
    ),
    "koemi_decode_memory_step": (
        c_int,
        (_P, _P, _P, c_int64, c_int64, _P, _P, _P, c_int64, _P, _P, _P, _P, c_int, c_int64, c_int64, c_int64, _P,
         _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, _P, _P, _P, _P, _P, _P,
         c_int64, c_int64, c_int64, _P),
    ),
    "koemi_read_step_pair_rings": (
        c_int,
        (_P, _P, _P, c_int64, c_int64, _P, _P, _P, c_int64, _P, _P, _P, _P, _P, c_int, c_int64, _P, _P, _P, _P, _P,
         _P, _P, _P, c_int64, c_int64, _P),
    ),
    "koemi_herm_greedy_tokens": (c_int, (_P, c_int64, c_int64, c_int64, c_int64, _P, _P)),
    "koemi_herm_token_context": (c_int, (_P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P)),
    "koemi_local_read": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_size_t, _P),
    ),
    "koemi_moe_permute_workspace_bytes": (c_size_t, (c_int64, c_int64, c_int64)),
    "koemi_moe_permute": (
        c_int,
        (_P, c_int, _P, c_int, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_moe_grouped_mlp_workspace_bytes": (c_size_t, (c_int64, c_int64, c_int64, c_int64, c_int)),
    "koemi_moe_grouped_mlp": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_size_t, _P),
    ),
    "koemi_moe_grouped_mlp_indexed": (
        c_int,
        (_P, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_moe_weights_to_fragments": (c_int, (_P, _P, c_int64, c_int64, c_int64, _P)),
    "koemi_moe_grouped_mlp_fragments": (
        c_int,
        (_P, c_int64, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_moe_combine_workspace_bytes": (c_size_t, (c_int64, c_int64)),
    "koemi_moe_combine": (
        c_int,
        (_P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, c_int, _P, c_size_t, _P),
    ),
    "koemi_herm_combine_norm_fusion": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, c_float, _P),
    ),
    "koemi_herm_combine_norm": (
        c_int,
        (_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, c_float, _P,
         c_size_t, _P),
    ),
    "koemi_moe_permute_hash_indices": (
        c_int,
        (_P, _P, c_int, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
    "koemi_moe_permute_indices": (
        c_int,
        (_P, c_int, _P, _P, _P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P, c_size_t, _P),
    ),
}

EXPORTED_SYMBOLS: tuple[str, ...] = tuple(_SIGNATURES)

_LOCK = threading.Lock()
_LIBRARY: ctypes.CDLL | None = None


def library_path() -> str:
    return str(LIBRARY_PATH)


def library_built() -> bool:
    return LIBRARY_PATH.is_file()


def load_library() -> ctypes.CDLL:
    """Load libkoemi_hip.so once per process and bind every declared entry point."""

    global _LIBRARY
    if _LIBRARY is not None:
        return _LIBRARY
    with _LOCK:
        if _LIBRARY is not None:
            return _LIBRARY
        if not LIBRARY_PATH.is_file():
            raise NativeLibraryUnavailableError(
                f"the gfx950 kernel library is not built: {LIBRARY_PATH} is missing "
                "(run __graft_entry__.build() or python -m koemi_amd._build)"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH), mode=ctypes.RTLD_LOCAL)
        except OSError as error:
            raise NativeLibraryUnavailableError(f"could not load {LIBRARY_PATH}: {error}") from error
        for name, (restype, argtypes) in _SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as error:
                raise NativeLibraryUnavailableError(f"{LIBRARY_PATH} does not export {name}") from error
            fn.restype = restype
            fn.argtypes = list(argtypes)
        version = lib.koemi_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryUnavailableError(f"{LIBRARY_PATH} exports ABI {version}; expected {ABI_VERSION}")
        _LIBRARY = lib
    return _LIBRARY


def dtype_code(dtype: torch.dtype) -> int:
    return _DTYPE_CODES[dtype]


def ptr(tensor: torch.Tensor | None) -> int | None:
    """Device address of a tensor's first element (None for an absent optional input)."""

    if tensor is None:
        return None
    return tensor.data_ptr()


def stream_of(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on `device`."""

    return torch.cuda.current_stream(device).cuda_stream


def ptr_array(tensors: list[torch.Tensor | None]) -> ctypes.Array:
    """A host array of device addresses (None for absent entries), for the
    entry points that take one pointer per layer."""

    return (c_void_p * len(tensors))(*(ptr(t) for t in tensors))


def call(name: str, *args: Any) -> None:
    """Invoke an entry point and raise NativeCallError on a non-zero status."""

    lib = load_library()
    status = getattr(lib, name)(*args)
    if status != OK:
        message = (lib.koemi_last_error() or b"").decode("utf-8", "replace")
        raise NativeCallError(name, status, message)


def query(name: str, *args: Any) -> int:
    """Invoke a size query entry point."""

    return int(getattr(load_library(), name)(*args))
