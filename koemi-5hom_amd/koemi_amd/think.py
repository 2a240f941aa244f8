"""Causal surprise and salience admission on the gfx950 HIP kernels.

``causal_surprise`` and ``benchmark_causal_surprise`` mirror
``src/koemi/cuda_kernels/think/surprise.py`` (signature, exceptions, messages,
autograd contract). As in the reference (surprise_kernel.cu:194-261) the
content-head logits come from a plain fp32 GEMM (here ``torch.mm``, i.e.
hipBLASLt) and the per-row work runs in ``csrc/surprise.hip``.

Build-side fronts (keyword-only extensions, no reference counterpart):

* ``surprise_from_logits`` — the row kernel on given fp32 logits
  (model/network.py:677-688 with the logits already computed);
* ``salience_admission`` — ``valid & (surprise > threshold)``
  (model/network.py:349) with a fixed threshold, or with the threshold at a
  quantile of the scores computed on device (``torch.quantile`` semantics).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from functools import lru_cache
from time import perf_counter

import torch
from torch import Tensor

from koemi_amd import _native

__all__ = [
    "CudaThinkBenchmark",
    "CudaThinkUnavailableError",
    "CudaThinkValidationError",
    "admission_above",
    "benchmark_causal_surprise",
    "causal_surprise",
    "salience_admission",
    "surprise_from_logits",
]

_SUPPORTED_DTYPES: tuple[torch.dtype, ...] = (torch.float16, torch.bfloat16, torch.float32)


class CudaThinkUnavailableError(RuntimeError):
    """Raised when the native think kernels cannot run (no GPU or no kernel library)."""


class CudaThinkValidationError(ValueError):
    """Raised when the causal-surprise tensors violate the native kernel contract."""


@dataclass(frozen=True)
class CudaThinkBenchmark:
    """Synchronized native-kernel timing for one causal-surprise shape."""

    elapsed_seconds: float
    latency_milliseconds: float
    positions_per_second: float
    position_count: int
    warmup_iterations: int
    measured_iterations: int


def _load() -> None:
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise CudaThinkUnavailableError(str(error)) from error


@lru_cache(maxsize=64)
def _log_vocab(vocab: int) -> float:
    # The reference computes std::log(static_cast<float>(V)) in float32.
    return float(torch.tensor(math.log(float(vocab)), dtype=torch.float32).item())


def _rows_forward(logits: Tensor, bias: Tensor | None, targets: Tensor, valid: Tensor, out_dtype: torch.dtype) -> Tensor:
    rows, vocab = logits.shape
    out = torch.empty((rows,), device=logits.device, dtype=out_dtype)
    if rows == 0:
        return out
    with torch.cuda.device(logits.device):
        _native.call(
            "koemi_surprise_rows_forward",
            logits.data_ptr(),
            _native.ptr(bias),
            targets.data_ptr(),
            valid.data_ptr(),
            out.data_ptr(),
            rows,
            vocab,
            _log_vocab(vocab),
            _native.dtype_code(out_dtype),
            _native.stream_of(logits.device),
        )
    return out


def _rows_backward(
    logits: Tensor, bias: Tensor | None, targets: Tensor, valid: Tensor, gradient: Tensor
) -> Tensor:
    rows, vocab = logits.shape
    grad_logits = torch.empty_like(logits)
    if rows == 0:
        return grad_logits
    with torch.cuda.device(logits.device):
        _native.call(
            "koemi_surprise_rows_backward",
            logits.data_ptr(),
            _native.ptr(bias),
            targets.data_ptr(),
            valid.data_ptr(),
            gradient.data_ptr(),
            grad_logits.data_ptr(),
            rows,
            vocab,
            _log_vocab(vocab),
            _native.dtype_code(gradient.dtype),
            _native.stream_of(logits.device),
        )
    return grad_logits


class _CausalSurpriseFunction(torch.autograd.Function):
    @staticmethod
    def forward(context, prior_states, content_weight, content_bias, target_ids, valid_mask):  # type: ignore[override]
        _load()
        inputs = tuple(t.contiguous() for t in (prior_states, content_weight, content_bias, target_ids, valid_mask))
        prior, weight, bias, targets, valid = inputs
        batch, sequence, width = prior.shape
        prior_float = prior.view(batch * sequence, width).float()
        logits = torch.mm(prior_float, weight.float().t())
        surprise = _rows_forward(logits, bias, targets.view(-1), valid.view(-1), prior.dtype)
        context.save_for_backward(*inputs)
        return surprise.view(batch, sequence)

    @staticmethod
    def backward(context, gradient):  # type: ignore[override]
        prior, weight, bias, targets, valid = context.saved_tensors
        batch, sequence, width = prior.shape
        prior_float = prior.view(batch * sequence, width).float()
        weight_float = weight.float()
        logits = torch.mm(prior_float, weight_float.t())
        grad_logits = _rows_backward(
            logits, bias, targets.view(-1), valid.view(-1), gradient.contiguous().view(-1).to(prior.dtype)
        )
        gradient_prior = torch.mm(grad_logits, weight_float).view(prior.shape)
        gradient_weight = torch.mm(grad_logits.t(), prior_float)
        gradient_bias = grad_logits.sum(0)
        return (
            gradient_prior.to(dtype=prior.dtype),
            gradient_weight.to(dtype=weight.dtype),
            gradient_bias.to(dtype=bias.dtype),
            None,
            None,
        )


def causal_surprise(
    prior_states: Tensor,
    content_weight: Tensor,
    content_bias: Tensor,
    target_ids: Tensor,
    valid_mask: Tensor,
    *,
    validate_targets: bool = True,
) -> Tensor:
    """Normalized causal surprise with a native forward/backward
    (reference think/surprise.py:91-128).

    Shapes ``[batch, sequence, width]``, ``[content_vocab, width]``,
    ``[content_vocab]``, ``[batch, sequence]`` (int64) and ``[batch, sequence]``
    (bool). ``prior_states[:, position]`` is the state before that position;
    invalid positions return zero and produce no gradient.
    ``validate_targets=False`` skips the host-side target range check.
    """

    _validate_inputs(prior_states, content_weight, content_bias, target_ids, valid_mask, validate_targets)
    if prior_states.shape[1] == 0:
        return prior_states.sum(dim=-1)[:, :0]
    return _CausalSurpriseFunction.apply(prior_states, content_weight, content_bias, target_ids, valid_mask)


def benchmark_causal_surprise(
    prior_states: Tensor,
    content_weight: Tensor,
    content_bias: Tensor,
    target_ids: Tensor,
    valid_mask: Tensor,
    *,
    warmup_iterations: int = 10,
    measured_iterations: int = 50,
    validate_targets: bool = True,
) -> CudaThinkBenchmark:
    """Synchronized native forward latency and positions per second
    (reference think/surprise.py:131-187)."""

    if isinstance(warmup_iterations, bool) or not isinstance(warmup_iterations, int) or warmup_iterations < 0:
        raise CudaThinkValidationError("warmup_iterations must be a non-negative integer")
    if isinstance(measured_iterations, bool) or not isinstance(measured_iterations, int) or measured_iterations <= 0:
        raise CudaThinkValidationError("measured_iterations must be a positive integer")
    _validate_inputs(prior_states, content_weight, content_bias, target_ids, valid_mask, validate_targets)
    with torch.no_grad():
        for _ in range(warmup_iterations):
            causal_surprise(prior_states, content_weight, content_bias, target_ids, valid_mask, validate_targets=False)
        torch.cuda.synchronize(prior_states.device)
        started_at = perf_counter()
        for _ in range(measured_iterations):
            causal_surprise(prior_states, content_weight, content_bias, target_ids, valid_mask, validate_targets=False)
        torch.cuda.synchronize(prior_states.device)
        elapsed_seconds = perf_counter() - started_at
    position_count = prior_states.shape[0] * prior_states.shape[1]
    average_seconds = elapsed_seconds / measured_iterations
    return CudaThinkBenchmark(
        elapsed_seconds=elapsed_seconds,
        latency_milliseconds=average_seconds * 1000.0,
        positions_per_second=position_count / average_seconds if average_seconds > 0.0 else math.inf,
        position_count=position_count,
        warmup_iterations=warmup_iterations,
        measured_iterations=measured_iterations,
    )


def _validate_inputs(
    prior_states: Tensor,
    content_weight: Tensor,
    content_bias: Tensor,
    target_ids: Tensor,
    valid_mask: Tensor,
    validate_targets: bool,
) -> int:
    """Contract checks in the reference order (think/surprise.py:190-251)."""

    tensors = {
        "prior_states": prior_states,
        "content_weight": content_weight,
        "content_bias": content_bias,
        "target_ids": target_ids,
        "valid_mask": valid_mask,
    }
    for name, tensor in tensors.items():
        if not isinstance(tensor, Tensor):
            raise CudaThinkValidationError(f"{name} must be a torch.Tensor")
    if prior_states.ndim != 3:
        raise CudaThinkValidationError("prior_states must have shape [batch, sequence, width]")
    if content_weight.ndim != 2:
        raise CudaThinkValidationError("content_weight must have shape [content_vocab, width]")
    if content_bias.ndim != 1:
        raise CudaThinkValidationError("content_bias must have shape [content_vocab]")
    expected_sequence_shape = prior_states.shape[:2]
    if target_ids.shape != expected_sequence_shape or valid_mask.shape != expected_sequence_shape:
        raise CudaThinkValidationError("target_ids and valid_mask must match [batch, sequence]")
    batch_size, _, width = prior_states.shape
    content_vocab = content_weight.shape[0]
    if content_weight.shape[1] != width or content_bias.shape[0] != content_vocab:
        raise CudaThinkValidationError("content head dimensions must match prior_states width")
    if batch_size < 1 or content_vocab < 2 or width < 1:
        raise CudaThinkValidationError("batch, content_vocab and width must be positive")
    if width > 4096:
        raise CudaThinkValidationError("width must be at most 4096 for the shared-memory backward kernel")
    if prior_states.dtype not in _SUPPORTED_DTYPES:
        raise CudaThinkValidationError("prior_states dtype must be float16, bfloat16 or float32")
    if content_weight.dtype != prior_states.dtype or content_bias.dtype != prior_states.dtype:
        raise CudaThinkValidationError("prior_states, content_weight and content_bias must share a dtype")
    if target_ids.dtype != torch.long:
        raise CudaThinkValidationError("target_ids must use torch.int64")
    if valid_mask.dtype != torch.bool:
        raise CudaThinkValidationError("valid_mask must use torch.bool")
    if isinstance(validate_targets, bool) is False:
        raise CudaThinkValidationError("validate_targets must be a boolean")
    if not torch.cuda.is_available():
        raise CudaThinkUnavailableError("native think kernel is unavailable: torch.cuda.is_available() is False")
    device_tensors = tuple(tensors.values())
    non_cuda = [str(tensor.device) for tensor in device_tensors if tensor.device.type != "cuda"]
    if non_cuda:
        raise CudaThinkValidationError(f"all think tensors must be on CUDA; found {', '.join(non_cuda)}")
    devices = {tensor.device for tensor in device_tensors}
    if len(devices) != 1:
        raise CudaThinkValidationError(
            f"all think tensors must use one CUDA device; found {', '.join(sorted(map(str, devices)))}"
        )
    if validate_targets and target_ids.numel() > 0:
        minimum_target = int(target_ids.amin().item())
        maximum_target = int(target_ids.amax().item())
        if minimum_target < 0 or maximum_target >= content_vocab:
            raise CudaThinkValidationError(
                f"target_ids must be in [0, {content_vocab}); found [{minimum_target}, {maximum_target}]"
            )
    return content_vocab


# ------------------------------------------------------------ build-side fronts


def surprise_from_logits(
    logits: Tensor,
    target_ids: Tensor,
    valid_mask: Tensor,
    *,
    content_bias: Tensor | None = None,
) -> Tensor:
    """Surprise ``1 - exp(-nll / ln V)`` from fp32 logits ``[..., V]``.

    ``nll = logsumexp(z) - z[target]`` with ``z = logits (+ content_bias)``;
    invalid positions are exactly 0 (model/network.py:677-688 with the head
    GEMM already applied). Returns fp32 ``[...]``. The exp/log routines and the
    summation order are fixed, so scores are reproducible bit for bit.
    """

    for name, tensor in (("logits", logits), ("target_ids", target_ids), ("valid_mask", valid_mask)):
        if not isinstance(tensor, Tensor):
            raise CudaThinkValidationError(f"{name} must be a torch.Tensor")
    if logits.ndim < 1 or logits.shape[-1] < 2:
        raise CudaThinkValidationError("logits must have shape [..., content_vocab] with content_vocab >= 2")
    if logits.dtype != torch.float32:
        raise CudaThinkValidationError("logits must use torch.float32")
    if target_ids.shape != logits.shape[:-1] or valid_mask.shape != logits.shape[:-1]:
        raise CudaThinkValidationError("target_ids and valid_mask must match logits.shape[:-1]")
    if target_ids.dtype != torch.long:
        raise CudaThinkValidationError("target_ids must use torch.int64")
    if valid_mask.dtype != torch.bool:
        raise CudaThinkValidationError("valid_mask must use torch.bool")
    vocab = logits.shape[-1]
    if content_bias is not None:
        if content_bias.shape != (vocab,) or content_bias.dtype != torch.float32:
            raise CudaThinkValidationError("content_bias must be a float32 tensor of shape [content_vocab]")
    if not torch.cuda.is_available():
        raise CudaThinkUnavailableError("native think kernel is unavailable: torch.cuda.is_available() is False")
    tensors = [logits, target_ids, valid_mask] + ([content_bias] if content_bias is not None else [])
    if any(t.device.type != "cuda" for t in tensors):
        raise CudaThinkValidationError("all think tensors must be on CUDA")
    if len({t.device for t in tensors}) != 1:
        raise CudaThinkValidationError("all think tensors must use one CUDA device")
    _load()
    flat = logits.reshape(-1, vocab).contiguous()
    if flat.data_ptr() % 16:
        flat = flat.clone()  # 16-byte row loads
    bias = content_bias.contiguous() if content_bias is not None else None
    out = _rows_forward(flat, bias, target_ids.reshape(-1).contiguous(), valid_mask.reshape(-1).contiguous(), torch.float32)
    return out.view(logits.shape[:-1])


def admission_above(surprise: Tensor, valid_mask: Tensor, threshold: float) -> Tensor:
    """The admission mask alone for a fixed threshold (network.py:349), as
    ``salience_admission(surprise, valid_mask, threshold=threshold)[0]`` without
    forming the tau tensor (one kernel)."""

    if not isinstance(surprise, Tensor) or not isinstance(valid_mask, Tensor):
        raise CudaThinkValidationError("surprise and valid_mask must be torch.Tensors")
    if surprise.shape != valid_mask.shape or valid_mask.dtype != torch.bool:
        raise CudaThinkValidationError("valid_mask must be a bool tensor of the surprise's shape")
    if surprise.dtype not in _SUPPORTED_DTYPES:
        raise CudaThinkValidationError("surprise dtype must be float16, bfloat16 or float32")
    if isinstance(threshold, bool) or not isinstance(threshold, (int, float)):
        raise CudaThinkValidationError("threshold must be a number")
    if surprise.device.type != "cuda" or valid_mask.device != surprise.device:
        raise CudaThinkValidationError("all think tensors must be on one CUDA device")
    _load()
    scores = surprise.reshape(-1).contiguous()
    valid = valid_mask.reshape(-1).contiguous()
    admission = torch.empty((scores.numel(),), device=scores.device, dtype=torch.bool)
    if scores.numel():
        _native.call("koemi_admission_threshold", scores.data_ptr(), valid.data_ptr(), admission.data_ptr(),
                     scores.numel(), float(threshold), _native.dtype_code(scores.dtype),
                     _native.stream_of(scores.device))
    return admission.view(surprise.shape)


def salience_admission(
    surprise: Tensor,
    valid_mask: Tensor,
    *,
    threshold: float | None = None,
    quantile: float | None = None,
) -> tuple[Tensor, Tensor]:
    """Admission mask ``valid & (surprise > tau)`` (model/network.py:349).

    Exactly one of ``threshold`` (fixed tau, the reference rule) or
    ``quantile`` (tau = ``torch.quantile(surprise, q)``, linear interpolation,
    over all scores, selected exactly on device) must be given. Returns
    ``(admission_mask, tau)`` with tau as a 0-d float32 device tensor; nothing
    is read back to the host.
    """

    if not isinstance(surprise, Tensor) or not isinstance(valid_mask, Tensor):
        raise CudaThinkValidationError("surprise and valid_mask must be torch.Tensors")
    if (threshold is None) == (quantile is None):
        raise CudaThinkValidationError("exactly one of threshold or quantile must be given")
    if surprise.shape != valid_mask.shape:
        raise CudaThinkValidationError("surprise and valid_mask must have the same shape")
    if valid_mask.dtype != torch.bool:
        raise CudaThinkValidationError("valid_mask must use torch.bool")
    if surprise.dtype not in _SUPPORTED_DTYPES:
        raise CudaThinkValidationError("surprise dtype must be float16, bfloat16 or float32")
    if not torch.cuda.is_available():
        raise CudaThinkUnavailableError("native think kernel is unavailable: torch.cuda.is_available() is False")
    if surprise.device.type != "cuda" or valid_mask.device != surprise.device:
        raise CudaThinkValidationError("all think tensors must be on one CUDA device")
    _load()
    scores = surprise.reshape(-1).contiguous()
    valid = valid_mask.reshape(-1).contiguous()
    count = scores.numel()
    admission = torch.empty((count,), device=scores.device, dtype=torch.bool)
    tau = torch.empty((), device=scores.device, dtype=torch.float32)
    with torch.cuda.device(scores.device):
        stream = _native.stream_of(scores.device)
        if threshold is not None:
            if isinstance(threshold, bool) or not isinstance(threshold, (int, float)):
                raise CudaThinkValidationError("threshold must be a number")
            tau.fill_(float(threshold))
            if count:
                _native.call(
                    "koemi_admission_threshold",
                    scores.data_ptr(),
                    valid.data_ptr(),
                    admission.data_ptr(),
                    count,
                    float(threshold),
                    _native.dtype_code(scores.dtype),
                    stream,
                )
        else:
            if isinstance(quantile, bool) or not isinstance(quantile, (int, float)) or not 0.0 <= float(quantile) <= 1.0:
                raise CudaThinkValidationError("quantile must be a number in [0, 1]")
            if count == 0:
                raise CudaThinkValidationError("quantile admission needs at least one score")
            scores32 = scores if scores.dtype == torch.float32 else scores.float()
            workspace_bytes = _native.query("koemi_admission_quantile_workspace_bytes", count)
            workspace = torch.empty((max(workspace_bytes, 1),), device=scores.device, dtype=torch.uint8)
            _native.call(
                "koemi_admission_quantile",
                scores32.data_ptr(),
                valid.data_ptr(),
                admission.data_ptr(),
                tau.data_ptr(),
                count,
                float(quantile),
                workspace.data_ptr(),
                workspace_bytes,
                stream,
            )
    return admission.view(surprise.shape), tau
