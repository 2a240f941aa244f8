"""MoE fronts on the gfx950 HIP kernels: route, permute, grouped GLU-FFN, combine.

Mirrors ``src/koemi/cuda_kernels/moe/__init__.py`` of the reference (names,
positional/keyword layout, return tuples, exception classes, validation order
and messages). The contract checks that the reference runs as several
``.item()`` synchronisations (moe/__init__.py:113-125, 213-220, 293-301,
345-353) run here as one device check and one read-back; ``validate=False``
(keyword-only, build-side) skips them for already checked inputs, like
``validate_targets=False`` of the think front.

Build-side keyword-only extensions (absent from the reference signatures):

* ``permute_topk(..., pair_weights=None)`` also returns the weights permuted
  into sorted order, for the learned gate;
* ``combine_topk(..., pair_weights=None)`` weighs each sorted pair by its gate
  probability (router.py:73) instead of ``1 / top_k`` (moe_kernels.cu:226-228);
* ``route_topk_learned`` — softmax top-k gate of router.py:46-49, with
  ``return_statistics=True`` also its ``RouterStatistics`` (router.py:11-22,
  50-58; ``merge_router_statistics`` router.py:25-32);
* ``expert_activation_counts`` — per-expert counts of network.py:48-70.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

import torch
from torch import Tensor

from koemi_amd import _native

__all__ = [
    "CudaMoeUnavailableError",
    "CudaMoeValidationError",
    "RouterStatistics",
    "combine_topk",
    "expert_activation_counts",
    "grouped_expert_mlp_fragments",
    "grouped_expert_mlp_inference",
    "load_native_extension",
    "merge_router_statistics",
    "permute_topk",
    "route_topk_learned",
    "route_topk_valid",
    "weights_to_fragments",
]

_MAX_PERMUTE_EXPERTS = 4095


class CudaMoeUnavailableError(RuntimeError):
    """Raised when the MoE kernels cannot run (no GPU or no kernel library)."""


class CudaMoeValidationError(ValueError):
    """Raised when a MoE operation receives an unsafe contract."""


def _require_library() -> None:
    if not torch.cuda.is_available():
        raise CudaMoeUnavailableError("Koemi MoE kernels require torch.cuda.is_available() == True")
    try:
        _native.load_library()
    except _native.NativeLibraryUnavailableError as error:
        raise CudaMoeUnavailableError(f"Koemi MoE kernel library is unavailable: {error}") from error


def _require_cuda_tensor(tensor: Tensor, name: str) -> None:
    if not isinstance(tensor, Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not tensor.is_cuda:
        raise CudaMoeValidationError(f"{name} must be a CUDA tensor")
    if not tensor.is_contiguous():
        raise CudaMoeValidationError(f"{name} must be contiguous")


def _require_same_cuda_device(tensors: dict[str, Tensor]) -> None:
    devices = {tensor.device for tensor in tensors.values()}
    if len(devices) != 1:
        rendered = ", ".join(sorted(str(device) for device in devices))
        raise CudaMoeValidationError(f"all MoE tensors must use one CUDA device, found {rendered}")


def _require_supported_context_dtype(tensor: Tensor, name: str) -> None:
    if tensor.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise CudaMoeValidationError(f"{name} must use float32, float16, or bfloat16; found {tensor.dtype}")


def _require_positive_bounded(value: int, name: str, upper_bound: int) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value < 1:
        raise CudaMoeValidationError(f"{name} must be a positive integer")
    if value > upper_bound:
        raise CudaMoeValidationError(f"{name} exceeds the CUDA MoE limit of {upper_bound}")
    return value


def _require_inference_only(tensors: dict[str, Tensor]) -> None:
    gradient_tensors = [name for name, tensor in tensors.items() if tensor.requires_grad]
    if gradient_tensors:
        raise RuntimeError("the native MoE path is inference-only; tensors require gradients: " + ", ".join(gradient_tensors))


def _aligned(tensor: Tensor) -> Tensor:
    """Contiguous tensor whose first element is 16-byte aligned (vector loads)."""

    return tensor if tensor.data_ptr() % 16 == 0 else tensor.clone()


def _assignment_flags(assignments: Tensor, valid_mask: Tensor, expert_count: int) -> tuple[bool, bool]:
    """(any valid assignment out of range, any valid token repeating an expert)."""

    flags = torch.zeros((2,), device=assignments.device, dtype=torch.int32)
    tokens, top_k = assignments.shape
    with torch.cuda.device(assignments.device):
        _native.call(
            "koemi_moe_check_assignments",
            assignments.data_ptr(),
            _native.dtype_code(assignments.dtype),
            valid_mask.data_ptr(),
            flags.data_ptr(),
            tokens,
            top_k,
            expert_count,
            _native.stream_of(assignments.device),
        )
    out_of_range, duplicate = flags.tolist()
    return bool(out_of_range), bool(duplicate)


def route_topk_valid(
    token_ids: Tensor,
    previous_token_ids: Tensor,
    valid_mask: Tensor,
    *,
    expert_count: int,
    top_k: int,
    validate: bool = True,
) -> Tensor:
    """Route tokens with HERM's content hash and reject duplicate valid slots
    (reference moe/__init__.py:128-176; int64 hash semantics of experts.py:283-289).

    Returns ``token_ids.shape + (top_k,)`` int64; invalid rows contain ``-1``.
    """

    tensors = {"token_ids": token_ids, "previous_token_ids": previous_token_ids, "valid_mask": valid_mask}
    for name, tensor in tensors.items():
        _require_cuda_tensor(tensor, name)
    _require_same_cuda_device(tensors)
    if token_ids.dtype not in (torch.int32, torch.int64):
        raise CudaMoeValidationError("token_ids must use int32 or int64")
    if previous_token_ids.dtype != token_ids.dtype:
        raise CudaMoeValidationError("token_ids and previous_token_ids must use one dtype")
    if valid_mask.dtype != torch.bool:
        raise CudaMoeValidationError("valid_mask must use boolean dtype")
    if token_ids.shape != previous_token_ids.shape or token_ids.shape != valid_mask.shape:
        raise CudaMoeValidationError("routing tensors must have equal shapes")
    expert_count = _require_positive_bounded(expert_count, "expert_count", 1 << 20)
    top_k = _require_positive_bounded(top_k, "top_k", 256)
    if top_k > expert_count:
        raise CudaMoeValidationError("top_k must not exceed expert_count")
    _require_library()
    count = token_ids.numel()
    assignments = torch.empty((count, top_k), device=token_ids.device, dtype=torch.int64)
    # the duplicate check's flag only when it is read (validate)
    duplicate = torch.zeros((1,), device=token_ids.device, dtype=torch.int32) if validate else None
    if count:
        with torch.cuda.device(token_ids.device):
            _native.call(
                "koemi_moe_route_hash",
                token_ids.data_ptr(),
                previous_token_ids.data_ptr(),
                valid_mask.data_ptr(),
                _native.dtype_code(token_ids.dtype),
                assignments.data_ptr(),
                duplicate.data_ptr() if duplicate is not None else None,
                count,
                expert_count,
                top_k,
                _native.stream_of(token_ids.device),
            )
    assignments = assignments.reshape(*token_ids.shape, top_k)
    if validate and count and top_k >= 2 and bool(duplicate.item()):
        raise CudaMoeValidationError("MoE routing produced duplicate experts for a valid token")
    return assignments


def route_topk_modulo(token_ids: Tensor, valid_mask: Tensor, *, expert_count: int, top_k: int) -> Tensor:
    """The benchmark's synthetic "token id mod E" route (C4 hash variant, no
    counterpart in the reference): slot ``s`` of a valid token takes expert
    ``(token_id + s) mod expert_count`` (``torch.remainder`` sign), invalid
    tokens ``-1``. Returns ``token_ids.shape + (top_k,)`` int64."""

    tensors = {"token_ids": token_ids, "valid_mask": valid_mask}
    for name, tensor in tensors.items():
        _require_cuda_tensor(tensor, name)
    _require_same_cuda_device(tensors)
    if token_ids.dtype not in (torch.int32, torch.int64):
        raise CudaMoeValidationError("token_ids must use int32 or int64")
    if valid_mask.dtype != torch.bool:
        raise CudaMoeValidationError("valid_mask must use boolean dtype")
    if token_ids.shape != valid_mask.shape:
        raise CudaMoeValidationError("routing tensors must have equal shapes")
    expert_count = _require_positive_bounded(expert_count, "expert_count", 1 << 20)
    top_k = _require_positive_bounded(top_k, "top_k", 256)
    if top_k > expert_count:
        raise CudaMoeValidationError("top_k must not exceed expert_count")
    _require_library()
    count = token_ids.numel()
    assignments = torch.empty((count, top_k), device=token_ids.device, dtype=torch.int64)
    if count:
        token_ids, valid_mask = token_ids.contiguous(), valid_mask.contiguous()
        with torch.cuda.device(token_ids.device):
            _native.call("koemi_moe_route_modulo", token_ids.data_ptr(), valid_mask.data_ptr(),
                         _native.dtype_code(token_ids.dtype), assignments.data_ptr(), count, expert_count, top_k,
                         _native.stream_of(token_ids.device))
    return assignments.reshape(*token_ids.shape, top_k)


@dataclass(frozen=True)
class RouterStatistics:
    """The learned gate's statistics of one forward (router.py:11-22): fp32
    device tensors ``probability_mass`` ``[E]`` (the valid tokens' softmax
    probabilities summed per expert), ``assignment_counts`` ``[E]`` (valid
    assignments per expert) and ``valid_count`` (0-dim, the valid tokens).
    ``balance_loss`` (0-dim fp32 device tensor) is
    ``E * sum((mass / max(valid, 1)) * (counts / max(sum(counts), 1)))``, formed
    on the device (``koemi_moe_router_balance_loss``) unless the route kernel
    already formed it."""

    probability_mass: Tensor
    assignment_counts: Tensor
    valid_count: Tensor
    _loss: Tensor | None = field(default=None, repr=False, compare=False)

    @property
    def balance_loss(self) -> Tensor:
        if self._loss is not None:
            return self._loss
        mass, counts = self.probability_mass.contiguous(), self.assignment_counts.contiguous()
        valid = self.valid_count.reshape(1).contiguous()
        tensors = {"probability_mass": mass, "assignment_counts": counts, "valid_count": valid}
        for name, tensor in tensors.items():
            _require_cuda_tensor(tensor, name)
            if tensor.dtype != torch.float32:
                raise CudaMoeValidationError(f"{name} must use float32")
        _require_same_cuda_device(tensors)
        if mass.ndim != 1 or counts.shape != mass.shape or mass.numel() < 1:
            raise CudaMoeValidationError("probability_mass and assignment_counts must be [expert_count]")
        _require_library()
        loss = torch.empty((), device=mass.device, dtype=torch.float32)
        with torch.cuda.device(mass.device):
            _native.call("koemi_moe_router_balance_loss", mass.data_ptr(), counts.data_ptr(), valid.data_ptr(),
                         mass.numel(), loss.data_ptr(), _native.stream_of(mass.device))
        return loss


def merge_router_statistics(statistics: list[RouterStatistics]) -> RouterStatistics | None:
    """Field-wise sums of several forwards' statistics (router.py:25-32: the
    windows of a sequence, network.py:835-837); None for an empty list."""

    if not statistics:
        return None
    return RouterStatistics(
        sum(item.probability_mass for item in statistics),
        sum(item.assignment_counts for item in statistics),
        sum(item.valid_count for item in statistics),
    )


def route_topk_learned(router_logits: Tensor, valid_mask: Tensor, *, top_k: int, return_statistics: bool = False
                       ) -> tuple[Tensor, Tensor] | tuple[Tensor, Tensor, RouterStatistics]:
    """Learned softmax top-k gate (router.py:46-49): returns int64 assignments and
    fp32 weights of shape ``router_logits.shape[:-1] + (top_k,)``, descending by
    probability (ties to the lower expert index); invalid rows get -1 and 0.
    With ``return_statistics`` also the ``RouterStatistics`` of router.py:50-58
    (one launch more: the route and the per-workgroup partials in one kernel,
    then a one-workgroup finisher that also forms the balance loss)."""

    tensors = {"router_logits": router_logits, "valid_mask": valid_mask}
    for name, tensor in tensors.items():
        _require_cuda_tensor(tensor, name)
    _require_same_cuda_device(tensors)
    if router_logits.dtype != torch.float32:
        raise CudaMoeValidationError("router_logits must use float32")
    if router_logits.ndim < 1 or valid_mask.shape != router_logits.shape[:-1]:
        raise CudaMoeValidationError("valid_mask must match router_logits.shape[:-1]")
    if valid_mask.dtype != torch.bool:
        raise CudaMoeValidationError("valid_mask must use boolean dtype")
    expert_count = _require_positive_bounded(int(router_logits.shape[-1]), "expert_count", 1024)
    top_k = _require_positive_bounded(top_k, "top_k", 256)
    if top_k > expert_count:
        raise CudaMoeValidationError("top_k must not exceed expert_count")
    _require_library()
    count = valid_mask.numel()
    assignments = torch.empty((count, top_k), device=router_logits.device, dtype=torch.int64)
    weights = torch.empty((count, top_k), device=router_logits.device, dtype=torch.float32)
    shape = (*valid_mask.shape, top_k)
    if return_statistics:
        device = router_logits.device
        mass = torch.empty((expert_count,), device=device, dtype=torch.float32)
        counts = torch.empty((expert_count,), device=device, dtype=torch.float32)
        valid_count = torch.empty((), device=device, dtype=torch.float32)
        loss = torch.empty((), device=device, dtype=torch.float32)
        need = _native.query("koemi_moe_route_learned_stats_workspace_bytes", count, expert_count)
        workspace = torch.empty((max(need, 1),), device=device, dtype=torch.uint8)
        logits_c, valid_c = router_logits.contiguous(), valid_mask.contiguous()
        with torch.cuda.device(device):
            _native.call("koemi_moe_route_learned_stats", logits_c.data_ptr(),
                         valid_c.data_ptr(), assignments.data_ptr(), weights.data_ptr(),
                         mass.data_ptr(), counts.data_ptr(), valid_count.data_ptr(), loss.data_ptr(), count,
                         expert_count, top_k, workspace.data_ptr(), need, _native.stream_of(device))
        statistics = RouterStatistics(mass, counts, valid_count, loss)
        return assignments.reshape(shape), weights.reshape(shape), statistics
    if count:
        with torch.cuda.device(router_logits.device):
            _native.call(
                "koemi_moe_route_learned",
                router_logits.data_ptr(),
                valid_mask.data_ptr(),
                assignments.data_ptr(),
                weights.data_ptr(),
                count,
                expert_count,
                top_k,
                _native.stream_of(router_logits.device),
            )
    return assignments.reshape(shape), weights.reshape(shape)


def expert_activation_counts(assignments: Tensor, valid_mask: Tensor, *, expert_count: int) -> Tensor:
    """int64 ``[expert_count]`` counts of valid in-range assignments (network.py:48-70)."""

    tensors = {"assignments": assignments, "valid_mask": valid_mask}
    for name, tensor in tensors.items():
        _require_cuda_tensor(tensor, name)
    _require_same_cuda_device(tensors)
    if assignments.dtype not in (torch.int32, torch.int64):
        raise CudaMoeValidationError("assignments must use int32 or int64")
    if assignments.ndim < 1 or valid_mask.shape != assignments.shape[:-1] or valid_mask.dtype != torch.bool:
        raise CudaMoeValidationError("valid_mask must be boolean with shape assignments.shape[:-1]")
    expert_count = _require_positive_bounded(expert_count, "expert_count", 1 << 20)
    _require_library()
    top_k = int(assignments.shape[-1])
    counts = torch.empty((expert_count,), device=assignments.device, dtype=torch.int64)
    with torch.cuda.device(assignments.device):
        _native.call(
            "koemi_moe_expert_counts",
            assignments.data_ptr(),
            _native.dtype_code(assignments.dtype),
            valid_mask.data_ptr(),
            counts.data_ptr(),
            valid_mask.numel(),
            max(top_k, 1),
            expert_count,
            _native.stream_of(assignments.device),
        )
    return counts


def permute_topk(
    context: Tensor,
    assignments: Tensor,
    valid_mask: Tensor,
    *,
    expert_count: int,
    pair_weights: Tensor | None = None,
    validate: bool = True,
    gather: bool = True,
) -> tuple[Tensor, ...]:
    """Sort valid token-expert pairs into stable expert segments
    (reference moe/__init__.py:179-228).

    Returns ``(sorted_context, sorted_rows, sorted_experts, segment_offsets)``;
    invalid pairs follow all expert segments with the sentinel expert
    ``expert_count`` and zero context rows. With ``pair_weights`` ([tokens,
    top_k] float32) a fifth tensor, the weights in sorted order, is returned.
    ``gather=False`` (build-side): the sorted copy of the context is not built
    and ``sorted_context`` is None (``grouped_expert_mlp_indexed`` reads the
    context rows by ``sorted_rows``).
    """

    tensors = {"context": context, "assignments": assignments, "valid_mask": valid_mask}
    for name, tensor in tensors.items():
        _require_cuda_tensor(tensor, name)
    _require_same_cuda_device(tensors)
    _require_supported_context_dtype(context, "context")
    if context.ndim < 2 or context.shape[-1] < 1:
        raise CudaMoeValidationError("context must have at least two dimensions and a non-empty width")
    if assignments.ndim != 2 or assignments.shape[0] != context.numel() // context.shape[-1]:
        raise CudaMoeValidationError("assignments must have shape [token_count, top_k]")
    if assignments.dtype not in (torch.int32, torch.int64):
        raise CudaMoeValidationError("assignments must use int32 or int64")
    if valid_mask.ndim != 1 or valid_mask.shape[0] != assignments.shape[0]:
        raise CudaMoeValidationError("valid_mask must have shape [token_count]")
    expert_count = _require_positive_bounded(expert_count, "expert_count", 1 << 20)
    top_k = _require_positive_bounded(int(assignments.shape[1]), "top_k", 256)
    if top_k > expert_count:
        raise CudaMoeValidationError("top_k must not exceed expert_count")
    if expert_count > _MAX_PERMUTE_EXPERTS:
        raise CudaMoeValidationError(f"expert_count exceeds the HIP MoE permute limit of {_MAX_PERMUTE_EXPERTS}")
    if pair_weights is not None:
        _require_cuda_tensor(pair_weights, "pair_weights")
        if pair_weights.shape != assignments.shape or pair_weights.dtype != torch.float32:
            raise CudaMoeValidationError("pair_weights must be float32 with the shape of assignments")
        if pair_weights.device != context.device:
            raise CudaMoeValidationError("all MoE tensors must use one CUDA device")
    _require_library()
    if validate and assignments.shape[0] > 0:
        out_of_range, duplicate = _assignment_flags(assignments, valid_mask, expert_count)
        if out_of_range:
            raise CudaMoeValidationError("valid MoE assignments must be in [0, expert_count)")
        if duplicate and top_k >= 2:
            raise CudaMoeValidationError("MoE permutation received duplicate experts for a valid token")
    flat = _aligned(context.reshape(-1, context.shape[-1]))
    tokens, width = flat.shape
    pairs = tokens * top_k
    device = context.device
    sorted_context = torch.empty((pairs, width), device=device, dtype=context.dtype) if gather else None
    sorted_rows = torch.empty((pairs,), device=device, dtype=torch.int64)
    sorted_experts = torch.empty((pairs,), device=device, dtype=torch.int64)
    segment_offsets = torch.empty((expert_count + 1,), device=device, dtype=torch.int64)
    sorted_weights = torch.empty((pairs,), device=device, dtype=torch.float32) if pair_weights is not None else None
    if tokens == 0:
        raise CudaMoeValidationError("context dimensions must be positive")
    workspace_bytes = _native.query("koemi_moe_permute_workspace_bytes", tokens, top_k, expert_count)
    workspace = torch.empty((workspace_bytes,), device=device, dtype=torch.uint8)
    with torch.cuda.device(device):
        _native.call(
            "koemi_moe_permute",
            flat.data_ptr(),
            _native.dtype_code(flat.dtype),
            assignments.data_ptr(),
            _native.dtype_code(assignments.dtype),
            valid_mask.data_ptr(),
            _native.ptr(pair_weights),
            _native.ptr(sorted_context),
            sorted_rows.data_ptr(),
            sorted_experts.data_ptr(),
            segment_offsets.data_ptr(),
            _native.ptr(sorted_weights),
            tokens,
            width,
            top_k,
            expert_count,
            workspace.data_ptr(),
            workspace_bytes,
            _native.stream_of(device),
        )
    if sorted_weights is not None:
        return sorted_context, sorted_rows, sorted_experts, segment_offsets, sorted_weights
    return sorted_context, sorted_rows, sorted_experts, segment_offsets


def grouped_expert_mlp_inference(
    sorted_context: Tensor,
    sorted_experts: Tensor,
    segment_offsets: Tensor,
    gate_weights: Tensor,
    gate_biases: Tensor,
    value_weights: Tensor,
    value_biases: Tensor,
    output_weights: Tensor,
    output_biases: Tensor,
    *,
    validate: bool = True,
) -> Tensor:
    """Grouped gated MLP for sorted MoE pairs (reference moe/__init__.py:231-312).

    Inference-only. Weights ``[E, H, D]``, ``[E, H]``, ``[E, H, D]``, ``[E, H]``,
    ``[E, D, H]``, ``[E, D]``; bf16 runs on MFMA with fp32 accumulation.
    """

    tensors = {
        "sorted_context": sorted_context,
        "sorted_experts": sorted_experts,
        "segment_offsets": segment_offsets,
        "gate_weights": gate_weights,
        "gate_biases": gate_biases,
        "value_weights": value_weights,
        "value_biases": value_biases,
        "output_weights": output_weights,
        "output_biases": output_biases,
    }
    for name, tensor in tensors.items():
        _require_cuda_tensor(tensor, name)
    _require_same_cuda_device(tensors)
    _require_supported_context_dtype(sorted_context, "sorted_context")
    _require_inference_only(tensors)
    if sorted_context.ndim != 2:
        raise CudaMoeValidationError("sorted_context must have shape [pair_count, width]")
    if sorted_experts.ndim != 1 or sorted_experts.shape[0] != sorted_context.shape[0]:
        raise CudaMoeValidationError("sorted_experts must have shape [pair_count]")
    if sorted_experts.dtype != torch.int64:
        raise CudaMoeValidationError("sorted_experts must use int64")
    if segment_offsets.dtype != torch.int64 or segment_offsets.ndim != 1:
        raise CudaMoeValidationError("segment_offsets must be a one-dimensional int64 tensor")
    if gate_weights.ndim != 3 or value_weights.ndim != 3 or output_weights.ndim != 3:
        raise CudaMoeValidationError("expert weights must be three-dimensional")
    expert_count, hidden_width, input_width = gate_weights.shape
    if input_width != sorted_context.shape[1]:
        raise CudaMoeValidationError("gate weight input width does not match sorted_context")
    if value_weights.shape != (expert_count, hidden_width, input_width):
        raise CudaMoeValidationError("value weights do not match gate weight shapes")
    if output_weights.shape[0] != expert_count or output_weights.shape[1] != input_width:
        raise CudaMoeValidationError("output weights do not match expert and output widths")
    if output_weights.shape[2] != hidden_width:
        raise CudaMoeValidationError("output weight hidden width does not match gate weights")
    if gate_biases.shape != (expert_count, hidden_width):
        raise CudaMoeValidationError("gate biases do not match gate weights")
    if value_biases.shape != (expert_count, hidden_width):
        raise CudaMoeValidationError("value biases do not match value weights")
    if output_biases.shape != (expert_count, input_width):
        raise CudaMoeValidationError("output biases do not match output weights")
    if segment_offsets.shape[0] != expert_count + 1:
        raise CudaMoeValidationError("segment_offsets must have expert_count + 1 entries")
    floating = [t for t in tensors.values() if t is not sorted_experts and t is not segment_offsets]
    if any(tensor.dtype != sorted_context.dtype for tensor in floating):
        raise CudaMoeValidationError("all grouped MLP floating tensors must use one dtype")
    _require_library()
    pairs = int(sorted_context.shape[0])
    if validate:
        offsets = segment_offsets.tolist()
        valid_pair_count = int(offsets[-1])
        if valid_pair_count < 0 or valid_pair_count > pairs:
            raise CudaMoeValidationError("segment_offsets final value is outside pair_count")
        if valid_pair_count:
            selected = sorted_experts[:valid_pair_count]
            bad = torch.stack(((selected < 0).any(), (selected >= expert_count).any())).tolist()
            if any(bad):
                raise CudaMoeValidationError("sorted expert ids are outside the expert catalog")
        if any(b < a for a, b in zip(offsets, offsets[1:])) or offsets[0] < 0:
            raise CudaMoeValidationError("segment_offsets must be non-decreasing")
    output = torch.empty_like(sorted_context)
    if pairs == 0:
        return output
    x = _aligned(sorted_context)
    weights = [_aligned(t) for t in (gate_weights, gate_biases, value_weights, value_biases, output_weights, output_biases)]
    workspace_bytes = _native.query(
        "koemi_moe_grouped_mlp_workspace_bytes",
        pairs,
        input_width,
        hidden_width,
        expert_count,
        _native.dtype_code(sorted_context.dtype),
    )
    workspace = torch.empty((workspace_bytes,), device=sorted_context.device, dtype=torch.uint8)
    with torch.cuda.device(sorted_context.device):
        _native.call(
            "koemi_moe_grouped_mlp",
            x.data_ptr(),
            sorted_experts.data_ptr(),
            segment_offsets.data_ptr(),
            *(w.data_ptr() for w in weights),
            output.data_ptr(),
            pairs,
            input_width,
            hidden_width,
            expert_count,
            _native.dtype_code(sorted_context.dtype),
            workspace.data_ptr(),
            workspace_bytes,
            _native.stream_of(sorted_context.device),
        )
    return output


def permute_indices(assignments: Tensor, valid_mask: Tensor, *, expert_count: int,
                    pair_weights: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor, Tensor | None, Tensor]:
    """The index phase of ``permute_topk`` without a context
    (``koemi_moe_permute_indices``, build-side): returns ``(sorted_rows,
    sorted_experts, segment_offsets, sorted_weights or None,
    pair_positions)``, the first four as ``permute_topk`` forms them and
    ``pair_positions`` [tokens * top_k] int64 the sorted position of each pair
    (valid pairs below ``segment_offsets[-1]``). No validation beyond shapes
    (the HERM block's own routing)."""

    if assignments.ndim != 2 or assignments.dtype not in (torch.int32, torch.int64):
        raise CudaMoeValidationError("assignments must be an int32 or int64 [token_count, top_k] tensor")
    tokens, top_k = assignments.shape
    if valid_mask.shape != (tokens,) or top_k > expert_count or expert_count > _MAX_PERMUTE_EXPERTS:
        raise CudaMoeValidationError("valid_mask must be [token_count] and top_k <= expert_count <= the permute limit")
    _require_library()
    device = assignments.device
    pairs = tokens * top_k
    sorted_rows = torch.empty((pairs,), device=device, dtype=torch.int64)
    sorted_experts = torch.empty((pairs,), device=device, dtype=torch.int64)
    segment_offsets = torch.empty((expert_count + 1,), device=device, dtype=torch.int64)
    sorted_weights = torch.empty((pairs,), device=device, dtype=torch.float32) if pair_weights is not None else None
    pair_positions = torch.empty((pairs,), device=device, dtype=torch.int64)
    need = _native.query("koemi_moe_permute_workspace_bytes", tokens, top_k, expert_count)
    workspace = torch.empty((need,), device=device, dtype=torch.uint8)
    with torch.cuda.device(device):
        _native.call("koemi_moe_permute_indices", assignments.contiguous().data_ptr(),
                     _native.dtype_code(assignments.dtype), valid_mask.contiguous().data_ptr(),
                     _native.ptr(pair_weights.contiguous() if pair_weights is not None else None),
                     sorted_rows.data_ptr(), sorted_experts.data_ptr(), segment_offsets.data_ptr(),
                     _native.ptr(sorted_weights), pair_positions.data_ptr(), tokens, top_k, expert_count,
                     workspace.data_ptr(), need, _native.stream_of(device))
    return sorted_rows, sorted_experts, segment_offsets, sorted_weights, pair_positions


def permute_hash_indices(token_ids: Tensor, previous_token_ids: Tensor, valid_mask: Tensor, *, expert_count: int,
                         top_k: int) -> tuple[Tensor, Tensor, Tensor, None, Tensor]:
    """``route_topk_valid`` then ``permute_indices`` in the same launches
    (``koemi_moe_permute_hash_indices``, build-side): each pair's expert is
    hashed from its token and previous token inside the permutation, the
    assignments never stored. Returns what ``permute_indices`` returns (no
    weights: the hash route has none)."""

    ids = token_ids.reshape(-1)
    prev = previous_token_ids.reshape(-1)
    tokens = ids.shape[0]
    if ids.dtype not in (torch.int32, torch.int64) or prev.dtype != ids.dtype or prev.shape != ids.shape:
        raise CudaMoeValidationError("token ids must be int32 or int64 tensors of one shape")
    if valid_mask.reshape(-1).shape != (tokens,) or top_k > expert_count or expert_count > _MAX_PERMUTE_EXPERTS:
        raise CudaMoeValidationError("valid_mask must be [token_count] and top_k <= expert_count <= the permute limit")
    _require_library()
    device = ids.device
    pairs = tokens * top_k
    sorted_rows = torch.empty((pairs,), device=device, dtype=torch.int64)
    sorted_experts = torch.empty((pairs,), device=device, dtype=torch.int64)
    segment_offsets = torch.empty((expert_count + 1,), device=device, dtype=torch.int64)
    pair_positions = torch.empty((pairs,), device=device, dtype=torch.int64)
    need = _native.query("koemi_moe_permute_workspace_bytes", tokens, top_k, expert_count)
    workspace = torch.empty((need,), device=device, dtype=torch.uint8)
    with torch.cuda.device(device):
        _native.call("koemi_moe_permute_hash_indices", ids.contiguous().data_ptr(), prev.contiguous().data_ptr(),
                     _native.dtype_code(ids.dtype), valid_mask.reshape(-1).contiguous().data_ptr(),
                     sorted_rows.data_ptr(), sorted_experts.data_ptr(), segment_offsets.data_ptr(),
                     pair_positions.data_ptr(), tokens, top_k, expert_count, workspace.data_ptr(), need,
                     _native.stream_of(device))
    return sorted_rows, sorted_experts, segment_offsets, None, pair_positions


def grouped_expert_mlp_indexed(
    context: Tensor,
    sorted_rows: Tensor,
    segment_offsets: Tensor,
    gate_weights: Tensor,
    gate_biases: Tensor,
    value_weights: Tensor,
    value_biases: Tensor,
    output_weights: Tensor,
    output_biases: Tensor,
) -> Tensor:
    """``grouped_expert_mlp_inference`` on the pairs of ``permute_topk(...,
    gather=False)`` without the sorted copy of the context: pair i reads row
    ``sorted_rows[i]`` of ``context`` ([tokens, width] bf16) straight into the
    first GEMM's operand tiles (``koemi_moe_grouped_mlp_indexed``). The
    output rows of the valid pairs ([pairs, width], pairs =
    ``sorted_rows.numel()``) equal ``grouped_expert_mlp_inference`` on the
    gathered rows bit for bit; the rows past them are left unwritten. bf16
    with width and hidden multiples of 64 only (the MFMA path); no validation
    of the index tensors beyond their shapes (indices are clamped on the
    device)."""

    if context.ndim != 2 or context.dtype != torch.bfloat16:
        raise CudaMoeValidationError("context must be a bf16 [tokens, width] tensor")
    expert_count, hidden_width, input_width = gate_weights.shape
    if input_width != context.shape[1] or input_width % 64 or hidden_width % 64:
        raise CudaMoeValidationError("the indexed grouped MLP needs width and hidden multiples of 64")
    if sorted_rows.dtype != torch.int64 or sorted_rows.ndim != 1 or segment_offsets.shape != (expert_count + 1,):
        raise CudaMoeValidationError("sorted_rows must be int64 [pairs] and segment_offsets int64 [experts + 1]")
    _require_library()
    pairs = int(sorted_rows.shape[0])
    output = torch.empty((pairs, input_width), device=context.device, dtype=context.dtype)
    if pairs == 0:
        return output
    x = _aligned(context.contiguous())
    weights = [_aligned(t.contiguous()) for t in
               (gate_weights, gate_biases, value_weights, value_biases, output_weights, output_biases)]
    workspace_bytes = _native.query("koemi_moe_grouped_mlp_workspace_bytes", pairs, input_width, hidden_width,
                                    expert_count, _native.dtype_code(torch.bfloat16))
    workspace = torch.empty((workspace_bytes,), device=context.device, dtype=torch.uint8)
    with torch.cuda.device(context.device):
        _native.call("koemi_moe_grouped_mlp_indexed", x.data_ptr(), int(x.shape[0]), sorted_rows.data_ptr(),
                     segment_offsets.data_ptr(), *(w.data_ptr() for w in weights), output.data_ptr(), pairs,
                     input_width, hidden_width, expert_count, workspace.data_ptr(), workspace_bytes,
                     _native.stream_of(context.device))
    return output


FEW_PAIRS_PER_EXPERT = 64  # pairs per expert on average up to which the skinny (decode) path runs


def weights_to_fragments(weights: Tensor) -> Tensor:
    """Expert weights [experts, rows, cols] bf16 (rows a multiple of 32, cols
    of 64) in the fragment order of ``grouped_expert_mlp_fragments``
    (``koemi_moe_weights_to_fragments``): each 32-row block stored as
    [cols / 64][4][64][8], so that every weight load of the few-rows kernels
    reads contiguous memory. A new tensor of the same shape whose element
    order alone differs."""

    if weights.ndim != 3 or weights.dtype != torch.bfloat16:
        raise CudaMoeValidationError("fragment order takes bf16 [experts, rows, cols] weights")
    matrices, rows, cols = weights.shape
    if rows % 32 or cols % 64:
        raise CudaMoeValidationError("fragment order needs rows a multiple of 32 and cols a multiple of 64")
    _require_library()
    src = _aligned(weights.contiguous())
    out = torch.empty_like(src)
    with torch.cuda.device(weights.device):
        _native.call("koemi_moe_weights_to_fragments", src.data_ptr(), out.data_ptr(), matrices, rows, cols,
                     _native.stream_of(weights.device))
    return out


def grouped_expert_mlp_fragments(
    context: Tensor,
    sorted_rows: Tensor,
    segment_offsets: Tensor,
    gate_fragments: Tensor,
    gate_biases: Tensor,
    value_fragments: Tensor,
    value_biases: Tensor,
    output_fragments: Tensor,
    output_biases: Tensor,
) -> Tensor:
    """``grouped_expert_mlp_indexed`` for a few rows per expert (a decode
    step; at most ``FEW_PAIRS_PER_EXPERT`` pairs per expert on average) with
    the three weight tensors given by ``weights_to_fragments``
    (``koemi_moe_grouped_mlp_fragments``). The same outputs bit for bit."""

    if context.ndim != 2 or context.dtype != torch.bfloat16:
        raise CudaMoeValidationError("context must be a bf16 [tokens, width] tensor")
    expert_count, hidden_width, input_width = gate_fragments.shape
    if input_width != context.shape[1] or input_width % 64 or hidden_width % 64:
        raise CudaMoeValidationError("the fragment-order grouped MLP needs width and hidden multiples of 64")
    if sorted_rows.dtype != torch.int64 or sorted_rows.ndim != 1 or segment_offsets.shape != (expert_count + 1,):
        raise CudaMoeValidationError("sorted_rows must be int64 [pairs] and segment_offsets int64 [experts + 1]")
    pairs = int(sorted_rows.shape[0])
    if pairs > FEW_PAIRS_PER_EXPERT * expert_count:
        raise CudaMoeValidationError("the fragment-order grouped MLP takes at most "
                                     f"{FEW_PAIRS_PER_EXPERT} pairs per expert on average")
    _require_library()
    output = torch.empty((pairs, input_width), device=context.device, dtype=context.dtype)
    if pairs == 0:
        return output
    x = _aligned(context.contiguous())
    weights = [_aligned(t.contiguous()) for t in
               (gate_fragments, gate_biases, value_fragments, value_biases, output_fragments, output_biases)]
    workspace_bytes = _native.query("koemi_moe_grouped_mlp_workspace_bytes", pairs, input_width, hidden_width,
                                    expert_count, _native.dtype_code(torch.bfloat16))
    workspace = torch.empty((workspace_bytes,), device=context.device, dtype=torch.uint8)
    with torch.cuda.device(context.device):
        _native.call("koemi_moe_grouped_mlp_fragments", x.data_ptr(), int(x.shape[0]), sorted_rows.data_ptr(),
                     segment_offsets.data_ptr(), *(w.data_ptr() for w in weights), output.data_ptr(), pairs,
                     input_width, hidden_width, expert_count, workspace.data_ptr(), workspace_bytes,
                     _native.stream_of(context.device))
    return output


def combine_topk(
    expert_outputs: Tensor,
    sorted_rows: Tensor,
    segment_offsets: Tensor,
    *,
    token_count: int,
    top_k: int,
    pair_weights: Tensor | None = None,
    validate: bool = True,
) -> Tensor:
    """Combine sorted expert outputs into token rows using ``1 / top_k``, or the
    per-pair ``pair_weights`` (sorted order, float32) of a learned gate
    (reference moe/__init__.py:315-360). Deterministic: no atomics in the sum."""

    tensors = {"expert_outputs": expert_outputs, "sorted_rows": sorted_rows, "segment_offsets": segment_offsets}
    for name, tensor in tensors.items():
        _require_cuda_tensor(tensor, name)
    _require_same_cuda_device(tensors)
    _require_supported_context_dtype(expert_outputs, "expert_outputs")
    _require_inference_only(tensors)
    if expert_outputs.ndim != 2:
        raise CudaMoeValidationError("expert_outputs must have shape [pair_count, width]")
    if sorted_rows.dtype != torch.int64 or sorted_rows.ndim != 1:
        raise CudaMoeValidationError("sorted_rows must be a one-dimensional int64 tensor")
    if sorted_rows.shape[0] != expert_outputs.shape[0]:
        raise CudaMoeValidationError("sorted_rows must match expert_outputs pair_count")
    if segment_offsets.dtype != torch.int64 or segment_offsets.ndim != 1:
        raise CudaMoeValidationError("segment_offsets must be a one-dimensional int64 tensor")
    token_count = _require_positive_bounded(token_count, "token_count", 1 << 31)
    top_k = _require_positive_bounded(top_k, "top_k", 256)
    if segment_offsets.shape[0] < 2:
        raise CudaMoeValidationError("segment_offsets must have at least two entries")
    if expert_outputs.shape[1] < 1:
        raise CudaMoeValidationError("expert_outputs must have shape [pair_count, width]")
    if pair_weights is not None:
        _require_cuda_tensor(pair_weights, "pair_weights")
        if pair_weights.shape != sorted_rows.shape or pair_weights.dtype != torch.float32:
            raise CudaMoeValidationError("pair_weights must be float32 of shape [pair_count]")
    _require_library()
    pairs = int(expert_outputs.shape[0])
    if validate:
        valid_pair_count = int(segment_offsets[-1].item())
        if valid_pair_count < 0 or valid_pair_count > pairs:
            raise CudaMoeValidationError("segment_offsets final value is outside pair_count")
        if valid_pair_count:
            selected = sorted_rows[:valid_pair_count]
            bad = torch.stack(((selected < 0).any(), (selected >= token_count).any())).tolist()
            if any(bad):
                raise CudaMoeValidationError("sorted rows are outside token_count")
    width = int(expert_outputs.shape[1])
    y = _aligned(expert_outputs)
    combined = torch.empty((token_count, width), device=expert_outputs.device, dtype=expert_outputs.dtype)
    workspace_bytes = _native.query("koemi_moe_combine_workspace_bytes", token_count, top_k)
    workspace = torch.empty((workspace_bytes,), device=expert_outputs.device, dtype=torch.uint8)
    with torch.cuda.device(expert_outputs.device):
        _native.call(
            "koemi_moe_combine",
            y.data_ptr(),
            sorted_rows.data_ptr(),
            segment_offsets.data_ptr(),
            _native.ptr(pair_weights),
            combined.data_ptr(),
            pairs,
            width,
            token_count,
            top_k,
            int(segment_offsets.shape[0]) - 1,
            _native.dtype_code(expert_outputs.dtype),
            workspace.data_ptr(),
            workspace_bytes,
            _native.stream_of(expert_outputs.device),
        )
    return combined


class _MoeExtension:
    """Object with the operator names of the reference's pybind MoE module
    (moe_kernels.cpp:256-262), over the C ABI."""

    KOEMI_CUDA_ABI_VERSION = _native.ABI_VERSION

    @staticmethod
    def route_topk(token_ids: Tensor, previous_token_ids: Tensor, valid_mask: Tensor, expert_count: int, top_k: int) -> Tensor:
        return route_topk_valid(
            token_ids, previous_token_ids, valid_mask, expert_count=expert_count, top_k=top_k, validate=False
        ).reshape(-1, top_k)

    @staticmethod
    def permute_topk(context: Tensor, assignments: Tensor, valid_mask: Tensor, expert_count: int) -> list[Tensor]:
        return list(permute_topk(context, assignments, valid_mask, expert_count=expert_count, validate=False))

    @staticmethod
    def grouped_expert_mlp(*tensors: Tensor) -> Tensor:
        return grouped_expert_mlp_inference(*tensors, validate=False)

    @staticmethod
    def combine_topk(expert_outputs: Tensor, sorted_rows: Tensor, segment_offsets: Tensor, token_count: int, top_k: int) -> Tensor:
        return combine_topk(expert_outputs, sorted_rows, segment_offsets, token_count=token_count, top_k=top_k, validate=False)


_MOE_EXTENSION = _MoeExtension()


def load_native_extension() -> Any:
    """Load the prebuilt kernel library (reference moe/__init__.py:24-70);
    returns an object exposing the reference's native op names."""

    _require_library()
    return _MOE_EXTENSION
