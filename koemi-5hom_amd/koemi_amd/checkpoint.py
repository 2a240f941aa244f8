"""Reference checkpoints and ``KoemiState`` in this package's stack layout.

The reference saves one ``KoemiModel`` (a single HERM block) as a format-7
payload ``{"format_version": 7, "model_settings": {...}, "model_state":
state_dict}`` (training/checkpoints.py:15, 36-57) and loads it back with
``torch.load(..., weights_only=True)`` (checkpoints.py:59-66). Its recurrent
state is the frozen ``KoemiState`` dataclass with the twelve tensor fields of
``KOEMI_STATE_FIELDS`` plus ``step_index`` (model/state.py:11-41).

This module maps both onto the layout of ``koemi_amd.herm``:

* ``block_parameters`` turns a reference ``state_dict`` into one layer's
  parameter dict (the names ``herm.init_stack`` produces), stacking the
  per-expert ``GatedFeedForward`` weights into ``[E, ...]`` tensors;
* ``load_reference_checkpoint`` reads a format-7 file with the weights-only
  loader (nothing in the file is executed) and returns ``HermSettings`` and
  the one-layer parameter list ``herm.prepare_stack`` takes;
* ``state_from_fields`` / ``state_to_fields`` convert between a ``KoemiState``
  (as a mapping of its field names, e.g. ``dataclasses.asdict``) and the
  per-layer state dict of ``herm.initial_states``; the refine memory, which
  the ``no_refine`` block neither reads nor writes, passes through unchanged.

Only the ``no_refine`` ablation and the two expert routings are mapped;
other ablations raise.
"""

from __future__ import annotations

from collections.abc import Mapping
from pathlib import Path

import torch
from torch import Tensor

__all__ = [
    "BLOCK_PARAMETERS",
    "CHECKPOINT_FORMAT_VERSION",
    "EXPERT_PARAMETERS",
    "STATE_FIELDS",
    "block_parameters",
    "load_reference_checkpoint",
    "settings_from_model_settings",
    "state_from_fields",
    "state_to_fields",
]

CHECKPOINT_FORMAT_VERSION = 7  # training/checkpoints.py:15

# reference module path (network.py:81-106; memory.py:14-20, 68-74, 291-295;
# experts.py:63-64; router.py:41) -> layer key of herm.init_stack
BLOCK_PARAMETERS: dict[str, str] = {
    "embedding.weight": "embedding",
    "input_normalizer.weight": "input_norm",
    "recurrent_state.retention_projection.weight": "retention_w",
    "recurrent_state.retention_projection.bias": "retention_b",
    "recurrent_state.candidate_projection.weight": "candidate_w",
    "recurrent_state.candidate_projection.bias": "candidate_b",
    "associative_memory.key_projection.weight": "key_w",
    "associative_memory.key_projection.bias": "key_b",
    "associative_memory.query_projection.weight": "query_w",
    "associative_memory.query_projection.bias": "query_b",
    "associative_memory.value_projection.weight": "value_w",
    "associative_memory.value_projection.bias": "value_b",
    "associative_memory.feature_projection.weight": "feature_w",
    "associative_memory.feature_projection.bias": "feature_b",
    "associative_memory.decay_projection.weight": "decay_w",
    "associative_memory.decay_projection.bias": "decay_b",
    "associative_memory.write_projection.weight": "write_w",
    "associative_memory.write_projection.bias": "write_b",
    "local_memory.local_key_projection.weight": "local_key_w",
    "local_memory.local_key_projection.bias": "local_key_b",
    "local_memory.local_value_projection.weight": "local_value_w",
    "local_memory.local_value_projection.bias": "local_value_b",
    "fusion_projection.weight": "fusion_w",
    "fusion_projection.bias": "fusion_b",
    "fusion_normalizer.weight": "fusion_norm",
    "experts.output_normalizer.weight": "expert_norm",
    "token_predictor.weight": "head_w",
    "token_predictor.bias": "head_b",
}
ROUTER_PARAMETER = ("experts.gate.weight", "router_w")  # LearnedExpertMixture.gate (router.py:41), no bias

# GatedFeedForward submodule (layers.py:19-29) -> stacked key prefix
EXPERT_PARAMETERS: dict[str, str] = {
    "gate_projection": "gate",
    "value_projection": "up",
    "output_projection": "down",
}

# KoemiState field (state.py:11-24) -> herm state key; refine_* are carried aside
STATE_FIELDS: dict[str, str] = {
    "working_state": "working",
    "memory_basis": "basis",
    "memory_normalizer": "normalizer",
    "local_keys": "local_keys",
    "local_values": "local_values",
    "local_valid": "local_valid",
    "salient_keys": "salient_keys",
    "salient_values": "salient_values",
    "salient_valid": "salient_valid",
    "last_token_ids": "last_token",
}
PASSTHROUGH_FIELDS = ("refine_basis", "refine_normalizer")


def block_parameters(model_state: Mapping[str, Tensor], expert_count: int) -> dict[str, Tensor]:
    """One layer's parameters from a reference ``KoemiModel.state_dict()``.

    Raises ``KeyError`` naming the first reference parameter that is missing
    and ``ValueError`` for parameters this layout does not know (for example
    the refine gate of a non-``no_refine`` model)."""

    out: dict[str, Tensor] = {}
    for name, key in BLOCK_PARAMETERS.items():
        if name not in model_state:
            raise KeyError(f"reference parameter {name!r} is missing")
        out[key] = model_state[name]
    known = set(BLOCK_PARAMETERS)
    for sub, prefix in EXPERT_PARAMETERS.items():
        for kind in ("weight", "bias"):
            names = [f"experts.experts.{e}.{sub}.{kind}" for e in range(expert_count)]
            missing = [n for n in names if n not in model_state]
            if missing:
                raise KeyError(f"reference parameter {missing[0]!r} is missing")
            out[f"{prefix}_{kind[0]}"] = torch.stack([model_state[n] for n in names])
            known.update(names)
    if ROUTER_PARAMETER[0] in model_state:
        out[ROUTER_PARAMETER[1]] = model_state[ROUTER_PARAMETER[0]]
        known.add(ROUTER_PARAMETER[0])
    unknown = sorted(set(model_state) - known)
    if unknown:
        raise ValueError(f"reference parameters without a place in the HERM layout: {unknown[:4]}")
    return out


def settings_from_model_settings(values: Mapping, *, layers: int = 1, linear_dtype: torch.dtype = torch.float32):
    """``herm.HermSettings`` for a reference ``ModelSettings.to_dict()`` payload
    (configuration/settings.py:14-32)."""

    from koemi_amd.herm import HermSettings

    ablation = values.get("ablation", "no_refine")
    if ablation != "no_refine":
        raise ValueError(f"only the no_refine ablation is mapped, not {ablation!r}")
    routing = values.get("expert_routing", "hash")
    if routing not in ("hash", "learned"):
        raise ValueError(f"unknown expert routing {routing!r}")
    return HermSettings(
        width=int(values.get("embedding_size", 64)),
        memory_features=int(values.get("memory_features", 16)),
        local_memory_size=int(values.get("local_memory_size", 16)),
        salience_memory_size=int(values.get("salience_memory_size", 16)),
        salience_threshold=float(values.get("salience_threshold", 0.75)),
        expert_count=int(values.get("expert_count", 0)),
        top_k=int(values.get("expert_top_k", 1)),
        vocabulary_size=int(values.get("vocabulary_size", 257)),
        layers=layers,
        scan_chunk=int(values.get("scan_chunk", 128)),
        linear_dtype=linear_dtype,
        expert_routing=routing,
    )


def load_reference_checkpoint(path: str | Path, *, linear_dtype: torch.dtype = torch.float32):
    """(settings, [layer params]) from a reference format-7 checkpoint file,
    read with ``torch.load(weights_only=True)`` on the CPU; the validation
    follows ``CheckpointStore.validate_checkpoint`` (checkpoints.py:80-93)."""

    raw = torch.load(Path(path), map_location="cpu", weights_only=True)
    if not isinstance(raw, dict):
        raise ValueError("checkpoint must contain a dictionary payload")
    if raw.get("format_version") != CHECKPOINT_FORMAT_VERSION:
        raise ValueError("checkpoint format version is not supported")
    if not isinstance(raw.get("model_settings"), dict):
        raise ValueError("checkpoint model settings are invalid")
    if not isinstance(raw.get("model_state"), dict):
        raise ValueError("checkpoint model state is invalid")
    settings = settings_from_model_settings(raw["model_settings"], linear_dtype=linear_dtype)
    params = block_parameters(raw["model_state"], settings.expert_count)
    if settings.expert_routing == "learned" and "router_w" not in params:
        raise KeyError(f"reference parameter {ROUTER_PARAMETER[0]!r} is missing")
    return settings, [params]


def state_from_fields(fields: Mapping[str, Tensor]) -> dict[str, Tensor]:
    """A herm layer state from ``KoemiState`` fields (a static state: the
    rings at their capacity, state.py:43-76)."""

    missing = [name for name in STATE_FIELDS if name not in fields]
    if missing:
        raise KeyError(f"KoemiState field {missing[0]!r} is missing")
    return {key: fields[name] for name, key in STATE_FIELDS.items()}


def state_to_fields(state: Mapping[str, Tensor], carried: Mapping[str, Tensor], step_index: int) -> dict:
    """``KoemiState`` fields (and ``step_index``) from a herm layer state; the
    refine basis and normalizer come from ``carried`` (the state before the
    window), as forward_window passes them on under ``no_refine``
    (network.py:368-371)."""

    out = {name: state[key] for name, key in STATE_FIELDS.items()}
    for name in PASSTHROUGH_FIELDS:
        out[name] = carried[name]
    out["step_index"] = int(step_index)
    return out
