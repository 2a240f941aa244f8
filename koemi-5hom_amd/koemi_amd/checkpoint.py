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

The ``no_refine`` and ``herm`` ablations and the two expert routings are
mapped; other ablations raise.
"""

from __future__ import annotations

import math
from collections.abc import Mapping
from pathlib import Path

import torch
from torch import Tensor

__all__ = [
    "BLOCK_PARAMETERS",
    "CHECKPOINT_FORMAT_VERSION",
    "EXPERT_PARAMETERS",
    "REFINE_GATE_PARAMETERS",
    "REFINE_STATE_FIELDS",
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
# the refine gate of the "herm" ablation (network.py:94-96: nn.Linear(4 width, 1))
REFINE_GATE_PARAMETERS: dict[str, str] = {
    "memory_refine_gate.weight": "refine_gate_w",
    "memory_refine_gate.bias": "refine_gate_b",
}

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
# with the refine memory ("herm" ablation) those two are part of the layer state
REFINE_STATE_FIELDS: dict[str, str] = {"refine_basis": "refine_basis", "refine_normalizer": "refine_normalizer"}


def block_parameters(model_state: Mapping[str, Tensor], expert_count: int) -> dict[str, Tensor]:
    """One layer's parameters from a reference ``KoemiModel.state_dict()``.

    Raises ``KeyError`` naming the first reference parameter that is missing
    and ``ValueError`` for parameters this layout does not know. The learned
    router's gate and the refine gate of a ``herm`` model are mapped when
    present (the refine gate's weight and bias together)."""

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
    if any(name in model_state for name in REFINE_GATE_PARAMETERS):
        for name, key in REFINE_GATE_PARAMETERS.items():
            if name not in model_state:
                raise KeyError(f"reference parameter {name!r} is missing")
            out[key] = model_state[name]
            known.add(name)
    unknown = sorted(set(model_state) - known)
    if unknown:
        raise ValueError(f"reference parameters without a place in the HERM layout: {unknown[:4]}")
    return out


# ModelSettings fields (configuration/settings.py:16-32) and their defaults.
_MODEL_SETTINGS_DEFAULTS = {
    "vocabulary_size": 257, "embedding_size": 64, "memory_features": 16, "local_memory_size": 16,
    "salience_memory_size": 16, "salience_threshold": 0.75, "expert_count": 0, "expert_top_k": 1,
    "expert_dispatch": "loop", "cache_capacity": 256, "scan_chunk": 128, "activation_checkpointing": False,
    "compile_forward": False, "refine_decay_rate": 0.0625, "ablation": "no_refine", "expert_routing": "hash",
    "expert_load_balance_weight": 0.01,
}


def _validate_model_settings(v: Mapping) -> None:
    """The checks of ModelSettings.__post_init__ (configuration/settings.py:
    34-75), with its messages, so a payload the reference would refuse is
    refused here too."""

    checks = (
        (v["vocabulary_size"] < 257, ValueError, "vocabulary_size must cover every byte value and the padding token"),
        (v["embedding_size"] < 8, ValueError, "embedding_size must be at least 8"),
        (v["memory_features"] < 2, ValueError, "memory_features must be at least 2"),
        (v["local_memory_size"] < 1, ValueError, "local_memory_size must be at least 1"),
        (v["salience_memory_size"] < 1, ValueError, "salience_memory_size must be at least 1"),
        (not 0.0 <= v["salience_threshold"] <= 1.0, ValueError, "salience_threshold must be between zero and one"),
        (v["scan_chunk"] < 1, ValueError, "scan_chunk must be at least 1"),
        (not 0 <= v["expert_count"] <= 128, ValueError, "expert_count must be between 0 and 128"),
        (v["expert_top_k"] < 1, ValueError, "expert_top_k must be at least 1"),
        (v["expert_count"] > 0 and v["expert_top_k"] > v["expert_count"], ValueError,
         "expert_top_k must not exceed expert_count"),
        (v["expert_dispatch"] not in {"loop", "segments"}, ValueError, "expert_dispatch must be loop or segments"),
        (v["expert_routing"] not in {"hash", "learned"}, ValueError, "expert_routing must be hash or learned"),
        (v["expert_routing"] == "learned" and (v["expert_count"] < 1 or v["ablation"] == "affine"), ValueError,
         "learned routing requires experts and a non-affine ablation"),
        (not math.isfinite(v["expert_load_balance_weight"]) or v["expert_load_balance_weight"] < 0, ValueError,
         "expert_load_balance_weight must be finite and non-negative"),
        (not isinstance(v["activation_checkpointing"], bool), TypeError, "activation_checkpointing must be a boolean"),
        (not isinstance(v["compile_forward"], bool), TypeError, "compile_forward must be a boolean"),
        (v["cache_capacity"] < 1, ValueError, "cache_capacity must be at least 1"),
        (not 0.0 < v["refine_decay_rate"] <= 1.0, ValueError,
         "refine_decay_rate must be greater than zero and at most one"),
        (v["ablation"] not in {"herm", "no_refine", "no_surprise", "affine"}, ValueError,
         "ablation must be herm, no_refine, no_surprise or affine"),
    )
    for failed, kind, message in checks:
        if failed:
            raise kind(message)


def settings_from_model_settings(values: Mapping, *, layers: int = 1, linear_dtype: torch.dtype = torch.float32):
    """``herm.HermSettings`` for a reference ``ModelSettings.to_dict()`` payload
    (configuration/settings.py:14-32). Unknown fields raise ``TypeError``
    (``ModelSettings.from_dict``'s ``cls(**values)``) and the values are checked
    as ``ModelSettings.__post_init__`` checks them. Fields that do not change
    this path's arithmetic are validated and then not carried:
    ``expert_dispatch`` (loop or segment dispatch of the same sums),
    ``cache_capacity`` (the runtime's token cache), ``activation_checkpointing``
    and ``compile_forward`` (training and compilation switches),
    and ``expert_load_balance_weight`` (the factor the caller applies
    to ``moe.RouterStatistics.balance_loss`` for ``router_loss``,
    network.py:42-46). The ``no_refine`` and ``herm`` ablations (with
    ``refine_decay_rate``) and at least one expert are mapped (``ValueError``
    otherwise)."""

    from koemi_amd.herm import HermSettings

    unknown = sorted(set(values) - set(_MODEL_SETTINGS_DEFAULTS))
    if unknown:
        raise TypeError(f"unknown ModelSettings fields: {unknown}")
    merged = {**_MODEL_SETTINGS_DEFAULTS, **values}
    _validate_model_settings(merged)
    ablation = merged["ablation"]
    if ablation not in ("no_refine", "herm"):
        raise ValueError(f"only the no_refine and herm ablations are mapped, not {ablation!r}")
    if merged["expert_count"] < 1:
        raise ValueError("the HERM block is mapped with experts only (expert_count >= 1)")
    routing = merged["expert_routing"]
    return HermSettings(
        width=int(merged["embedding_size"]),
        memory_features=int(merged["memory_features"]),
        local_memory_size=int(merged["local_memory_size"]),
        salience_memory_size=int(merged["salience_memory_size"]),
        salience_threshold=float(merged["salience_threshold"]),
        expert_count=int(merged["expert_count"]),
        top_k=int(merged["expert_top_k"]),
        vocabulary_size=int(merged["vocabulary_size"]),
        layers=layers,
        scan_chunk=int(merged["scan_chunk"]),
        linear_dtype=linear_dtype,
        expert_routing=routing,
        ablation=ablation,
        refine_decay_rate=float(merged["refine_decay_rate"]),
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
    if raw.get("vocabulary") is not None and not isinstance(raw["vocabulary"], dict):
        raise ValueError("checkpoint vocabulary payload is invalid")
    if raw.get("identity") is not None and not isinstance(raw["identity"], dict):
        raise ValueError("checkpoint identity payload is invalid")
    settings = settings_from_model_settings(raw["model_settings"], linear_dtype=linear_dtype)
    params = block_parameters(raw["model_state"], settings.expert_count)
    if settings.expert_routing == "learned" and "router_w" not in params:
        raise KeyError(f"reference parameter {ROUTER_PARAMETER[0]!r} is missing")
    if (settings.ablation == "herm") != ("refine_gate_w" in params):
        raise ValueError("the refine gate parameters are present exactly for the herm ablation")
    return settings, [params]


def state_from_fields(fields: Mapping[str, Tensor], *, refine: bool = False) -> dict[str, Tensor]:
    """A herm layer state from ``KoemiState`` fields (a static state: the
    rings at their capacity, state.py:43-76); with ``refine`` (a ``herm``
    ablation stack) the refine basis and normalizer as well."""

    names = {**STATE_FIELDS, **(REFINE_STATE_FIELDS if refine else {})}
    missing = [name for name in names if name not in fields]
    if missing:
        raise KeyError(f"KoemiState field {missing[0]!r} is missing")
    return {key: fields[name] for name, key in names.items()}


def state_to_fields(state: Mapping[str, Tensor], carried: Mapping[str, Tensor], step_index: int) -> dict:
    """``KoemiState`` fields (and ``step_index``) from a herm layer state; the
    refine basis and normalizer come from the state when it holds them (the
    ``herm`` ablation), else from ``carried`` (the state before the window),
    as forward_window passes them on under ``no_refine`` (network.py:368-371)."""

    out = {name: state[key] for name, key in STATE_FIELDS.items()}
    for name in PASSTHROUGH_FIELDS:
        out[name] = state[REFINE_STATE_FIELDS[name]] if REFINE_STATE_FIELDS[name] in state else carried[name]
    out["step_index"] = int(step_index)
    return out
