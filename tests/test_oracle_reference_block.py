"""The HERM block oracle against the reference's own forward_window.

``tests/golden/herm_block_{hash,learned}.npz`` hold the reference
``KoemiModel`` (model/network.py:296-441) at toy size in float64: its
``state_dict``, three windows of ids (11 tokens, 11 more with the state
carried, one decode position; padding inside and at the end of rows) and every
output (logits, surprise, admission, expert assignments, each ``KoemiState``
field after the window). They were written by
``tests/golden/make_herm_block_fixture.py`` in the CPU container from the
reference package; nothing from the reference is imported here.

The weights go through ``koemi_amd.checkpoint`` (the reference state-dict and
``KoemiState`` layout map) into ``oracle.herm.block_window``, so these tests
pin both the oracle's block composition (fusion order, residuals, norm
placement, ring updates, routing) and the layout map. Tolerances, relative to
each output's largest magnitude: 1e-12 for everything the associative memory
does not feed (working state, surprise, local and salient rings), float64
against float64; 1e-7 for the basis, normalizer and logits, because the
reference forms the memory's log-decay factors in fp32 (memory.py:106-129)
with torch's fp32 log/exp, which differ from the oracle's correctly rounded
ones by at most an ulp on some inputs (measured: <= 1e-8), and the learned
gate's fp32 softmax weights (router.py:46) likewise. Assignments, admission
masks, ring valid bits and last tokens are exact.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from koemi_amd import checkpoint
from oracle import herm

GOLDEN = Path(__file__).resolve().parent / "golden"
FIELDS = tuple(checkpoint.STATE_FIELDS) + tuple(checkpoint.REFINE_STATE_FIELDS)


def load(routing: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / f"herm_block_{routing}.npz", allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def params_of(data: dict[str, np.ndarray], expert_count: int = 4) -> dict[str, np.ndarray]:
    model_state = {k[len("param."):]: torch.from_numpy(v) for k, v in data.items() if k.startswith("param.")}
    return {k: v.numpy() for k, v in checkpoint.block_parameters(model_state, expert_count).items()}


def cfg_of(data: dict[str, np.ndarray], routing: str) -> dict:
    """``routing``: the fixture name ("hash", "learned", or "refine": hash
    routing under the herm ablation, refine_decay_rate at the reference's
    default 0.0625)."""
    return dict(width=16, memory_features=4, local_memory_size=4, salience_memory_size=3,
                salience_threshold=float(data["settings.salience_threshold"]), expert_count=4, top_k=2,
                expert_routing="learned" if routing == "learned" else "hash",
                ablation="herm" if routing == "refine" else "no_refine", refine_decay_rate=0.0625)


def state_in(data: dict[str, np.ndarray], w: int, refine: bool = False) -> dict[str, np.ndarray]:
    fields = {name: data[f"w{w}.state_in.{name}"] for name in FIELDS}
    return {k: np.asarray(v) for k, v in checkpoint.state_from_fields(fields, refine=refine).items()}


def close(got, want, rel):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    scale = max(float(np.abs(want).max()), 1e-30)
    err = float(np.abs(got - want).max()) if want.size else 0.0
    assert err <= rel * scale, f"max abs err {err:.3e} > {rel:.0e} x scale {scale:.3e}"


@pytest.mark.parametrize("routing", ["hash", "learned", "refine"])
def test_block_window_matches_reference_fixture(routing):
    data = load(routing)
    p = params_of(data)
    cfg = cfg_of(data, routing)
    refine = routing == "refine"
    fine, memory_fed = 1e-12, 1e-7
    tol = lambda key: memory_fed if key in ("basis", "normalizer", "refine_basis", "refine_normalizer") else fine
    windows = [int(n) for n in data["settings.windows"]]
    assert windows == [11, 11, 1]
    state = state_in(data, 0, refine)
    for w in range(len(windows)):
        # each window from the reference's own incoming state: errors do not compound
        if w:
            carried = state_in(data, w, refine)
            for key in carried:
                if carried[key].dtype == bool or carried[key].dtype.kind == "i":
                    np.testing.assert_array_equal(state[key], carried[key], err_msg=key)
                else:
                    close(state[key], carried[key], tol(key))
            state = carried
        logits, final, nxt, surprise, admission, assign, stats = herm.block_window(
            p, state, data[f"w{w}.ids"], cfg, return_assignments=True, return_statistics=True)
        close(logits, data[f"w{w}.logits"], memory_fed)
        if routing == "learned":
            # RouterStatistics (router.py:50-58): the reference's are fp32 sums of
            # fp32 probabilities; counts and the valid count are exact
            close(stats["probability_mass"], data[f"w{w}.router.probability_mass"], 1e-6)
            np.testing.assert_array_equal(stats["assignment_counts"], data[f"w{w}.router.assignment_counts"])
            assert stats["valid_count"] == float(data[f"w{w}.router.valid_count"])
            close(stats["balance_loss"], data[f"w{w}.router.balance_loss"], 1e-6)
        else:
            assert stats is None
        close(surprise, data[f"w{w}.surprise"], fine)
        np.testing.assert_array_equal(admission, data[f"w{w}.admission"])
        np.testing.assert_array_equal(assign, data[f"w{w}.assignments"])
        want = {k: np.asarray(v) for k, v in checkpoint.state_from_fields(
            {name: data[f"w{w}.state_out.{name}"] for name in FIELDS}, refine=refine).items()}
        for key, value in want.items():
            if value.dtype == bool or value.dtype.kind == "i":
                np.testing.assert_array_equal(nxt[key], value, err_msg=f"window {w} {key}")
            else:
                close(nxt[key], value, tol(key))
        state = nxt


def test_fixture_exercises_the_block():
    """The fixture covers what the pins need: admissions on and off in every
    window, carried ring entries, padding, both slots of each routing."""

    for routing in ("hash", "learned"):
        data = load(routing)
        for w in range(2):
            adm = data[f"w{w}.admission"]
            assert adm.any() and not adm.all()
        assert data["w2.admission"].any()
        assert data["w1.state_in.salient_valid"].any() and data["w1.state_in.local_valid"].any()
        assert (data["w0.ids"] == herm.PAD).any() and (data["w1.ids"] == herm.PAD).any()
        assert (data["w0.assignments"] >= 0).any() and (data["w0.assignments"] == -1).any()
    learned = load("learned")
    for w in range(3):  # statistics with padding excluded (windows 0 and 1 hold padding)
        if w < 2:
            assert float(learned[f"w{w}.router.valid_count"]) < learned[f"w{w}.ids"].size
        assert learned[f"w{w}.router.assignment_counts"].sum() == 2 * float(learned[f"w{w}.router.valid_count"])


def test_layout_map_roundtrip_and_errors():
    data = load("learned")
    model_state = {k[len("param."):]: torch.from_numpy(v) for k, v in data.items() if k.startswith("param.")}
    p = checkpoint.block_parameters(model_state, 4)
    assert p["gate_w"].shape == (4, 32, 16) and p["down_w"].shape == (4, 16, 32) and p["router_w"].shape == (4, 16)
    np.testing.assert_array_equal(p["up_w"][2].numpy(), data["param.experts.experts.2.value_projection.weight"])
    with pytest.raises(KeyError, match="experts.experts.3"):
        checkpoint.block_parameters({k: v for k, v in model_state.items() if "experts.3." not in k}, 4)
    with pytest.raises(ValueError, match="without a place"):
        checkpoint.block_parameters({**model_state, "memory_refine_extra.weight": torch.zeros(1, 64)}, 4)
    with pytest.raises(KeyError, match="memory_refine_gate.bias"):
        checkpoint.block_parameters({**model_state, "memory_refine_gate.weight": torch.zeros(1, 64)}, 4)
    refine = load("refine")
    refine_state = {k[len("param."):]: torch.from_numpy(v) for k, v in refine.items() if k.startswith("param.")}
    rp = checkpoint.block_parameters(refine_state, 4)
    assert rp["refine_gate_w"].shape == (1, 64) and rp["refine_gate_b"].shape == (1,)
    fields = {name: torch.from_numpy(data[f"w1.state_out.{name}"]) for name in
              (*checkpoint.STATE_FIELDS, *checkpoint.PASSTHROUGH_FIELDS)}
    back = checkpoint.state_to_fields(checkpoint.state_from_fields(fields), fields, 22)
    assert back["step_index"] == 22
    for name, tensor in fields.items():
        assert back[name] is tensor


def test_reference_checkpoint_loads_weights_only(tmp_path):
    """A format-7 payload (checkpoints.py:36-57) written with torch.save loads
    through the weights-only loader into the stack layout."""

    data = load("hash")
    model_state = {k[len("param."):]: torch.from_numpy(v) for k, v in data.items() if k.startswith("param.")}
    settings = {"vocabulary_size": 257, "embedding_size": 16, "memory_features": 4, "local_memory_size": 4,
                "salience_memory_size": 3, "salience_threshold": 0.6, "expert_count": 4, "expert_top_k": 2,
                "scan_chunk": 11, "ablation": "no_refine", "expert_routing": "hash"}
    path = tmp_path / "model.pt"
    torch.save({"format_version": 7, "model_settings": settings, "model_state": model_state}, path)
    hs, params = checkpoint.load_reference_checkpoint(path)
    assert (hs.width, hs.memory_features, hs.expert_count, hs.top_k, hs.layers) == (16, 4, 4, 2, 1)
    assert hs.expert_routing == "hash" and hs.scan_chunk == 11
    torch.testing.assert_close(params[0]["fusion_w"], model_state["fusion_projection.weight"], rtol=0, atol=0)
    torch.save({"format_version": 6, "model_settings": settings, "model_state": model_state}, path)
    with pytest.raises(ValueError, match="format version"):
        checkpoint.load_reference_checkpoint(path)
    with pytest.raises(ValueError, match="ablation"):
        checkpoint.settings_from_model_settings({**settings, "ablation": "no_surprise"})
    hs_refine = checkpoint.settings_from_model_settings({**settings, "ablation": "herm", "refine_decay_rate": 0.125})
    assert hs_refine.refine and hs_refine.refine_decay_rate == 0.125
    torch.save({"format_version": 7, "model_settings": {**settings, "ablation": "herm"}, "model_state": model_state},
               path)
    with pytest.raises(ValueError, match="exactly for the herm ablation"):
        checkpoint.load_reference_checkpoint(path)
    # CheckpointStore.validate_checkpoint's optional payload types (checkpoints.py:87-92)
    for key in ("vocabulary", "identity"):
        torch.save({"format_version": 7, "model_settings": settings, "model_state": model_state, key: [1, 2]}, path)
        with pytest.raises(ValueError, match=f"{key} payload is invalid"):
            checkpoint.load_reference_checkpoint(path)
    torch.save({"format_version": 7, "model_settings": settings, "model_state": model_state,
                "vocabulary": None, "identity": {"name": "x"}}, path)
    assert checkpoint.load_reference_checkpoint(path)[0].width == 16


@pytest.mark.parametrize("change, kind, message", [
    ({"expert_top_k": 5}, ValueError, "must not exceed expert_count"),
    ({"salience_threshold": 1.5}, ValueError, "between zero and one"),
    ({"embedding_size": 4}, ValueError, "at least 8"),
    ({"expert_dispatch": "scatter"}, ValueError, "loop or segments"),
    ({"expert_routing": "learned", "ablation": "affine"}, ValueError, "non-affine"),
    ({"compile_forward": 1}, TypeError, "boolean"),
    ({"refine_decay_rate": 0.0}, ValueError, "refine_decay_rate"),
    ({"expert_load_balance_weight": float("nan")}, ValueError, "finite"),
    ({"not_a_field": 1}, TypeError, "unknown ModelSettings fields"),
    ({"expert_count": 0, "expert_top_k": 1}, ValueError, "experts only"),
])
def test_model_settings_checks_follow_the_reference(change, kind, message):
    """ModelSettings.__post_init__ (configuration/settings.py:34-75) refuses
    these payloads, and so does the settings map (the last two: a field
    ModelSettings does not have, and a block without experts, which the map
    does not carry)."""
    settings = {"vocabulary_size": 257, "embedding_size": 16, "memory_features": 4, "expert_count": 4,
                "expert_top_k": 2, "ablation": "no_refine", "expert_routing": "hash"}
    with pytest.raises(kind, match=message):
        checkpoint.settings_from_model_settings({**settings, **change})
    ok = checkpoint.settings_from_model_settings({**settings, "expert_dispatch": "segments", "cache_capacity": 8})
    assert (ok.width, ok.expert_count, ok.top_k, ok.local_memory_size) == (16, 4, 2, 16)
