"""The C5 workload on the GPU: 12 HERM blocks, width 1024, state 1024, 16
experts top-2 (hash-routed), rings of 16, byte vocabulary + PAD, bf16
projections and expert FFNs, admission threshold 0.75 -- the benchmark's
configuration, at its shapes.

* The prefill of 8 x 2048 ids (config5) replayed from the window graph:
  finite logits of the right shape, the carried last tokens equal the last ids,
  the local rings full of valid entries, the first window's graph replay equal
  to the eager window (1e-5 of the logit scale: the same kernels; the library
  GEMMs may be replayed from other algorithms inside the capture), and a
  second replayed prefill bit-identical to the first.
* The first layer's first 128-token window and one decode step at batch 64
  (layer 0 with its token head) against oracle.herm in float64 on every row.
  Tolerances for the bf16 path against float64: relative Frobenius error of
  each output <= 1e-2 and max abs error <= 1.5e-2 of its largest magnitude,
  about five bf16 unit roundoffs (2^-9): every GEMM operand (weights and
  activations of the gate, working-state, fusion, expert and head products)
  is rounded to bf16 and about two such products feed each output in series
  (measured: 2.4e-3 to 4.3e-3, normalizer 1e-3). The surprise scores within
  2e-3 relative and the admission masks equal wherever the oracle's score is
  5e-3 or more from the threshold (with the random-initialised head every
  score is near 1 - 1/e, below the 0.75 threshold: nothing is admitted at
  this configuration; the reference fixtures cover admission).
* Decode steps replayed from the decode graph equal eager steps (ids exact,
  logits 1e-5 of scale).
* The wavefront prefill (per-layer streams) equals the window-by-window
  prefill bit for bit; the sequence-parallel prefill equals it within the bf16
  tolerances (layer 0's state bit for bit).
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from koemi_amd import herm, workloads
from oracle import herm as oherm

pytestmark = pytest.mark.gpu

WINDOW = 128


@pytest.fixture(scope="module")
def c5(device):
    settings = herm.HermSettings()
    assert (settings.layers, settings.width, settings.expert_count, settings.top_k) == (12, 1024, 16, 2)
    assert settings.linear_dtype == torch.bfloat16 and settings.salience_threshold == 0.75
    raw = herm.init_stack(settings, 1005, device)
    params = herm.prepare_stack(raw, settings, device)
    return settings, raw, params


def _report(name, got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = float(np.abs(want).max()) + 1e-30
    rel = float(np.linalg.norm(got - want) / (np.linalg.norm(want) + 1e-30))
    mx = float(np.abs(got - want).max()) / scale
    print(f"{name}: rel_frobenius={rel:.3e} max_abs/scale={mx:.3e}", flush=True)
    assert rel <= 1e-2, name
    assert mx <= 1.5e-2, name


def test_c5_prefill_properties_and_graph_replay(device, c5):
    settings, _, params = c5
    ids = workloads.config5().prefill_ids.to(device)
    batch = ids.shape[0]
    eager_logits, _ = herm.stack_window(params, settings, ids[:, :WINDOW].contiguous(),
                                        herm.initial_states(settings, batch, device))
    logits, states, graph = herm.prefill_graphed(params, settings, ids, herm.initial_states(settings, batch, device))
    torch.cuda.synchronize()
    assert logits.shape == (batch, ids.shape[1], settings.vocabulary_size)
    assert torch.isfinite(logits).all()
    scale = float(eager_logits.abs().max())
    assert float((logits[:, :WINDOW] - eager_logits).abs().max()) <= 1e-5 * scale
    first = logits.clone()
    for layer, st in enumerate(states):
        assert torch.equal(st["last_token"], ids[:, -1]), f"layer {layer} last token"
        assert bool(st["local_valid"].all()), f"layer {layer} local ring"
        assert st["salient_valid"].shape == (batch, settings.salience_memory_size)
        assert torch.isfinite(st["working"]).all() and torch.isfinite(st["basis"]).all()
    again, _, graph = herm.prefill_graphed(params, settings, ids, herm.initial_states(settings, batch, device), graph)
    torch.cuda.synchronize()
    assert torch.equal(again, first)


def _oracle_layer(raw_layer):
    return {k: v.double().cpu().numpy() for k, v in raw_layer.items()}


def test_c5_first_layer_window_and_decode_step_match_the_oracle(device, c5):
    settings, raw, params = c5
    cfg = settings.oracle_config()
    p_np = _oracle_layer(raw[0])
    c = workloads.config5()
    for name, ids in (("prefill window", c.prefill_ids[:, :WINDOW].contiguous()), ("decode step", c.decode_ids)):
        batch = ids.shape[0]
        state = herm.initial_states(dataclasses.replace(settings, layers=1), batch, device)[0]
        logits, final, nxt, surprise = herm.block_window(params[0], settings, ids.to(device), state)
        torch.cuda.synchronize()
        w_logits, w_final, w_next, w_surprise, w_adm = oherm.block_window(p_np, oherm.initial_state(batch, cfg),
                                                                          ids.numpy(), cfg)
        _report(f"{name} logits", logits.cpu().numpy(), w_logits)
        _report(f"{name} final context", final.cpu().numpy(), w_final)
        for key in ("working", "basis", "normalizer", "local_keys", "local_values"):
            _report(f"{name} {key}", nxt[key].cpu().numpy(), w_next[key])
        got_s = surprise.cpu().numpy()
        assert np.all(np.abs(got_s - w_surprise) <= 2e-3 * np.abs(w_surprise) + 1e-6), name
        clear = np.abs(w_surprise - settings.salience_threshold) >= 5e-3
        got_adm = (got_s > settings.salience_threshold) & (ids.numpy() != herm.PAD_TOKEN_ID)
        np.testing.assert_array_equal(got_adm[clear], w_adm[clear])
        np.testing.assert_array_equal(nxt["last_token"].cpu().numpy(), w_next["last_token"])
        np.testing.assert_array_equal(nxt["local_valid"].cpu().numpy(), w_next["local_valid"])
        print(f"{name}: admitted (oracle) {int(w_adm.sum())} of {w_adm.size}", flush=True)


def test_c5_decode_graph_replays_equal_eager_steps(device, c5):
    settings, _, params = c5
    ids = workloads.config5().decode_ids.to(device)
    batch = ids.shape[0]
    decode = herm.DecodeGraph(params, settings, ids, herm.initial_states(settings, batch, device))
    eager_ids, eager_states = ids.clone(), herm.initial_states(settings, batch, device)
    for step in range(4):
        logits = decode.run().clone()
        eager_logits, eager_states = herm.stack_window(params, settings, eager_ids, eager_states)
        torch.cuda.synchronize()
        scale = float(eager_logits.abs().max())
        assert float((logits - eager_logits).abs().max()) <= 1e-5 * scale, f"step {step}"
        scores = eager_logits[:, -1].clone()
        scores[:, herm.PAD_TOKEN_ID] = float("-inf")
        eager_ids = scores.argmax(dim=-1, keepdim=True)
        assert torch.equal(decode.ids, eager_ids), f"step {step}"


def test_c5_wavefront_prefill_equals_the_window_by_window_prefill(device, c5):
    settings, _, params = c5
    ids = workloads.config5().prefill_ids.to(device)
    batch = ids.shape[0]
    want, want_states, _ = herm.prefill_graphed(params, settings, ids, herm.initial_states(settings, batch, device))
    wave = herm.WavefrontPrefill(params, settings, herm.initial_states(settings, batch, device), batch, device)
    logits = wave.run(ids)
    torch.cuda.synchronize()
    assert torch.equal(logits, want)
    for got, exp in zip(wave.states, want_states):
        for key, tensor in exp.items():
            assert torch.equal(got[key], tensor), key


def test_c5_sequence_prefill_matches_the_window_by_window_prefill(device, c5):
    """The sequence-parallel prefill (one HIP graph) at C5. Layer 0's carried
    state does not depend on any product whose rows change with the batching
    (its expert FFN feeds only the next layer); the sequence path forms its
    working state with the fused gate projection + scan kernel (its own MFMA
    accumulation order, carries composed per 256-position tile) where the
    window path takes the library GEMM and the scan kernel, so layer 0 agrees
    within 1e-6 relative (1e-4 for what passes through a bf16 projection of
    the state) rather than bit for bit. The later layers and the
    logits carry the bf16 rounding of products computed over other row sets
    (the split-K expert tiles of a window against whole tiles of the
    sequence): within the tolerances of the bf16 path above (measured 6.1e-3
    relative Frobenius, 1.0e-2 max/scale). Ring bits and last tokens exact."""

    settings, _, params = c5
    ids = workloads.config5().prefill_ids.to(device)
    batch = ids.shape[0]
    want, want_states, _ = herm.prefill_graphed(params, settings, ids, herm.initial_states(settings, batch, device))
    seq = herm.SequencePrefill(params, settings, herm.initial_states(settings, batch, device), ids)
    got = seq.run(ids)
    torch.cuda.synchronize()
    rel = float((got - want).norm() / want.norm())
    mx = float((got - want).abs().max() / want.abs().max())
    print(f"C5 sequence-parallel vs window-by-window logits: rel_frobenius={rel:.3e} max/scale={mx:.3e}", flush=True)
    assert rel <= 1e-2 and mx <= 2e-2
    for key, tensor in want_states[0].items():
        got0 = seq.states[0][key]
        if tensor.dtype.is_floating_point:
            rel0 = float((got0 - tensor).norm() / (tensor.norm() + 1e-30))
            print(f"layer 0 {key}: rel_frobenius={rel0:.3e}", flush=True)
            # the working state and what the scan feeds in fp32: 1e-6; what passes
            # through the bf16 copy of the state and a bf16 projection (a value
            # may round to the neighbouring bf16 value): 1e-4
            assert rel0 <= (1e-6 if key in ("working", "basis", "normalizer") else 1e-4), f"layer 0 {key}"
        else:
            assert torch.equal(got0, tensor), f"layer 0 {key}"
    for layer, (st, exp) in enumerate(zip(seq.states, want_states)):
        for key in ("local_valid", "salient_valid", "last_token"):
            assert torch.equal(st[key], exp[key]), f"layer {layer} {key}"
        for key in ("working", "basis", "local_keys"):
            assert float((st[key] - exp[key]).norm() / exp[key].norm()) <= 1e-2, f"layer {layer} {key}"
