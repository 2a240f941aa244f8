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
  this configuration).
* The benchmarked path, SequencePrefill over the whole 12-layer stack, on a
  2 x 256 prefix against the float64 oracle at every layer, once at C5 and
  once with every head scaled by 8 so that admission fires in every layer
  (test_c5_sequence_prefill_stack_matches_the_oracle, tolerances there).
* Decode steps replayed from the decode graph equal eager steps (ids exact,
  logits 1e-5 of scale).
* The wavefront prefill (per-layer streams) equals the window-by-window
  prefill bit for bit; the sequence-parallel prefill equals it within the bf16
  tolerances (layer 0's fp32 states within 1e-6 relative: the fused gate
  kernel accumulates in its own order).
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


STACK_IDS = (2, 256)  # two sequences of two windows: the fused gate kernel's whole 256-position tiles


def _stack_oracle_params(raw):
    return [_oracle_layer(layer) for layer in raw]


def _rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    rel = float(np.linalg.norm(got - want) / (np.linalg.norm(want) + 1e-30))
    mx = float(np.abs(got - want).max() / (np.abs(want).max() + 1e-30))
    return rel, mx


@pytest.mark.parametrize("head_scale", [1.0, 8.0], ids=["c5", "c5-admitting"])
def test_c5_sequence_prefill_stack_matches_the_oracle(device, c5, head_scale):
    """The benchmarked path itself -- SequencePrefill, the whole 12-layer
    width-1024 stack replayed from one HIP graph (the gate projection fused
    with the scan over 256-position tiles, the window rings, the windowed
    associative memory, the batched window reads, surprise and admission in
    one kernel, the hash route inside the permutation, the indexed expert
    GEMM, the combine with both norms) -- over a 2 x 256 prefix of the C5
    ids, against oracle.herm.prefill in float64 (windows of 128, state
    carried), every layer.

    Admission: with the random-initialised head every score sits near
    1 - 1/e, below the 0.75 threshold, so the C5 case admits nothing; the
    second case scales every layer's head (weights and bias) by 8, as the
    reference fixture script does, so that scores spread and 15-55% of the
    tokens of each layer are admitted and the salient rings and reads run
    full. A score within rounding distance of the threshold may fall on
    either side in bf16 arithmetic; the oracle therefore takes the GPU's
    admission mask as its decision, and the test asserts that this mask
    equals the oracle's own rule valid & (s > threshold) for every score
    at least MARGIN from the threshold. Given equal decisions the ring bits
    (local and salient valid flags) and last tokens must be equal exactly.

    Tolerances (bf16 path against float64). Each layer's bf16 products add
    roundings of about the same relative size to the context it passes on,
    independent from layer to layer, and every layer renormalises its input,
    so relative errors grow like a random walk, as sqrt(l + 1) for layer l
    (0-based): measured relative Frobenius errors 2.7-3.8e-3 at layer 0 and
    0.99-1.06e-2 at layer 11, max abs / scale up to 4.8e-3 and 2.3e-2,
    surprise up to 0.9e-3 and 5.0e-3. Bounds, about twice the measurements:
    relative Frobenius <= REL0 * sqrt(l + 1) and max abs <= MAX0 * sqrt(l + 1)
    of the largest magnitude for every carried state and the last logits,
    surprise max abs <= SURPRISE0 * sqrt(l + 1), and MARGIN (twice the
    largest surprise bound) around the threshold for the admission rule."""

    REL0, MAX0, SURPRISE0, MARGIN = 8e-3, 1.5e-2, 3e-3, 2e-2
    settings, raw, params = c5
    if head_scale != 1.0:
        raw = [dict(layer) for layer in raw]
        for layer in raw:
            layer["head_w"] = layer["head_w"] * head_scale
            layer["head_b"] = layer["head_b"] * head_scale
        params = herm.prepare_stack(raw, settings, device)
    cfg = settings.oracle_config()
    b, length = STACK_IDS
    ids = workloads.config5().prefill_ids[:b, :length].contiguous()
    print(f"case head_scale={head_scale}: SequencePrefill [{b}, {length}] x {settings.layers} layers", flush=True)
    seq = herm.SequencePrefill(params, settings, herm.initial_states(settings, b, device), ids.to(device))
    logits = seq.run().clone()
    torch.cuda.synchronize()
    seq.check()
    surprise = [s.cpu().numpy().astype(np.float64) for s in seq.surprise]
    valid = ids.numpy() != herm.PAD_TOKEN_ID
    tau = settings.salience_threshold
    gpu_adm = [valid & (s > tau) for s in surprise]
    states = [{k: v.cpu().numpy() for k, v in st.items()} for st in seq.states]
    p_np = _stack_oracle_params(raw)
    o_logits, o_states, o_surprise, o_adm = oherm.prefill(
        p_np, [oherm.initial_state(b, cfg) for _ in p_np], ids.numpy(), cfg, settings.scan_chunk, gpu_adm,
        return_layers=True)
    admitted = [int(a.sum()) for a in gpu_adm]
    print(f"admitted per layer: {admitted}", flush=True)
    if head_scale != 1.0:
        assert min(admitted) >= 0.1 * valid.sum(), "the admitting case must admit in every layer"
    else:
        assert max(admitted) == 0
    worst = {}
    for layer in range(settings.layers):
        grow = float(np.sqrt(layer + 1.0))
        ds = float(np.abs(surprise[layer] - o_surprise[layer]).max())
        rule = valid & (o_surprise[layer] > tau)
        clear = np.abs(o_surprise[layer] - tau) >= MARGIN
        flips = int((rule != gpu_adm[layer])[clear].sum())
        print(f"layer {layer}: surprise max abs {ds:.2e}; decisions within {MARGIN} of tau "
              f"{int((~clear).sum())}; flips outside {flips}", flush=True)
        assert ds <= SURPRISE0 * grow, f"layer {layer} surprise"
        assert flips == 0, f"layer {layer} admission"
        got, want = states[layer], o_states[layer]
        for key in ("local_valid", "salient_valid", "last_token"):
            np.testing.assert_array_equal(got[key], want[key], err_msg=f"layer {layer} {key}")
        for key in ("working", "basis", "normalizer", "local_keys", "local_values", "salient_keys",
                    "salient_values"):
            if not np.any(want[key]):
                assert not np.any(got[key]), f"layer {layer} {key}"
                continue
            rel, mx = _rel(got[key], want[key])
            worst[key] = max(worst.get(key, (0, 0)), (rel, mx))
            print(f"layer {layer} {key}: rel_frobenius={rel:.3e} max/scale={mx:.3e}", flush=True)
            assert rel <= REL0 * grow and mx <= MAX0 * grow, f"layer {layer} {key}"
    rel, mx = _rel(logits.cpu().numpy(), o_logits)
    print(f"last logits: rel_frobenius={rel:.3e} max/scale={mx:.3e}; worst per key {worst}", flush=True)
    grow = float(np.sqrt(settings.layers))
    assert rel <= REL0 * grow and mx <= MAX0 * grow
