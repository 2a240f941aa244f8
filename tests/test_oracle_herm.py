"""CPU checks of the HERM block oracle (oracle/herm.py) and its new parts.

Pins, beyond the formulas themselves:
* the associative scan-and-read (parallel, memory.py:97-144) equals the
  sequential read/update recurrence (memory.py:91-95, 279-288);
* the local sliding-window read (memory.py:332-383) equals the per-position
  ring read of the sequential path (memory.py:307-330, 457-475);
* with admission switched off (threshold above every score), the stack's
  output does not depend on how the sequence is cut into windows (the carried
  state reproduces a longer window exactly): exercises every state carry;
* a window of padding tokens leaves the recurrent and associative state, the
  last token and the salient ring unchanged.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import herm

PAD = oracle.PAD_TOKEN_ID


def _linear(rng, o, i):
    bound = 1.0 / np.sqrt(i)
    return rng.uniform(-bound, bound, (o, i)), rng.uniform(-bound, bound, (o,))


def _params(rng, layers, d, m, e, head_scale=8.0):
    out = []
    for layer in range(layers):
        p = {}
        if layer == 0:
            p["embedding"] = rng.normal(size=(PAD + 1, d))
            p["embedding"][PAD] = 0.0
        p["input_norm"] = 1.0 + 0.1 * rng.normal(size=d)
        for n in ("retention", "candidate", "key", "query", "value", "local_key", "local_value"):
            p[n + "_w"], p[n + "_b"] = _linear(rng, d, d)
        p["feature_w"], p["feature_b"] = _linear(rng, m, d)
        p["decay_w"], p["decay_b"] = _linear(rng, 1, d)
        p["write_w"], p["write_b"] = _linear(rng, 1, d)
        p["fusion_w"], p["fusion_b"] = _linear(rng, d, 4 * d)
        p["fusion_norm"] = np.ones(d)
        for n, (o, i) in (("gate", (2 * d, d)), ("up", (2 * d, d)), ("down", (d, 2 * d))):
            pairs = [_linear(rng, o, i) for _ in range(e)]
            p[n + "_w"] = np.stack([w for w, _ in pairs])
            p[n + "_b"] = np.stack([b for _, b in pairs])
        p["expert_norm"] = np.ones(d)
        p["head_w"], p["head_b"] = _linear(rng, PAD + 1, d)
        p["head_w"] *= head_scale
        out.append(p)
    return out


def _cfg(threshold=0.6):
    # exact-arithmetic invariants: the memory's log-decay factors in float64
    # (the reference's fp32 log domain is pinned by test_oracle_reference_block)
    return dict(width=16, memory_features=4, local_memory_size=4, salience_memory_size=3,
                salience_threshold=threshold, expert_count=4, top_k=2, memory_log_dtype=np.float64)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_associative_scan_read_matches_the_sequential_recurrence(seed):
    rng = np.random.default_rng(seed)
    b, length, d, m = 2, 11, 6, 4
    basis = rng.normal(size=(b, d, m))
    normalizer = rng.random((b, m))
    decay = rng.uniform(2.0**-12, 1.0, (b, length))
    decay[:, 3] = 1.0  # a masked (padding) position
    value = np.tanh(rng.normal(size=(b, length, d)))
    features = herm.softmax(rng.normal(size=(b, length, m)))
    weight = rng.random((b, length))
    weight[:, 3] = 0.0
    query = herm.softmax(rng.normal(size=(b, length, m)))
    parallel = herm.associative_scan_read(basis, normalizer, decay, value, features, weight, query,
                                          log_dtype=np.float64)
    sequential = herm.associative_sequential(basis, normalizer, decay, value, features, weight, query)
    for got, want in zip(parallel, sequential):
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("b, carried, length, d, window, p", [
    (2, 4, 9, 5, 4, 0.7), (3, 0, 7, 3, 2, 0.5), (1, 6, 12, 4, 6, 0.9), (2, 6, 5, 4, 3, 0.0), (2, 4, 10, 3, 1, 1.0)])
def test_local_read_matches_the_sequential_ring_read(b, carried, length, d, window, p):
    rng = np.random.default_rng(b * 100 + length)
    ck, cv, k, v, q = (rng.normal(size=s) for s in [(b, carried, d), (b, carried, d), (b, length, d), (b, length, d),
                                                     (b, length, d)])
    cvalid, valid = rng.random((b, carried)) < p, rng.random((b, length)) < p
    got = oracle.read_local_window(ck, cv, cvalid, k, v, valid, q, window)
    want = oracle.read_local_sequential(ck, cv, cvalid, k, v, valid, q, window)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_stack_output_does_not_depend_on_the_window_cut_without_admission():
    rng = np.random.default_rng(5)
    cfg = _cfg(threshold=2.0)  # above every surprise value: nothing is admitted
    params = _params(rng, 2, 16, 4, 4)
    ids = rng.integers(0, 256, (2, 12))
    ids[1, 4] = PAD
    results = []
    for window in (12, 5, 1):
        states = [herm.initial_state(2, cfg) for _ in params]
        logits, states = herm.prefill(params, states, ids, cfg, window)
        results.append((logits, states))
    for logits, states in results[1:]:
        np.testing.assert_allclose(logits, results[0][0], rtol=1e-9, atol=1e-9)
        for got, want in zip(states, results[0][1]):
            for key in ("working", "basis", "normalizer", "local_keys", "local_values"):
                np.testing.assert_allclose(got[key], want[key], rtol=1e-9, atol=1e-9)
            np.testing.assert_array_equal(got["local_valid"], want["local_valid"])
            np.testing.assert_array_equal(got["last_token"], want["last_token"])


def test_padding_window_leaves_the_carried_state():
    rng = np.random.default_rng(6)
    cfg = _cfg()
    params = _params(rng, 2, 16, 4, 4)
    states = [herm.initial_state(2, cfg) for _ in params]
    _, states = herm.prefill(params, states, rng.integers(0, 256, (2, 9)), cfg, 9)
    logits, after, surprise = herm.stack_window(params, states, np.full((2, 4), PAD), cfg)
    assert np.isfinite(logits).all()
    for before, now, s in zip(states, after, surprise):
        np.testing.assert_array_equal(s, 0.0)
        for key in ("working", "basis", "normalizer", "salient_keys", "salient_values"):
            np.testing.assert_allclose(now[key], before[key], rtol=1e-12, atol=1e-12)
        np.testing.assert_array_equal(now["salient_valid"], before["salient_valid"])
        np.testing.assert_array_equal(now["last_token"], before["last_token"])
        assert not now["local_valid"].any()  # the ring shifted in four invalid entries


def test_admission_fills_the_salient_ring_with_the_latest_admitted_entries():
    rng = np.random.default_rng(7)
    cfg = _cfg(threshold=0.0)  # every valid token is admitted
    params = _params(rng, 1, 16, 4, 4)
    states = [herm.initial_state(2, cfg)]
    ids = rng.integers(0, 256, (2, 6))
    ids[0, 5] = PAD
    _, next_states, _ = herm.stack_window(params, states, ids, cfg)
    st = next_states[0]
    assert st["salient_valid"].all()  # five or six admitted entries for three slots
    _, _, _, _, admission = herm.block_window(params[0], states[0], ids, cfg)
    np.testing.assert_array_equal(admission, ids != PAD)
