"""Pins of the CPU oracle (CPU only).

The oracle is only trusted as far as these checks fix it. For each oracle
function, the checks below are chosen so that a plausible slip (dropped term,
wrong sign, swapped operand, wrong rounding order) fails at least one:

* exp/log (the fixed routines behind the bit-exact surprise and router):
  <= 2 ulp from float64 math over a dense sweep; exact special values.
* scan_sequential: brute-force Python recurrence (tiny shapes); closed forms
  a=0 -> h=b, a=1,b=0 -> h=h0, constant (a,b) -> geometric series; fp32 path
  bit-identical to a torch fp32 loop (test_dense_cuda.py:21-33); finiteness at
  the bounded retention range (test_scan.py:40-45); Hillis-Steele agrees
  (test_scan.py:20-30 sizes).
* rmsnorm_silu: torch float64 closed form (test_core_cuda.py:70-71); constant
  rows; fp32 port within the reference tolerance 2e-5.
* surprise_rows: float64 logsumexp formula and torch cross_entropy
  (network.py:677-688) within a few ulp; uniform logits -> 1 - 1/e; invalid
  -> exactly 0; bias[65] = 12 monotonic known case (test_network.py:61-70).
* quantile: torch.quantile (linear) on many sizes / q; NaN propagation.
* salient_tail: the ring KAT (test_salience_memory.py:13-30); the reference's
  own torch expression (topk over valid ? t : -1, sorted) on every case where
  it is unambiguous (at least `capacity` valid entries), and its valid slots
  on every case; fit-in-capacity returns the concatenation unchanged.
* hash route: the network KAT (test_network.py:95-101) and the dispatch
  properties of test_dispatch.py:50-108; uint32-vs-int64 closed form (E power
  of two agrees, E = 6 does not).
* learned route: torch softmax + topk indices, weights to 1e-6; exact ties.
* router statistics / balance loss: the reference's own forward_window
  statistics (tests/test_oracle_reference_block.py); closed forms (uniform
  gate with balanced counts -> loss 1; all mass and every assignment on one
  expert -> loss E; an empty mask -> loss 0, test_learned_router.py:82-87);
  invariants (the mass sums to the valid count, the counts to k x valid,
  test_learned_router.py:34); a brute-force Python loop over tokens; merging
  two halves equals the statistics of the whole.
* permute: the stable-pairs KAT and torch.argsort(stable=True) on random data.
* grouped_mlp / combine: torch per-row loops of test_moe_cuda.py:79-113.
* sample_tokens: the reference's own torch expression (index_fill PAD,
  topk threshold, softmax of scores / temperature; fast_decode.py:57-95) for
  the probabilities; top_k = 1 -> the masked argmax; u = 0 -> the first
  column with p > 0; a hand-made three-column case.
* local_novelty: a brute-force loop over each query's sliding window of
  cosine similarities; closed forms (a query parallel to an eligible key ->
  0, no eligible slot -> 1, a query orthogonal to every key -> 1); the
  reference's refine-ablation forward_window fixture (through the block).
* grouped_mlp_bound: its values equal grouped_mlp's with bf16 hidden values;
  a torch fp32 implementation with bf16 operands (another summation order)
  stays inside the bound; a dropped output bias or swapped gate and value
  projections fall outside it; round_bf16_f64 equals torch's float32 ->
  bfloat16 rounding on float32 inputs.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

GOLDEN = json.loads((Path(__file__).parent / "golden" / "kats.json").read_text())


def ulp_error(got: np.ndarray, want64: np.ndarray) -> np.ndarray:
    want32 = want64.astype(np.float32)
    spacing = np.spacing(np.abs(want32)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want64) / spacing


# ----------------------------------------------------------------- exp / log


def test_det_exp_within_two_ulp_over_the_used_range():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-86.0, 88.0, 400_000), rng.uniform(-1, 1, 100_000), np.arange(-86, 89)]).astype(np.float32)
    got = oracle.det_expf_array(x)
    assert ulp_error(got, np.exp(x.astype(np.float64))).max() <= 2.0


def test_det_exp_special_values():
    assert oracle.det_expf(0.0) == 1.0
    assert oracle.det_expf(-100.0) == 0.0
    assert math.isinf(oracle.det_expf(100.0))
    assert math.isnan(oracle.det_expf(float("nan")))


def test_det_log_within_two_ulp():
    rng = np.random.default_rng(1)
    x = np.concatenate([np.exp(rng.uniform(-80, 80, 400_000)), rng.uniform(0.5, 2.0, 100_000), [1.0, 2.0, 256.0]]).astype(np.float32)
    got = oracle.det_logf_array(x)
    want = np.log(x.astype(np.float64))
    err = np.abs(got - want)
    # relative ulp except near log(1) = 0 where the absolute error is what matters
    ok = (ulp_error(got, want) <= 2.0) | (err <= 2 * np.spacing(np.float32(1.0)) * np.abs(x.astype(np.float64) - 1.0) + 1e-12)
    assert ok.all()
    assert oracle.det_logf(1.0) == 0.0
    assert math.isinf(oracle.det_logf(0.0)) and oracle.det_logf(0.0) < 0


# ---------------------------------------------------------------------- scan


def brute_force_scan(a, b, h0):
    B, L = b.shape[:2]
    out = np.empty_like(b)
    for bi in range(B):
        state = h0[bi].copy()
        for t in range(L):
            state = a[bi, t] * state + b[bi, t]
            out[bi, t] = state
    return out


@pytest.mark.parametrize("shape", [(3, 1, 5), (3, 2, 5), (4, 17, 8), (2, 96, 48)])
def test_scan_matches_brute_force_float64(shape):
    rng = np.random.default_rng(2)
    a = rng.uniform(0.004, 0.994, shape)
    b = rng.standard_normal(shape)
    h0 = rng.standard_normal((shape[0], shape[2]))
    np.testing.assert_array_equal(oracle.scan_sequential(a, b, h0), brute_force_scan(a, b, h0))


def test_scan_broadcast_retention_matches_expanded():
    rng = np.random.default_rng(3)
    a = rng.uniform(0.05, 0.95, (2, 29, 1, 1))
    b = rng.standard_normal((2, 29, 4, 8))
    h0 = rng.standard_normal((2, 4, 8))
    expanded = oracle.scan_sequential(np.broadcast_to(a, b.shape).copy(), b, h0)
    np.testing.assert_array_equal(oracle.scan_sequential(a, b, h0).reshape(b.shape), expanded.reshape(b.shape))


def test_scan_closed_forms():
    rng = np.random.default_rng(4)
    b = rng.standard_normal((2, 50, 3))
    h0 = rng.standard_normal((2, 3))
    np.testing.assert_array_equal(oracle.scan_sequential(np.zeros_like(b), b, h0), b)
    np.testing.assert_array_equal(oracle.scan_sequential(np.ones_like(b), np.zeros_like(b), h0), np.broadcast_to(h0[:, None], b.shape))
    a_c, b_c = 0.9, 0.3
    h = oracle.scan_sequential(np.full_like(b, a_c), np.full_like(b, b_c), h0)
    t = np.arange(1, 51)[None, :, None]
    closed = a_c**t * h0[:, None] + b_c * (1 - a_c**t) / (1 - a_c)
    np.testing.assert_allclose(h, closed, rtol=1e-12, atol=1e-12)


def test_scan_fp32_is_the_torch_fp32_recurrence_bit_for_bit():
    torch.manual_seed(101)
    a = torch.rand((2, 37, 64)) * 0.9 + 0.05
    b = torch.randn((2, 37, 64))
    h0 = torch.randn((2, 64))
    state, states = h0, []
    for t in range(b.shape[1]):  # test_dense_cuda.py:21-33
        state = a[:, t] * state + b[:, t]
        states.append(state)
    expected = torch.stack(states, dim=1).numpy()
    np.testing.assert_array_equal(oracle.scan_sequential(a.numpy(), b.numpy(), h0.numpy()), expected)


def test_scan_stays_finite_at_the_bounded_retention_range():
    b = np.random.default_rng(5).standard_normal((1, 2048, 8)).astype(np.float32)
    for value in (2.0**-8, 1.0 - 2.0**-8):
        assert np.isfinite(oracle.scan_sequential(np.full_like(b, value), b, np.zeros((1, 8), np.float32))).all()


@pytest.mark.parametrize("shape", [(3, 1, 5), (4, 17, 8), (2, 96, 48)])
def test_hillis_steele_window_scan_agrees(shape):
    rng = np.random.default_rng(6)
    a = (rng.uniform(0, 1, shape) * 0.99 + 0.004).astype(np.float32)
    b = rng.standard_normal(shape).astype(np.float32)
    h0 = rng.standard_normal((shape[0], shape[2])).astype(np.float32)
    np.testing.assert_allclose(oracle.scan_hillis_steele(a, b, h0), oracle.scan_sequential(a, b, h0), atol=1e-5)


# ------------------------------------------------------------- rmsnorm-silu


def test_rmsnorm_silu_matches_the_torch_closed_form():
    torch.manual_seed(11)
    x = torch.randn((5, 257), dtype=torch.float64)
    w = torch.randn((257,), dtype=torch.float64)
    expected = F.silu(x * torch.rsqrt(x.square().mean(dim=-1, keepdim=True) + 1e-6) * w)
    y, inv = oracle.rmsnorm_silu_f64(x.numpy(), w.numpy())
    np.testing.assert_allclose(y, expected.numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(inv, torch.rsqrt(x.square().mean(dim=-1) + 1e-6).numpy(), rtol=1e-14)


def test_rmsnorm_silu_constant_rows():
    c, eps = -0.37, 1e-6
    x = np.full((2, 16), c)
    w = np.linspace(0.5, 1.5, 16)
    y, _ = oracle.rmsnorm_silu_f64(x, w, eps)
    v = np.sign(c) * w * abs(c) / math.sqrt(c * c + eps)
    np.testing.assert_allclose(y[0], v / (1 + np.exp(-v)), rtol=1e-13)


def test_rmsnorm_silu_fp32_port_within_reference_tolerance():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(512)).astype(np.float32)
    y32, inv32 = oracle.rmsnorm_silu_f32(x, w)
    y64, inv64 = oracle.rmsnorm_silu_f64(x, w)
    np.testing.assert_allclose(y32, y64, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(inv32, inv64, rtol=2e-6)


def test_bf16_round_trip_and_rounding():
    values = np.array([1.0, 1.00390625, 1.005859375, -2.5, 3.0e38, 1e-40], dtype=np.float32)
    torch_bits = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(oracle.f32_to_bf16(values), torch_bits)


# ------------------------------------------------------------------ surprise


def test_surprise_matches_float64_and_torch_cross_entropy():
    g = torch.Generator().manual_seed(21)
    logits = 2.0 * torch.randn((2048, 256), generator=g)
    targets = torch.randint(0, 256, (2048,), generator=g)
    valid = torch.rand((2048,), generator=g) > 0.1
    got = oracle.surprise_rows(logits.numpy(), targets.numpy(), valid.numpy())
    want64 = oracle.surprise_rows_f64(logits.numpy(), targets.numpy(), valid.numpy())
    assert np.abs(got - want64).max() <= 4 * np.spacing(np.float32(1.0))
    # reference model path: cross_entropy / log(V), 1 - exp(-.), zero where invalid
    nll = F.cross_entropy(logits, targets, reduction="none")
    ref = torch.where(valid, 1.0 - torch.exp(-(nll / math.log(256))), torch.zeros(()))
    assert np.abs(got - ref.numpy()).max() <= 3e-6
    assert (got[~valid.numpy()] == 0).all()


@pytest.mark.parametrize("vocab", [2, 19, 257, 1000, 1030])
def test_surprise_ragged_vocabularies(vocab):
    rng = np.random.default_rng(vocab)
    logits = rng.normal(0, 3, (64, vocab)).astype(np.float32)
    bias = rng.normal(0, 1, vocab).astype(np.float32)
    targets = rng.integers(0, vocab, 64)
    valid = np.ones(64, dtype=bool)
    got = oracle.surprise_rows(logits, targets, valid, bias)
    want = oracle.surprise_rows_f64(logits.astype(np.float64) + bias.astype(np.float32).astype(np.float64), targets, valid)
    assert np.abs(got - want).max() <= 8 * np.spacing(np.float32(1.0))


def test_surprise_uniform_logits_is_one_minus_inverse_e():
    s = oracle.surprise_rows(np.zeros((4, 256), np.float32), np.array([0, 7, 100, 255]), np.ones(4, bool))
    assert np.abs(s - (1 - math.exp(-1))).max() <= 2 * np.spacing(np.float32(0.63))


def test_surprise_bias_known_case():
    kat = GOLDEN["surprise_bias_monotonic"]
    bias = np.zeros(kat["vocab"], np.float32)
    bias[kat["bias_index"]] = kat["bias_value"]
    s = oracle.surprise_rows(np.zeros((2, kat["vocab"]), np.float32), np.array(kat["tokens"]), np.ones(2, bool), bias)
    assert s[0] < s[1]


@pytest.mark.parametrize("n", [1, 2, 7, 100, 1001, 32768])
@pytest.mark.parametrize("q", [0.0, 0.1, 0.5, 0.9, 0.999, 1.0])
def test_quantile_matches_torch(n, q):
    values = torch.rand((n,), generator=torch.Generator().manual_seed(n)) * 0.3 + 0.55
    got = oracle.quantile(values.numpy(), q)
    want = float(torch.quantile(values, q))
    assert got == want or abs(got - want) <= np.spacing(np.float32(want))


def test_quantile_with_ties_and_nan():
    v = np.array([0.5, 0.5, 0.5, 0.7, 0.7], np.float32)
    assert oracle.quantile(v, 0.5) == float(torch.quantile(torch.from_numpy(v), 0.5))
    assert math.isnan(oracle.quantile(np.array([0.1, float("nan"), 0.3], np.float32), 0.9))


def test_admission_is_strictly_above_the_threshold():
    s = np.array([0.7, 0.75, 0.8, 0.9], np.float32)
    mask, _ = oracle.admission(s, np.array([True, True, True, False]), threshold=0.75)
    assert mask.tolist() == [False, False, True, False]


def _torch_salient_tail(ck, cv, cvalid, k, v, adm, capacity):
    """The reference expression of model/memory.py:431-455, in torch on the CPU."""
    all_keys = torch.cat((ck, k), dim=1)
    all_values = torch.cat((cv, v), dim=1)
    all_valid = torch.cat((cvalid, adm), dim=1)
    if all_keys.shape[1] <= capacity:
        return all_keys, all_values, all_valid
    t = torch.arange(all_keys.shape[1]).unsqueeze(0).expand_as(all_valid)
    ranked = torch.where(all_valid, t, torch.full_like(t, -1))
    sel = ranked.topk(capacity, dim=1, largest=True).indices.sort(dim=1).values
    ok = all_valid.gather(1, sel)
    idx = sel.unsqueeze(-1).expand(-1, -1, all_keys.shape[-1])
    sk = torch.where(ok.unsqueeze(-1), all_keys.gather(1, idx), torch.zeros(()))
    sv = torch.where(ok.unsqueeze(-1), all_values.gather(1, idx), torch.zeros(()))
    return sk, sv, ok


def _torch_read_salient_window(ck, cv, cvalid, k, v, adm, q):
    """The reference expression of model/memory.py:405-429, in torch on the CPU (float64)."""
    batch_size, length, width = q.shape
    carried_length = ck.shape[1]
    all_keys = torch.cat((ck, k), dim=1)
    all_values = torch.cat((cv, v), dim=1)
    carried_eligible = cvalid.unsqueeze(1).expand(batch_size, length, carried_length)
    positions = torch.arange(length)
    prior = positions.unsqueeze(1) > positions.unsqueeze(0)
    current_eligible = adm.unsqueeze(1) & prior.unsqueeze(0)
    eligible = torch.cat((carried_eligible, current_eligible), dim=-1)
    scores = torch.einsum("bsd,btd->bts", all_keys, q) / math.sqrt(width)
    masked = scores.masked_fill(~eligible, float("-inf"))
    any_slot = eligible.any(dim=-1, keepdim=True)
    weights = torch.where(any_slot, torch.softmax(masked, dim=-1), torch.zeros(()))
    return torch.einsum("bts,bsd->btd", weights, all_values)


def _read_case(rng, b, s, length, d, p):
    ck, cv = rng.normal(size=(b, s, d)), rng.normal(size=(b, s, d))
    k, v, q = rng.normal(size=(b, length, d)), rng.normal(size=(b, length, d)), rng.normal(size=(b, length, d))
    return ck, cv, rng.random((b, s)) < p, k, v, rng.random((b, length)) < p, q


@pytest.mark.parametrize("seed", range(8))
def test_read_salient_window_matches_the_reference_expression(seed):
    rng = np.random.default_rng(100 + seed)
    case = _read_case(rng, 2, int(rng.integers(0, 5)), int(rng.integers(1, 24)), int(rng.integers(1, 9)),
                      rng.uniform(0.0, 1.0))
    got = oracle.read_salient_window(*case)
    want = _torch_read_salient_window(*(torch.from_numpy(np.asarray(x)) for x in case)).numpy()
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_read_salient_window_closed_forms():
    rng = np.random.default_rng(7)
    ck, cv, _, k, v, _, q = _read_case(rng, 1, 3, 6, 4, 0.5)
    none = oracle.read_salient_window(ck, cv, np.zeros((1, 3), bool), k, v, np.zeros((1, 6), bool), q)
    assert np.all(none == 0.0)  # no eligible slot: zeros
    # only carried slot 1 valid, nothing admitted: every query reads value 1 exactly
    one = oracle.read_salient_window(ck, cv, np.array([[False, True, False]]), k, v, np.zeros((1, 6), bool), q)
    np.testing.assert_array_equal(one[0], np.broadcast_to(cv[0, 1], (6, 4)))
    # window slot 2 admitted only: queries t <= 2 read zeros, later ones value 2 exactly
    adm = np.zeros((1, 6), bool)
    adm[0, 2] = True
    w2 = oracle.read_salient_window(ck, cv, np.zeros((1, 3), bool), k, v, adm, q)
    assert np.all(w2[0, :3] == 0.0)
    np.testing.assert_array_equal(w2[0, 3:], np.broadcast_to(v[0, 2], (3, 4)))
    # zero queries: equal scores, so the read is the mean of the eligible values
    cvalid = np.array([[True, False, True]])
    adm = np.ones((1, 6), bool)
    mean = oracle.read_salient_window(ck, cv, cvalid, k, v, adm, np.zeros_like(q))
    for t in range(6):
        rows = np.concatenate([cv[0, [0, 2]], v[0, :t]], axis=0)
        np.testing.assert_allclose(mean[0, t], rows.mean(axis=0), rtol=1e-13, atol=1e-13)


def test_read_salient_window_is_causal():
    rng = np.random.default_rng(9)
    case = list(_read_case(rng, 2, 4, 10, 3, 0.6))
    base = oracle.read_salient_window(*case)
    for i in (3, 4, 5):  # keys, values, admission of the window from position 5 on
        case[i] = case[i].copy()
        case[i][:, 5:] = rng.normal(size=case[i][:, 5:].shape) if i != 5 else ~case[i][:, 5:]
    changed = oracle.read_salient_window(*case)
    np.testing.assert_array_equal(changed[:, :6], base[:, :6])  # query t sees window slots j < t only


def _torch_gates(u, wr, br, wc, bc):
    """BoundedRecurrentState.gates (model/memory.py:14-30) with torch.nn on the CPU (float64)."""
    lin_r, lin_c = torch.nn.Linear(u.shape[-1], u.shape[-1]).double(), torch.nn.Linear(u.shape[-1], u.shape[-1]).double()
    with torch.no_grad():
        lin_r.weight.copy_(wr), lin_r.bias.copy_(br), lin_c.weight.copy_(wc), lin_c.bias.copy_(bc)
        retention = torch.sigmoid(lin_r(u))
        bounded = 2.0**-8 + ((1.0 - 2.0**-8) - 2.0**-8) * retention
        return bounded, (1.0 - bounded) * torch.tanh(lin_c(u))


@pytest.mark.parametrize("seed", range(4))
def test_recurrent_gates_match_the_reference_module(seed):
    rng = np.random.default_rng(200 + seed)
    d = int(rng.integers(1, 12))
    u = rng.normal(size=(3, 5, d))
    wr, wc = rng.normal(size=(d, d)), rng.normal(size=(d, d))
    br, bc = rng.normal(size=d), rng.normal(size=d)
    a, b = oracle.recurrent_gates(u, wr, br, wc, bc)
    ta, tb = _torch_gates(*(torch.from_numpy(x) for x in (u, wr, br, wc, bc)))
    np.testing.assert_allclose(a, ta.numpy(), rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(b, tb.numpy(), rtol=1e-13, atol=1e-15)


def test_recurrent_gates_closed_forms():
    d = 4
    u = np.random.default_rng(3).normal(size=(2, 6, d))
    zeros = np.zeros((d, d))
    a, b = oracle.recurrent_gates(u, zeros, np.zeros(d), zeros, np.zeros(d))
    assert np.all(a == 0.5) and np.all(b == 0.0)  # sigmoid(0) = 1/2: 2^-8 + (1 - 2^-7) / 2 = 1/2
    a, b = oracle.recurrent_gates(u, zeros, np.full(d, 1e4), zeros, np.full(d, -1e4))
    assert np.all(a == 1.0 - 2.0**-8) and np.all(b == -(2.0**-8))  # saturated bounds
    valid = np.array([[True, False, True, True, False, True]] * 2)
    a, b = oracle.recurrent_gates(u, np.eye(d), np.zeros(d), np.eye(d), np.zeros(d), valid)
    assert np.all(a[~valid] == 1.0) and np.all(b[~valid] == 0.0)
    assert np.all((a[valid] >= 2.0**-8) & (a[valid] <= 1.0 - 2.0**-8)) and np.all(np.abs(b[valid]) < 1.0 - a[valid] + 1e-15)


def test_salient_tail_known_answer():
    kat = GOLDEN["salient_tail_latest"]
    adm = np.array([kat["admission"]])
    keys = np.arange(4 * 3, dtype=np.float32).reshape(1, 4, 3)
    empty = np.zeros((1, 0, 3), np.float32)
    k, v, ok = oracle.salient_tail(empty, empty, np.zeros((1, 0), bool), keys, keys + 100, adm, kat["capacity"])
    np.testing.assert_array_equal(k[0], keys[0, kat["kept_positions"]])
    np.testing.assert_array_equal(v[0], keys[0, kat["kept_positions"]] + 100)
    assert ok.tolist() == [[True, True]]


@pytest.mark.parametrize("seed", range(12))
def test_salient_tail_matches_the_reference_expression(seed):
    rng = np.random.default_rng(seed)
    b, s, length, d = 3, int(rng.integers(0, 6)), int(rng.integers(1, 40)), 5
    capacity = int(rng.integers(1, 20))
    p = rng.uniform(0.05, 0.95)
    ck, cv = rng.normal(size=(b, s, d)).astype(np.float32), rng.normal(size=(b, s, d)).astype(np.float32)
    k, v = rng.normal(size=(b, length, d)).astype(np.float32), rng.normal(size=(b, length, d)).astype(np.float32)
    cvalid, adm = rng.random((b, s)) < p, rng.random((b, length)) < p
    got = oracle.salient_tail(ck, cv, cvalid, k, v, adm, capacity)
    want = _torch_salient_tail(*(torch.from_numpy(x) for x in (ck, cv, cvalid, k, v, adm)), capacity)
    valid_counts = np.concatenate([cvalid, adm], axis=1).sum(axis=1)
    for bi in range(b):
        if s + length <= capacity or valid_counts[bi] >= capacity:  # no tie: the whole output is fixed
            for g, w in zip(got, want):
                np.testing.assert_array_equal(g[bi], w[bi].numpy())
        else:  # ties among invalid filler: the valid slots, in order, are still fixed
            gv, wv = got[2][bi], want[2][bi].numpy()
            np.testing.assert_array_equal(got[0][bi][gv], want[0][bi].numpy()[wv])
            np.testing.assert_array_equal(got[1][bi][gv], want[1][bi].numpy()[wv])
            assert not got[0][bi][~gv].any() and not got[1][bi][~gv].any()


# ------------------------------------------------------------------------ MoE


def test_network_hash_route_known_answer():
    kat = GOLDEN["network_hash_route"]
    tok, prev = np.array(kat["token_ids"]), np.array(kat["previous_token_ids"])
    valid = tok != oracle.PAD_TOKEN_ID
    a = oracle.route_hash(tok, prev, valid, kat["expert_count"], kat["top_k"])
    assert a[..., 0].tolist() == kat["expert_indices"]
    assert oracle.expert_counts(a, valid, kat["expert_count"]).tolist() == kat["activation_counts"]


def test_modulo_route_known_answer_and_torch_expression():
    """The synthetic "token id mod 16" variant: slot s -> (tok + s) mod 16,
    hand-computed, and torch.remainder's expression on random ids (negative
    ids included, for the sign convention)."""

    tok = np.array([0, 15, 16, 17, 255, 256, 3])
    valid = np.array([True, True, True, True, True, False, True])
    got = oracle.route_modulo(tok, valid, 16, 2)
    assert got.tolist() == [[0, 1], [15, 0], [0, 1], [1, 2], [15, 0], [-1, -1], [3, 4]]
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(-300, 300, (2048,), generator=g)
    ok = torch.rand((2048,), generator=g) < 0.9
    want = (ids.unsqueeze(-1) + torch.arange(3)).remainder(13).masked_fill(~ok.unsqueeze(-1), -1)
    np.testing.assert_array_equal(oracle.route_modulo(ids.numpy(), ok.numpy(), 13, 3), want.numpy())


def test_hash_route_properties_of_the_reference_dispatch_tests():
    six = oracle.route_hash(np.array([[97, 98, 99]]), np.array([[32, 97, 98]]), np.ones((1, 3), bool), 128, 6)
    assert all(len(set(row)) == 6 for row in six[0].tolist())
    tokens = np.arange(1, 256)
    reachable = set(oracle.route_hash(tokens, tokens - 1, np.ones(255, bool), 64, 1)[:, 0].tolist())
    assert len(reachable) >= 48
    mixed = oracle.content_hash(tokens, tokens - 1)
    affine = tokens * 1_000_003 + (tokens - 1) * 97_409
    for e in (4, 64):
        assert len(set((mixed % e).tolist())) > len(set((affine % e).tolist()))
    all_tokens = np.arange(0, 257)
    assert (oracle.content_hash(all_tokens, np.full_like(all_tokens, 256)) >= 0).all()
    padded = oracle.route_hash(np.array([65, 256, 66]), np.array([32, 65, 256]), np.array([True, False, True]), 8, 1)
    assert padded[1, 0] == -1 and padded[0, 0] >= 0 and padded[2, 0] >= 0


def test_hash_route_against_torch_int64_expression():
    g = torch.Generator().manual_seed(31)
    tok = torch.randint(0, 257, (4096,), generator=g)
    prev = torch.randint(0, 257, (4096,), generator=g)
    value = (tok * 1_000_003 + prev * 97_409) & 0xFFFFFFFF  # experts.py:30-38, in torch int64
    value = value ^ (value >> 16)
    value = (value * 0x45D9F3B) & 0xFFFFFFFF
    value = value ^ (value >> 16)
    value = (value * 0x45D9F3B) & 0xFFFFFFFF
    value = value ^ (value >> 16)
    expected = (value.unsqueeze(-1) + torch.arange(3) * 0x9E3779B9).remainder(16)
    got = oracle.route_hash(tok.numpy(), prev.numpy(), np.ones(4096, bool), 16, 3)
    np.testing.assert_array_equal(got, expected.numpy())


def test_uint32_slot_offsets_agree_only_for_power_of_two_expert_counts():
    tokens = np.arange(40_000) % 257
    prev = (np.arange(40_000) * 7) % 257
    h = oracle.content_hash(tokens, prev)
    for experts, expect_equal in ((16, True), (128, True), (6, False)):
        wide = (h + 0x9E3779B9) % experts
        wrapped = ((h + 0x9E3779B9) & 0xFFFFFFFF) % experts
        assert bool((wide == wrapped).all()) == expect_equal


def test_learned_route_matches_torch_softmax_topk():
    g = torch.Generator().manual_seed(41)
    logits = torch.randn((4096, 16), generator=g)
    valid = torch.rand((4096,), generator=g) > 0.05
    probs = logits.softmax(dim=-1)
    w_ref, idx_ref = probs.topk(2, dim=-1)
    idx, w = oracle.route_learned(logits.numpy(), valid.numpy(), 2)
    v = valid.numpy()
    np.testing.assert_array_equal(idx[v], idx_ref.numpy()[v])
    np.testing.assert_allclose(w[v], w_ref.numpy()[v], rtol=1e-6, atol=0)
    assert (idx[~v] == -1).all() and (w[~v] == 0).all()
    assert oracle.expert_counts(idx, v, 16).sum() == v.sum() * 2


def test_learned_route_ties_go_to_the_lower_index():
    logits = np.zeros((1, 8), np.float32)
    logits[0, [2, 5, 6]] = 1.0
    idx, w = oracle.route_learned(logits, np.ones(1, bool), 3)
    assert idx[0].tolist() == [2, 5, 6] and w[0, 0] == w[0, 1] == w[0, 2]


def _router_loop(logits, valid, assignments):
    """RouterStatistics by a plain loop over tokens (router.py:50-58)."""
    T, E = logits.shape
    mass, counts, n = [0.0] * E, [0.0] * E, 0
    for t in range(T):
        if not valid[t]:
            continue
        n += 1
        z = [float(x) for x in logits[t]]
        top = max(z)
        ex = [math.exp(x - top) for x in z]
        total = sum(ex)
        for e in range(E):
            mass[e] += ex[e] / total
        for e in assignments[t]:
            counts[int(e)] += 1.0
    loss = E * sum((mass[e] / max(n, 1)) * (counts[e] / max(sum(counts), 1.0)) for e in range(E))
    return mass, counts, n, loss


def test_router_statistics_brute_force_and_invariants():
    g = torch.Generator().manual_seed(43)
    logits = (2.0 * torch.randn((300, 6), generator=g)).numpy()
    valid = (torch.rand((300,), generator=g) > 0.2).numpy()
    idx, _ = oracle.route_learned(logits, valid, 2)
    stats = oracle.router_statistics(logits, valid, idx)
    mass, counts, n, loss = _router_loop(logits, valid, idx)
    np.testing.assert_allclose(stats["probability_mass"], mass, rtol=1e-12)
    np.testing.assert_array_equal(stats["assignment_counts"], counts)
    assert stats["valid_count"] == n == valid.sum()
    assert abs(stats["balance_loss"] - loss) <= 1e-12 * loss
    assert abs(stats["probability_mass"].sum() - n) <= 1e-9 * n
    assert stats["assignment_counts"].sum() == 2 * n
    # merging the two halves gives the statistics of the whole (router.py:25-32)
    halves = [oracle.router_statistics(logits[s], valid[s], idx[s]) for s in (slice(0, 150), slice(150, 300))]
    merged = oracle.merge_router_statistics(halves)
    np.testing.assert_allclose(merged["probability_mass"], stats["probability_mass"], rtol=1e-12)
    np.testing.assert_array_equal(merged["assignment_counts"], stats["assignment_counts"])
    assert merged["valid_count"] == stats["valid_count"]
    assert abs(merged["balance_loss"] - stats["balance_loss"]) <= 1e-12
    assert oracle.merge_router_statistics([]) is None


def test_router_statistics_closed_forms():
    # uniform gate, every expert taken equally often: importance = load = 1/E -> loss 1
    E, k = 8, 2
    logits = np.zeros((64, E), np.float32)
    valid = np.ones(64, bool)
    balanced = np.stack([np.arange(64) % E, (np.arange(64) + 1) % E], axis=1)
    stats = oracle.router_statistics(logits, valid, balanced)
    assert abs(stats["balance_loss"] - 1.0) < 1e-12
    np.testing.assert_allclose(stats["probability_mass"], np.full(E, 64 / E), rtol=1e-12)
    # every token certain of expert 3 and routed there alone: importance_3 = load_3 = 1 -> loss E
    peaked = np.full((32, E), -1e4, np.float32)
    peaked[:, 3] = 0.0
    stats = oracle.router_statistics(peaked, np.ones(32, bool), np.full((32, 1), 3))
    assert abs(stats["balance_loss"] - E) < 1e-9
    # an empty mask: zero statistics and zero loss (test_learned_router.py:82-87)
    empty = oracle.router_statistics(np.random.default_rng(0).normal(size=(10, 4)).astype(np.float32),
                                     np.zeros(10, bool), np.full((10, 2), -1))
    assert empty["valid_count"] == 0 and empty["balance_loss"] == 0.0
    assert not empty["probability_mass"].any() and not empty["assignment_counts"].any()


def test_permute_known_answer():
    kat = GOLDEN["permute_stable_pairs"]
    ctx = np.arange(kat["context_rows"] * kat["context_width"], dtype=np.float32).reshape(kat["context_rows"], -1)
    sc, rows, experts, offsets = oracle.permute(ctx, np.array(kat["assignments"]), np.array(kat["valid"]), kat["expert_count"])
    assert rows.tolist() == kat["sorted_rows"]
    assert experts.tolist() == kat["sorted_experts"]
    assert offsets.tolist() == kat["segment_offsets"]
    k = len(kat["assignments"][0])
    np.testing.assert_array_equal(sc[: kat["zero_rows_from"]], ctx[np.array(kat["sorted_pairs"][: kat["zero_rows_from"]]) // k])
    assert (sc[kat["zero_rows_from"]:] == 0).all()


def test_permute_matches_torch_stable_argsort_with_invalid_and_repeated_slots():
    g = torch.Generator().manual_seed(51)
    T, k, E = 3000, 3, 11
    assignments = torch.randint(-1, E + 1, (T, k), generator=g)
    valid = torch.rand((T,), generator=g) > 0.2
    ctx = torch.randn((T, 5), generator=g)
    # experts.py:181-196 in torch
    pair_rows = torch.arange(T).repeat_interleave(k)
    pair_experts = assignments.reshape(-1)
    slots = torch.arange(k)
    repeated = (assignments.unsqueeze(-1) == assignments.unsqueeze(-2)) & (slots.unsqueeze(0) < slots.unsqueeze(1))
    first = ~repeated.any(dim=-1)
    pair_valid = pair_experts.ge(0) & pair_experts.lt(E) & valid.repeat_interleave(k) & first.reshape(-1)
    keys = torch.where(pair_valid, pair_experts, torch.full((), E))
    order = torch.argsort(keys, stable=True)
    sc, rows, experts, offsets = oracle.permute(ctx.numpy(), assignments.numpy(), valid.numpy(), E)
    np.testing.assert_array_equal(rows, pair_rows[order].numpy())
    np.testing.assert_array_equal(experts, keys[order].numpy())
    counts = torch.bincount(keys, minlength=E + 1)
    np.testing.assert_array_equal(offsets[1:], torch.cumsum(counts[:E], 0).numpy())
    n_valid = int(offsets[-1])
    np.testing.assert_array_equal(sc[:n_valid], ctx[pair_rows[order][:n_valid]].numpy())
    assert (sc[n_valid:] == 0).all()


def test_grouped_mlp_and_combine_match_the_reference_loops():
    g = torch.Generator().manual_seed(61)
    E, D, H, P = 3, 8, 6, 10
    x = torch.randn((P, D), generator=g, dtype=torch.float64)
    experts = torch.tensor([0, 0, 0, 1, 2, 2, 2, 2, 3, 3])
    offsets = torch.tensor([0, 3, 4, 8])
    gw, vw = torch.randn((E, H, D), generator=g, dtype=torch.float64), torch.randn((E, H, D), generator=g, dtype=torch.float64)
    gb, vb = torch.randn((E, H), generator=g, dtype=torch.float64), torch.randn((E, H), generator=g, dtype=torch.float64)
    ow, ob = torch.randn((E, D, H), generator=g, dtype=torch.float64), torch.randn((E, D), generator=g, dtype=torch.float64)
    got = oracle.grouped_mlp(x.numpy(), experts.numpy(), offsets.numpy(), gw.numpy(), gb.numpy(), vw.numpy(), vb.numpy(), ow.numpy(), ob.numpy())
    rows = []
    for row, e in enumerate(experts[:8].tolist()):  # test_moe_cuda.py:106-112
        gate = F.linear(x[row], gw[e], gb[e])
        value = F.linear(x[row], vw[e], vb[e])
        rows.append(F.linear(F.silu(gate) * value, ow[e], ob[e]))
    np.testing.assert_allclose(got[:8], torch.stack(rows).numpy(), rtol=1e-12, atol=1e-12)
    assert (got[8:] == 0).all()
    # combine: test_moe_cuda.py:79-82
    y = torch.randn((P, D), generator=g)
    sorted_rows = torch.tensor([0, 1, 2, 0, 1, 3, 2, 3, 4, 4])
    combined = oracle.combine(y.numpy(), sorted_rows.numpy(), offsets.numpy(), 5, 2)
    expected = torch.zeros((5, D))
    for pair in range(8):
        expected[sorted_rows[pair]] += y[pair] / 2.0
    np.testing.assert_array_equal(combined, expected.numpy())


def test_grouped_mlp_bound_accepts_fp32_and_rejects_slips():
    g = torch.Generator().manual_seed(71)
    E, D, H, P = 3, 128, 256, 300
    sizes = [100, 0, 200]
    off = np.concatenate([[0], np.cumsum(sizes)])
    bf = lambda *shape, s=1.0: (s * torch.randn(shape, generator=g)).to(torch.bfloat16).float()
    x = bf(P, D)
    gw, gb, vw, vb = bf(E, H, D, s=0.05), bf(E, H, s=0.05), bf(E, H, D, s=0.05), bf(E, H, s=0.05)
    ow, ob = bf(E, D, H, s=0.05), bf(E, D, s=0.05)
    ws = [t.numpy() for t in (gw, gb, vw, vb, ow, ob)]
    y, bound = oracle.grouped_mlp_bound(x.numpy(), off, *ws)
    want = oracle.grouped_mlp(x.numpy(), np.repeat(np.arange(E), sizes), off, *ws, round_hidden_bf16=True)
    assert np.abs(y - want).max() <= 1e-2 * np.abs(want).max() * 2.0 ** -7  # double rounding of a few h only

    def fp32_impl(gate_w, value_w, out_b):
        out = torch.zeros((P, D))
        for e in range(E):
            lo, hi = int(off[e]), int(off[e + 1])
            xe = x[lo:hi]
            hg = xe @ gate_w[e].T + gb[e]
            hv = xe @ value_w[e].T + vb[e]
            h = (torch.nn.functional.silu(hg) * hv).to(torch.bfloat16).float()
            out[lo:hi] = (h.flip(1) @ ow[e].flip(1).T + out_b[e]).to(torch.bfloat16).float()
        return out.double().numpy()

    assert np.all(np.abs(fp32_impl(gw, vw, ob) - y) <= bound)
    assert not np.all(np.abs(fp32_impl(gw, vw, torch.zeros_like(ob)) - y) <= bound)
    assert not np.all(np.abs(fp32_impl(vw, gw, ob) - y) <= bound)


def test_round_bf16_f64_is_one_rounding():
    x = torch.randn(200000, generator=torch.Generator().manual_seed(3)) * 7
    np.testing.assert_array_equal(oracle.round_bf16_f64(x.double().numpy()),
                                  x.to(torch.bfloat16).double().numpy())
    # a float64 value just above a bf16 midpoint rounds up (torch's float64
    # conversion first rounds to float32, which lands on the midpoint and ties to even)
    mid = 1.0 + 2.0 ** -8 + 2.0 ** -40
    assert oracle.round_bf16_f64(np.array([mid]))[0] == 1.0 + 2.0 ** -7


def test_local_novelty_brute_force_and_closed_forms():
    rng = np.random.default_rng(8)
    b, cap, length, d, window = 3, 4, 7, 6, 3
    ck = rng.normal(size=(b, cap, d))
    cv = rng.random((b, cap)) < 0.6
    k = rng.normal(size=(b, length, d))
    kv = rng.random((b, length)) < 0.7
    q = rng.normal(size=(b, length, d))
    got = oracle.local_novelty(ck, cv, k, kv, q, window)
    for bi in range(b):
        allk = np.concatenate([ck[bi], k[bi]])
        allv = np.concatenate([cv[bi], kv[bi]])
        for t in range(length):
            sims = [float(allk[s] @ q[bi, t] / (np.linalg.norm(allk[s]) * np.linalg.norm(q[bi, t])))
                    for s in range(max(cap + t - window, 0), cap + t) if allv[s]]
            want = min(max(1.0 - max(sims), 0.0), 1.0) if sims else 1.0
            assert abs(got[bi, t] - want) <= 1e-12
    # closed forms: parallel -> 0, none eligible -> 1, orthogonal -> 1
    e = np.eye(4)[None]
    keys = np.stack([e[0, 0], e[0, 1]])[None]
    qs = np.stack([3.0 * e[0, 0], e[0, 2]])[None]
    nov = oracle.local_novelty(np.zeros((1, 0, 4)), np.zeros((1, 0), bool), keys, np.ones((1, 2), bool), qs, 2)
    assert nov[0, 0] == 1.0  # no slot before the first entry
    assert nov[0, 1] == 1.0  # e2 is orthogonal to e0
    qs2 = np.stack([e[0, 1], 2.0 * e[0, 0]])[None]
    assert oracle.local_novelty(np.zeros((1, 0, 4)), np.zeros((1, 0), bool), keys, np.ones((1, 2), bool), qs2,
                                2)[0, 1] == 0.0


@pytest.mark.parametrize("temperature, top_k", [(1.0, None), (0.7, 5), (2.5, 40), (1.0, 300)])
def test_sample_tokens_probabilities_match_the_torch_expression(temperature, top_k):
    g = torch.Generator().manual_seed(12)
    logits = 3.0 * torch.randn((16, 257), generator=g)
    logits[3, 10] = logits[3, 11] = 50.0  # a tie at the top
    scores = logits.float().index_fill(-1, torch.tensor([256]), float("-inf"))
    if top_k is not None:
        kept = min(top_k, scores.shape[-1])
        thr = torch.topk(scores, kept, dim=-1).values[..., -1:]
        scores = scores.masked_fill(scores < thr, float("-inf"))
    want = torch.softmax(scores / temperature, dim=-1).double().numpy()
    u = torch.rand((16,), generator=g).numpy()
    ids, p = oracle.sample_tokens(logits.numpy(), 256, temperature, top_k, u)
    np.testing.assert_allclose(p, want, rtol=1e-5, atol=1e-7)
    assert p[:, 256].max() == 0.0
    cum = np.cumsum(p, axis=1)
    for r in range(16):
        assert cum[r, ids[r]] > u[r] and (ids[r] == 0 or cum[r, ids[r] - 1] <= u[r])


def test_sample_tokens_closed_forms():
    logits = np.array([[0.0, np.log(2.0), np.log(5.0), 99.0]], np.float32)
    ids, p = oracle.sample_tokens(logits, 3, 1.0, None, np.array([0.0]))
    np.testing.assert_allclose(p[0], [1 / 8, 2 / 8, 5 / 8, 0.0], rtol=1e-7)
    assert ids[0] == 0  # u = 0: the first column with p > 0
    assert oracle.sample_tokens(logits, 3, 1.0, None, np.array([0.2]))[0][0] == 1  # 1/8 <= 0.2 < 3/8
    assert oracle.sample_tokens(logits, 3, 1.0, None, np.array([0.999]))[0][0] == 2
    # top_k = 1: the masked argmax, whatever the uniform
    rng = np.random.default_rng(3)
    big = rng.normal(size=(8, 257)).astype(np.float32)
    for u in (0.0, 0.5, 0.999):
        ids, _ = oracle.sample_tokens(big, 256, 1.3, 1, np.full(8, u))
        np.testing.assert_array_equal(ids, big[:, :256].argmax(axis=1))
