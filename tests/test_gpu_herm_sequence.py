"""The sequence-parallel HERM block (koemi_amd.herm.block_sequence, stack_sequence,
SequencePrefill) against the window-by-window block and the oracle.

* window_rings: the ring carried into every window equals, bit for bit, the
  ring a window-by-window run carries: the salient ring against
  oracle.salient_tail applied window after window (memory.py:431-455), the
  local ring against the tail of [ring ; entries] (memory.py:385-403).
* associative_scan_read_windows: reads and final state bit-identical to
  associative_scan_read run window after window with the state carried (the
  same kernel arithmetic: the per-window terms, then e^{c_{L-1}} state +
  terms).
* stack_sequence over a three-layer stack (width 32, fp32 projections, five
  windows of six tokens with padding and admissions): logits and float states
  within 1e-5 of the window-by-window prefill's scale, ring bits and last
  tokens exact; and against oracle.herm's prefill (float64) within 1e-4 (the
  tolerance of tests/test_gpu_herm.py), the admission threshold placed
  >= 2e-3 from every oracle score.
* SequencePrefill (one HIP graph) replays equal the eager stack_sequence
  (1e-5) and each other (exactly).
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

import oracle
from koemi_amd import herm
from oracle import herm as oherm

from test_gpu_herm import _close, _ids, _oracle_params, _params, _pick_threshold, _settings

pytestmark = pytest.mark.gpu


def _rand_rings(rng, b, s, length, d, p_flag):
    ck = rng.normal(size=(b, s, d)).astype(np.float32)
    cv = rng.normal(size=(b, s, d)).astype(np.float32)
    cok = rng.random((b, s)) < 0.5
    ck[~cok] = 0.0
    cv[~cok] = 0.0
    k = rng.normal(size=(b, length, d)).astype(np.float32)
    v = rng.normal(size=(b, length, d)).astype(np.float32)
    flags = rng.random((b, length)) < p_flag
    return ck, cv, cok, k, v, flags


@pytest.mark.parametrize("p_flag", [0.02, 0.3, 0.9])
def test_window_rings_equal_the_window_by_window_rings(device, p_flag):
    rng = np.random.default_rng(int(p_flag * 100))
    b, s, window, windows, d = 3, 5, 7, 6, 12
    ck, cv, cok, k, v, flags = _rand_rings(rng, b, s, window * windows, d, p_flag)
    t = lambda x: torch.from_numpy(x).to(device)
    for tail in (False, True):
        rings, final = herm.window_rings(t(ck), t(cv), t(cok), t(k), t(v), t(flags), window=window, capacity=s,
                                         tail=tail)
        per_row = [x.view(b, windows, *x.shape[1:]) for x in rings]
        got_k = torch.cat((per_row[0], final[0].unsqueeze(1)), dim=1)
        got_v = torch.cat((per_row[1], final[1].unsqueeze(1)), dim=1)
        got_ok = torch.cat((per_row[2], final[2].unsqueeze(1)), dim=1)
        rk, rv, rok = ck, cv, cok
        for w in range(windows + 1):
            np.testing.assert_array_equal(got_ok[:, w].cpu().numpy(), rok, err_msg=f"tail={tail} w={w}")
            np.testing.assert_array_equal(got_k[:, w].cpu().numpy(), rk, err_msg=f"tail={tail} w={w}")
            np.testing.assert_array_equal(got_v[:, w].cpu().numpy(), rv, err_msg=f"tail={tail} w={w}")
            if w == windows:
                break
            sl = slice(w * window, (w + 1) * window)
            if tail:
                rk = np.concatenate([rk, k[:, sl]], axis=1)[:, -s:]
                rv = np.concatenate([rv, v[:, sl]], axis=1)[:, -s:]
                rok = np.concatenate([rok, flags[:, sl]], axis=1)[:, -s:]
            else:
                rk, rv, rok = (np.asarray(x) for x in oracle.salient_tail(rk, rv, rok, k[:, sl], v[:, sl],
                                                                          flags[:, sl], s))
                rk, rv = rk.astype(np.float32), rv.astype(np.float32)


@pytest.mark.parametrize("key_dtype", [torch.bfloat16, torch.float32])
def test_window_rings_read_projection_columns_in_place(device, key_dtype):
    """Keys and values read in place from column blocks of a wider projection
    (bf16 or fp32, rows C apart) with key_valid give the same ring bits as the
    contiguous fp32 entries with invalid rows zeroed (network.py:337-340);
    final_only (with and without final_out buffers) gives the final ring of
    the full call, and with a carried ring below capacity the rings of
    oracle.salient_tail and of the tail of [ring ; entries]."""

    rng = np.random.default_rng(11)
    b, s, window, windows, d = 3, 5, 7, 4, 12
    length, c = window * windows, 2 * d + 8
    ck, cv, cok, _, _, flags = _rand_rings(rng, b, s, length, d, 0.4)
    valid = rng.random((b, length)) < 0.7
    flags &= valid
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device)
    projected = torch.randn((b, length, c), device=device).to(key_dtype)
    keys, values = projected[..., :d], projected[..., d:2 * d]
    vmask = t(valid)
    masked = [torch.where(vmask[..., None], x.float(), torch.zeros((), device=device)).contiguous()
              for x in (keys, values)]
    for tail, fl in ((True, valid), (False, flags)):
        want_rings, want_final = herm.window_rings(t(ck), t(cv), t(cok), *masked, t(fl), window=window, capacity=s,
                                                   tail=tail)
        got_rings, got_final = herm.window_rings(t(ck), t(cv), t(cok), keys, values, t(fl), window=window,
                                                 capacity=s, tail=tail, key_valid=vmask)
        for w, g in zip(want_rings + want_final, got_rings + got_final):
            assert torch.equal(w, g), f"tail={tail}"
        none, final = herm.window_rings(t(ck), t(cv), t(cok), keys, values, t(fl), window=length, capacity=s,
                                        tail=tail, key_valid=vmask, final_only=True)
        assert none is None
        for w, g in zip(want_final, final):
            assert torch.equal(w, g), f"final_only tail={tail}"
        bufs = tuple(torch.full_like(x, 1) for x in want_final)
        herm.window_rings(t(ck), t(cv), t(cok), keys, values, t(fl), window=length, capacity=s, tail=tail,
                          key_valid=vmask, final_only=True, final_out=bufs)
        for w, g in zip(want_final, bufs):
            assert torch.equal(w, g), f"final_out tail={tail}"
        # a carried ring below capacity (two entries, capacity 9)
        cap, short = 9, 2
        head = projected[:, :window].contiguous()
        _, final = herm.window_rings(t(ck[:, :short]), t(cv[:, :short]), t(cok[:, :short]), head[..., :d],
                                     head[..., d:2 * d], t(fl[:, :window]), window=window, capacity=cap, tail=tail,
                                     key_valid=vmask[:, :window].contiguous(), final_only=True)
        mk, mv = (m[:, :window].cpu().numpy() for m in masked)
        if tail:
            rk = np.concatenate([ck[:, :short], mk], axis=1)[:, -cap:]
            rv = np.concatenate([cv[:, :short], mv], axis=1)[:, -cap:]
            rok = np.concatenate([cok[:, :short], fl[:, :window]], axis=1)[:, -cap:]
        else:
            rk, rv, rok = (np.asarray(x) for x in oracle.salient_tail(ck[:, :short], cv[:, :short], cok[:, :short],
                                                                      mk, mv, fl[:, :window], cap))
        np.testing.assert_array_equal(final[2].cpu().numpy(), rok, err_msg=f"short tail={tail}")
        np.testing.assert_array_equal(final[0].cpu().numpy(), rk.astype(np.float32), err_msg=f"short tail={tail}")
        np.testing.assert_array_equal(final[1].cpu().numpy(), rv.astype(np.float32), err_msg=f"short tail={tail}")


@pytest.mark.parametrize("key_dtype, slots", [(torch.bfloat16, 16), (torch.float32, 5)])
def test_read_step_with_rings_equals_the_read_and_the_two_rings(device, key_dtype, slots):
    """koemi_read_step_pair_rings (a decode step's reads and both ring
    updates, one launch) equals koemi_read_step_pair plus window_rings of the
    local (tail) and salient rings, bit for bit; the entries are column blocks
    of a wider projection, some positions invalid, some admitted."""

    from koemi_amd import _native

    rng = np.random.default_rng(slots)
    b, d = 37, 64
    c = 2 * d + 8
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device)
    lk, lv, lok, _, _, _ = _rand_rings(rng, b, slots, 1, d, 0.5)
    sk, sv, sok, _, _, _ = _rand_rings(rng, b, slots, 1, d, 0.5)
    valid = rng.random((b, 1)) < 0.8
    admission = valid & (rng.random((b, 1)) < 0.5)
    projected = torch.randn((b, 1, c), device=device).to(key_dtype)
    keys, values = projected[..., :d], projected[..., d:2 * d]
    q = torch.randn((b, d), device=device)
    lk, lv, lok, sk, sv, sok, vmask, amask = (t(x) for x in (lk, lv, lok, sk, sv, sok, valid, admission))
    stream = _native.stream_of(q.device)
    common = lambda lo, so: (_native.ptr(lk), _native.ptr(lv), _native.ptr(lok), slots, slots, _native.ptr(sk),
                             _native.ptr(sv), _native.ptr(sok), slots, _native.ptr(q), _native.ptr(lo),
                             _native.ptr(so))
    want_l, want_s = torch.empty_like(q), torch.empty_like(q)
    _native.call("koemi_read_step_pair", *common(want_l, want_s), b, d, stream)
    _, want_lr = herm.window_rings(lk, lv, lok, keys, values, vmask, window=1, capacity=slots, tail=True,
                                   key_valid=vmask, final_only=True)
    _, want_sr = herm.window_rings(sk, sv, sok, keys, values, amask, window=1, capacity=slots, tail=False,
                                   key_valid=vmask, final_only=True)
    got_l, got_s = torch.full_like(q, 7.0), torch.full_like(q, 7.0)
    got_lr = tuple(torch.full_like(x, 1) for x in want_lr)
    got_sr = tuple(torch.full_like(x, 1) for x in want_sr)
    _native.call("koemi_read_step_pair_rings", *common(got_l, got_s), _native.ptr(keys), _native.ptr(values),
                 _native.dtype_code(key_dtype), keys.stride(1), _native.ptr(vmask), _native.ptr(amask),
                 *(_native.ptr(x) for x in got_lr + got_sr), b, d, stream)
    assert torch.equal(got_l, want_l) and torch.equal(got_s, want_s)
    for w, g in zip(want_lr + want_sr, got_lr + got_sr):
        assert torch.equal(w, g)


@pytest.mark.parametrize("proj_dtype, m", [(torch.bfloat16, 16), (torch.float32, 5)])
def test_decode_memory_step_equals_the_reads_rings_and_associative_step(device, proj_dtype, m):
    """koemi_decode_memory_step (the two reads, both ring updates and the
    associative memory's one-position step in one launch) equals
    koemi_read_step_pair_rings plus associative_scan_read at length 1, bit
    for bit, on a stacked projection [local keys ; local values ; values ;
    feature logits ; decay ; write] with padding columns."""

    from koemi_amd import _native

    rng = np.random.default_rng(m)
    b, d, slots = 19, 64, 16
    c = 3 * d + 2 * m + 2
    c += -c % 4
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device)
    lk, lv, lok, _, _, _ = _rand_rings(rng, b, slots, 1, d, 0.5)
    sk, sv, sok, _, _, _ = _rand_rings(rng, b, slots, 1, d, 0.5)
    valid = rng.random((b, 1)) < 0.8
    admission = valid & (rng.random((b, 1)) < 0.5)
    lk, lv, lok, sk, sv, sok, vmask, amask = (t(x) for x in (lk, lv, lok, sk, sv, sok, valid, admission))
    projected = torch.randn((b, 1, c), device=device).to(proj_dtype)
    q = torch.randn((b, d), device=device)
    surprise = torch.rand((b, 1), device=device)
    basis = torch.randn((b, d, m), device=device) * 0.1
    normalizer = torch.rand((b, m), device=device)
    stream = _native.stream_of(q.device)
    common = lambda lo, so: (_native.ptr(lk), _native.ptr(lv), _native.ptr(lok), slots, slots, _native.ptr(sk),
                             _native.ptr(sv), _native.ptr(sok), slots, _native.ptr(q), _native.ptr(lo),
                             _native.ptr(so))
    rings = lambda: tuple(torch.full_like(x, 1) for x in (lk, lv, lok, sk, sv, sok))
    want_l, want_s, want_r = torch.empty_like(q), torch.empty_like(q), rings()
    keys, values = projected[..., :d], projected[..., d:2 * d]
    _native.call("koemi_read_step_pair_rings", *common(want_l, want_s), _native.ptr(keys), _native.ptr(values),
                 _native.dtype_code(proj_dtype), c, _native.ptr(vmask), _native.ptr(amask),
                 *(_native.ptr(x) for x in want_r), b, d, stream)
    want_fast, want_basis, want_norm = herm.associative_scan_read(projected, surprise, vmask, basis, normalizer,
                                                                  width=d, features=m)
    got_l, got_s, got_r = torch.full_like(q, 7.0), torch.full_like(q, 7.0), rings()
    got_fast = torch.full((b, 1, d), 7.0, device=device)
    got_basis, got_norm = torch.full_like(basis, 7.0), torch.full_like(normalizer, 7.0)
    _native.call("koemi_decode_memory_step", *common(got_l, got_s), _native.ptr(projected),
                 _native.dtype_code(proj_dtype), c, 0, d, _native.ptr(vmask), _native.ptr(amask),
                 *(_native.ptr(x) for x in got_r), 2 * d, 3 * d, 3 * d + m, 3 * d + 2 * m, 3 * d + 2 * m + 1,
                 _native.ptr(surprise), _native.ptr(basis), _native.ptr(normalizer), _native.ptr(got_fast),
                 _native.ptr(got_basis), _native.ptr(got_norm), m, b, d, stream)
    assert torch.equal(got_l, want_l) and torch.equal(got_s, want_s)
    for w, g in zip(want_r, got_r):
        assert torch.equal(w, g)
    assert torch.equal(got_fast, want_fast)
    assert torch.equal(got_basis, want_basis) and torch.equal(got_norm, want_norm)


def test_windowed_associative_memory_equals_window_by_window(device):
    g = torch.Generator(device=device).manual_seed(9)
    b, windows, window, d, m = 3, 5, 40, 96, 16
    stride = 3 * d + 2 * m + 2 + 2
    proj = torch.randn((b, windows * window, stride), generator=g, device=device)
    surprise = torch.rand((b, windows * window), generator=g, device=device)
    valid = torch.rand((b, windows * window), generator=g, device=device) < 0.9
    basis = torch.randn((b, d, m), generator=g, device=device) * 0.1
    norm = torch.rand((b, m), generator=g, device=device)
    read, nb, nn = herm.associative_scan_read_windows(proj, surprise, valid, basis, norm, width=d, features=m,
                                                      window=window)
    cur_b, cur_n = basis, norm
    for w in range(windows):
        sl = slice(w * window, (w + 1) * window)
        r, cur_b, cur_n = herm.associative_scan_read(proj[:, sl].contiguous(), surprise[:, sl], valid[:, sl], cur_b,
                                                     cur_n, width=d, features=m)
        assert torch.equal(read[:, sl], r), f"window {w}"
    assert torch.equal(nb, cur_b) and torch.equal(nn, cur_n)


def test_stack_sequence_matches_window_by_window_and_the_oracle(device):
    b, length = 2, 30
    settings = _settings(layers=3, scan_chunk=6)
    params = _params(settings, seed=23)
    params_np = _oracle_params(params)
    ids = _ids(b, length, seed=12)
    ids[1, 20:23] = herm.PAD_TOKEN_ID
    tau = _pick_threshold(params_np, ids, settings)
    settings = dataclasses.replace(settings, salience_threshold=tau)
    cfg = settings.oracle_config()
    prepared = herm.prepare_stack(params, settings, device)
    ids_t = torch.from_numpy(ids).to(device)
    want_logits, want_states = herm.prefill(prepared, settings, ids_t, herm.initial_states(settings, b, device))
    logits, states = herm.stack_sequence(prepared, settings, ids_t, herm.initial_states(settings, b, device))
    torch.cuda.synchronize()
    scale = float(want_logits.abs().max())
    assert float((logits - want_logits).abs().max()) <= 1e-5 * scale
    for layer, (got, want) in enumerate(zip(states, want_states)):
        for key, tensor in want.items():
            if tensor.dtype.is_floating_point:
                tol = 1e-5 * float(tensor.abs().max()) + 1e-7
                assert float((got[key] - tensor).abs().max()) <= tol, f"layer {layer} {key}"
            else:
                assert torch.equal(got[key], tensor), f"layer {layer} {key}"
    assert any(bool(st["salient_valid"].any()) for st in want_states)
    o_logits, o_states = oherm.prefill(params_np, [oherm.initial_state(b, cfg) for _ in params_np], ids, cfg,
                                       settings.scan_chunk)
    _close(logits.cpu().numpy(), o_logits, float(np.abs(o_logits).max()), "sequence-parallel logits vs oracle")
    for got, want in zip(states, o_states):
        for key in ("local_valid", "salient_valid", "last_token"):
            np.testing.assert_array_equal(got[key].cpu().numpy(), want[key])


def test_sequence_prefill_graph_replays_equal_eager(device):
    b, length = 2, 24
    settings = _settings(layers=2, scan_chunk=6, salience_threshold=0.55)
    prepared = herm.prepare_stack(_params(settings, seed=25), settings, device)
    ids = torch.from_numpy(_ids(b, length, seed=13)).to(device)
    want, want_states = herm.stack_sequence(prepared, settings, ids, herm.initial_states(settings, b, device))
    seq = herm.SequencePrefill(prepared, settings, herm.initial_states(settings, b, device), ids)
    first = None
    for run in range(2):
        got = seq.run(ids).clone()
        torch.cuda.synchronize()
        # the library GEMMs may be replayed from other algorithms inside the capture
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5 * float(want.abs().max()))
        for g_state, w_state in zip(seq.states, want_states):
            for key, tensor in w_state.items():
                if tensor.dtype.is_floating_point:
                    torch.testing.assert_close(g_state[key], tensor, rtol=1e-5, atol=1e-6)
                else:
                    assert torch.equal(g_state[key], tensor), f"run {run} {key}"
        if first is None:
            first = got
        else:
            assert torch.equal(got, first)
