"""HERM block stack on the GPU (koemi_amd.herm) against the float64 oracle.

Parity setting: fp32 projections (``linear_dtype=torch.float32``), a two-layer
stack of width 32 run over two windows from the static initial state, then
greedy decode steps. The admission threshold is placed in a gap of the
oracle's surprise values (at least 2e-3 from every score), so the GPU's fp32
surprise (within ~1e-6 of the oracle's) admits exactly the same entries.
Tolerances: logits and states 1e-4 relative + 1e-4 x max|logit| absolute
(fp32 products and fp32 state against float64); masks and token ids exact.
The bf16 setting (the benchmark's) is compared with the fp32 setting with
admission off, within 5e-2 relative (bf16 rounding of every projection input).
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from koemi_amd import _native, herm, moe, think
from oracle import herm as oherm

pytestmark = pytest.mark.gpu

PAD = herm.PAD_TOKEN_ID


def _settings(**kw):
    base = dict(width=32, memory_features=4, local_memory_size=4, salience_memory_size=3, expert_count=4, top_k=2,
                layers=2, scan_chunk=6, linear_dtype=torch.float32)
    base.update(kw)
    return herm.HermSettings(**base)


def _params(settings, seed=11):
    params = herm.init_stack(settings, seed)
    for p in params:
        p["head_w"] *= 8.0  # spread the surprise scores over (0, 1)
    return params


def _oracle_params(params):
    return [{k: v.double().numpy() for k, v in p.items()} for p in params]


def _ids(b, length, seed=3):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, 256, (b, length))
    ids[1, 2] = PAD
    ids[0, 9] = PAD
    return ids


def _pick_threshold(params_np, ids, settings):
    """A threshold 2e-3 or more from every surprise score of the oracle run
    with it, with scores on both sides."""

    cfg = settings.oracle_config()
    for tau in (0.5, 0.55, 0.6, 0.65, 0.45, 0.7, 0.4):
        cfg["salience_threshold"] = tau
        scores = _oracle_scores(params_np, ids, settings, cfg)
        if np.abs(scores - tau).min() >= 2e-3 and (scores > tau).any() and (scores < tau).any():
            return tau
    pytest.skip("no threshold with a 2e-3 margin for this seed")


def _oracle_scores(params_np, ids, settings, cfg):
    states = [oherm.initial_state(ids.shape[0], cfg) for _ in params_np]
    scores = []
    for start in range(0, ids.shape[1], settings.scan_chunk):
        piece = ids[:, start:start + settings.scan_chunk]
        _, states, surprise = oherm.stack_window(params_np, states, piece, cfg)
        scores += [s[piece != PAD] for s in surprise]
    return np.concatenate(scores)


def _close(got, want, scale, what):
    err = np.abs(np.asarray(got, np.float64) - want)
    bound = 1e-4 * np.abs(want) + 1e-4 * scale
    print(f"{what}: max_abs={err.max():.3e} scale={scale:.3e}", flush=True)
    assert np.all(err <= bound), what


def test_stack_prefill_and_decode_match_the_oracle(device):
    b, length = 2, 12
    settings = _settings()
    params = _params(settings)
    params_np = _oracle_params(params)
    ids = _ids(b, length)
    tau = _pick_threshold(params_np, ids, settings)
    settings = dataclasses.replace(settings, salience_threshold=tau)
    cfg = settings.oracle_config()

    prepared = herm.prepare_stack(params, settings, device)
    states = herm.initial_states(settings, b, device)
    logits, states = herm.prefill(prepared, settings, torch.from_numpy(ids).to(device), states)
    want_states = [oherm.initial_state(b, cfg) for _ in params_np]
    want_logits, want_states = oherm.prefill(params_np, want_states, ids, cfg, settings.scan_chunk)
    scale = float(np.abs(want_logits).max())
    _close(logits.cpu().numpy(), want_logits, scale, "prefill logits")
    for layer, (got, want) in enumerate(zip(states, want_states)):
        for key in ("working", "basis", "normalizer", "local_keys", "salient_keys", "salient_values"):
            _close(got[key].cpu().numpy(), want[key], float(np.abs(want[key]).max()) + 1e-30, f"layer {layer} {key}")
        for key in ("local_valid", "salient_valid", "last_token"):
            np.testing.assert_array_equal(got[key].cpu().numpy(), want[key])
    assert any(w["salient_valid"].any() for w in want_states)  # admission happened

    # three greedy decode steps from the prefill state
    next_ids = torch.from_numpy(ids[:, -1:]).to(device)
    want_next = ids[:, -1:]
    for step in range(3):
        got_logits, states = herm.stack_window(prepared, settings, next_ids, states)
        want_step_logits, want_states, _ = oherm.stack_window(params_np, want_states, want_next, cfg)
        _close(got_logits.cpu().numpy(), want_step_logits, scale, f"decode step {step} logits")
        scores = want_step_logits[:, -1].copy()
        scores[:, PAD] = -np.inf
        want_next = scores.argmax(axis=-1)[:, None]
        top2 = np.sort(scores, axis=-1)[:, -2:]
        assert np.all(top2[:, 1] - top2[:, 0] > 1e-3)  # no near-tie in this case
        got_scores = got_logits[:, -1].clone()
        got_scores[:, PAD] = float("-inf")
        next_ids = got_scores.argmax(dim=-1, keepdim=True)
        np.testing.assert_array_equal(next_ids.cpu().numpy(), want_next)


def test_decode_graph_replays_match_eager_steps(device):
    b = 3
    settings = _settings(layers=2, salience_threshold=0.55)
    params = herm.prepare_stack(_params(settings, seed=12), settings, device)
    states = herm.initial_states(settings, b, device)
    _, states = herm.prefill(params, settings, torch.from_numpy(_ids(b, 12, seed=4)).to(device), states)
    ids = torch.tensor([[65], [66], [PAD]], device=device)
    graph = herm.DecodeGraph(params, settings, ids, states)
    eager_ids, eager_states = ids, states
    for step in range(4):
        eager_ids, eager_states = herm.decode_step(params, settings, eager_ids, eager_states)
        torch.cuda.synchronize()
        got = graph.step().clone()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), eager_ids.cpu().numpy())
        for layer, (g, e) in enumerate(zip(graph.states, eager_states)):
            for key, tensor in e.items():
                if tensor.dtype.is_floating_point:
                    torch.testing.assert_close(g[key], tensor, rtol=1e-5, atol=1e-5,
                                               msg=lambda m: f"step {step} layer {layer} {key}: {m}")
                else:
                    assert torch.equal(g[key], tensor), f"step {step} layer {layer} {key}"


def test_decode_surprise_of_all_layers_equals_the_per_layer_surprise(device):
    """A decode step's surprise and admission of every layer, formed at once
    (one batched content-head launch, one scoring launch), equal the
    per-layer path (koemi_linear_rows + koemi_herm_surprise_shifted) bit for
    bit: the same arithmetic per row."""

    b = 5
    settings = _settings(width=64, layers=3, linear_dtype=torch.bfloat16, salience_threshold=0.5)
    params = herm.prepare_stack(_params(settings, seed=21), settings, device)
    gen = torch.Generator().manual_seed(5)
    states = [{"working": torch.randn((b, 64), generator=gen).to(device)} for _ in range(3)]
    targets = torch.tensor([[3], [250], [0], [77], [128]], device=device)
    valid = torch.tensor([[True], [True], [False], [True], [True]], device=device)
    got = herm._surprise_layers(params, settings, states, targets, valid)
    assert got is not None
    for p, st, (s_got, a_got) in zip(params, states, got):
        s_want, a_want = herm._surprise_carried(p, settings, st["working"], targets, valid)
        assert torch.equal(s_got, s_want) and torch.equal(a_got, a_want)
    assert bool(valid.logical_not().logical_or(got[0][0] > 0).all())


def test_greedy_tokens_equal_the_masked_argmax(device):
    """koemi_herm_greedy_tokens equals torch's argmax of the last position's
    logits with the padding id set to -inf: random rows, ties (the first
    maximum wins), the padding id holding the maximum, an all -inf row and a
    row with NaNs (torch.argmax takes the first NaN)."""

    g = torch.Generator().manual_seed(8)
    b, length, vocab = 9, 2, 257
    logits = torch.randn((b, length, vocab), generator=g)
    logits[1, -1, [3, 77, 200]] = 9.0              # a three-way tie
    logits[2, -1, PAD] = 50.0                        # the padding id holds the maximum
    logits[3, -1, :] = float("-inf")                 # nothing but -inf
    logits[4, -1, [10, 20]] = float("nan")           # NaNs
    logits[5, -1, :] = 1.5                           # a constant row
    logits = logits.to(device)
    got = herm._greedy_tokens(logits)
    scores = logits[:, -1].clone()
    scores[:, PAD] = float("-inf")
    want = scores.cpu().argmax(dim=-1, keepdim=True)
    assert torch.equal(got.cpu(), want), (got.cpu().reshape(-1), want.reshape(-1))


def test_bf16_projections_stay_close_to_fp32(device):
    b = 2
    base = _settings(width=64, salience_threshold=2.0)  # admission off: no discrete flips
    params = _params(base, seed=13)
    ids = torch.from_numpy(_ids(b, 12, seed=5)).to(device)
    out = {}
    for dtype in (torch.float32, torch.bfloat16):
        settings = dataclasses.replace(base, linear_dtype=dtype)
        prepared = herm.prepare_stack(params, settings, device)
        logits, _ = herm.prefill(prepared, settings, ids, herm.initial_states(settings, b, device))
        assert torch.isfinite(logits).all()
        out[dtype] = logits.double()
    rel = float((out[torch.bfloat16] - out[torch.float32]).norm() / out[torch.float32].norm())
    print(f"bf16 vs fp32 projections: relative error {rel:.3e}", flush=True)
    assert rel < 5e-2


def test_graphed_prefill_matches_the_eager_prefill(device):
    b = 2
    settings = _settings(salience_threshold=0.55)
    params = herm.prepare_stack(_params(settings, seed=14), settings, device)
    ids = torch.from_numpy(_ids(b, 12, seed=6)).to(device)
    want_logits, want_states = herm.prefill(params, settings, ids, herm.initial_states(settings, b, device))
    graph = None
    for run in range(2):  # the second call reuses the captured window
        logits, states, graph = herm.prefill_graphed(params, settings, ids, herm.initial_states(settings, b, device),
                                                     graph)
        torch.cuda.synchronize()
        torch.testing.assert_close(logits, want_logits, rtol=1e-5, atol=1e-5)
        for g, e in zip(states, want_states):
            for key, tensor in e.items():
                if tensor.dtype.is_floating_point:
                    torch.testing.assert_close(g[key], tensor, rtol=1e-5, atol=1e-5)
                else:
                    assert torch.equal(g[key], tensor), f"run {run} {key}"


@pytest.mark.parametrize("b, length, d, m", [(2, 130, 100, 16), (3, 1, 64, 16), (2, 9, 36, 5), (1, 70, 128, 32),
                                              (2, 130, 100, 5), (1, 130, 264, 15)])
def test_associative_kernel_matches_the_oracle(device, b, length, d, m):
    """koemi_assoc_scan_read (memory.py:82-144, 244-255; network.py:734-740)
    against oracle/herm.py's float64 scan-and-read fed with the same terms
    (features = softmax of the given key/query feature logits, value = tanh,
    bounded decay, surprise-scaled write weight, masking): several 64-row
    influence tiles, partial 64-column chunks, one position (the decode step)
    and 5 or 32 features; fp32 tolerance 1e-4 relative + 1e-5 x max|result|.
    The last two cases have row strides and widths that are multiples of four
    (the reads' two-columns-per-lane layout with its causal stop): a last
    query tile of two rows, a partly filled 64-column wave tile, and two
    256-column groups."""

    rng = np.random.default_rng(b * 1000 + length)
    proj = rng.normal(size=(b, length, 3 * d + 2 * m + 2)).astype(np.float32)
    surprise = rng.random((b, length)).astype(np.float32)
    valid = rng.random((b, length)) < 0.8
    basis = rng.normal(size=(b, d, m)).astype(np.float32)
    normalizer = rng.random((b, m)).astype(np.float32)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(device)
    read, nb, nn = herm.associative_scan_read(t(proj), t(surprise), t(valid), t(basis), t(normalizer), width=d,
                                              features=m)
    p64 = proj.astype(np.float64)
    value = np.tanh(p64[..., 2 * d:3 * d])
    features = oherm.softmax(p64[..., 3 * d:3 * d + m])
    qf = oherm.softmax(p64[..., 3 * d + m:3 * d + 2 * m])
    decay = oherm.MIN_DECAY + (oherm.MAX_DECAY - oherm.MIN_DECAY) * oherm.sigmoid(p64[..., 3 * d + 2 * m])
    weight = oherm.sigmoid(p64[..., 3 * d + 2 * m + 1]) * (0.25 + 0.75 * np.clip(surprise, 0, 1))
    decay = np.where(valid, decay, 1.0)
    weight = np.where(valid, weight, 0.0)
    want = oherm.associative_scan_read(basis.astype(np.float64), normalizer.astype(np.float64), decay, value,
                                       features, weight, qf)
    for got, ref, name in zip((read, nb, nn), want, ("read", "basis", "normalizer")):
        err = np.abs(got.cpu().numpy().astype(np.float64) - ref)
        scale = float(np.abs(ref).max())
        print(f"assoc {name} b={b} L={length} d={d} m={m}: max_abs={err.max():.3e} scale={scale:.3e}", flush=True)
        assert np.all(err <= 1e-4 * np.abs(ref) + 1e-5 * scale), name


@pytest.mark.parametrize("length", [130, 128])
def test_associative_reads_into_a_bf16_block_and_from_bf16_projections(device, length):
    """The reads written into a bf16 column block of a wider matrix equal the
    fp32 reads rounded to bf16 (one launch, the same arithmetic), for the
    one-window and the windowed entry; projections given in bf16 give the
    reads of their fp32 widening bit for bit (the kernels widen on load)."""

    b, d, m, window = 2, 96, 16, 64
    g = torch.Generator(device=device).manual_seed(length)
    # rows padded to a multiple of 4 columns: the four-columns-per-lane read
    proj = torch.randn((b, length, 3 * d + 2 * m + 4), generator=g, device=device)
    surprise = torch.rand((b, length), generator=g, device=device)
    valid = torch.rand((b, length), generator=g, device=device) < 0.8
    basis = torch.randn((b, d, m), generator=g, device=device) * 0.1
    norm = torch.rand((b, m), generator=g, device=device)
    wide = torch.zeros((b, length, 3 * d), device=device, dtype=torch.bfloat16)
    read, nb, nn = herm.associative_scan_read(proj, surprise, valid, basis, norm, width=d, features=m)
    got, nb2, nn2 = herm.associative_scan_read(proj, surprise, valid, basis, norm, width=d, features=m,
                                               out=wide[..., d:2 * d])
    assert got.data_ptr() == wide[..., d:2 * d].data_ptr()
    assert torch.equal(wide[..., d:2 * d], read.to(torch.bfloat16))
    assert torch.equal(nb2, nb) and torch.equal(nn2, nn)
    assert not wide[..., :d].any() and not wide[..., 2 * d:].any()
    low = proj.to(torch.bfloat16)
    r16, b16, n16 = herm.associative_scan_read(low, surprise, valid, basis, norm, width=d, features=m)
    r32, b32, n32 = herm.associative_scan_read(low.float(), surprise, valid, basis, norm, width=d, features=m)
    assert torch.equal(r16, r32) and torch.equal(b16, b32) and torch.equal(n16, n32)
    if length % window == 0:
        wide.zero_()
        rw, bw, nw = herm.associative_scan_read_windows(proj, surprise, valid, basis, norm, width=d, features=m,
                                                        window=window)
        herm.associative_scan_read_windows(proj, surprise, valid, basis, norm, width=d, features=m, window=window,
                                           out=wide[..., 2 * d:])
        assert torch.equal(wide[..., 2 * d:], rw.to(torch.bfloat16))


@pytest.mark.parametrize("b, length", [(3, 130), (64, 1)])
def test_shifted_surprise_equals_the_row_kernel_on_shifted_logits(device, b, length):
    """koemi_herm_surprise_shifted scores row t on the logits of row t - 1
    (the carried state's for t = 0): equal, bit for bit, to
    koemi_surprise_rows_forward on the explicitly shifted logits, and its
    admission to valid & (surprise > threshold)."""

    g = torch.Generator(device=device).manual_seed(b + length)
    logits = torch.randn((b * length, 256), generator=g, device=device) * 2.0
    first = torch.randn((b, 256), generator=g, device=device) * 2.0
    bias = torch.randn((256,), generator=g, device=device) * 0.1
    targets = torch.randint(0, 256, (b, length), generator=g, device=device)
    valid = torch.rand((b, length), generator=g, device=device) < 0.8
    surprise = torch.empty((b, length), device=device)
    admission = torch.empty((b, length), device=device, dtype=torch.bool)
    threshold = 0.6
    _native.call("koemi_herm_surprise_shifted", _native.ptr(logits), _native.ptr(first), _native.ptr(bias),
                 _native.ptr(targets), _native.ptr(valid), _native.ptr(surprise), _native.ptr(admission), threshold,
                 b, length, 256, think._log_vocab(256), _native.stream_of(device))
    shifted = torch.cat((first.unsqueeze(1), logits.view(b, length, 256)[:, :-1]), dim=1).reshape(b * length, 256)
    want = think.surprise_from_logits(shifted.contiguous(), targets.reshape(-1), valid.reshape(-1),
                                      content_bias=bias).view(b, length)
    assert torch.equal(surprise, want)
    assert torch.equal(admission, valid & (want > threshold))


def test_bf16_copies_written_by_the_kernels_equal_the_casts(device):
    """The bf16 GEMM inputs the block's kernels write beside their fp32 results
    (RMSNorm, the gated scan, the fusion concatenation) equal torch's
    round-to-nearest-even casts of those results bit for bit."""

    from koemi_amd import _native, recurrent

    g = torch.Generator().manual_seed(21)
    x = torch.randn((37, 1024), generator=g).to(device)
    w = (1.0 + 0.1 * torch.randn((1024,), generator=g)).to(device)
    out, out16 = herm._rms(x, w, low=torch.bfloat16)
    assert out16.dtype == torch.bfloat16 and torch.equal(out16, out.to(torch.bfloat16))
    only16 = herm._rms(x, w, fp32=False, low=torch.bfloat16)
    assert only16[0] is None and torch.equal(only16[1], out16)

    for length in (1, 40):
        z = torch.randn((3, length, 2 * 96), generator=g).to(device)
        h0 = torch.randn((3, 96), generator=g).to(device)
        valid = (torch.rand((3, length), generator=g) < 0.7).to(device)
        states, states16 = recurrent.gated_scan(z, valid, h0, width=96, with_bf16=True)
        assert torch.equal(states, recurrent.gated_scan(z, valid, h0, width=96))
        assert torch.equal(states16, states.to(torch.bfloat16))

    pieces = [torch.randn((5, 7, 64), generator=g).to(device) for _ in range(4)]
    cat16 = torch.empty((5, 7, 256), device=device, dtype=torch.bfloat16)
    _native.call("koemi_herm_concat_bf16", *(_native.ptr(p) for p in pieces), 4, 35, 64, _native.ptr(cat16),
                 _native.stream_of(device))
    assert torch.equal(cat16, torch.cat(pieces, dim=-1).to(torch.bfloat16))


def test_wavefront_prefill_equals_the_window_by_window_prefill(device):
    """Layer windows scheduled as a wavefront on per-layer streams give the
    sequential prefill's logits and states bit for bit (same kernels, same
    inputs), over five windows and three layers, with admissions."""

    b = 2
    settings = _settings(layers=3, salience_threshold=0.55)
    params = herm.prepare_stack(_params(settings, seed=21), settings, device)
    ids = torch.from_numpy(_ids(b, 30, seed=8)).to(device)
    want_logits, want_states, _ = herm.prefill_graphed(params, settings, ids, herm.initial_states(settings, b, device))
    wave = herm.WavefrontPrefill(params, settings, herm.initial_states(settings, b, device), b, device)
    for run in range(2):
        logits = wave.run(ids)
        torch.cuda.synchronize()
        assert torch.equal(logits, want_logits), f"run {run}"
        for got, want in zip(wave.states, want_states):
            for key, tensor in want.items():
                assert torch.equal(got[key], tensor), f"run {run} {key}"
    assert any(bool(st["salient_valid"].any()) for st in want_states)


@pytest.mark.parametrize("tokens, learned", [(4096, False), (64, False), (300, True)])
def test_combine_norm_equals_combine_then_the_two_norms(device, tokens, learned):
    """koemi_herm_combine_norm (the expert tail of a stack's inner block: the
    combine, the expert normalizer with its residual and valid-row select, the
    next block's input norm) gives the bits of combine_topk followed by the
    two herm_rmsnorm calls it replaces, for hash (mean of the k outputs) and
    learned (weighted) mixtures, at prefill and decode row counts."""
    g = torch.Generator(device=device).manual_seed(tokens + learned)
    d, E, k, hidden = 1024, 16, 2, 256
    ctx = torch.randn((tokens, d), generator=g, device=device).to(torch.bfloat16)
    valid = torch.rand((tokens,), generator=g, device=device) < 0.9
    if learned:
        a, w = moe.route_topk_learned(torch.randn((tokens, E), generator=g, device=device), valid, top_k=k)
    else:
        ids = torch.randint(0, 256, (tokens,), generator=g, device=device)
        a = moe.route_topk_valid(ids, torch.roll(ids, 1), valid, expert_count=E, top_k=k, validate=False)
        w = None
    permuted = moe.permute_topk(ctx, a, valid, expert_count=E, pair_weights=w, gather=False)
    _, rows, _, offsets = permuted[:4]
    sw = permuted[4] if learned else None
    ws = [(0.05 * torch.randn(shape, generator=g, device=device)).to(torch.bfloat16)
          for shape in ((E, hidden, d), (E, hidden), (E, hidden, d), (E, hidden), (E, d, hidden), (E, d))]
    y = moe.grouped_expert_mlp_indexed(ctx, rows, offsets, *ws)
    flat = torch.randn((tokens, d), generator=g, device=device)
    w_e = 1.0 + 0.1 * torch.randn((d,), generator=g, device=device)
    w_n = 1.0 + 0.1 * torch.randn((d,), generator=g, device=device)
    update = moe.combine_topk(y, rows, offsets, token_count=tokens, top_k=k, pair_weights=sw, validate=False)
    want_final = herm._rms(flat, w_e, residual=update, mask=valid)
    want_next = herm._rms(want_final, w_n, fp32=False, low=torch.bfloat16)[1]
    need = _native.query("koemi_moe_combine_workspace_bytes", tokens, k)
    workspace = torch.empty((need,), device=device, dtype=torch.uint8)
    # pairs from the inversion of sorted_rows, and from the permutation's own map
    rows3, _, offsets3, sw3, positions = moe.permute_indices(a, valid, expert_count=E, pair_weights=w)
    assert torch.equal(rows3, rows) and torch.equal(offsets3, offsets)
    for by_position in (False, True):
        final = torch.empty_like(flat)
        nxt = torch.empty((tokens, d), device=device, dtype=torch.bfloat16)
        _native.call("koemi_herm_combine_norm", _native.ptr(y), _native.ptr(rows),
                     _native.ptr(positions if by_position else None), _native.ptr(offsets), _native.ptr(sw),
                     _native.ptr(flat), _native.ptr(valid), _native.ptr(w_e), _native.ptr(w_n), _native.ptr(final),
                     _native.ptr(nxt), int(y.shape[0]), d, tokens, k, E, herm._EPS, _native.ptr(workspace), need,
                     _native.stream_of(device))
        torch.cuda.synchronize()
        assert torch.equal(final, want_final), by_position
        assert torch.equal(nxt, want_next), by_position


@pytest.mark.parametrize("tokens, d, k", [(4096, 1024, 2), (300, 1024, 2), (64, 2048, 3), (129, 256, 1)])
def test_combine_norm_fusion_equals_the_fusion_norm_then_combine_norm(device, tokens, d, k):
    """koemi_herm_combine_norm_fusion (the fusion normalizer formed inside the
    expert tail from the bf16 fusion rows) gives the bits of herm_rmsnorm on
    those rows followed by koemi_herm_combine_norm on its fp32 result, with
    all three outputs (final, next input) and invalid rows."""
    g = torch.Generator(device=device).manual_seed(tokens + d + k)
    E, hidden = 8, 128
    ctx = torch.randn((tokens, d), generator=g, device=device).to(torch.bfloat16)
    valid = torch.rand((tokens,), generator=g, device=device) < 0.9
    ids = torch.randint(0, 256, (tokens,), generator=g, device=device)
    a = moe.route_topk_valid(ids, torch.roll(ids, 1), valid, expert_count=E, top_k=k, validate=False)
    rows, _, offsets, _, positions = moe.permute_indices(a, valid, expert_count=E)
    ws = [(0.05 * torch.randn(shape, generator=g, device=device)).to(torch.bfloat16)
          for shape in ((E, hidden, d), (E, hidden), (E, hidden, d), (E, hidden), (E, d, hidden), (E, d))]
    y = moe.grouped_expert_mlp_indexed(ctx, rows, offsets, *ws)
    fusion = (3.0 * torch.randn((tokens, d), generator=g, device=device)).to(torch.bfloat16)
    w_f, w_e, w_n = (1.0 + 0.1 * torch.randn((d,), generator=g, device=device) for _ in range(3))
    flat = herm._rms(fusion, w_f)
    outs = []
    for fused_form in (False, True):
        final = torch.empty((tokens, d), device=device, dtype=torch.float32)
        nxt = torch.empty((tokens, d), device=device, dtype=torch.bfloat16)
        if fused_form:
            _native.call("koemi_herm_combine_norm_fusion", _native.ptr(y), _native.ptr(positions),
                         _native.ptr(offsets), None, _native.ptr(fusion), _native.ptr(w_f), _native.ptr(valid),
                         _native.ptr(w_e), _native.ptr(w_n), _native.ptr(final), _native.ptr(nxt),
                         int(y.shape[0]), d, tokens, k, E, herm._EPS, _native.stream_of(device))
        else:
            _native.call("koemi_herm_combine_norm", _native.ptr(y), _native.ptr(rows), _native.ptr(positions),
                         _native.ptr(offsets), None, _native.ptr(flat), _native.ptr(valid), _native.ptr(w_e),
                         _native.ptr(w_n), _native.ptr(final), _native.ptr(nxt), int(y.shape[0]), d, tokens, k, E,
                         herm._EPS, None, 0, _native.stream_of(device))
        outs.append((final, nxt))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    assert not valid.all() and torch.equal(outs[1][0][~valid], flat[~valid])  # invalid rows keep the context
