"""Salient memory on the GPU against the oracle: ring update (model/memory.py:431-455)
bit for bit, ring read (memory.py:405-429) within the tolerances stated below."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from koemi_amd import memory, think

pytestmark = pytest.mark.gpu


def _case(seed, b, s, length, d, p, dtype):
    g = torch.Generator().manual_seed(seed)
    ck, cv = torch.randn((b, s, d), generator=g).to(dtype), torch.randn((b, s, d), generator=g).to(dtype)
    k, v = torch.randn((b, length, d), generator=g).to(dtype), torch.randn((b, length, d), generator=g).to(dtype)
    cvalid, adm = torch.rand((b, s), generator=g) < p, torch.rand((b, length), generator=g) < p
    return ck, cv, cvalid, k, v, adm


@pytest.mark.parametrize(
    "b, s, length, d, p, capacity, dtype",
    [
        (2, 0, 4, 3, 0.75, 2, torch.float32),       # the ring KAT shape
        (4, 16, 2048, 64, 0.1, 16, torch.float32),  # C2-like window, sparse admission
        (3, 16, 64, 32, 0.9, 16, torch.bfloat16),   # many admitted
        (3, 5, 9, 8, 0.3, 32, torch.float16),       # fits: plain concatenation
        (2, 7, 300, 17, 0.02, 16, torch.float32),   # fewer valid than capacity: filler slots
        (5, 0, 1000, 128, 0.5, 100, torch.bfloat16),
    ],
)
def test_salient_tail_bit_exact(device, b, s, length, d, p, capacity, dtype):
    ck, cv, cvalid, k, v, adm = _case(b * 31 + length, b, s, length, d, p, dtype)
    got = memory.salient_tail(*(t.to(device) for t in (ck, cv, cvalid, k, v, adm)), capacity)
    as_np = (lambda t: t.view(torch.int16).numpy()) if dtype != torch.float32 else (lambda t: t.numpy())
    want = oracle.salient_tail(as_np(ck), as_np(cv), cvalid.numpy(), as_np(k), as_np(v), adm.numpy(), capacity)
    for g, w, is_flag in zip(got, want, (False, False, True)):
        g = g.cpu()
        g = g.numpy() if is_flag or dtype == torch.float32 else g.view(torch.int16).numpy()
        np.testing.assert_array_equal(g, w)


def test_salient_tail_known_answer(device):
    keys = torch.arange(12, dtype=torch.float32).view(1, 4, 3)
    empty = torch.zeros((1, 0, 3))
    k, v, ok = memory.salient_tail(empty.to(device), empty.to(device), torch.zeros((1, 0), dtype=torch.bool, device=device),
                                   keys.to(device), (keys + 100).to(device),
                                   torch.tensor([[True, False, True, True]], device=device), 2)
    assert torch.equal(k.cpu(), keys[:, [2, 3]]) and torch.equal(v.cpu(), keys[:, [2, 3]] + 100)
    assert ok.cpu().tolist() == [[True, True]]


def test_salient_tail_rejects_bad_inputs(device):
    k = torch.zeros((1, 4, 3), device=device)
    with pytest.raises(ValueError, match="positive integer"):
        memory.salient_tail(k[:, :0], k[:, :0], torch.zeros((1, 0), dtype=torch.bool, device=device), k, k,
                            torch.ones((1, 4), dtype=torch.bool, device=device), 0)
    with pytest.raises(ValueError, match="share a dtype"):
        memory.salient_tail(k[:, :0].half(), k[:, :0].half(), torch.zeros((1, 0), dtype=torch.bool, device=device), k, k,
                            torch.ones((1, 4), dtype=torch.bool, device=device), 2)


# ------------------------------------------------------------ salient read
# read_salient_window (model/memory.py:405-429) against the float64 oracle on
# the same (rounded) inputs. fp32: rtol 1e-4, atol 1e-5 x max|value| (fp32
# products on fp32 MFMA or rocBLAS, fp32 softmax). f16/bf16: the weights and the output are
# rounded to the input dtype as in the reference, so |err| <= 2^-7 x max|value|.


def _read_case(seed, b, s, length, d, p, dtype):
    g = torch.Generator().manual_seed(seed)
    t = lambda *shape: torch.randn(shape, generator=g).to(dtype)
    ck, cv, k, v, q = t(b, s, d), t(b, s, d), t(b, length, d), t(b, length, d), t(b, length, d)
    cvalid, adm = torch.rand((b, s), generator=g) < p, torch.rand((b, length), generator=g) < p
    return ck, cv, cvalid, k, v, adm, q


@pytest.mark.parametrize(
    "b, s, length, d, p, dtype",
    [
        (2, 16, 128, 64, 0.3, torch.float32),      # default model: 16 salient slots, 128-token window
        (8, 16, 128, 1024, 0.1, torch.float32),    # C5 width
        (3, 16, 128, 256, 0.5, torch.bfloat16),
        (2, 5, 37, 24, 0.7, torch.float16),
        (2, 0, 20, 8, 0.5, torch.float32),         # empty ring
        (1, 4, 1, 16, 1.0, torch.float32),         # one query: carried slots only (the one-position kernel)
        (64, 16, 1, 1024, 0.6, torch.float32),     # a C5 decode step
        (3, 16, 1, 100, 0.0, torch.bfloat16),      # one position, nothing eligible: zeros
        (2, 0, 1, 8, 0.5, torch.float32),          # one position, empty ring
        (3, 16, 64, 32, 0.0, torch.bfloat16),      # nothing eligible: zeros
        (1, 16, 984, 48, 0.3, torch.float32),      # 1000 slots (16 per softmax lane)
        (1, 24, 1000, 36, 0.3, torch.float32),     # 1024 slots: the largest of the HIP kernels
        (1, 16, 1100, 40, 0.3, torch.float32),     # 1116 slots: the rocBLAS path
        (2, 3, 45, 130, 0.6, torch.bfloat16),      # odd slot count and width (two-byte scalar loads)
        (2, 7, 33, 12, 0.8, torch.float32),        # one 64-column chunk, three empty width parts
        (1, 9, 70, 4100, 0.5, torch.float32),      # 65 chunks: 17 per width part, the last part short
        (2, 40, 90, 200, 0.9, torch.float16),      # carried slots fill two slot tiles
    ],
)
def test_read_salient_window_matches_oracle(device, b, s, length, d, p, dtype):
    case = _read_case(b * 7 + length + d, b, s, length, d, p, dtype)
    got = memory.read_salient_window(*(x.to(device) for x in case)).float().cpu().numpy()
    want = oracle.read_salient_window(*(x.float().numpy() if x.is_floating_point() else x.numpy() for x in case))
    vmax = max(float(case[1].float().abs().max()) if s else 0.0, float(case[4].float().abs().max()))
    err = np.abs(got - want)
    print(f"salient read b={b} s={s} L={length} d={d} {dtype}: max_abs={err.max():.3e} max|v|={vmax:.3e}", flush=True)
    if dtype == torch.float32:
        assert np.all(err <= 1e-4 * np.abs(want) + 1e-5 * vmax)
    else:
        assert np.all(err <= 2.0**-7 * vmax)
    if p == 0.0:
        assert np.all(got == 0.0)


@pytest.mark.parametrize("window, s, length", [(0, 16, 128), (16, 16, 128), (0, 16, 200), (40, 16, 50)])
def test_reads_into_a_bf16_block_equal_the_rounded_reads(device, window, s, length):
    """read_*_window(out=...) writes the read into a bf16 column block of a
    wider matrix: equal to the fp32 read rounded to bf16, the neighbouring
    columns untouched. (0, 16, 128) and (16, 16, 128) take the one-launch
    read (koemi_memory_read_into); (0, 16, 200) (215 candidate slots) and
    (40, 16, 50) (a window past 33) the fallback through the fp32 read."""

    b, d = 3, 64
    ck, cv, cvalid, k, v, flags, q = (x.to(device) for x in _read_case(7 + window + length, b, s, length, d, 0.6,
                                                                       torch.float32))
    wide = torch.zeros((b, length, 3 * d), device=device, dtype=torch.bfloat16)
    if window:
        want = memory.read_local_window(ck, cv, cvalid, k, v, flags, q, window=window)
        memory.read_local_window(ck, cv, cvalid, k, v, flags, q, window=window, out=wide[..., d:2 * d])
    else:
        want = memory.read_salient_window(ck, cv, cvalid, k, v, flags, q)
        memory.read_salient_window(ck, cv, cvalid, k, v, flags, q, out=wide[..., d:2 * d])
    assert torch.equal(wide[..., d:2 * d], want.to(torch.bfloat16))
    assert not wide[..., :d].any() and not wide[..., 2 * d:].any()


@pytest.mark.parametrize("window", [0, 16])
def test_reads_of_bf16_projection_columns_equal_the_widened_reads(device, window):
    """The fused read with the window's keys and values as bf16 column blocks
    of a wider projection (rows 2 D + 8 apart, read in place) equals the read
    of the same entries widened to contiguous fp32 to fp32 rounding (1e-6 of
    the output scale: the bf16 rows run on bf16 MFMA with the fp32 operand
    split in three parts, exact products; fp32 rows on fp32 MFMA); entries of
    positions the flags exclude do not matter (garbage there changes nothing,
    bit for bit)."""

    b, s, length, d = 3, 16, 64, 64
    ck, cv, cvalid, _, _, flags, q = (x.to(device) for x in _read_case(31 + window, b, s, length, d, 0.6,
                                                                       torch.float32))
    projected = torch.randn((b, length, 2 * d + 8), device=device).to(torch.bfloat16)
    keys, values = projected[..., :d], projected[..., d:2 * d]
    read = memory.read_local_window if window else memory.read_salient_window
    kw = {"window": window} if window else {}
    want = torch.zeros((b, length, d), device=device, dtype=torch.float32)
    read(ck, cv, cvalid, keys.float(), values.float(), flags, q, out=want, **kw)
    got = torch.zeros_like(want)
    read(ck, cv, cvalid, keys, values, flags, q, out=got, **kw)
    err = (got - want).abs().max().item()
    print(f"bf16 in place vs widened fp32 (window {window}): max_abs={err:.3e}", flush=True)
    assert err <= 1e-6 * want.abs().max().item()
    # a read that cannot take them in place (no out) widens them first
    assert torch.equal(read(ck, cv, cvalid, keys, values, flags, q, **kw),
                       read(ck, cv, cvalid, keys.float(), values.float(), flags, q, **kw))
    # the fused read lists only flagged slots: what the others hold is never read
    projected[..., :2 * d].masked_fill_(~flags[..., None], float("nan"))
    got2 = torch.zeros_like(want)
    read(ck, cv, cvalid, keys, values, flags, q, out=got2, **kw)
    assert torch.equal(got2, got)


def test_read_salient_window_rejects_bad_inputs(device):
    ck, cv, cvalid, k, v, adm, q = (x.to(device) for x in _read_case(1, 2, 3, 5, 4, 0.5, torch.float32))
    with pytest.raises(think.CudaThinkValidationError, match="share a dtype"):
        memory.read_salient_window(ck, cv, cvalid, k.half(), v, adm, q)
    with pytest.raises(think.CudaThinkValidationError, match="must be on CUDA"):
        memory.read_salient_window(ck, cv, cvalid, k, v, adm, q.cpu())
    with pytest.raises(think.CudaThinkValidationError, match="same shape"):
        memory.read_salient_window(ck, cv, cvalid, k[:, :4], v, adm, q)


# ------------------------------------------------------------ local read
# read_local_window (value output of model/memory.py:332-383) against the
# float64 oracle (itself pinned to the per-position ring read); same
# tolerances as the salient read.


@pytest.mark.parametrize(
    "b, s, length, d, window, p, dtype",
    [
        (8, 16, 128, 64, 16, 0.9, torch.float32),    # C5 shape (width reduced): ring of 16, window of 128
        (2, 16, 300, 48, 16, 0.8, torch.float32),    # several query tiles: the lower bound skips slot tiles
        (2, 4, 9, 12, 40, 0.7, torch.float32),       # window longer than the sequence
        (3, 5, 33, 20, 1, 0.6, torch.bfloat16),      # window of one entry
        (1, 16, 1100, 40, 24, 0.9, torch.float32),   # 1116 slots: the rocBLAS path
        (2, 0, 17, 8, 4, 0.5, torch.float16),        # empty ring
        (64, 16, 1, 1024, 16, 0.7, torch.float32),   # a C5 decode step (one-position kernel)
        (3, 20, 1, 72, 6, 0.8, torch.float16),       # one position: only the newest `window` ring slots
    ],
)
def test_read_local_window_matches_oracle(device, b, s, length, d, window, p, dtype):
    case = _read_case(b * 11 + length + d, b, s, length, d, p, dtype)
    got = memory.read_local_window(*(x.to(device) for x in case), window=window).float().cpu().numpy()
    ck, cv, cvalid, k, v, valid, q = (x.float().numpy() if x.is_floating_point() else x.numpy() for x in case)
    want = oracle.read_local_window(ck, cv, cvalid, k, v, valid, q, window)
    vmax = max(float(np.abs(cv).max()) if s else 0.0, float(np.abs(v).max()))
    err = np.abs(got - want)
    print(f"local read b={b} s={s} L={length} d={d} window={window} {dtype}: max_abs={err.max():.3e}", flush=True)
    if dtype == torch.float32:
        assert np.all(err <= 1e-4 * np.abs(want) + 1e-5 * vmax)
    else:
        assert np.all(err <= 2.0**-7 * vmax)


def test_read_local_window_rejects_a_bad_window(device):
    case = [x.to(device) for x in _read_case(3, 2, 3, 5, 4, 0.5, torch.float32)]
    with pytest.raises(think.CudaThinkValidationError, match="positive integer"):
        memory.read_local_window(*case, window=0)


@pytest.mark.parametrize("b, length, p", [(3, 300, 0.7), (2, 1, 0.5), (4, 64, 0.0), (1, 257, 1.0)])
def test_token_context_matches_the_oracle(device, b, length, p):
    """koemi_herm_token_context: previous valid token per position and last
    valid token per row (network.py:742-761) against the oracle's loop, over
    several 256-position chunks, one position, no valid token and all valid."""

    from koemi_amd import herm

    g = torch.Generator().manual_seed(b * 31 + length)
    ids = torch.randint(0, 256, (b, length), generator=g)
    valid = torch.rand((b, length), generator=g) < p
    carried = torch.randint(0, 257, (b,), generator=g)
    previous, last = herm._token_context(ids.to(device), valid.to(device), carried.to(device))
    want = oracle.previous_token_ids(ids.numpy(), valid.numpy(), carried.numpy())
    np.testing.assert_array_equal(previous.cpu().numpy(), want)
    want_last = np.array([ids[r][valid[r]][-1].item() if valid[r].any() else carried[r].item() for r in range(b)])
    np.testing.assert_array_equal(last.cpu().numpy(), want_last)
    # the same kernel forming the validity from the padding id, and the surprise targets
    padded = torch.where(valid, ids, torch.full_like(ids, herm.PAD_TOKEN_ID))
    previous2, last2, valid2, targets = herm._token_context(padded.to(device), None, carried.to(device))
    np.testing.assert_array_equal(valid2.cpu().numpy(), valid.numpy())
    np.testing.assert_array_equal(targets.cpu().numpy(), np.where(valid.numpy(), ids.numpy(), 0))
    np.testing.assert_array_equal(previous2.cpu().numpy(), want)
    np.testing.assert_array_equal(last2.cpu().numpy(), want_last)


def test_read_step_pair_equals_the_two_reads(device):
    """koemi_read_step_pair (the decode step's local and salient reads in one
    launch) against read_local_window and read_salient_window with one query."""
    from koemi_amd import _native

    g = torch.Generator().manual_seed(77)
    b, d, w, s = 5, 96, 16, 12
    lk, lv = (torch.randn((b, w, d), generator=g).to(device) for _ in range(2))
    sk, sv = (torch.randn((b, s, d), generator=g).to(device) for _ in range(2))
    lvalid = (torch.rand((b, w), generator=g) < 0.7).to(device)
    svalid = (torch.rand((b, s), generator=g) < 0.5).to(device)
    svalid[0] = False  # a row with nothing eligible
    q = torch.randn((b, 1, d), generator=g).to(device)
    new_k, new_v = (torch.randn((b, 1, d), generator=g).to(device) for _ in range(2))
    one = torch.ones((b, 1), dtype=torch.bool, device=device)
    for window in (16, 5):
        lo, so = torch.empty_like(q), torch.empty_like(q)
        _native.call("koemi_read_step_pair", _native.ptr(lk), _native.ptr(lv), _native.ptr(lvalid), w, window,
                     _native.ptr(sk), _native.ptr(sv), _native.ptr(svalid), s, _native.ptr(q), _native.ptr(lo),
                     _native.ptr(so), b, d, _native.stream_of(device))
        want_l = memory.read_local_window(lk, lv, lvalid, new_k, new_v, one, q, window=window)
        want_s = memory.read_salient_window(sk, sv, svalid, new_k, new_v, one, q)
        torch.testing.assert_close(lo, want_l, rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(so, want_s, rtol=1e-6, atol=1e-6)
        assert torch.equal(so[0], torch.zeros_like(so[0]))
