"""Bounded recurrent gates (model/memory.py:14-30) and the window's working-state
scan (network.py:306-310) on the GPU against the float64 oracle.

Tolerances: fp32 products accumulate in fp32 over the width, so gates are
within 2e-5 absolute (|a|, |b| < 1) and the scanned states within 1e-4 (a < 1
keeps the recurrence contractive); bf16/f16 outputs are rounded to the dtype,
within 2^-7 absolute of values below 1 and 2^-6 of the scanned states.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from koemi_amd import dense, recurrent

pytestmark = pytest.mark.gpu


def _case(seed, b, length, d, p, dtype):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn((b, length, d), generator=g).to(dtype)
    scale = d ** -0.5  # nn.Linear's initialisation scale
    wr, wc = ((scale * torch.randn((d, d), generator=g)).to(dtype) for _ in range(2))
    br, bc = ((scale * torch.randn((d,), generator=g)).to(dtype) for _ in range(2))
    valid = torch.rand((b, length), generator=g) < p
    return u, wr, br, wc, bc, valid


def _np(t):
    return t.float().numpy() if t.is_floating_point() else t.numpy()


@pytest.mark.parametrize(
    "b, length, d, p, dtype",
    [
        (2, 128, 64, 0.9, torch.float32),      # default model window (embedding 64, scan window 128)
        (4, 256, 1024, 0.8, torch.float32),    # C5 width
        (2, 64, 256, 0.7, torch.bfloat16),
        (3, 17, 12, 0.5, torch.float16),
    ],
)
def test_recurrent_gates_match_oracle(device, b, length, d, p, dtype):
    u, wr, br, wc, bc, valid = _case(b * 13 + d, b, length, d, p, dtype)
    a, inc = recurrent.recurrent_gates(*(t.to(device) for t in (u, wr, br, wc, bc)), valid.to(device))
    want_a, want_b = oracle.recurrent_gates(*(_np(t) for t in (u, wr, br, wc, bc, valid)))
    tol = 2e-5 if dtype == torch.float32 else 2.0**-7
    err_a = np.abs(a.float().cpu().numpy() - want_a).max()
    err_b = np.abs(inc.float().cpu().numpy() - want_b).max()
    print(f"gates b={b} L={length} d={d} {dtype}: max_abs a={err_a:.3e} b={err_b:.3e}", flush=True)
    assert err_a <= tol and err_b <= tol
    inv = ~valid.numpy()
    assert np.all(a.float().cpu().numpy()[inv] == 1.0) and np.all(inc.float().cpu().numpy()[inv] == 0.0)


@pytest.mark.parametrize("b, length, d, dtype", [(2, 128, 64, torch.float32), (2, 300, 128, torch.bfloat16)])
def test_recurrent_scan_matches_oracle(device, b, length, d, dtype):
    u, wr, br, wc, bc, valid = _case(b + length + d, b, length, d, 0.85, dtype)
    h0 = torch.randn((b, d), generator=torch.Generator().manual_seed(5)).to(dtype)
    h = recurrent.recurrent_scan(*(t.to(device) for t in (u, wr, br, wc, bc, valid, h0)))
    a, inc = oracle.recurrent_gates(*(_np(t) for t in (u, wr, br, wc, bc, valid)))
    if dtype != torch.float32:  # the kernel hands a and b to the scan in the input dtype
        a = a.astype(np.float32).astype(np.float64) if dtype == torch.float16 else oracle.round_bf16(a.astype(np.float32)).astype(np.float64)
        inc = inc.astype(np.float32).astype(np.float64) if dtype == torch.float16 else oracle.round_bf16(inc.astype(np.float32)).astype(np.float64)
    want = oracle.scan_sequential(a, inc, _np(h0).astype(np.float64))
    err = np.abs(h.float().cpu().numpy() - want).max()
    print(f"recurrent scan b={b} L={length} d={d} {dtype}: max_abs={err:.3e}", flush=True)
    assert err <= (1e-4 if dtype == torch.float32 else 2.0**-6)


@pytest.mark.parametrize(
    "b, length, d, p, with_mask",
    [
        (64, 40, 512, 0.8, True),    # two columns per lane (64 x 4 column strips fill the chip)
        (32, 33, 1024, 0.9, False),  # C3 width, no mask
        (2, 300, 100, 0.7, True),    # one column per lane, a partial column strip
        (3, 1, 64, 0.5, True),       # one-token window (decode)
        (8, 129, 1024, 0.85, True),  # C5 batch and width, one column per lane
    ],
)
def test_fused_recurrent_scan_equals_gates_then_scan(device, b, length, d, p, with_mask):
    """koemi_recurrent_scan forms the gates inside the scan kernel with the
    gate kernel's expressions: its states match gates + dense_affine_scan to
    fp32 rounding (the oracle fixes both within 1e-4)."""
    u, wr, br, wc, bc, valid = _case(b * 7 + length + d, b, length, d, p, torch.float32)
    h0 = torch.randn((b, d), generator=torch.Generator().manual_seed(9))
    args = [t.to(device) for t in (u, wr, br, wc, bc)]
    mask = valid.to(device) if with_mask else None
    fused = recurrent.recurrent_scan(*args, mask, h0.to(device))
    a, inc = recurrent.recurrent_gates(*args, mask)
    split = dense.dense_affine_scan(a, inc, h0.to(device))
    torch.cuda.synchronize()
    diff = (fused - split).abs().max().item()
    print(f"fused scan b={b} L={length} d={d} mask={with_mask}: max_abs vs split={diff:.3e} "
          f"exact={torch.equal(fused, split)}", flush=True)
    assert diff <= 1e-6
    if length * d <= 300 * 128:
        want = oracle.scan_sequential(*oracle.recurrent_gates(*(_np(t) for t in (u, wr, br, wc, bc, valid if with_mask
                                                                                  else torch.ones_like(valid)))),
                                      _np(h0).astype(np.float64))
        assert np.abs(fused.cpu().numpy() - want).max() <= 1e-4


@pytest.mark.parametrize(
    "b, length, d, r_off, c_off, cols",
    [
        (64, 40, 512, 0, 512, 1024),    # stacked gate GEMM output, two columns per lane
        (8, 129, 1024, 0, 1024, 2048),  # C5 window shape, one column per lane
        (2, 37, 100, 3, 105, 210),      # odd offsets inside wider rows
        (64, 1, 1024, 0, 1024, 2048),   # decode step (one-position kernel)
        (3, 1, 36, 41, 2, 80),          # candidate columns before the retention columns
    ],
)
def test_gated_scan_from_preactivations(device, b, length, d, r_off, c_off, cols):
    """koemi_gated_scan against the oracle's gates (u = the pre-activation
    row, W_r and W_c selecting the two column ranges, zero biases) and scan."""
    g = torch.Generator().manual_seed(b * 1000 + length + d)
    z = 1.5 * torch.randn((b, length, cols), generator=g)
    valid = torch.rand((b, length), generator=g) < 0.8
    h0 = torch.randn((b, d), generator=g)
    h = recurrent.gated_scan(z.to(device), valid.to(device), h0.to(device), width=d, retention_offset=r_off,
                             candidate_offset=c_off)
    select = lambda off: np.eye(cols)[off:off + d]
    a, inc = oracle.recurrent_gates(z.double().numpy(), select(r_off), np.zeros(d), select(c_off), np.zeros(d),
                                    valid.numpy())
    want = oracle.scan_sequential(a, inc, h0.double().numpy())
    err = np.abs(h.cpu().numpy() - want).max()
    print(f"gated scan b={b} L={length} d={d} offsets=({r_off},{c_off}): max_abs={err:.3e}", flush=True)
    assert err <= 1e-4
    # a one-position call (the decode kernel) reproduces the window's first state bit for bit
    first = recurrent.gated_scan(z[:, :1].to(device), valid[:, :1].to(device), h0.to(device), width=d,
                                 retention_offset=r_off, candidate_offset=c_off)
    assert torch.equal(first, h[:, :1])


@pytest.mark.parametrize(
    "b, length, d, r_off, c_off, cols",
    [
        (8, 2048, 1024, 0, 1024, 2048),  # C5 prefill: 128 column tiles, eight chunks of 256 positions
        (3, 1000, 100, 3, 105, 210),     # ragged: the last chunk and the last column tile short
        (1, 777, 64, 0, 64, 128),        # one column tile: a chunk of 64 positions per workgroup
    ],
)
def test_two_phase_gated_scan_equals_the_one_pass_scan(device, b, length, d, r_off, c_off, cols):
    """The two-phase scan (segment transfers, then chunks from their composed
    carries) gives the one-pass scan's bits, fp32 states and bf16 copy, and
    stays within 1e-4 of the oracle's float64 scan."""
    g = torch.Generator().manual_seed(b * 7 + length)
    z = (1.5 * torch.randn((b, length, cols), generator=g)).to(device)
    valid = (torch.rand((b, length), generator=g) < 0.8).to(device)
    h0 = torch.randn((b, d), generator=g).to(device)
    kw = dict(width=d, retention_offset=r_off, candidate_offset=c_off, with_bf16=True)
    one, one16 = recurrent.gated_scan(z, valid, h0, two_phase=False, **kw)
    two, two16 = recurrent.gated_scan(z, valid, h0, two_phase=True, **kw)
    # the bf16 copy written into a column block of a wider matrix
    wide = torch.zeros((b, length, 3 * d), device=device, dtype=torch.bfloat16)
    three, _ = recurrent.gated_scan(z, valid, h0, two_phase=True, out_bf16=wide[..., d:2 * d], **kw)
    torch.cuda.synchronize()
    assert torch.equal(one, two) and torch.equal(one16, two16)
    assert torch.equal(three, one) and torch.equal(wide[..., d:2 * d], one16)
    assert not wide[..., :d].any() and not wide[..., 2 * d:].any()
    select = lambda off: np.eye(cols)[off:off + d]
    zc = z.double().cpu().numpy()
    a, inc = oracle.recurrent_gates(zc, select(r_off), np.zeros(d), select(c_off), np.zeros(d), valid.cpu().numpy())
    want = oracle.scan_sequential(a, inc, h0.double().cpu().numpy())
    err = np.abs(two.cpu().numpy() - want).max()
    print(f"two-phase gated scan b={b} L={length} d={d}: max_abs={err:.3e}", flush=True)
    assert err <= 1e-4


@pytest.mark.parametrize("b, length, d, two_phase", [(8, 256, 1024, True), (64, 40, 512, True), (3, 300, 100, True),
                                                     (64, 1, 1024, False), (1, 777, 64, True)])
def test_gated_scan_from_bf16_preactivations_equals_their_widening(device, b, length, d, two_phase):
    """bf16 pre-activations (a bf16 GEMM's own output) give the states of
    their exact fp32 widening, bit for bit: every path (wide, lane-group,
    two-phase, one position) widens on load and computes in fp32."""

    g = torch.Generator(device=device).manual_seed(b + length + d)
    z = (1.5 * torch.randn((b, length, 2 * d), generator=g, device=device)).to(torch.bfloat16)
    valid = torch.rand((b, length), generator=g, device=device) < 0.8
    h0 = torch.randn((b, d), generator=g, device=device)
    bias = torch.randn((2 * d,), generator=g, device=device) * 0.1
    kw = dict(width=d, with_bf16=True, two_phase=two_phase, retention_bias=bias[:d], candidate_bias=bias[d:])
    low, low16 = recurrent.gated_scan(z, valid, h0, **kw)
    wide, wide16 = recurrent.gated_scan(z.float(), valid, h0, **kw)
    torch.cuda.synchronize()
    assert torch.equal(low, wide) and torch.equal(low16, wide16)


def _exact_projection_case(seed, b, length, k, d, p, device):
    """bf16 inputs and weights on grids fine enough that every product and
    partial sum of the gate projection is exact in fp32 (u in {-3..3} / 8, W
    in {-3..3} / 64: products are multiples of 2^-9 and |sums| <= 18 for K <=
    1024, so 15 significant bits), so the projection does not depend on the
    order of accumulation and every implementation forms the same
    pre-activations."""
    g = torch.Generator().manual_seed(seed)
    u = (torch.randint(-3, 4, (b, length, k), generator=g) / 8.0).to(torch.bfloat16)
    w = (torch.randint(-3, 4, (2 * d, k), generator=g) / 64.0).to(torch.bfloat16)
    bias = (torch.randint(-8, 9, (2 * d,), generator=g) / 64.0).to(torch.bfloat16)
    valid = torch.rand((b, length), generator=g) < p
    valid[:, 255::256] = False  # masked positions at tile ends
    h0 = torch.randn((b, d), generator=g)
    return (t.to(device) for t in (u, w, bias, valid, h0))


@pytest.mark.parametrize(
    "b, length, k, d, p",
    [
        (2, 512, 256, 256, 0.9),     # two tiles per sequence, four ticket groups
        (3, 768, 128, 384, 0.8),     # nine chains: one ticket group
        (1, 256, 64, 128, 1.0),      # one tile, two K steps
        (8, 2048, 1024, 1024, 0.9),  # C5 prefill: 512 tiles, two rounds of the chip
    ],
)
def test_gated_projection_scan_matches_oracle(device, b, length, k, d, p):
    """koemi_gated_projection_scan against the oracle's gates and float64
    scan of the bf16-rounded pre-activations (exact projection), and against
    koemi_gated_scan on the same pre-activations: the gates are the same
    bits, the states differ only by how carries are composed (within 1e-5);
    the bf16 copy is the states rounded, written into a column block."""
    u, w, bias, valid, h0 = _exact_projection_case(b * 31 + length + d, b, length, k, d, p, device)
    z = torch.addmm(bias.float(), u.reshape(-1, k).float(), w.float().t()).view(b, length, 2 * d)
    z16 = z.to(torch.bfloat16)
    wide = torch.zeros((b, length, 3 * d), device=device, dtype=torch.bfloat16)
    fin = torch.full((b, d), float("nan"), device=device)
    got, got16 = recurrent.gated_projection_scan(u, w, bias, valid, h0, with_bf16=True, out_bf16=wide[..., d:2 * d],
                                                 final_out=fin)
    ref = recurrent.gated_scan(z16, valid, h0, width=d)
    torch.cuda.synchronize()
    assert torch.equal(got16, got.to(torch.bfloat16))
    assert torch.equal(fin, got[:, -1])
    assert not wide[..., :d].any() and not wide[..., 2 * d:].any()
    diff = (got - ref).abs().max().item()
    select = lambda off: np.eye(2 * d)[off:off + d]
    a, inc = oracle.recurrent_gates(z16.double().cpu().numpy(), select(0), np.zeros(d), select(d), np.zeros(d),
                                    valid.cpu().numpy())
    want = oracle.scan_sequential(a, inc, h0.double().cpu().numpy())
    err = np.abs(got.cpu().numpy() - want).max()
    print(f"gated projection scan b={b} L={length} K={k} d={d}: max_abs vs oracle {err:.3e}, "
          f"vs gates+scan {diff:.3e}", flush=True)
    assert err <= 1e-4
    assert diff <= 1e-5


def test_gated_projection_scan_random_weights_match_library_gemm_then_scan(device):
    """C5 shape with normal inputs and nn.Linear-scale weights: the fused
    kernel against hipBLASLt's bf16 GEMM (bias in the epilogue) then
    koemi_gated_scan. The two GEMMs accumulate in different orders, so a
    pre-activation can round to the neighbouring bf16 value (2^-8 relative);
    the states then differ by at most a few 1e-3 and almost everywhere by
    much less. Two calls in a row (the second with other inputs) check that
    each call starts from cleared flags."""
    g = torch.Generator(device=device).manual_seed(5)
    b, length, k, d = 8, 2048, 1024, 1024
    w = (torch.randn((2 * d, k), generator=g, device=device) * k ** -0.5).to(torch.bfloat16)
    bias = (torch.randn((2 * d,), generator=g, device=device) * k ** -0.5).to(torch.bfloat16)
    h0 = torch.randn((b, d), generator=g, device=device)
    for call in range(2):
        u = torch.randn((b, length, k), generator=g, device=device).to(torch.bfloat16)
        valid = torch.rand((b, length), generator=g, device=device) < 0.9
        got = recurrent.gated_projection_scan(u, w, bias, valid, h0)
        z16 = torch.addmm(bias, u.reshape(-1, k), w.t()).view(b, length, 2 * d)
        ref = recurrent.gated_scan(z16, valid, h0, width=d)
        torch.cuda.synchronize()
        diff = (got - ref).abs()
        big = (diff > 1e-4).float().mean().item()
        print(f"call {call}: max_abs {diff.max().item():.3e}, mean {diff.mean().item():.3e}, "
              f"share above 1e-4 {big:.2e}", flush=True)
        assert diff.max().item() <= 2e-2
        assert big <= 1e-3


def test_gated_projection_scan_graph_replays_equal_eager(device):
    """The kernel (its flag clearing included) captured in a HIP graph and
    replayed three times, with eager work between the replays, gives the
    eager call's bits each time: the carries do not depend on timing. Under
    capture the timeout is reported into a caller's status word, read after
    the replays."""
    u, w, bias, valid, h0 = _exact_projection_case(11, 4, 1024, 256, 256, 0.9, device)
    eager = recurrent.gated_projection_scan(u, w, bias, valid, h0)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        recurrent.gated_projection_scan(u, w, bias, valid, h0, status=status)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = recurrent.gated_projection_scan(u, w, bias, valid, h0, status=status)
    for _ in range(3):
        recurrent.gated_projection_scan(u, w, bias, valid, h0 * 0.5)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    recurrent.check_gated_scan_status(status)
    assert int(status.item()) == 0


def test_gated_projection_scan_timeout_is_an_error(device):
    """The bounded carry wait, driven to its timeout from the host: with
    KOEMI_GP_WITHHOLD_TRANSFERS no tile publishes its transfer, so every tile
    past the first of its sequence gives up after 64 polls (every wave still
    exits normally). The status word reads 1, the front raises, the first
    tile's states equal a normal call's and every later state is NaN (never
    silently wrong); a normal call afterwards is unaffected."""
    u, w, bias, valid, h0 = _exact_projection_case(12, 2, 768, 256, 256, 0.9, device)
    good = recurrent.gated_projection_scan(u, w, bias, valid, h0)
    status = torch.zeros(1, dtype=torch.int32, device=device)
    final = torch.empty((2, 256), device=device)
    got = recurrent.gated_projection_scan(u, w, bias, valid, h0, status=status, final_out=final,
                                          spin_limit=recurrent.GP_WITHHOLD_TRANSFERS | 64)
    torch.cuda.synchronize()
    assert int(status.item()) == 1
    with pytest.raises(recurrent.GatedScanTimeoutError, match="timed out"):
        recurrent.check_gated_scan_status(status)
    assert torch.equal(got[:, :256], good[:, :256])
    assert torch.isnan(got[:, 256:]).all() and torch.isnan(final).all()
    with pytest.raises(recurrent.GatedScanTimeoutError):
        recurrent.gated_projection_scan(u, w, bias, valid, h0, spin_limit=recurrent.GP_WITHHOLD_TRANSFERS | 64)
    assert torch.equal(recurrent.gated_projection_scan(u, w, bias, valid, h0), good)


def test_gated_projection_scan_needs_status_under_capture(device):
    """Under graph capture the front cannot read a status word back, so it
    refuses to run without the caller's."""
    u, w, bias, valid, h0 = _exact_projection_case(13, 1, 256, 64, 128, 1.0, device)
    recurrent.gated_projection_scan(u, w, bias, valid, h0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(dense.DenseCudaValidationError, match="status"):
        with torch.cuda.graph(graph):
            recurrent.gated_projection_scan(u, w, bias, valid, h0)


def test_gated_projection_scan_rejects_unsupported_shapes(device):
    u = torch.zeros((2, 200, 64), device=device, dtype=torch.bfloat16)
    w = torch.zeros((256, 64), device=device, dtype=torch.bfloat16)
    h0 = torch.zeros((2, 128), device=device)
    assert not recurrent.gated_projection_fits(u, w)
    with pytest.raises(dense.DenseCudaValidationError):
        recurrent.gated_projection_scan(u, w, None, None, h0)


def test_gated_scan_rejects_bad_columns(device):
    z = torch.zeros((2, 3, 10), device=device)
    h0 = torch.zeros((2, 4), device=device)
    with pytest.raises(dense.DenseCudaValidationError, match="inside"):
        recurrent.gated_scan(z, None, h0, width=4, retention_offset=0, candidate_offset=7)
    with pytest.raises(dense.DenseCudaValidationError, match="initial"):
        recurrent.gated_scan(z, None, h0[:, :3], width=4)
    assert recurrent.gated_scan(z, None, h0, width=4).shape == (2, 3, 4)


def test_recurrent_scan_rejects_bad_initial(device):
    u, wr, br, wc, bc, valid = (t.to(device) for t in _case(2, 2, 4, 8, 0.5, torch.float32))
    with pytest.raises(dense.DenseCudaValidationError, match="initial"):
        recurrent.recurrent_scan(u, wr, br, wc, bc, valid, torch.zeros((2, 4), device=device))
    h = recurrent.recurrent_scan(u[:, :0], wr, br, wc, bc, valid[:, :0])
    assert h.shape == (2, 0, 8)


def test_recurrent_gates_reject_bad_inputs(device):
    u, wr, br, wc, bc, valid = (t.to(device) for t in _case(1, 2, 4, 8, 0.5, torch.float32))
    with pytest.raises(dense.DenseCudaValidationError, match="must be on CUDA"):
        recurrent.recurrent_gates(u.cpu(), wr, br, wc, bc)
    with pytest.raises(dense.DenseCudaValidationError, match="same dtype"):
        recurrent.recurrent_gates(u, wr.double(), br, wc, bc)
    with pytest.raises(dense.DenseCudaValidationError, match="shape"):
        recurrent.recurrent_gates(u, wr[:4], br, wc, bc)
    with pytest.raises(dense.DenseCudaValidationError, match="valid_mask"):
        recurrent.recurrent_gates(u, wr, br, wc, bc, valid[:, :2])
