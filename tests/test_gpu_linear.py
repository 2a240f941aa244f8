"""koemi_linear_rows (few-row projections with bf16 weights) against a
float64 product of the same bf16-rounded operands.

Tolerance: fp32 accumulation of K bf16 products, so within 1e-5 of the
largest |output| (plus 1e-6 absolute); fp32 inputs are rounded to bf16 on
load, as torch's cast does (round to nearest even).
"""

from __future__ import annotations

import pytest
import torch

from koemi_amd import dense, linear

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize(
    "rows, n_out, width, pieces, dtype, with_bias",
    [
        (64, 3106, 1024, 1, torch.float32, True),   # stacked working-state projections of a decode step
        (64, 2048, 1024, 1, torch.float32, True),   # the two gate projections
        (64, 1024, 1024, 4, torch.float32, True),   # fusion over [working ; memory ; local ; salient]
        (64, 257, 1024, 1, torch.float32, True),    # head (a partial last column group)
        (5, 96, 1024, 2, torch.bfloat16, False),    # few rows, bf16 input, no bias
        (70, 40, 1024, 3, torch.float32, True),     # two row passes
        (3, 64, 1600, 1, torch.float32, True),      # a partial last K chunk
        (1, 33, 192, 1, torch.bfloat16, True),
    ],
)
def test_linear_rows_matches_float64(device, rows, n_out, width, pieces, dtype, with_bias):
    g = torch.Generator().manual_seed(rows * 7 + n_out + width + pieces)
    xs = [torch.randn((rows, width), generator=g).to(dtype) for _ in range(pieces)]
    w = (torch.randn((n_out, width * pieces), generator=g) * (width * pieces) ** -0.5).to(torch.bfloat16)
    b = torch.randn((n_out,), generator=g) if with_bias else None
    got = linear.linear_rows([x.to(device) for x in xs], w.to(device), b.to(device) if b is not None else None)
    x64 = torch.cat([x.to(torch.bfloat16).double() for x in xs], dim=-1)
    want = x64 @ w.double().T + (b.double() if b is not None else 0.0)
    err = (got.double().cpu() - want).abs().max().item()
    scale = want.abs().max().item()
    print(f"linear rows {rows}x{width * pieces}->{n_out} {dtype}: max_abs={err:.3e} scale={scale:.3e}", flush=True)
    assert err <= 1e-5 * scale + 1e-6


def test_linear_rows_rejects_bad_inputs(device):
    x = torch.zeros((4, 64), device=device)
    w = torch.zeros((8, 64), device=device, dtype=torch.bfloat16)
    with pytest.raises(dense.DenseCudaValidationError, match="bfloat16"):
        linear.linear_rows([x], w.float(), None)
    with pytest.raises(dense.DenseCudaValidationError, match="multiples of 64"):
        linear.linear_rows([x[:, :32]], w[:, :32], None)
    with pytest.raises(dense.DenseCudaValidationError, match="float32"):
        linear.linear_rows([x], w, torch.zeros(8, device=device, dtype=torch.float64))
    assert linear.linear_rows([x[:0]], w, None).shape == (0, 8)


@pytest.mark.parametrize("rows, splits, dtype", [(64, 8, torch.float32), (37, 4, torch.float32),
                                                  (16, 4, torch.bfloat16)])
def test_split_linear_rows_partials_sum_to_the_projection(device, rows, splits, dtype):
    """koemi_linear_rows_split: the partial blocks, added in order, equal the
    float64 product of the bf16-rounded operands (the tolerance above), the
    bias in block 0 only; each block alone is the product over its K range."""

    from koemi_amd import _native

    width, pieces, n_out = 1024, 4, 1024
    g = torch.Generator().manual_seed(rows + splits)
    xs = [torch.randn((rows, width), generator=g).to(dtype).to(device) for _ in range(pieces)]
    w = (torch.randn((n_out, width * pieces), generator=g) * (width * pieces) ** -0.5).to(torch.bfloat16).to(device)
    b = torch.randn((n_out,), generator=g).to(device)
    partials = torch.empty((splits, rows, n_out), device=device)
    _native.call("koemi_linear_rows_split", *(_native.ptr(x) for x in xs), pieces, width, _native.dtype_code(dtype),
                 _native.ptr(w), _native.ptr(b), _native.ptr(partials), rows, n_out, splits,
                 _native.stream_of(partials.device))
    x64 = torch.cat([x.to(torch.bfloat16).double() for x in xs], dim=-1).cpu()
    w64 = w.double().cpu()
    k = width * pieces // splits
    for s in range(splits):
        want = x64[:, s * k:(s + 1) * k] @ w64[:, s * k:(s + 1) * k].T + (b.double().cpu() if s == 0 else 0.0)
        err = (partials[s].double().cpu() - want).abs().max().item()
        assert err <= 1e-5 * want.abs().max().item() + 1e-6, f"block {s}"
    total = partials.double().sum(0).cpu()
    want = x64 @ w64.T + b.double().cpu()
    assert (total - want).abs().max().item() <= 1e-5 * want.abs().max().item() + 1e-6


def test_split_fusion_and_norm_match_the_concatenated_projection(device):
    """The decode-step fusion layer as a split projection of its four fp32
    pieces plus the parts-summing norm (bf16 bias, bf16 rounding of the
    result) against float64: the projection of the bf16-rounded pieces plus
    the bf16 bias, rounded to bf16 (the autocast result), then the RMS norm.
    A rounding boundary may fall either way in fp32 accumulation, so an
    element may differ by one bf16 step of the pre-norm value (2^-8
    relative) and the norm by as much; the fp32 and bf16 outputs agree."""

    from koemi_amd import herm

    rows, d = 64, 1024
    g = torch.Generator().manual_seed(9)
    pieces = tuple(torch.randn((rows, 1, d), generator=g).to(device) for _ in range(4))
    p = {"fusion_w": (torch.randn((d, 4 * d), generator=g) * (4 * d) ** -0.5).to(torch.bfloat16).to(device),
         "fusion_b16": torch.randn((d,), generator=g).to(torch.bfloat16).to(device),
         "fusion_norm": (1.0 + 0.1 * torch.randn((d,), generator=g)).to(device)}
    assert herm._fusion_split_fits(p, pieces, d)
    out, out16 = herm._fusion_split(p, pieces, d)
    x64 = torch.cat([t.to(torch.bfloat16).double().cpu() for t in pieces], dim=-1).reshape(rows, 4 * d)
    y = (x64 @ p["fusion_w"].double().cpu().T + p["fusion_b16"].double().cpu()).to(torch.bfloat16).double()
    want = y * torch.rsqrt((y * y).mean(-1, keepdim=True) + herm._EPS) * p["fusion_norm"].double().cpu()
    got = out.reshape(rows, d).double().cpu()
    err = (got - want).abs()
    assert (err <= 2.0**-7 * want.abs() + 1e-5).all(), err.max().item()
    assert (err > 1e-5 + 1e-6 * want.abs()).float().mean().item() < 0.01  # rounding flips are rare
    assert torch.equal(out16, out.to(torch.bfloat16))


@pytest.mark.parametrize("rows, width, k, dtype", [(64, 1024, 1024, torch.bfloat16), (5, 40, 64, torch.float32),
                                                   (70, 96, 128, torch.bfloat16)])
def test_gated_linear_rows_equal_the_projection_then_the_gated_step(device, rows, width, k, dtype):
    """koemi_linear_rows_gated (a decode step's gate projections with the
    gates and the one-position scan in the epilogue) equals, bit for bit,
    koemi_linear_rows followed by the gated scan at length 1: the same sums
    in the same order, then the same gate arithmetic; invalid rows carry the
    state."""

    from koemi_amd import _native, recurrent

    g = torch.Generator().manual_seed(rows + width)
    u = torch.randn((rows, 1, k), generator=g).to(dtype).to(device)
    w = (torch.randn((2 * width, k), generator=g) * k ** -0.5).to(torch.bfloat16).to(device)
    bias = torch.randn((2 * width,), generator=g).to(device)
    h0 = torch.randn((rows, width), generator=g).to(device)
    valid = (torch.rand((rows, 1), generator=g) < 0.8).to(device)
    z = linear.linear_rows([u.reshape(rows, k)], w, None).reshape(rows, 1, 2 * width)
    want, want16 = recurrent.gated_scan(z, valid, h0, width=width, with_bf16=True, retention_bias=bias[:width],
                                        candidate_bias=bias[width:])
    got = torch.full((rows, 1, width), 7.0, device=device)
    wide16 = torch.zeros((rows, 1, width + 8), device=device, dtype=torch.bfloat16)
    _native.call("koemi_linear_rows_gated", _native.ptr(u), _native.dtype_code(dtype), _native.ptr(w),
                 _native.ptr(bias[:width]), _native.ptr(bias[width:]), _native.ptr(valid), _native.ptr(h0),
                 _native.ptr(got), _native.ptr(wide16), width + 8, rows, width, k, _native.stream_of(got.device))
    assert torch.equal(got, want)
    assert torch.equal(wide16[..., :width], want16) and not wide16[..., width:].any()
    assert torch.equal(got[~valid.reshape(-1)].reshape(-1, width), h0[~valid.reshape(-1)])
