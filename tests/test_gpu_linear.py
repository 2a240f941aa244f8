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
