"""GPU parity of the affine scan (dense_affine_scan / cuda_affine_scan).

Tolerances: fp32 atol = rtol = 1e-5 against the fp32 sequential recurrence
(tests/cuda/test_dense_cuda.py:78), f16/bf16 5e-3 (test_dense_cuda.py:110),
first-order gradients 2e-5 (test_dense_cuda.py:147); float64 1e-12. The full
C1 and C3 configurations are compared element by element with the C oracle and
the max abs / rel errors are printed.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from koemi_amd import cuda_scan, workloads
from koemi_amd.dense import dense_affine_scan

pytestmark = pytest.mark.gpu
GOLDEN = json.loads((Path(__file__).parent / "golden" / "kats.json").read_text())


def sequential_torch(retention, increment, initial):
    state, states = initial, []
    for t in range(increment.shape[1]):
        state = retention[:, t] * state + increment[:, t]
        states.append(state)
    return torch.stack(states, dim=1)


def report(name, got, want):
    got64, want64 = np.asarray(got, dtype=np.float64), np.asarray(want, dtype=np.float64)
    abs_err = np.abs(got64 - want64)
    rel_err = abs_err / np.maximum(np.abs(want64), 1e-30)
    print(f"{name}: max_abs={abs_err.max():.3e} max_rel={rel_err.max():.3e} (n={want64.size})", flush=True)
    return abs_err.max()


def test_exact_retention_forward(device):
    torch.manual_seed(101)
    r = torch.rand((2, 37, 64)) * 0.9 + 0.05
    i = torch.randn((2, 37, 64))
    h0 = torch.randn((2, 64))
    got = dense_affine_scan(r.to(device), i.to(device), h0.to(device)).cpu()
    want = oracle.scan_sequential(r.numpy(), i.numpy(), h0.numpy())
    torch.testing.assert_close(got, torch.from_numpy(want), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("r_shape,i_shape", [((2, 29, 1, 1), (2, 29, 4, 8)), ((2, 17, 1, 3), (2, 17, 4, 3)), ((3, 100, 1), (3, 100, 70))])
def test_broadcast_retention_forward(device, r_shape, i_shape):
    torch.manual_seed(102)
    r = torch.rand(r_shape) * 0.9 + 0.05
    i = torch.randn(i_shape)
    h0 = torch.randn((i_shape[0],) + i_shape[2:])
    got = dense_affine_scan(r.to(device), i.to(device), h0.to(device)).cpu()
    want = sequential_torch(r.double(), i.double(), h0.double()).float()
    torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_low_precision_forward(device, dtype):
    torch.manual_seed(104)
    r = (torch.rand((1, 13, 32)) * 0.8 + 0.1).to(dtype)
    i = torch.randn((1, 13, 32)).to(dtype)
    h0 = torch.randn((1, 32)).to(dtype)
    got = dense_affine_scan(r.to(device), i.to(device), h0.to(device)).cpu().float()
    want = sequential_torch(r.float(), i.float(), h0.float())
    torch.testing.assert_close(got, want, atol=5e-3, rtol=5e-3)


def test_float64_matches_the_oracle(device):
    rng = np.random.default_rng(7)
    r = rng.uniform(0.05, 0.99, (3, 300, 130))
    i = rng.standard_normal((3, 300, 130))
    h0 = rng.standard_normal((3, 130))
    got = dense_affine_scan(*(torch.from_numpy(x).to(device) for x in (r, i, h0))).cpu().numpy()
    np.testing.assert_allclose(got, oracle.scan_sequential(r, i, h0), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("broadcast", [True, False])
def test_forward_and_first_order_gradients(device, broadcast):
    torch.manual_seed(105)
    r_shape = (2, 19, 1, 1) if broadcast else (2, 19, 4, 8)
    rv = torch.rand(r_shape) * 0.8 + 0.1
    iv = torch.randn((2, 19, 4, 8))
    hv = torch.randn((2, 4, 8))
    up = torch.randn_like(iv)
    leaves = [t.to(device).requires_grad_() for t in (rv, iv, hv)]
    states = dense_affine_scan(*leaves)
    states.backward(up.to(device))
    ref_leaves = [t.double().requires_grad_() for t in (rv, iv, hv)]
    ref = sequential_torch(*ref_leaves)
    ref.backward(up.double())
    torch.testing.assert_close(states.detach().cpu(), ref.detach().float(), atol=1e-5, rtol=1e-5)
    for got, want in zip(leaves, ref_leaves):
        assert got.grad.shape == want.grad.shape
        torch.testing.assert_close(got.grad.cpu(), want.grad.float(), atol=2e-5, rtol=2e-5)


def test_closed_forms_are_exact(device):
    torch.manual_seed(9)
    b = torch.randn((2, 200, 96), device=device)
    h0 = torch.randn((2, 96), device=device)
    assert torch.equal(dense_affine_scan(torch.zeros_like(b), b, h0), b)
    assert torch.equal(dense_affine_scan(torch.ones_like(b), torch.zeros_like(b), h0), h0.unsqueeze(1).expand_as(b))


def test_cuda_scan_chunk_known_answer_and_diagnostics(device):
    kat = GOLDEN["scan_chunk_count"]
    shape = tuple(kat["shape"])
    r = torch.full(shape, kat["retention"], device=device)
    i = torch.full(shape, kat["increment"], device=device)
    h0 = torch.zeros((shape[0], shape[2]), device=device)
    diag = cuda_scan.diagnose_cuda_affine_scan(r, i, h0, chunk_size=kat["chunk_size"])
    assert diag.token_count == kat["token_count"] and diag.chunk_count == kat["chunk_count"]
    t = torch.arange(1, shape[1] + 1, dtype=torch.float64)
    closed = (1 - kat["retention"] ** t) / (1 - kat["retention"])
    torch.testing.assert_close(diag.states[0, :, 0].cpu().double(), closed, atol=1e-6, rtol=1e-6)
    empty = cuda_scan.cuda_affine_scan(torch.empty((2, 0, 4), device=device), torch.empty((2, 0, 4), device=device), chunk_size=3)
    assert tuple(empty.shape) == (2, 0, 4)
    for chunk in (1, 5, 64, None):
        got = cuda_scan.cuda_affine_scan(r, i, h0, chunk_size=chunk)
        torch.testing.assert_close(got, diag.states)


def test_config1_full_against_the_oracle(device):
    c = workloads.config1()
    got = dense_affine_scan(c.retention.to(device), c.increment.to(device), c.initial.to(device)).cpu().numpy()
    want = oracle.scan_sequential(c.retention.numpy(), c.increment.numpy(), c.initial.numpy())
    report("C1 scan fp32 vs sequential fp32", got, want)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)


def test_config3_full_against_the_oracle(device):
    c = workloads.config3()
    got = dense_affine_scan(c.retention.to(device), c.increment.to(device), c.initial.to(device)).cpu().numpy()
    want = oracle.scan_sequential(c.retention.numpy(), c.increment.numpy(), c.initial.numpy())
    report("C3 scan fp32 vs sequential fp32", got, want)
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-5)
    # chunk 64 through the model-path seam gives the same states
    chunked = cuda_scan.cuda_affine_scan(c.retention[:2].to(device), c.increment[:2].to(device), chunk_size=c.chunk)
    np.testing.assert_array_equal(chunked.cpu().numpy(), got[:2])
