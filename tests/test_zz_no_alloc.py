"""The allocation-free quantile admission (koemi_admission_quantile_noalloc)
against the workspace entry point (koemi_admission_quantile), through the C ABI.

The no-alloc variant keeps the partitioned select's records and candidate
slots in a static device array; its results must be bit-identical to the
existing entry point's (mask bytes and tau) and to the oracle's, on calls in a
row that reuse the array, the later ones smaller (1024-thread partition,
256-thread partition, single workgroup), and the first call on the device
resolves the array's address.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from koemi_amd import _native

pytestmark = pytest.mark.gpu


def _run(name: str, scores: torch.Tensor, valid: torch.Tensor, q: float) -> tuple[np.ndarray, float]:
    count = scores.numel()
    mask = torch.full((count,), 7, dtype=torch.uint8, device=scores.device)
    tau = torch.full((1,), float("nan"), dtype=torch.float32, device=scores.device)
    stream = _native.stream_of(scores.device)
    if name == "koemi_admission_quantile":
        nbytes = _native.query("koemi_admission_quantile_workspace_bytes", count)
        workspace = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=scores.device)
        _native.call(name, scores.data_ptr(), valid.data_ptr(), mask.data_ptr(), tau.data_ptr(), count, q,
                     workspace.data_ptr(), nbytes, stream)
    else:
        _native.call(name, scores.data_ptr(), valid.data_ptr(), mask.data_ptr(), tau.data_ptr(), count, q, stream)
    torch.cuda.synchronize()
    return mask.cpu().numpy().astype(bool), float(tau.item())


def test_noalloc_quantile_admission_matches_the_workspace_entry_point(device):
    rng = np.random.default_rng(2026)
    # three calls in a row on the shared static array, each smaller than the last
    for count, q in ((120_000, 0.9), (20_001, 0.25), (5_000, 0.9)):
        scores_np = rng.normal(0.63, 0.05, count).astype(np.float32)
        valid_np = rng.random(count) > 0.2
        scores = torch.from_numpy(scores_np).to(device)
        valid = torch.from_numpy(valid_np).to(device)
        want_mask, want_tau = _run("koemi_admission_quantile", scores, valid, q)
        got_mask, got_tau = _run("koemi_admission_quantile_noalloc", scores, valid, q)
        assert got_tau == want_tau, (count, got_tau, want_tau)
        np.testing.assert_array_equal(got_mask, want_mask)
        oracle_mask, oracle_tau = oracle.admission(scores_np, valid_np, q=q)
        assert got_tau == oracle_tau
        np.testing.assert_array_equal(got_mask, oracle_mask)
        print(f"no-alloc admission n={count} q={q}: tau={got_tau:.9g} admitted={int(got_mask.sum())}", flush=True)


def test_noalloc_quantile_admission_rejects_bad_arguments(device):
    scores = torch.zeros(16, device=device)
    valid = torch.ones(16, dtype=torch.bool, device=device)
    out = torch.empty(16, dtype=torch.uint8, device=device)
    tau = torch.empty(1, device=device)
    lib = _native.load_library()
    stream = _native.stream_of(device)
    status = lib.koemi_admission_quantile_noalloc(scores.data_ptr(), valid.data_ptr(), out.data_ptr(), tau.data_ptr(),
                                                  0, 0.5, stream)
    assert status == _native.ERR_INVALID
    assert b"at least one score" in lib.koemi_last_error()
