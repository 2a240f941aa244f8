"""Salient-memory ring update (model/memory.py:431-455) on the GPU against the oracle, bit for bit."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from koemi_amd import memory

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
