"""The PyTorch-CPU block restatement (oracle/herm_torch.py, the CPU baseline of
the end-to-end configuration) against the reference fixtures and oracle.herm.

Float64 throughout. Against the reference's forward_window fixtures
(tests/golden/herm_block_*.npz) the restatement runs the same torch fp32
log-decay domain, so the memory-fed outputs agree to 1e-9 of their scale and
everything else to 1e-12; routing, admission and ring bits are exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import herm, herm_torch

from test_oracle_reference_block import FIELDS, cfg_of, checkpoint, close, load, params_of, state_in


def _t(d: dict) -> dict:
    return {k: torch.from_numpy(np.asarray(v)) for k, v in d.items()}


@pytest.mark.parametrize("routing", ["hash", "learned"])
def test_torch_block_matches_reference_fixture(routing):
    data = load(routing)
    p = _t(params_of(data))
    cfg = cfg_of(data, routing)
    for w in range(3):
        state = _t(state_in(data, w))
        logits, _, nxt, surprise, admission, assign = herm_torch.block_window(p, state, torch.from_numpy(
            data[f"w{w}.ids"]), cfg)
        close(logits.numpy(), data[f"w{w}.logits"], 1e-9)
        close(surprise.numpy(), data[f"w{w}.surprise"], 1e-12)
        np.testing.assert_array_equal(admission.numpy(), data[f"w{w}.admission"])
        np.testing.assert_array_equal(assign.numpy(), data[f"w{w}.assignments"])
        want = checkpoint.state_from_fields({n: data[f"w{w}.state_out.{n}"] for n in FIELDS})
        for key, value in want.items():
            value = np.asarray(value)
            got = nxt[key].numpy()
            if value.dtype.kind in "bi":
                np.testing.assert_array_equal(got, value, err_msg=f"window {w} {key}")
            else:
                close(got, value, 1e-9 if key in ("basis", "normalizer") else 1e-12)


def test_torch_block_matches_numpy_oracle_on_a_longer_window():
    """Width 32, 8 features, 4 experts, a 40-token window with padding: the
    torch restatement and oracle.herm (both float64, fp32 log domain)."""

    rng = np.random.default_rng(11)
    d, m, e = 32, 8, 4
    import test_oracle_herm as toh

    p = toh._params(rng, 1, d, m, e)[0]
    cfg = dict(width=d, memory_features=m, local_memory_size=6, salience_memory_size=5, salience_threshold=0.55,
               expert_count=e, top_k=2)
    state = herm.initial_state(3, cfg)
    ids = rng.integers(0, 256, (3, 40))
    ids[0, 7] = oracle.PAD_TOKEN_ID
    ids[2, -5:] = oracle.PAD_TOKEN_ID
    want = herm.block_window(p, state, ids, cfg, return_assignments=True)
    got = herm_torch.block_window(_t(p), _t(state), torch.from_numpy(ids), cfg)
    for w_item, g_item in zip(want[:2], got[:2]):
        close(g_item.numpy(), w_item, 1e-8)
    close(got[3].numpy(), want[3], 1e-12)
    np.testing.assert_array_equal(got[4].numpy(), want[4])
    np.testing.assert_array_equal(got[5].numpy(), want[5])
    assert want[4].any() and not want[4].all()
