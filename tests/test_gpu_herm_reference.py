"""The GPU HERM block (koemi_amd.herm.block_window) on the reference's own
forward_window fixtures (tests/golden/herm_block_{hash,learned,refine}.npz:
the reference KoemiModel at toy size in float64, three windows with the state
carried, padding and admissions, the third under the herm ablation with the
refine memory; written in the CPU container by
tests/golden/make_herm_block_fixture.py).

The reference weights go through koemi_amd.checkpoint (the state-dict /
KoemiState layout map) into prepare_stack with fp32 projections; each window
starts from the reference's own incoming state. Tolerances: logits, states and
surprise within 1e-4 of each output's largest magnitude (fp32 arithmetic
against float64); admission (through the salient ring bits), ring valid bits
and last tokens exact (every fixture score is >= 1.5e-3 from the threshold).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from koemi_amd import checkpoint, herm

from test_oracle_reference_block import FIELDS, close, load

pytestmark = pytest.mark.gpu


def _settings(routing: str) -> herm.HermSettings:
    """``routing``: the fixture ("hash", "learned", or "refine": hash routing
    under the herm ablation)."""
    return herm.HermSettings(width=16, memory_features=4, local_memory_size=4, salience_memory_size=3,
                             salience_threshold=0.6, expert_count=4, top_k=2, layers=1, scan_chunk=11,
                             linear_dtype=torch.float32, expert_routing="learned" if routing == "learned" else "hash",
                             ablation="herm" if routing == "refine" else "no_refine")


@pytest.mark.parametrize("routing", ["hash", "learned", "refine"])
def test_gpu_block_window_matches_reference_fixture(device, routing):
    data = load(routing)
    settings = _settings(routing)
    refine = settings.refine
    model_state = {k[len("param."):]: torch.from_numpy(v).float() for k, v in data.items() if k.startswith("param.")}
    params = herm.prepare_stack([checkpoint.block_parameters(model_state, 4)], settings, device)
    for w in range(3):
        fields = {n: torch.from_numpy(data[f"w{w}.state_in.{n}"]) for n in FIELDS}
        state = {k: (v.float() if v.is_floating_point() else v).to(device).contiguous()
                 for k, v in checkpoint.state_from_fields(fields, refine=refine).items()}
        ids = torch.from_numpy(data[f"w{w}.ids"]).to(device)
        routing_out: dict = {}
        logits, _, nxt, surprise = herm.block_window(params[0], settings, ids, state, routing=routing_out)
        torch.cuda.synchronize()
        close(logits.cpu().numpy(), data[f"w{w}.logits"], 1e-4)
        if routing == "learned":
            # the window's RouterStatistics (router.py:50-58): fp32 sums over fp32
            # probabilities; counts and the valid count exact
            (stats,) = routing_out["statistics"]
            close(stats.probability_mass.cpu().numpy(), data[f"w{w}.router.probability_mass"], 1e-4)
            np.testing.assert_array_equal(stats.assignment_counts.cpu().numpy(),
                                          data[f"w{w}.router.assignment_counts"])
            assert float(stats.valid_count) == float(data[f"w{w}.router.valid_count"])
            close(stats.balance_loss.cpu().numpy(), data[f"w{w}.router.balance_loss"], 1e-4)
        else:
            assert "statistics" not in routing_out
        close(surprise.cpu().numpy(), data[f"w{w}.surprise"], 1e-4)
        want = checkpoint.state_from_fields({n: data[f"w{w}.state_out.{n}"] for n in FIELDS}, refine=refine)
        for key, value in want.items():
            value = np.asarray(value)
            got = nxt[key].cpu().numpy()
            if value.dtype.kind in "bi":
                np.testing.assert_array_equal(got, value, err_msg=f"{routing} window {w} {key}")
            else:
                close(got, value, 1e-4)
