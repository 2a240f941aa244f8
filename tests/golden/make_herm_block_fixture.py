#!/usr/bin/env python3
"""Write the HERM block fixtures: the reference KoemiModel.forward_window at toy size.

Run in the CPU container only, where the reference tree is mounted:

    PYTHONPATH=/root/reference/src python tests/golden/make_herm_block_fixture.py

It imports the reference's model package (torch + numpy only), builds a
single-block ``KoemiModel`` (width 16, 4 memory features, 4 experts, top-2,
local ring 4, salient ring 3, ablation ``no_refine``) in float64, scales the
token head by 8 so that surprise spreads around the admission threshold, and
runs three windows from ``KoemiState.create_static``: 11 tokens, 11 more
(state carried, both with padding inside), then one decode position. The
weights, ids and every output (logits, surprise, admission, expert
assignments, each next state field and, for learned routing, the window's
RouterStatistics with its balance loss) go to ``herm_block_<routing>.npz`` beside
this script: with hash routing, with learned routing, and with hash routing
under the ``herm`` ablation (the refine memory, its gate and the local read's
novelty; ``herm_block_refine.npz``). Only data
is written; nothing from the reference is copied. The GPU box never runs this.

Reference: model/network.py:296-441 (forward_window), state.py:43-76
(create_static), experts.py:109-150 (static dispatch), router.py:43-97
(learned routing).
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
SEED = 20261202
HEAD_SCALE = 8.0
WINDOWS = (11, 11, 1)
BATCH = 2


def _ids(rng: np.random.Generator, length: int, pad: int) -> np.ndarray:
    ids = rng.integers(0, 256, (BATCH, length))
    if length > 1:
        ids[0, 3] = pad          # padding inside a row
        ids[1, -2:] = pad        # padding at the end of a row
    return ids


def make(routing: str, ablation: str = "no_refine") -> dict[str, np.ndarray]:
    from koemi.configuration.settings import PAD_TOKEN_ID, ModelSettings
    from koemi.model.network import KoemiModel
    from koemi.model.state import KOEMI_STATE_FIELDS, KoemiState

    settings = ModelSettings(embedding_size=16, memory_features=4, local_memory_size=4, salience_memory_size=3,
                             salience_threshold=0.6, expert_count=4, expert_top_k=2, scan_chunk=11,
                             ablation=ablation, expert_routing=routing)
    torch.manual_seed(SEED)
    model = KoemiModel(settings).double().eval()
    with torch.no_grad():
        model.token_predictor.weight.mul_(HEAD_SCALE)
        model.token_predictor.bias.mul_(HEAD_SCALE)
    state = KoemiState.create_static(BATCH, 16, 4, 4, 3, torch.device("cpu"), torch.float64)
    out: dict[str, np.ndarray] = {f"param.{k}": v.detach().numpy().copy() for k, v in model.state_dict().items()}
    out["settings.salience_threshold"] = np.array(settings.salience_threshold)
    out["settings.windows"] = np.array(WINDOWS)
    rng = np.random.default_rng(SEED)
    for w, length in enumerate(WINDOWS):
        ids = _ids(rng, length, PAD_TOKEN_ID)
        for field in KOEMI_STATE_FIELDS:
            out[f"w{w}.state_in.{field}"] = getattr(state, field).detach().numpy().copy()
        with torch.no_grad():
            result = model.forward_window(torch.from_numpy(ids), state, None)
        out[f"w{w}.ids"] = ids
        out[f"w{w}.logits"] = result.logits.numpy()
        out[f"w{w}.surprise"] = result.surprise_values.numpy()
        out[f"w{w}.admission"] = (result.valid_positions & (result.surprise_values > settings.salience_threshold)).numpy()
        out[f"w{w}.assignments"] = (result.active_expert_indices if result.active_expert_indices is not None
                                    else result.expert_indices.unsqueeze(-1)).numpy()
        for field in KOEMI_STATE_FIELDS:
            out[f"w{w}.state_out.{field}"] = getattr(result.state, field).detach().numpy().copy()
        stats = result.router_statistics
        if stats is not None:  # learned routing: RouterStatistics of the window (router.py:50-58)
            out[f"w{w}.router.probability_mass"] = stats.probability_mass.detach().numpy().copy()
            out[f"w{w}.router.assignment_counts"] = stats.assignment_counts.detach().numpy().copy()
            out[f"w{w}.router.valid_count"] = stats.valid_count.detach().numpy().copy()
            out[f"w{w}.router.balance_loss"] = stats.balance_loss.detach().numpy().copy()
        state = result.state
    return out


def main() -> int:
    src = os.environ.get("KOEMI_REFERENCE_SRC", "/root/reference/src")
    if src not in sys.path:
        sys.path.insert(0, src)
    torch.set_num_threads(1)
    for name, routing, ablation in (("hash", "hash", "no_refine"), ("learned", "learned", "no_refine"),
                                    ("refine", "hash", "herm")):
        data = make(routing, ablation)
        path = HERE / f"herm_block_{name}.npz"
        np.savez_compressed(path, **data)
        print(f"wrote {path} ({path.stat().st_size} bytes, {len(data)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
