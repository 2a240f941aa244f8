"""PyTorch-CPU restatement of one HERM block window: the CPU baseline of the
end-to-end configuration.

TEST INFRASTRUCTURE ONLY (see the package docstring): the CPU baseline leg of
bench.py and tests/ run it; nothing in the product imports it.

``block_window`` follows KoemiModel.forward_window (reference
model/network.py:296-441) with torch tensor operations on the host, in the
parameters' dtype (fp32 for the baseline, float64 in the parity tests), under
the default ``no_refine`` ablation and static rings (state.py:43-76):

* embedding + input normalizer (network.py:703-707; layers.py:14-16);
* gates, masking and the Hillis-Steele window scan (memory.py:22-26;
  network.py:306-310; scan.py:17-34);
* surprise from the content head, PAD column removed (network.py:677-698);
* local entries and the sliding-window read (memory.py:297-383);
* the associative memory's projection, write terms, masking and
  scan_and_read with its fp32 log-decay domain (memory.py:82-144, 244-255;
  network.py:734-740);
* admission, salient read and salient tail (network.py:349;
  memory.py:405-455);
* fusion (network.py:723-732); experts by the reference's sorted-segment
  dispatch (experts.py:171-216; hash routing, 1/k weights) or learned routing
  (router.py:43-97); the token head (network.py:700-701);
* local tail and last valid token (memory.py:385-403; network.py:742-761).

The expert mixture uses the segment dispatch, not the static one
(experts.py:109-150): both compute the same sums, but the static form gathers
a full copy of the expert weights for every (token, slot) pair, 17 GB per
projection at width 1024 and 2048 pairs, which no host can hold.

Pinned by tests/test_oracle_torch_block.py against the reference fixtures
(tests/golden/herm_block_*.npz) and against oracle.herm in float64.
"""

from __future__ import annotations

import math

import torch
from torch.nn import functional

PAD = 256
EPS = 1e-6
HASH_TOKEN, HASH_PREVIOUS, HASH_MIX, SLOT_OFFSET = 1_000_003, 97_409, 0x45D9F3B, 0x9E3779B9


def rms(x, weight):
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + EPS) * weight


def window_scan(retention, increment, initial):
    """Hillis-Steele over the window (scan.py:17-30), then the carried state."""

    coef, val, offset, n = retention, increment, 1, retention.shape[1]
    while offset < n:
        shifted_coef = torch.cat((torch.ones_like(coef[:, :offset]), coef[:, : n - offset]), dim=1)
        shifted_val = torch.cat((torch.zeros_like(val[:, :offset]), val[:, : n - offset]), dim=1)
        val = coef * shifted_val + val
        coef = coef * shifted_coef
        offset *= 2
    return coef * initial.unsqueeze(1) + val


def content_hash(tokens, previous):
    v = (tokens * HASH_TOKEN + previous * HASH_PREVIOUS) & 0xFFFFFFFF
    v = ((v ^ (v >> 16)) * HASH_MIX) & 0xFFFFFFFF
    v = ((v ^ (v >> 16)) * HASH_MIX) & 0xFFFFFFFF
    return v ^ (v >> 16)


def previous_tokens(ids, valid, carried):
    """network.py:742-750 as a running maximum of valid positions."""

    length = ids.shape[1]
    positions = torch.arange(length).expand_as(ids)
    marked = torch.where(valid, positions, torch.full_like(positions, -1))
    latest = torch.cummax(marked, dim=1).values
    before = torch.cat((torch.full_like(latest[:, :1], -1), latest[:, :-1]), dim=1)
    gathered = ids.gather(1, before.clamp_min(0))
    previous = torch.where(before >= 0, gathered, carried.unsqueeze(1).expand_as(ids))
    last_pos = latest[:, -1]
    last = torch.where(last_pos >= 0, ids.gather(1, last_pos.clamp_min(0).unsqueeze(1)).squeeze(1), carried)
    return previous, last


def ffn(p, e, x):
    gate = functional.linear(x, p["gate_w"][e], p["gate_b"][e])
    up = functional.linear(x, p["up_w"][e], p["up_b"][e])
    return functional.linear(functional.silu(gate) * up, p["down_w"][e], p["down_b"][e])


def experts(p, cfg, context, ids, previous, valid):
    """Returns (mixed context, assignments [B, L, k])."""

    k, count = cfg["top_k"], cfg["expert_count"]
    flat = context.reshape(-1, context.shape[-1])
    rows_valid = valid.reshape(-1)
    pair_rows = torch.arange(flat.shape[0]).repeat_interleave(k)
    if cfg.get("expert_routing", "hash") == "learned":
        gate_context = context.masked_fill(~valid.unsqueeze(-1), 0)
        probabilities = functional.linear(gate_context, p["router_w"]).float().softmax(dim=-1)
        weights, assignments = probabilities.topk(k, dim=-1)
        assignments = assignments.masked_fill(~valid.unsqueeze(-1), -1)
        pair_weight = weights.masked_fill(~valid.unsqueeze(-1), 0).reshape(-1).to(flat.dtype)
        pair_ok = assignments.reshape(-1) >= 0
    else:
        h = content_hash(ids, previous)
        assignments = (h.unsqueeze(-1) + torch.arange(k) * SLOT_OFFSET).remainder(count)
        assignments = assignments.masked_fill(~valid.unsqueeze(-1), -1)
        flat_a = assignments.reshape(-1, k)
        first = ~((flat_a.unsqueeze(-1) == flat_a.unsqueeze(-2))
                  & (torch.arange(k).unsqueeze(0) < torch.arange(k).unsqueeze(1))).any(dim=-1)
        pair_ok = (flat_a >= 0).reshape(-1) & first.reshape(-1) & rows_valid.repeat_interleave(k)
        pair_weight = torch.full((pair_ok.numel(),), 1.0 / k, dtype=flat.dtype)
    keys = torch.where(pair_ok, assignments.reshape(-1), torch.full_like(pair_rows, count))
    order = torch.argsort(keys, stable=True)
    sizes = torch.bincount(keys, minlength=count + 1)[:count].tolist()
    rows = pair_rows[order]
    sorted_context = flat.index_select(0, rows)
    sorted_weight = pair_weight[order]
    update = torch.zeros_like(flat)
    offset = 0
    for e, size in enumerate(sizes):
        if size:
            end = offset + size
            y = ffn(p, e, sorted_context[offset:end]) * sorted_weight[offset:end, None]
            update.index_add_(0, rows[offset:end], y)
            offset = end
    mixed = rms(flat + update, p["expert_norm"])
    return torch.where(rows_valid.unsqueeze(-1), mixed, flat).reshape_as(context), assignments


def block_window(p, state, ids, cfg, context=None):
    """One forward_window; ``p``/``state`` as oracle.herm (torch tensors),
    ``ids`` int64 [B, L]. Returns (logits, final_context, next_state,
    surprise, admission, assignments)."""

    batch, length = ids.shape
    width = p["input_norm"].shape[0]
    valid = ids != PAD
    keep = valid.unsqueeze(-1)
    source = functional.embedding(ids, p["embedding"]) if context is None else context
    u = rms(source, p["input_norm"])
    lo, hi = 2.0**-8, 1.0 - 2.0**-8
    retention = lo + (hi - lo) * torch.sigmoid(functional.linear(u, p["retention_w"], p["retention_b"]))
    increment = (1.0 - retention) * torch.tanh(functional.linear(u, p["candidate_w"], p["candidate_b"]))
    retention = torch.where(keep, retention, torch.ones_like(retention))
    increment = torch.where(keep, increment, torch.zeros_like(increment))
    ws = window_scan(retention, increment, state["working"])
    prior = torch.cat((state["working"].unsqueeze(1), ws[:, :-1]), dim=1)

    content = functional.linear(prior, p["head_w"][:PAD], p["head_b"][:PAD])
    targets = torch.where(valid, ids, torch.zeros_like(ids))
    nll = functional.cross_entropy(content.reshape(-1, PAD), targets.reshape(-1), reduction="none").view(batch, length)
    surprise = torch.where(valid, 1.0 - torch.exp(-nll / math.log(PAD)), torch.zeros_like(nll))

    local_keys = torch.where(keep, functional.linear(ws, p["local_key_w"], p["local_key_b"]), 0.0)
    local_values = torch.where(keep, functional.linear(ws, p["local_value_w"], p["local_value_b"]), 0.0)
    window = cfg["local_memory_size"]
    carried = state["local_keys"].shape[1]
    all_keys = torch.cat((state["local_keys"], local_keys), dim=1)
    all_values = torch.cat((state["local_values"], local_values), dim=1)
    all_valid = torch.cat((state["local_valid"], valid), dim=1)
    own = carried + torch.arange(length).unsqueeze(1)
    src = torch.arange(all_valid.shape[1]).unsqueeze(0)
    eligible = ((src < own) & (src >= own - window)).unsqueeze(0) & all_valid.unsqueeze(1)
    local_value = masked_attention(all_keys, all_values, ws, eligible)

    key = functional.linear(ws, p["key_w"], p["key_b"])
    features = torch.softmax(functional.linear(key, p["feature_w"], p["feature_b"]), dim=-1)
    value = torch.tanh(functional.linear(ws, p["value_w"], p["value_b"]))
    min_decay, max_decay = 2.0**-12, 1.0 - 2.0**-12
    decay = min_decay + (max_decay - min_decay) * torch.sigmoid(functional.linear(ws, p["decay_w"], p["decay_b"]))
    decay = torch.where(keep, decay, torch.ones_like(decay)).squeeze(-1)
    write = torch.sigmoid(functional.linear(ws, p["write_w"], p["write_b"])).squeeze(-1)
    write = write * (0.25 + 0.75 * surprise.clamp(0.0, 1.0))
    write = torch.where(valid, write, torch.zeros_like(write))
    query = torch.softmax(functional.linear(functional.linear(ws, p["query_w"], p["query_b"]), p["feature_w"],
                                            p["feature_b"]), dim=-1)
    fast, basis, normalizer = scan_and_read(state["basis"], state["normalizer"], decay, value, features, write, query)

    admission = valid & (surprise > cfg["salience_threshold"])
    s_carried = state["salient_keys"].shape[1]
    positions = torch.arange(length)
    earlier = positions.unsqueeze(1) > positions.unsqueeze(0)
    s_eligible = torch.cat((state["salient_valid"].unsqueeze(1).expand(batch, length, s_carried),
                            admission.unsqueeze(1) & earlier.unsqueeze(0)), dim=-1)
    salient_value = masked_attention(torch.cat((state["salient_keys"], local_keys), dim=1),
                                     torch.cat((state["salient_values"], local_values), dim=1), ws, s_eligible)

    fused = rms(functional.linear(torch.cat((ws, fast, local_value, salient_value), dim=-1), p["fusion_w"],
                                  p["fusion_b"]), p["fusion_norm"])
    previous, last = previous_tokens(ids, valid, state["last_token"])
    final, assignments = experts(p, cfg, fused, ids, previous, valid)
    logits = functional.linear(final, p["head_w"], p["head_b"])

    capacity = cfg["salience_memory_size"]
    s_all_k = torch.cat((state["salient_keys"], local_keys), dim=1)
    s_all_v = torch.cat((state["salient_values"], local_values), dim=1)
    s_all_ok = torch.cat((state["salient_valid"], admission), dim=1)
    temporal = torch.arange(s_all_ok.shape[1]).expand_as(s_all_ok)
    ranked = torch.where(s_all_ok, temporal, torch.full_like(temporal, -1))
    chosen = ranked.topk(capacity, dim=1).indices.sort(dim=1).values
    chosen_ok = s_all_ok.gather(1, chosen)
    gather = chosen.unsqueeze(-1).expand(-1, -1, s_all_k.shape[-1])
    zero_bad = lambda t: torch.where(chosen_ok.unsqueeze(-1), t, torch.zeros_like(t))
    next_state = {
        "working": ws[:, -1],
        "basis": basis,
        "normalizer": normalizer,
        "local_keys": all_keys[:, -window:],
        "local_values": all_values[:, -window:],
        "local_valid": all_valid[:, -window:],
        "salient_keys": zero_bad(s_all_k.gather(1, gather)),
        "salient_values": zero_bad(s_all_v.gather(1, gather)),
        "salient_valid": chosen_ok,
        "last_token": last,
    }
    return logits, final, next_state, surprise, admission, assignments


def masked_attention(keys, values, queries, eligible):
    """softmax(K q / sqrt(d)) over eligible slots, zero rows where none is
    (memory.py:355-367, 418-429)."""

    scores = torch.einsum("bsd,btd->bts", keys, queries) / math.sqrt(queries.shape[-1])
    weights = torch.softmax(scores.masked_fill(~eligible, float("-inf")), dim=-1)
    weights = torch.where(eligible.any(dim=-1, keepdim=True), weights, torch.zeros_like(weights))
    return torch.einsum("bts,bsd->btd", weights, values)


def scan_and_read(basis, normalizer, decay, value, features, write, query):
    """memory.py:97-144 with the fp32 log-decay domain."""

    log_decay = torch.log(decay.float())
    cumulative = torch.cumsum(log_decay, dim=1)
    prior = cumulative - log_decay
    initial = torch.exp(prior).to(value.dtype)
    length = value.shape[1]
    positions = torch.arange(length)
    past = positions.unsqueeze(1) > positions.unsqueeze(0)
    pair = torch.exp((prior.unsqueeze(-1) - cumulative.unsqueeze(1)).masked_fill(~past, float("-inf"))).to(value.dtype)
    influence = pair * torch.einsum("bsm,btm->bts", features, query) * write.unsqueeze(1)
    numerator = initial.unsqueeze(-1) * torch.einsum("bdm,btm->btd", basis, query)
    numerator = numerator + torch.einsum("bts,bsd->btd", influence, value)
    denominator = (initial * torch.einsum("bm,btm->bt", normalizer, query) + influence.sum(dim=-1)).unsqueeze(-1)
    regularized = denominator + 2.0**-8
    read = (denominator / regularized) * numerator / regularized
    total = cumulative[:, -1]
    total_factor = torch.exp(total).to(value.dtype)
    final_weight = torch.exp(total.unsqueeze(1) - cumulative).to(value.dtype) * write
    next_basis = total_factor[:, None, None] * basis + torch.einsum("bs,bsd,bsm->bdm", final_weight, value, features)
    next_normalizer = total_factor[:, None] * normalizer + torch.einsum("bs,bsm->bm", final_weight, features)
    return read, next_basis, next_normalizer
