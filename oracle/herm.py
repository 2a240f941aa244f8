"""CPU oracle of one HERM block window and of the block stack, in float64.

TEST INFRASTRUCTURE ONLY (see the package docstring): imported by tests/ and
nowhere in the product.

Restates KoemiModel.forward_window (reference model/network.py:296-441) under
the ablation it runs by default ("no_refine": memory_value is the fast
associative read) or, with ``cfg["ablation"] == "herm"``, with the refine
memory (memory.py:257-268 refine write terms from the reconstruction error
and the local read's novelty, a second scan_and_read over the refine state,
the refine gate of network.py:714-721), with hash expert routing (the static dispatch of
experts.py:109-150) or learned routing (router.py:43-97), from the
reference's own formulas:

* embed + input normalizer (network.py:703-707, layers.py:8-16);
* gates, masking and scan (memory.py:22-26; network.py:306-310; scan.py);
* previous states and surprise (scan.py:33-34; network.py:677-698);
* local entries and the local read (memory.py:297-383);
* associative projection, fast write terms, masking and scan_and_read
  (memory.py:82-144, 244-255; network.py:734-740);
* admission, salient read and salient tail (network.py:349; memory.py:405-455);
* fusion (network.py:723-732), experts (experts.py:109-150, 283-289;
  layers.py:19-29), token head (network.py:700-701);
* local tail and last valid token (memory.py:385-403; network.py:751-761).

The block stack is this repository's composition for the 12-layer
configuration (the reference model is one block): layer 0 embeds the token ids,
layer l > 0 takes layer l - 1's final context in place of the embedding (its
own input normalizer applied), every layer keeps its own state and uses the
token ids for validity, routing and surprise targets; the last layer's head
gives the logits.

Pinned against the reference itself by tests/test_oracle_reference_block.py:
the reference KoemiModel.forward_window at toy size in float64 (hash and
learned routing, three windows with the state carried, padding, admissions;
fixtures tests/golden/herm_block_*.npz). Pinned beyond that by
tests/test_oracle_herm.py: the associative scan-and-read against the
sequential read/update recurrence (memory.py:91-95, 279-288), the local read
against the per-position ring read (oracle.read_local_sequential), window-cut
independence of the stack, and the reused oracle functions' own pins.

``cfg`` keys: the HermSettings names (width, memory_features,
local_memory_size, salience_memory_size, salience_threshold, expert_count,
top_k), optionally ``expert_routing`` ("hash" or "learned"; learned needs the
layer's ``router_w``), ``ablation`` ("no_refine" or "herm"; herm needs the
layer's ``refine_gate_w`` [1, 4 width] and ``refine_gate_b`` [1], the state's
``refine_basis`` and ``refine_normalizer``, and ``refine_decay_rate``) and
``memory_log_dtype`` (fp32 by default, as the
reference forms the memory's log-decays; float64 for exact-arithmetic checks).
"""

from __future__ import annotations

import math

import numpy as np

import oracle

PAD = oracle.PAD_TOKEN_ID
EPS = 1e-6                  # RootMeanSquareNorm default epsilon (layers.py:9)
MIN_DECAY = 2.0**-12        # memory.py:74-75
MAX_DECAY = 1.0 - 2.0**-12
MAX_REFINE_DECAY = 1.0 - 2.0**-16   # memory.py:79
READ_EPSILON = 2.0**-8      # memory.py:77


def rms(x: np.ndarray, weight: np.ndarray) -> np.ndarray:
    """RootMeanSquareNorm.forward (layers.py:14-16)."""

    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + EPS) * weight


def linear(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None) -> np.ndarray:
    y = x @ np.asarray(weight, np.float64).T
    return y if bias is None else y + np.asarray(bias, np.float64)


def softmax(z: np.ndarray) -> np.ndarray:
    e = np.exp(z - z.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def sigmoid(z: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-z))


def confidence_read(numerator: np.ndarray, denominator: np.ndarray) -> np.ndarray:
    """confidence_weighted_read (memory.py:248-251)."""

    regularized = denominator + READ_EPSILON
    return (denominator / regularized) * numerator / regularized


def associative_scan_read(basis, normalizer, decay, value, features, weight, query_features, *,
                          log_dtype=np.float32):
    """scan_and_read of memory.py:97-144 (parallel form): reads for every
    position from the state before its own write, and the final state.

    The reference forms the log-decays, their cumulative sums and the decay
    factors in fp32 whatever the model's dtype (``torch.log(decay.float())``,
    memory.py:106-115, 126-129) and casts the factors back; ``log_dtype``
    follows that (float64 gives the exact-arithmetic form, used to pin the
    parallel form against the sequential recurrence)."""

    ld = np.dtype(log_dtype)
    # log and exp at log_dtype, correctly rounded (evaluated in float64, then
    # rounded): torch's fp32 log/exp agree with that to within one ulp
    log = lambda v: np.log(np.asarray(v, ld).astype(np.float64)).astype(ld)
    exp = lambda v: np.exp(np.asarray(v, np.float64)).astype(ld).astype(np.float64)
    log_decay = log(decay)
    # torch's CPU cumsum accumulates fp32 in float64 and rounds each prefix
    cumulative = np.cumsum(log_decay.astype(np.float64), axis=1).astype(ld)
    prior = cumulative - log_decay
    initial = exp(prior)
    length = decay.shape[1]
    past = np.arange(length)[:, None] > np.arange(length)[None, :]
    pair_log = np.where(past[None], prior[:, :, None] - cumulative[:, None, :], ld.type(0))
    pair = np.where(past[None], exp(pair_log), 0.0)
    similarity = np.einsum("bsm,btm->bts", features, query_features)
    influence = pair * similarity * weight[:, None, :]
    numerator = initial[..., None] * np.einsum("bdm,btm->btd", basis, query_features)
    numerator = numerator + np.einsum("bts,bsd->btd", influence, value)
    denominator = initial * np.einsum("bm,btm->bt", normalizer, query_features) + influence.sum(axis=-1)
    read = confidence_read(numerator, denominator[..., None])
    total = cumulative[:, -1]
    final_weight = exp(total[:, None] - cumulative) * weight
    total_factor = exp(total)
    final_basis = total_factor[:, None, None] * basis + np.einsum("bs,bsd,bsm->bdm", final_weight, value, features)
    final_normalizer = total_factor[:, None] * normalizer + np.einsum("bs,bsm->bm", final_weight, features)
    return read, final_basis, final_normalizer


def associative_sequential(basis, normalizer, decay, value, features, weight, query_features):
    """The same reads and final state position by position: read (memory.py:
    91-95) from the current state, then update (memory.py:279-288)."""

    basis = basis.copy()
    normalizer = normalizer.copy()
    reads = np.zeros_like(value)
    for t in range(value.shape[1]):
        qf = query_features[:, t]
        numerator = np.einsum("bdm,bm->bd", basis, qf)
        denominator = (normalizer * qf).sum(axis=-1, keepdims=True)
        reads[:, t] = confidence_read(numerator, denominator)
        d = decay[:, t]
        basis = d[:, None, None] * basis + weight[:, t, None, None] * (value[:, t, :, None] * features[:, t, None, :])
        normalizer = d[:, None] * normalizer + weight[:, t, None] * features[:, t]
    return reads, basis, normalizer


def initial_state(batch: int, cfg: dict) -> dict:
    """KoemiState.create_static (state.py:43-76): zero state, rings at capacity,
    all slots invalid; with the refine ablation also the zero refine basis
    and normalizer."""

    d, m, w, s = cfg["width"], cfg["memory_features"], cfg["local_memory_size"], cfg["salience_memory_size"]
    refine = {"refine_basis": np.zeros((batch, d, m)), "refine_normalizer": np.zeros((batch, m))} \
        if cfg.get("ablation", "no_refine") == "herm" else {}
    return {**refine,
        "working": np.zeros((batch, d)),
        "basis": np.zeros((batch, d, m)),
        "normalizer": np.zeros((batch, m)),
        "local_keys": np.zeros((batch, w, d)),
        "local_values": np.zeros((batch, w, d)),
        "local_valid": np.zeros((batch, w), bool),
        "salient_keys": np.zeros((batch, s, d)),
        "salient_values": np.zeros((batch, s, d)),
        "salient_valid": np.zeros((batch, s), bool),
        "last_token": np.full((batch,), PAD, np.int64),
    }


def learned_route(router_w: np.ndarray, context: np.ndarray, valid: np.ndarray, top_k: int):
    """LearnedExpertMixture.forward's gate (router.py:46-50): the context with
    invalid rows zeroed through the bias-free gate, the logits rounded to fp32,
    softmax and top-k in fp32 (oracle.route_learned); invalid rows -1 and 0.
    Returns (assignments [..., k] int64, weights [..., k] fp32, the
    RouterStatistics of router.py:50-58 as ``oracle.router_statistics``)."""

    gate_context = np.where(valid[..., None], context, 0.0)
    logits = linear(gate_context, router_w, None).astype(np.float32)
    assignments, weights = oracle.route_learned(logits, valid, top_k)
    return assignments, weights, oracle.router_statistics(logits, valid, assignments)


def experts(p: dict, context: np.ndarray, ids: np.ndarray, previous: np.ndarray, valid: np.ndarray, cfg: dict):
    """The expert mixture of a block, then output_normalizer(context + update)
    where valid (experts.py:134-136; router.py:96-97).

    Hash routing (the default): DeterministicExpertMixture's static dispatch
    (experts.py:109-150), every valid token adds FFN_e(context) / k over its
    distinct assigned experts. ``cfg["expert_routing"] == "learned"``:
    LearnedExpertMixture (router.py:43-97), every valid token adds
    w_slot * FFN_e(context) over its top-k experts, w the fp32 softmax weight.
    Returns (context, assignments, router statistics or None for hash
    routing)."""

    k, count = cfg["top_k"], cfg["expert_count"]
    b, length, d = context.shape
    flat = context.reshape(-1, d)
    ok = valid.reshape(-1)
    statistics = None
    if cfg.get("expert_routing", "hash") == "learned":
        assignments, weights, statistics = learned_route(p["router_w"], context, valid, k)
        a = assignments.reshape(-1, k)
        scale = weights.reshape(-1, k).astype(np.float64)
        take = ok[:, None] & (a >= 0)
    else:
        assignments = oracle.route_hash(ids, previous, valid, count, k)
        a = assignments.reshape(-1, k)
        scale = np.full(a.shape, 1.0 / k)
        # a slot counts when the token is valid, the expert in range and not
        # already taken by an earlier slot of the token (experts.py:120-127, 261-267)
        take = ok[:, None] & (a >= 0) & (a < count)
        for slot in range(1, k):
            take[:, slot] &= ~(a[:, :slot] == a[:, slot:slot + 1]).any(axis=1)
    update = np.zeros_like(flat)
    for e in range(count):
        rows, slots = np.nonzero(take & (a == e))
        if rows.size == 0:
            continue
        x = flat[rows]
        gate = linear(x, p["gate_w"][e], p["gate_b"][e])
        up = linear(x, p["up_w"][e], p["up_b"][e])
        y = linear(gate / (1.0 + np.exp(-gate)) * up, p["down_w"][e], p["down_b"][e])
        np.add.at(update, rows, y * scale[rows, slots][:, None])
    mixed = rms(flat + update, p["expert_norm"])
    out = np.where(ok[:, None], mixed, flat).reshape(b, length, d)
    return out, assignments, statistics


def block_window(p: dict, state: dict, ids: np.ndarray, cfg: dict, input_context: np.ndarray | None = None, *,
                 return_assignments: bool = False, return_statistics: bool = False,
                 admission_in: np.ndarray | None = None):
    """One forward_window of one block. Returns (logits, final_context,
    next_state, surprise, admission), the expert assignments [B, L, k] as a
    further item with ``return_assignments``, and the learned gate's router
    statistics (``oracle.router_statistics``; None for hash routing) as the
    last item with ``return_statistics``. ``admission_in`` ([B, L] bool, or
    None) replaces the admission decision ``valid & (surprise > threshold)``
    (network.py:349), so that a checker can follow another implementation's
    decision for scores that lie within rounding distance of the threshold;
    the returned admission is then ``admission_in``."""

    f = lambda name: np.asarray(p[name], np.float64)
    ids = np.asarray(ids, np.int64)
    valid = ids != PAD
    source = f("embedding")[ids] if input_context is None else input_context
    u = rms(source, f("input_norm"))
    retention, increment = oracle.recurrent_gates(u, f("retention_w"), f("retention_b"), f("candidate_w"),
                                                  f("candidate_b"), valid)
    ws = oracle.scan_sequential(np.asarray(retention, np.float64), np.asarray(increment, np.float64), state["working"])
    prior = np.concatenate([state["working"][:, None], ws[:, :-1]], axis=1)

    content = linear(prior, f("head_w")[:PAD], f("head_b")[:PAD])
    targets = np.where(valid, ids, 0)
    zmax = content.max(axis=-1, keepdims=True)
    lse = np.log(np.exp(content - zmax).sum(axis=-1)) + zmax[..., 0]
    nll = lse - np.take_along_axis(content, targets[..., None], axis=-1)[..., 0]
    surprise = np.where(valid, 1.0 - np.exp(-nll / math.log(PAD)), 0.0)

    keep = valid[..., None]
    local_keys = np.where(keep, linear(ws, f("local_key_w"), f("local_key_b")), 0.0)
    local_values = np.where(keep, linear(ws, f("local_value_w"), f("local_value_b")), 0.0)
    local_value = oracle.read_local_window(state["local_keys"], state["local_values"], state["local_valid"],
                                           local_keys, local_values, valid, ws, cfg["local_memory_size"])

    key = linear(ws, f("key_w"), f("key_b"))
    features = softmax(linear(key, f("feature_w"), f("feature_b")))
    value = np.tanh(linear(ws, f("value_w"), f("value_b")))
    decay = MIN_DECAY + (MAX_DECAY - MIN_DECAY) * sigmoid(linear(ws, f("decay_w"), f("decay_b")))[..., 0]
    write = sigmoid(linear(ws, f("write_w"), f("write_b")))[..., 0] * (0.25 + 0.75 * np.clip(surprise, 0.0, 1.0))
    decay = np.where(valid, decay, 1.0)
    write = np.where(valid, write, 0.0)
    query_features = softmax(linear(linear(ws, f("query_w"), f("query_b")), f("feature_w"), f("feature_b")))
    fast, basis, normalizer = associative_scan_read(state["basis"], state["normalizer"], decay, value, features,
                                                    write, query_features,
                                                    log_dtype=cfg.get("memory_log_dtype", np.float32))

    refine_next = {}
    if cfg.get("ablation", "no_refine") == "herm":
        # the refine memory (network.py:359-384): write terms from the
        # reconstruction error and the local read's novelty (memory.py:257-268),
        # masked as the fast terms, a second scan_and_read over the refine
        # state with the same query features, and the refine gate
        # (network.py:714-721) mixing it into the memory value
        novelty = oracle.local_novelty(state["local_keys"], state["local_valid"], local_keys, valid, ws,
                                       cfg["local_memory_size"])
        bounded = MIN_DECAY + (MAX_DECAY - MIN_DECAY) * sigmoid(linear(ws, f("decay_w"), f("decay_b")))[..., 0]
        refine_decay = np.minimum(1.0 - (1.0 - bounded) * cfg["refine_decay_rate"], MAX_REFINE_DECAY)
        refine_weight = (sigmoid(linear(ws, f("write_w"), f("write_b")))[..., 0] * np.clip(surprise, 0.0, 1.0)
                         * np.clip(novelty, 0.0, 1.0))
        error = np.clip(value - fast, -2.0, 2.0)
        refine, refine_basis, refine_normalizer = associative_scan_read(
            state["refine_basis"], state["refine_normalizer"], np.where(valid, refine_decay, 1.0), error, features,
            np.where(valid, refine_weight, 0.0), query_features, log_dtype=cfg.get("memory_log_dtype", np.float32))
        gate_in = np.concatenate([ws, fast, refine, local_value], axis=-1)
        gate = sigmoid(linear(gate_in, f("refine_gate_w"), f("refine_gate_b")))
        fast = fast + gate * refine
        refine_next = {"refine_basis": refine_basis, "refine_normalizer": refine_normalizer}

    admission = valid & (surprise > cfg["salience_threshold"])
    if admission_in is not None:
        admission = np.asarray(admission_in, bool).reshape(admission.shape)
    salient_value = oracle.read_salient_window(state["salient_keys"], state["salient_values"], state["salient_valid"],
                                               local_keys, local_values, admission, ws)
    fused = rms(linear(np.concatenate([ws, fast, local_value, salient_value], axis=-1), f("fusion_w"),
                       f("fusion_b")), f("fusion_norm"))
    previous = oracle.previous_token_ids(ids, valid, state["last_token"])
    names = ("gate_w", "gate_b", "up_w", "up_b", "down_w", "down_b", "expert_norm", "router_w")
    final, assignments, statistics = experts({k: f(k) for k in names if k in p}, fused, ids, previous, valid, cfg)
    logits = linear(final, f("head_w"), f("head_b"))

    w = cfg["local_memory_size"]
    all_lk = np.concatenate([state["local_keys"], local_keys], axis=1)
    all_lv = np.concatenate([state["local_values"], local_values], axis=1)
    all_ok = np.concatenate([state["local_valid"], valid], axis=1)
    sk, sv, sok = oracle.salient_tail(state["salient_keys"], state["salient_values"], state["salient_valid"],
                                      local_keys, local_values, admission, cfg["salience_memory_size"])
    positions = np.where(valid, np.arange(ids.shape[1])[None, :], -1).max(axis=1)
    last = np.where(positions >= 0, ids[np.arange(ids.shape[0]), np.maximum(positions, 0)], state["last_token"])
    next_state = {
        "working": ws[:, -1],
        "basis": basis,
        "normalizer": normalizer,
        "local_keys": all_lk[:, -w:],
        "local_values": all_lv[:, -w:],
        "local_valid": all_ok[:, -w:],
        "salient_keys": np.asarray(sk, np.float64),
        "salient_values": np.asarray(sv, np.float64),
        "salient_valid": np.asarray(sok, bool),
        "last_token": last,
        **refine_next,
    }
    out = (logits, final, next_state, surprise, admission)
    if return_assignments:
        out += (assignments,)
    if return_statistics:
        out += (statistics,)
    return out


def stack_window(params: list[dict], states: list[dict], ids: np.ndarray, cfg: dict,
                 admissions: list[np.ndarray] | None = None, *, return_admissions: bool = False):
    """One window through every layer (the composition in the module docstring).
    Returns (last layer's logits, next states, per-layer surprise), and the
    per-layer admission masks with ``return_admissions``. ``admissions``: per
    layer the ``admission_in`` of ``block_window`` (or None)."""

    context = None
    next_states, surprises, admitted = [], [], []
    logits = None
    for layer, (p, st) in enumerate(zip(params, states)):
        forced = None if admissions is None else admissions[layer]
        logits, context, nst, surprise, admission = block_window(p, st, ids, cfg, context, admission_in=forced)
        next_states.append(nst)
        surprises.append(surprise)
        admitted.append(admission)
    if return_admissions:
        return logits, next_states, surprises, admitted
    return logits, next_states, surprises


def prefill(params: list[dict], states: list[dict], ids: np.ndarray, cfg: dict, window: int,
            admissions: list[np.ndarray] | None = None, *, return_layers: bool = False):
    """forward_parallel (network.py:176-197): the sequence in windows of `window`, state carried.
    Returns (logits, final states), and with ``return_layers`` also every
    layer's surprise and admission over the whole sequence ([B, L] each).
    ``admissions``: per layer a [B, L] mask replacing the admission decision
    (``block_window``'s ``admission_in``), or None."""

    pieces, surprise, admitted = [], [], []
    for start in range(0, ids.shape[1], window):
        forced = None if admissions is None else [a[:, start:start + window] for a in admissions]
        logits, states, s, a = stack_window(params, states, ids[:, start:start + window], cfg, forced,
                                            return_admissions=True)
        pieces.append(logits)
        surprise.append(s)
        admitted.append(a)
    logits = np.concatenate(pieces, axis=1)
    if not return_layers:
        return logits, states
    per_layer = lambda parts: [np.concatenate([w[layer] for w in parts], axis=1) for layer in range(len(params))]
    return logits, states, per_layer(surprise), per_layer(admitted)
