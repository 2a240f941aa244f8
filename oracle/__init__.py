"""CPU oracle of the Koemi-5HOM HERM hot path (numpy + the C restatement).

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the CPU baseline — never as the thing measured or shipped. The
product package ``koemi_amd`` does not import it and has no CPU fallback.

Each function names the reference lines it restates. Pinning (which checks in
tests/test_oracle.py fix each function beyond its own formula) is listed in the
module docstring of that test file.
"""

from __future__ import annotations

import ctypes
import math
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import numpy as np

from oracle.build import LIBRARY, build

PAD_TOKEN_ID = 256  # configuration/settings.py:10-11

# ----------------------------------------------------------------- C library

_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The C restatement, built on first use if the shared object is missing."""

    global _LIB
    if _LIB is None:
        if not LIBRARY.is_file():
            build()
        handle = ctypes.CDLL(str(LIBRARY))
        handle.oracle_det_expf.restype = c_float
        handle.oracle_det_expf.argtypes = [c_float]
        handle.oracle_det_logf.restype = c_float
        handle.oracle_det_logf.argtypes = [c_float]
        handle.oracle_quantile.restype = c_float
        handle.oracle_quantile.argtypes = [c_void_p, c_int64, c_float]
        for name in ("oracle_scan_sequential_f32", "oracle_scan_sequential_f64"):
            fn = getattr(handle, name)
            fn.restype = None
            fn.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int]
        handle.oracle_surprise_rows.restype = None
        handle.oracle_surprise_rows.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_float]
        handle.oracle_route_learned.restype = None
        handle.oracle_route_learned.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64]
        for name in ("oracle_det_expf_array", "oracle_det_logf_array"):
            fn = getattr(handle, name)
            fn.restype = None
            fn.argtypes = [c_void_p, c_void_p, c_int64]
        handle.oracle_rmsnorm_silu_f32.restype = None
        handle.oracle_rmsnorm_silu_f32.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_float]
        _LIB = handle
    return _LIB


def _p(array: np.ndarray | None) -> int | None:
    return None if array is None else array.ctypes.data


# ---------------------------------------------------------------- bfloat16

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32."""

    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even; NaN kept quiet."""

    u = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(values)
    if nan.any():
        rounded = rounded.copy()
        rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def round_bf16(values: np.ndarray) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(np.asarray(values, dtype=np.float32)))


# -------------------------------------------------------------------- scan

def scan_sequential(retention: np.ndarray, increment: np.ndarray, initial: np.ndarray | None = None) -> np.ndarray:
    """h_t = a_t * h_{t-1} + b_t in the input dtype (float32 or float64), h_{-1} =
    initial (zeros if None). Retention is full-shape or [B, L] (+ trailing 1s).
    Restates tests/model/test_scan.py:10-16 and tests/cuda/test_dense_cuda.py:21-33."""

    dtype = increment.dtype
    assert dtype in (np.float32, np.float64)
    b = np.ascontiguousarray(increment)
    B, L = b.shape[:2]
    F = int(np.prod(b.shape[2:])) if b.ndim > 2 else 1
    a = np.ascontiguousarray(retention, dtype=dtype)
    broadcast = a.size == B * L and b.size != B * L
    if not broadcast and a.shape != b.shape:
        a = np.ascontiguousarray(np.broadcast_to(a, b.shape))
    h0 = np.zeros((B, F), dtype=dtype) if initial is None else np.ascontiguousarray(initial, dtype=dtype).reshape(B, F)
    out = np.empty_like(b)
    fn = lib().oracle_scan_sequential_f32 if dtype == np.float32 else lib().oracle_scan_sequential_f64
    fn(_p(a), _p(b), _p(h0), _p(out), B, L, F, int(broadcast))
    return out


def scan_hillis_steele(retention: np.ndarray, increment: np.ndarray, initial: np.ndarray | None = None) -> np.ndarray:
    """The model-path window scan of model/scan.py:17-30 (log2 L doubling rounds),
    vectorized over the state columns; used as the second CPU baseline."""

    coefficient = np.broadcast_to(retention, increment.shape).astype(increment.dtype)
    value = increment.copy()
    length = increment.shape[1]
    offset = 1
    while offset < length:
        shifted_c = np.concatenate((np.ones_like(coefficient[:, :offset]), coefficient[:, : length - offset]), axis=1)
        shifted_v = np.concatenate((np.zeros_like(value[:, :offset]), value[:, : length - offset]), axis=1)
        value = coefficient * shifted_v + value
        coefficient = coefficient * shifted_c
        offset *= 2
    if initial is None:
        return value
    return value + coefficient * initial[:, None]


# ------------------------------------------------------------ rmsnorm-silu

def rmsnorm_silu_f64(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> tuple[np.ndarray, np.ndarray]:
    """silu(x * rsqrt(mean(x^2) + eps) * w) in float64 (test_core_cuda.py:70-71,
    layers.py:14-16 followed by silu). Returns (y, inverse_rms)."""

    xf = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(xf * xf, axis=-1) + eps)
    v = xf * inv[:, None] * np.asarray(weight, dtype=np.float64)
    return v / (1.0 + np.exp(-v)), inv


def rmsnorm_silu_f32(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> tuple[np.ndarray, np.ndarray]:
    """fp32 port of the fused forward (core/rmsnorm_silu.cu:62-91), for the CPU baseline."""

    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(weight, dtype=np.float32)
    rows, hidden = x.shape
    y = np.empty_like(x)
    inv = np.empty((rows,), dtype=np.float32)
    lib().oracle_rmsnorm_silu_f32(_p(x), _p(w), _p(y), _p(inv), rows, hidden, c_float(eps))
    return y, inv


# --------------------------------------------------------------- surprise

def log_vocab_f32(vocab: int) -> float:
    return float(np.float32(math.log(float(np.float32(vocab)))))


def det_expf(x: float) -> float:
    return float(lib().oracle_det_expf(float(x)))


def det_logf(x: float) -> float:
    return float(lib().oracle_det_logf(float(x)))


def det_expf_array(x: np.ndarray) -> np.ndarray:
    xs = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(xs)
    lib().oracle_det_expf_array(_p(xs), _p(out), xs.size)
    return out


def det_logf_array(x: np.ndarray) -> np.ndarray:
    xs = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(xs)
    lib().oracle_det_logf_array(_p(xs), _p(out), xs.size)
    return out


def surprise_rows(
    logits: np.ndarray, targets: np.ndarray, valid: np.ndarray, bias: np.ndarray | None = None
) -> np.ndarray:
    """Per-row surprise with the kernel's rounding steps (network.py:677-688;
    surprise_kernel.cu:84-134). logits float32 [R, V]."""

    z = np.ascontiguousarray(logits, dtype=np.float32)
    rows, vocab = z.shape
    t = np.ascontiguousarray(targets, dtype=np.int64).reshape(rows)
    v = np.ascontiguousarray(valid, dtype=np.uint8).reshape(rows)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    out = np.empty((rows,), dtype=np.float32)
    lib().oracle_surprise_rows(_p(z), _p(b), _p(t), _p(v), _p(out), rows, vocab, c_float(log_vocab_f32(vocab)))
    return out


def surprise_rows_f64(logits: np.ndarray, targets: np.ndarray, valid: np.ndarray) -> np.ndarray:
    """Surprise in float64 via a max-shifted logsumexp (reference_causal_surprise,
    tests/cuda/test_think_cuda.py:19-32), as the accuracy yardstick."""

    z = np.asarray(logits, dtype=np.float64)
    m = z.max(axis=-1, keepdims=True)
    lse = np.log(np.exp(z - m).sum(axis=-1)) + m[..., 0]
    zt = np.take_along_axis(z, np.asarray(targets, dtype=np.int64)[..., None], axis=-1)[..., 0]
    s = 1.0 - np.exp(-(lse - zt) / math.log(z.shape[-1]))
    return np.where(np.asarray(valid, dtype=bool), s, 0.0)


def quantile(scores: np.ndarray, q: float) -> float:
    s = np.ascontiguousarray(scores, dtype=np.float32).reshape(-1)
    return float(lib().oracle_quantile(_p(s), s.size, c_float(q)))


def admission(scores: np.ndarray, valid: np.ndarray, *, threshold: float | None = None, q: float | None = None) -> tuple[np.ndarray, float]:
    """valid & (s > tau) with strict '>' (network.py:349); tau fixed or the q-quantile."""

    s = np.asarray(scores, dtype=np.float32)
    tau = float(np.float32(threshold)) if threshold is not None else quantile(s, q)
    return np.asarray(valid, dtype=bool) & (s > np.float32(tau)), tau


def recurrent_gates(u, retention_weight, retention_bias, candidate_weight, candidate_bias, valid=None):
    """BoundedRecurrentState.gates (model/memory.py:14-30) in float64, with the
    masking of network.py:307-309 when `valid` is given:
    a = 2^-8 + ((1 - 2^-8) - 2^-8) sigmoid(u W_r^T + b_r), b = (1 - a) tanh(u W_c^T + b_c),
    invalid rows a = 1, b = 0."""

    x = np.asarray(u, dtype=np.float64)
    zr = x @ np.asarray(retention_weight, np.float64).T + np.asarray(retention_bias, np.float64)
    zc = x @ np.asarray(candidate_weight, np.float64).T + np.asarray(candidate_bias, np.float64)
    lo, hi = 2.0**-8, 1.0 - 2.0**-8
    a = lo + (hi - lo) / (1.0 + np.exp(-zr))
    b = (1.0 - a) * np.tanh(zc)
    if valid is not None:
        keep = np.asarray(valid, bool)[..., None]
        a = np.where(keep, a, 1.0)
        b = np.where(keep, b, 0.0)
    return a, b


def read_salient_window(
    carried_keys: np.ndarray,
    carried_values: np.ndarray,
    carried_valid: np.ndarray,
    keys: np.ndarray,
    values: np.ndarray,
    admission: np.ndarray,
    queries: np.ndarray,
) -> np.ndarray:
    """Salient read (model/memory.py:405-429), in float64: scores of every query
    against [carried keys ; window keys] divided by sqrt(width); carried slot s
    eligible when carried_valid, window slot j when admitted and j < t; softmax
    over the eligible slots (rows with none read zeros); weighted sum of
    [carried values ; window values]."""

    ck = np.asarray(carried_keys, dtype=np.float64)
    k = np.asarray(keys, dtype=np.float64)
    q = np.asarray(queries, dtype=np.float64)
    all_k = np.concatenate([ck, k], axis=1)
    all_v = np.concatenate([np.asarray(carried_values, np.float64), np.asarray(values, np.float64)], axis=1)
    b, length, width = q.shape
    s = ck.shape[1]
    pos = np.arange(length)
    current = np.asarray(admission, bool)[:, None, :] & (pos[:, None] > pos[None, :])[None]
    carried = np.broadcast_to(np.asarray(carried_valid, bool)[:, None, :], (b, length, s))
    eligible = np.concatenate([carried, current], axis=-1)
    scores = np.einsum("bsd,btd->bts", all_k, q) / np.sqrt(width)
    scores = np.where(eligible, scores, -np.inf)
    any_slot = eligible.any(axis=-1, keepdims=True)
    m = np.where(any_slot, scores.max(axis=-1, keepdims=True, initial=-np.inf), 0.0)
    e = np.where(eligible, np.exp(scores - m), 0.0)
    total = e.sum(axis=-1, keepdims=True)
    w = np.where(any_slot, e / np.where(total > 0, total, 1.0), 0.0)
    return np.einsum("bts,bsd->btd", w, all_v)


def read_local_window(
    carried_keys: np.ndarray,
    carried_values: np.ndarray,
    carried_valid: np.ndarray,
    keys: np.ndarray,
    values: np.ndarray,
    valid: np.ndarray,
    queries: np.ndarray,
    window: int,
) -> np.ndarray:
    """Local read (value output of LocalKeyValueMemory.read_window, model/memory.py:
    332-362, with sliding_window_mask 364-383), in float64: slot s of
    [carried ; window entries] is eligible for query t when valid and
    C + t - window <= s < C + t; softmax of key . query / sqrt(width) over the
    eligible slots (rows with none read zeros)."""

    ck = np.asarray(carried_keys, dtype=np.float64)
    all_k = np.concatenate([ck, np.asarray(keys, np.float64)], axis=1)
    all_v = np.concatenate([np.asarray(carried_values, np.float64), np.asarray(values, np.float64)], axis=1)
    all_valid = np.concatenate([np.asarray(carried_valid, bool), np.asarray(valid, bool)], axis=1)
    q = np.asarray(queries, dtype=np.float64)
    b, length, width = q.shape
    c = ck.shape[1]
    own = c + np.arange(length)[:, None]
    src = np.arange(all_k.shape[1])[None, :]
    eligible = ((src < own) & (src >= own - window))[None] & all_valid[:, None, :]
    scores = np.einsum("bsd,btd->bts", all_k, q) / np.sqrt(width)
    scores = np.where(eligible, scores, -np.inf)
    any_slot = eligible.any(axis=-1, keepdims=True)
    m = np.where(any_slot, scores.max(axis=-1, keepdims=True, initial=-np.inf), 0.0)
    e = np.where(eligible, np.exp(scores - m), 0.0)
    total = e.sum(axis=-1, keepdims=True)
    w = np.where(any_slot, e / np.where(total > 0, total, 1.0), 0.0)
    return np.einsum("bts,bsd->btd", w, all_v)


def local_novelty(
    carried_keys: np.ndarray,
    carried_valid: np.ndarray,
    keys: np.ndarray,
    valid: np.ndarray,
    queries: np.ndarray,
    window: int,
) -> np.ndarray:
    """Novelty output of LocalKeyValueMemory.read_window (model/memory.py:
    354-361), in float64: over the slots eligible for query t (the local
    read's sliding window, memory.py:364-383), the largest cosine similarity
    of the query with a key (both normalised as functional.normalize does,
    x / max(|x|, 1e-12)); novelty = clamp(1 - largest, 0, 1), and 1 for a
    query with no eligible slot. Returns [B, L]."""

    all_k = np.concatenate([np.asarray(carried_keys, np.float64), np.asarray(keys, np.float64)], axis=1)
    all_valid = np.concatenate([np.asarray(carried_valid, bool), np.asarray(valid, bool)], axis=1)
    q = np.asarray(queries, dtype=np.float64)
    length = q.shape[1]
    c = np.asarray(carried_keys).shape[1]
    own = c + np.arange(length)[:, None]
    src = np.arange(all_k.shape[1])[None, :]
    eligible = ((src < own) & (src >= own - window))[None] & all_valid[:, None, :]
    nk = all_k / np.maximum(np.linalg.norm(all_k, axis=-1, keepdims=True), 1e-12)
    nq = q / np.maximum(np.linalg.norm(q, axis=-1, keepdims=True), 1e-12)
    similarity = np.where(eligible, np.einsum("bsd,btd->bts", nk, nq), -np.inf)
    any_slot = eligible.any(axis=-1)
    highest = similarity.max(axis=-1, initial=-np.inf)
    return np.clip(np.where(any_slot, 1.0 - highest, 1.0), 0.0, 1.0)


def read_local_sequential(
    carried_keys: np.ndarray,
    carried_values: np.ndarray,
    carried_valid: np.ndarray,
    keys: np.ndarray,
    values: np.ndarray,
    valid: np.ndarray,
    queries: np.ndarray,
    window: int,
) -> np.ndarray:
    """The same read position by position, as the sequential path does it
    (LocalKeyValueMemory.read, memory.py:274-295, then append, 457-475): a
    ring of the last `window` entries, read before the query's own entry is
    appended. An independent restatement used to pin read_local_window."""

    ring_k = [row for row in np.asarray(carried_keys, np.float64).transpose(1, 0, 2)]
    ring_v = [row for row in np.asarray(carried_values, np.float64).transpose(1, 0, 2)]
    ring_ok = [row for row in np.asarray(carried_valid, bool).T]
    ring_k, ring_v, ring_ok = ring_k[-window:], ring_v[-window:], ring_ok[-window:]
    q = np.asarray(queries, np.float64)
    b, length, width = q.shape
    out = np.zeros_like(q)
    for t in range(length):
        if ring_k:
            k = np.stack(ring_k, 1)
            v = np.stack(ring_v, 1)
            ok = np.stack(ring_ok, 1)
            scores = np.einsum("bsd,bd->bs", k, q[:, t]) / np.sqrt(width)
            for r in range(b):
                if ok[r].any():
                    z = scores[r][ok[r]]
                    e = np.exp(z - z.max())
                    out[r, t] = (e / e.sum()) @ v[r][ok[r]]
        ring_k.append(np.asarray(keys, np.float64)[:, t])
        ring_v.append(np.asarray(values, np.float64)[:, t])
        ring_ok.append(np.asarray(valid, bool)[:, t])
        ring_k, ring_v, ring_ok = ring_k[-window:], ring_v[-window:], ring_ok[-window:]
    return out


def salient_tail(
    carried_keys: np.ndarray,
    carried_values: np.ndarray,
    carried_valid: np.ndarray,
    keys: np.ndarray,
    values: np.ndarray,
    admission: np.ndarray,
    capacity: int,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Salient ring update (model/memory.py:431-455): concatenate carried and new
    entries; if they fit, return them unchanged; else keep the entries ranked
    highest by (valid ? t : -1), in ascending t, zeroing invalid slots. The
    reference's torch.topk leaves the choice among tied invalid entries
    unspecified; this restatement (and the kernel) takes the latest ones."""

    all_k = np.concatenate([carried_keys, keys], axis=1)
    all_v = np.concatenate([carried_values, values], axis=1)
    all_ok = np.concatenate([carried_valid, admission], axis=1).astype(bool)
    n = all_k.shape[1]
    if n <= capacity:
        return all_k, all_v, all_ok
    out_k = np.zeros((all_k.shape[0], capacity) + all_k.shape[2:], dtype=all_k.dtype)
    out_v = np.zeros_like(out_k)
    out_ok = np.zeros((all_k.shape[0], capacity), dtype=bool)
    for b in range(all_k.shape[0]):
        valid_idx = np.flatnonzero(all_ok[b])
        invalid_idx = np.flatnonzero(~all_ok[b])
        m = min(valid_idx.size, capacity)
        chosen = list(valid_idx[valid_idx.size - m:]) + list(invalid_idx[invalid_idx.size - (capacity - m):]
                                                            if capacity > m else [])
        sel = np.sort(np.asarray(chosen, dtype=np.int64))
        ok = all_ok[b, sel]
        out_ok[b] = ok
        out_k[b] = np.where(ok[:, None], all_k[b, sel], 0)
        out_v[b] = np.where(ok[:, None], all_v[b, sel], 0)
    return out_k, out_v, out_ok


# ------------------------------------------------------------------- MoE

TOKEN_HASH_FACTOR = 1_000_003          # experts.py:12
PREVIOUS_TOKEN_HASH_FACTOR = 97_409    # experts.py:13
HASH_MIX_MULTIPLIER = 0x45D9F3B        # experts.py:15
SLOT_OFFSET = 0x9E3779B9               # experts.py:288


def content_hash(token_ids: np.ndarray, previous_token_ids: np.ndarray) -> np.ndarray:
    """experts.py:30-38 in int64 arithmetic (two's-complement wrap of the
    products, masked to 32 bits)."""

    mask = np.int64(0xFFFFFFFF)
    with np.errstate(over="ignore"):
        v = (np.asarray(token_ids, dtype=np.int64) * TOKEN_HASH_FACTOR
             + np.asarray(previous_token_ids, dtype=np.int64) * PREVIOUS_TOKEN_HASH_FACTOR) & mask
        v = v ^ (v >> 16)
        v = (v * HASH_MIX_MULTIPLIER) & mask
        v = v ^ (v >> 16)
        v = (v * HASH_MIX_MULTIPLIER) & mask
    return v ^ (v >> 16)


def route_hash(token_ids: np.ndarray, previous_token_ids: np.ndarray, valid: np.ndarray, expert_count: int, top_k: int) -> np.ndarray:
    """assign_top_k of experts.py:283-289: (hash + s * 0x9E3779B9) mod E in int64; invalid -> -1."""

    h = content_hash(token_ids, previous_token_ids)
    offsets = np.arange(top_k, dtype=np.int64) * SLOT_OFFSET
    a = np.remainder(h[..., None] + offsets, expert_count)
    return np.where(np.asarray(valid, dtype=bool)[..., None], a, -1).astype(np.int64)


def route_modulo(token_ids: np.ndarray, valid: np.ndarray, expert_count: int, top_k: int) -> np.ndarray:
    """The benchmark's synthetic "token id mod E" variant (
    no reference counterpart): slot s -> (tok + s) mod E with Python's
    (torch.remainder's) sign; invalid -> -1."""

    a = np.remainder(np.asarray(token_ids, np.int64)[..., None] + np.arange(top_k, dtype=np.int64), expert_count)
    return np.where(np.asarray(valid, bool)[..., None], a, -1).astype(np.int64)


def route_learned(router_logits: np.ndarray, valid: np.ndarray, top_k: int) -> tuple[np.ndarray, np.ndarray]:
    """router.py:46-49 with the kernel's rounding steps: (assignments, weights)."""

    z = np.ascontiguousarray(router_logits, dtype=np.float32)
    E = z.shape[-1]
    T = z.size // E
    v = np.ascontiguousarray(valid, dtype=np.uint8).reshape(T)
    idx = np.empty((T, top_k), dtype=np.int64)
    w = np.empty((T, top_k), dtype=np.float32)
    lib().oracle_route_learned(_p(z), _p(v), _p(idx), _p(w), T, E, top_k)
    shape = tuple(z.shape[:-1]) + (top_k,)
    return idx.reshape(shape), w.reshape(shape)


def router_statistics(router_logits: np.ndarray, valid: np.ndarray, assignments: np.ndarray) -> dict:
    """RouterStatistics of LearnedExpertMixture.forward (router.py:11-22, 50-58)
    in float64: ``probability_mass`` [E] = the softmax probabilities of the
    valid tokens summed per expert, ``assignment_counts`` [E] = the valid
    (token, slot) assignments per expert (scatter_add of the valid flags over
    the assignments clamped at 0), ``valid_count`` = the valid tokens, and
    ``balance_loss`` (``balance_loss`` below)."""

    z = np.asarray(router_logits, np.float64)
    E = z.shape[-1]
    z = z.reshape(-1, E)
    ok = np.asarray(valid, bool).reshape(-1)
    a = np.asarray(assignments, np.int64).reshape(ok.size, -1)
    e = np.exp(z - z.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    mass = (p * ok[:, None]).sum(axis=0)
    counts = np.zeros(E, np.float64)
    np.add.at(counts, np.maximum(a, 0).reshape(-1), np.repeat(ok, a.shape[1]).astype(np.float64))
    valid_count = float(ok.sum())
    return {"probability_mass": mass, "assignment_counts": counts, "valid_count": valid_count,
            "balance_loss": balance_loss(mass, counts, valid_count)}


def balance_loss(probability_mass: np.ndarray, assignment_counts: np.ndarray, valid_count: float) -> float:
    """RouterStatistics.balance_loss (router.py:17-22) in float64:
    E * sum((mass / max(valid, 1)) * (counts / max(sum(counts), 1)))."""

    mass = np.asarray(probability_mass, np.float64)
    counts = np.asarray(assignment_counts, np.float64)
    importance = mass / max(float(valid_count), 1.0)
    load = counts / max(float(counts.sum()), 1.0)
    return float(mass.size * (importance * load).sum())


def merge_router_statistics(statistics: list[dict]) -> dict | None:
    """merge_router_statistics (router.py:25-32): field-wise sums (None when
    empty), the balance loss formed again from the sums."""

    if not statistics:
        return None
    mass = sum(np.asarray(item["probability_mass"], np.float64) for item in statistics)
    counts = sum(np.asarray(item["assignment_counts"], np.float64) for item in statistics)
    valid_count = float(sum(float(item["valid_count"]) for item in statistics))
    return {"probability_mass": mass, "assignment_counts": counts, "valid_count": valid_count,
            "balance_loss": balance_loss(mass, counts, valid_count)}


def sample_tokens(logits: np.ndarray, exclude: int, temperature: float, top_k: int | None,
                  uniforms: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """TokenSampler's non-greedy draw (runtime/fast_decode.py:57-95) in
    float64 from the fp32 scores: the excluded (PAD) column at -inf, with
    top_k every score below the min(top_k, V)-th largest at -inf (ties kept),
    p = softmax(score / temperature), the id the first column whose
    cumulative p exceeds the row's uniform. Returns (ids [rows], p [rows, V])."""

    s = np.asarray(logits, np.float32).astype(np.float64).copy()
    s[:, exclude] = -np.inf
    rows, vocab = s.shape
    if top_k is not None and top_k < vocab:
        thr = np.sort(s, axis=1)[:, vocab - top_k][:, None]
        s = np.where(s < thr, -np.inf, s)
    y = s / temperature
    e = np.exp(y - y.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    cum = np.cumsum(p, axis=1)
    ids = np.array([int(np.argmax(cum[r] > uniforms[r])) if (cum[r] > uniforms[r]).any()
                    else int(np.nonzero(p[r] > 0)[0][-1]) for r in range(rows)])
    return ids, p


def expert_counts(assignments: np.ndarray, valid: np.ndarray, expert_count: int) -> np.ndarray:
    """network.py:48-70: counts of valid, in-range assignments per expert."""

    a = np.asarray(assignments, dtype=np.int64)
    counted = np.asarray(valid, dtype=bool)[..., None] & (a >= 0) & (a < expert_count)
    return np.bincount(a[counted].reshape(-1), minlength=expert_count).astype(np.int64)


def pair_keys(assignments: np.ndarray, valid: np.ndarray, expert_count: int) -> np.ndarray:
    """Sort key per (token, slot) pair (moe_kernels.cu:68-91; experts.py:183-191):
    the expert, or expert_count for an invalid token, an out-of-range expert or a
    slot repeating an earlier slot's expert."""

    a = np.asarray(assignments, dtype=np.int64)
    T, k = a.shape
    ok = np.asarray(valid, dtype=bool)[:, None] & (a >= 0) & (a < expert_count)
    for s in range(1, k):
        ok[:, s] &= ~(a[:, :s] == a[:, s : s + 1]).any(axis=1)
    return np.where(ok, a, expert_count).reshape(-1)


def permute(context: np.ndarray, assignments: np.ndarray, valid: np.ndarray, expert_count: int,
            pair_weights: np.ndarray | None = None):
    """permute_topk contract (moe/__init__.py:179-228; moe_kernels.cu:390-499):
    stable argsort of the pair keys (experts.py:189-197). Returns
    (sorted_context, sorted_rows, sorted_experts, segment_offsets[, sorted_weights])."""

    T, k = np.asarray(assignments).shape
    keys = pair_keys(assignments, valid, expert_count)
    order = np.argsort(keys, kind="stable")
    sorted_keys = keys[order]
    counts = np.bincount(keys, minlength=expert_count + 1)
    offsets = np.zeros(expert_count + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts[:expert_count])
    rows = order // k
    ctx = np.asarray(context).reshape(T, -1)
    sorted_ctx = ctx[rows].copy()
    sorted_ctx[offsets[-1]:] = 0
    result = [sorted_ctx, rows.astype(np.int64), sorted_keys.astype(np.int64), offsets]
    if pair_weights is not None:
        sw = np.asarray(pair_weights, dtype=np.float32).reshape(-1)[order].copy()
        sw[offsets[-1]:] = 0.0
        result.append(sw)
    return tuple(result)


def grouped_mlp(sorted_context: np.ndarray, sorted_experts: np.ndarray, offsets: np.ndarray,
                gate_w, gate_b, value_w, value_b, out_w, out_b, *, dtype=np.float64,
                round_hidden_bf16: bool = False) -> np.ndarray:
    """Per-expert GLU FFN over the sorted segments (GatedFeedForward, layers.py:27-29;
    moe_kernels.cu:147-199): y = W_o (silu(W_g x + b_g) * (W_v x + b_v)) + b_o,
    rows past offsets[-1] zero. With round_hidden_bf16 the GLU product is rounded
    to bfloat16 before the second product, as the bf16 MFMA path stores it."""

    x = np.asarray(sorted_context, dtype=dtype)
    out = np.zeros((x.shape[0], np.asarray(out_w).shape[1]), dtype=dtype)
    off = np.asarray(offsets, dtype=np.int64)
    for e in range(off.shape[0] - 1):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi <= lo:
            continue
        xe = x[lo:hi]
        g = xe @ np.asarray(gate_w[e], dtype=dtype).T + np.asarray(gate_b[e], dtype=dtype)
        v = xe @ np.asarray(value_w[e], dtype=dtype).T + np.asarray(value_b[e], dtype=dtype)
        h = g / (1.0 + np.exp(-g)) * v
        if round_hidden_bf16:
            h = round_bf16(h.astype(np.float32)).astype(dtype)
        out[lo:hi] = h @ np.asarray(out_w[e], dtype=dtype).T + np.asarray(out_b[e], dtype=dtype)
    return out


def round_bf16_f64(x: np.ndarray) -> np.ndarray:
    """float64 values rounded to the nearest bfloat16 (8 significant bits,
    ties to even), kept in float64; one rounding, no detour through float32."""

    m, ex = np.frexp(np.asarray(x, np.float64))
    return np.ldexp(np.round(np.ldexp(m, 8)), ex - 8)


def grouped_mlp_bound(sorted_context: np.ndarray, offsets: np.ndarray, gate_w, gate_b, value_w, value_b, out_w,
                      out_b) -> tuple[np.ndarray, np.ndarray]:
    """The bf16 grouped GLU FFN (moe_kernels.cu:147-199 contract) in float64
    with the hidden activations stored as bf16 (one rounding), and for every
    output the error a bf16-operand, fp32-accumulating implementation is
    allowed against it. Returns (y [P, D] float64, bound [P, D]); rows past
    offsets[-1] are zero with bound 0.

    bound = ulp(y) / 2 + 2^-7 sqrt(sum_k (h_k W_o[j, k])^2)
            + 4 sqrt(H) 2^-24 (sum_k |h_k W_o[j, k]| + |b_o[j]|)

    * ulp(y) / 2: the output's rounding to bf16 (ulp of bf16 at |y|);
    * the hidden term: a stored hidden value may round to the neighbouring
      bf16 value where the implementation's fp32 sums of the first GEMM land
      on the other side of a rounding boundary, a change of at most one bf16
      ulp (2^-7 |h_k|); such changes have independent signs, so their effect
      on an output is bounded by the root of the sum of squares (if every
      hidden value moved by a full ulp), not by the sum;
    * the accumulation term: the second GEMM's fp32 sum over H terms in any
      order, Higham's sqrt(n) rounding-error model with a factor of 4.

    A worst-case bound (gamma_n = n u for both GEMMs and every hidden value
    that could round either way taken at its full ulp in the same direction)
    is above 0.19 |y| at C4, which checks nothing. The largest ratio of
    |y_gpu - y| to this bound measured at C4 (65,536 pairs x 1024 outputs)
    is 0.33."""

    u = 2.0 ** -24
    x = np.asarray(sorted_context, np.float64)
    D = np.asarray(out_w).shape[1]
    y = np.zeros((x.shape[0], D), np.float64)
    bound = np.zeros_like(y)
    off = np.asarray(offsets, np.int64)
    for e in range(off.shape[0] - 1):
        lo, hi = int(off[e]), int(off[e + 1])
        if hi <= lo:
            continue
        xe = x[lo:hi]
        wg, wv, wo = (np.asarray(w[e], np.float64) for w in (gate_w, value_w, out_w))
        bg, bv, bo = (np.asarray(b[e], np.float64) for b in (gate_b, value_b, out_b))
        g = xe @ wg.T + bg
        v = xe @ wv.T + bv
        hb = round_bf16_f64(g / (1.0 + np.exp(-g)) * v)
        ye = hb @ wo.T + bo
        rms = np.sqrt((hb * hb).astype(np.float32) @ (wo * wo).T.astype(np.float32))
        s2 = np.abs(hb).astype(np.float32) @ np.abs(wo).T.astype(np.float32) + np.abs(bo)
        _, ex = np.frexp(ye)
        y[lo:hi] = ye
        bound[lo:hi] = np.ldexp(1.0, ex - 9) + 2.0 ** -7 * rms + 4.0 * math.sqrt(hb.shape[1]) * u * s2
    return y, bound


def combine(expert_outputs: np.ndarray, sorted_rows: np.ndarray, offsets: np.ndarray, token_count: int,
            top_k: int, pair_weights: np.ndarray | None = None) -> np.ndarray:
    """combine_topk (moe_kernels.cu:201-229; router.py:73): out[t] = sum over valid
    sorted pairs of y * (1/k or w), accumulated in float32 in ascending pair order."""

    y = np.asarray(expert_outputs, dtype=np.float32)
    out = np.zeros((token_count, y.shape[1]), dtype=np.float32)
    valid_pairs = int(np.asarray(offsets)[-1])
    for i in range(valid_pairs):
        t = int(sorted_rows[i])
        contribution = y[i] * np.float32(pair_weights[i]) if pair_weights is not None else y[i] / np.float32(top_k)
        out[t] = out[t] + contribution
    return out


def previous_token_ids(input_ids: np.ndarray, valid: np.ndarray, carried: np.ndarray) -> np.ndarray:
    """network.py:742-750: the previous valid token of each position, or the carried
    last token before the first valid one."""

    B, L = input_ids.shape
    out = np.empty_like(input_ids)
    for b in range(B):
        last = carried[b]
        for t in range(L):
            out[b, t] = last
            if valid[b, t]:
                last = input_ids[b, t]
    return out

