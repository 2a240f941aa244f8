#!/usr/bin/env python3
"""Benchmark of the MI355X HERM hot path (one GPU).

Headline ("C5", the largest single-GPU
configuration): a random-initialised stack of 12 HERM blocks (width 1024,
state 1024, 16 experts top-2, byte vocabulary + PAD). One step is one prefill
of 8 x 2048 byte ids through all 12 layers in windows of 128 tokens (the state
carried from window to window), with the ids, the weights and the state
resident in HBM. The prefill runs sequence-parallel (``herm.SequencePrefill``:
each layer over all positions at once, the state carried into every window
formed by one scan, window rings and a windowed associative memory; the whole
stack replayed from one HIP graph), checked against the window-by-window
prefill (within the bf16 path's rounding), whose rate is reported beside it
with that of the wavefront schedule (``herm.WavefrontPrefill``, bit-identical
to it). ``value`` is prefill HERM tokens/s over K steps; greedy
decode tokens/s (256 steps at batch 64, fixed-shape state) is reported beside
it under ``kernels["C5.decode"]``.

``roofline`` is the prefill's dominant hand-written kernel, the grouped
expert FFN of one layer over the whole prefill, timed live with HIP events on
its launch stream over graphs of repeated launches at the exact shape (its
expert segments come from the same ids), with weights rotated so the Infinity
Cache cannot hold them.

``cpu_baseline`` is the reference's block window restated in PyTorch on the
host (oracle/herm_torch.py: the reference's forward_window formulas with its
sorted-segment expert dispatch), fp32, on all host cores, median of 5 runs
after a warmup, on one window of the same configuration (8 x 128 tokens, one
layer), scaled to the 12 layers of the stack.

Also reported under ``kernels``: the C1/C3 affine scan, the C2 step (fused
RMSNorm-SiLU + surprise + 0.9-quantile admission), the C3 RMSNorm-SiLU, the
C4 MoE route/permute/grouped-FFN/combine, the C3-shape recurrent gates and
one C5 window's salient read, each as the median per-launch time from HIP
events, GB/s or TFLOP/s and the roofline fraction, with inputs rotated over
more than 256 MiB where the working set would otherwise fit the Infinity
Cache; and the reference's PyTorch formulas for those rows on the host cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _path in (ROOT, ROOT / "koemi-5hom_amd"):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
FP32_PEAK_TFLOPS = 157.3       # MI355X dense fp32 MFMA
MALL_BYTES = 256 * 2**20       # Infinity Cache

# C5: the stack
C5_LAYERS, C5_WIDTH, C5_HIDDEN, C5_E, C5_K = 12, 1024, 2048, 16, 2
C5_BATCH, C5_LEN, C5_WINDOW = 8, 2048, 128
C5_PREFILL_TOKENS = C5_BATCH * C5_LEN
C5_DECODE_BATCH, C5_DECODE_STEPS = 64, 256
C5_PAIRS = C5_PREFILL_TOKENS * C5_K
C5_FFN_FLOP = 6 * C5_WIDTH * C5_HIDDEN * C5_PAIRS                   # GEMM 1 (gate + value) + GEMM 2, per layer
# Algorithmic HBM bytes of that FFN (bf16): the sorted context read, the gate
# and value weights, the hidden rows written and read back, the output weights
# and the output rows.
C5_FFN_BYTES = 2 * (C5_PAIRS * C5_WIDTH + 2 * C5_E * C5_HIDDEN * C5_WIDTH + 2 * C5_PAIRS * C5_HIDDEN
                    + C5_E * C5_WIDTH * C5_HIDDEN + C5_PAIRS * C5_WIDTH)

# Algorithmic bytes / FLOPs per launch of the other rows.
C2_TOKENS = 16 * 2048
C2_NORM_BYTES = 32768 * 512 * 2 * 2 + 512 * 2 + 32768 * 4            # x read, y write, gamma, inv
C2_SURPRISE_BYTES = 32768 * 256 * 4 + 32768 * 8 + 32768 + 32768 * 4   # logits, targets, valid, s
C2_ADMISSION_BYTES = 32768 * 4 + 32768 + 32768 + 4                     # s, valid, mask, tau
C1_SCAN_BYTES = 12 * 4 * 1024 * 256 + 4 * 256 * 4
C3_SCAN_BYTES = 12 * 32 * 4096 * 1024 + 32 * 1024 * 4
C3_NORM_BYTES = 131072 * 1024 * 2 * 2 + 1024 * 2 + 131072 * 4
C4_T, C4_D, C4_H, C4_E, C4_K = 32768, 1024, 2816, 16, 2
C4_PAIRS = C4_T * C4_K
C4_ROUTE_BYTES = C4_T * (8 + 8 + 1) + C4_PAIRS * 8
C4_PERMUTE_BYTES = C4_T * C4_D * 2 + C4_PAIRS * C4_D * 2 + C4_PAIRS * 8 + C4_T + 2 * C4_PAIRS * 8 + (C4_E + 1) * 8
C4_GEMM_FLOP = 6 * C4_D * C4_H * C4_PAIRS
C3G_FLOP = 2 * 2 * 32 * 4096 * 1024 * 1024                              # two width x width products
C4_COMBINE_BYTES = C4_PAIRS * C4_D * 2 + C4_T * C4_D * 2 + C4_PAIRS * 8 + (C4_E + 1) * 8


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10, help="timed C5 prefill steps (8 x 2048 tokens, 12 layers each)")
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--configs", default="1,2,3,4,5,g",
                    help="extra rows to measure (comma list of 1,2,3,4,5,g; '' for none)")
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="budget of each CPU reference row")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the C5 prefill steps (for rocprofv3 runs of the headline alone)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the C5 greedy decode steps (for rocprofv3 runs of the decode step alone); prints them "
                         "as JSON")
    ap.add_argument("--rows-only", action="store_true",
                    help="only the kernel rows of --configs (for rocprofv3 runs of one configuration's kernels); "
                         "prints them as JSON")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run each HBM kernel a few times at its config plus a device copy of known size, for "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes (prints nothing else)")
    ap.add_argument("--read-floor", action="store_true",
                    help="sweep the launch shape of a plain streaming read (koemi_stream_read) over the C2 "
                         "surprise and RMSNorm-SiLU byte counts, six rotating input sets each, and print the "
                         "fastest shapes as JSON (the floor the memory-bound C2 kernels are judged against)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn the two --pmc passes over --traffic-probe into profiles/traffic.json")
    return ap.parse_args()


def roofline(achieved: float, peak: float, unit: str, bound: str, traffic) -> dict:
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def load_traffic(kernel: str):
    """HBM bytes per launch from the committed rocprofv3 counter summary, if any."""

    path = ROOT / "profiles" / "traffic.json"
    if not path.is_file():
        return None
    try:
        return json.loads(path.read_text()).get(kernel, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


# Kernels of the traffic probe: name fragment in the rocprofv3 kernel name -> bench key
# and algorithmic bytes per launch.
# (The PMC passes run rocprofv3 with --mangled-kernels, so the fragments are
# parts of mangled names.)
TRAFFIC_KERNELS = {
    ("rmsnorm_silu_fwd_groupIDF16bLi4ELi16ELb0E",): ("C2.rmsnorm_silu", C2_NORM_BYTES),
    ("surprise_rows16_kernel",): ("C2.surprise_rows", C2_SURPRISE_BYTES),
    ("scan_forward_wide_kernel",): ("C3.affine_scan", C3_SCAN_BYTES),
    ("rmsnorm_silu_fwd_groupIDF16bLi4ELi32ELb1E",): ("C3.rmsnorm_silu", C3_NORM_BYTES),
    ("permute_gather_kernel",): ("C4.permute_gather", C4_T * C4_D * 2 + C4_PAIRS * C4_D * 2 + C4_PAIRS * 8),
    ("combine_rows_small_kernel",): ("C4.combine_rows", C4_PAIRS * C4_D * 2 + C4_T * C4_D * 2 + C4_PAIRS * 8),
}
# Groups of the traffic probe: every launch of these kernels belongs to one of
# `calls` calls of the group's operation -> bench key, calls, algorithmic bytes
# per call.
TRAFFIC_GROUPS = {
    ("grouped_gemm_bf16_kernel", "split_fixup_kernel", "build_schedule_kernel", "zero_tail_rows_kernel"):
        ("C5.expert_ffn_layer", 3, C5_FFN_BYTES),
}
COPY_BYTES = 512 * 2**20  # the calibration copy reads and writes this many bytes


def median_s(fn, runs: int = 5, budget_s: float = 1e9) -> tuple[float, int]:
    """Median wall time of ``fn`` over ``runs`` runs after one warmup (fewer
    runs, never below one, if ``budget_s`` is spent first)."""

    fn()
    times, t0 = [], time.perf_counter()
    while len(times) < runs and (not times or time.perf_counter() - t0 < budget_s):
        t1 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t1)
    return statistics.median(times), len(times)


def cpu_stack_baseline(threads: int, ids_window, decode_ids) -> dict:
    """The C5 CPU baseline: oracle/herm_torch.py's block window (the
    reference's forward_window formulas, fp32) on the host cores, one layer
    of the stack's shapes with its own seeded fp32 weights; tokens/s of the
    12-layer stack = window tokens / (12 x the median window time)."""

    import torch

    from koemi_amd import herm
    from oracle import herm_torch

    torch.set_num_threads(threads)
    settings = herm.HermSettings(layers=1)
    p = herm.init_stack(settings, 1005, "cpu")[0]
    cfg = settings.oracle_config()

    def state(batch):
        return {k: v.cpu() for k, v in herm.initial_states(settings, batch, torch.device("cpu"))[0].items()}

    prefill_state = state(ids_window.shape[0])
    decode_state = state(decode_ids.shape[0])
    with torch.inference_mode():
        window_s, runs = median_s(lambda: herm_torch.block_window(p, prefill_state, ids_window, cfg), 5)
        step_s, step_runs = median_s(lambda: herm_torch.block_window(p, decode_state, decode_ids, cfg), 5)
    tokens = ids_window.numel()
    return {
        "value": round(tokens / (C5_LAYERS * window_s), 1),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"one C5 prefill window ({ids_window.shape[0]} x {ids_window.shape[1]} tokens) through one layer, "
                   f"oracle/herm_torch.py fp32 on {threads} threads, median of {runs} runs after a warmup: "
                   f"{window_s * 1e3:.1f} ms; value = tokens / (12 layers x that)"),
        "decode": {"tokens_per_s": round(decode_ids.numel() / (C5_LAYERS * step_s), 1),
                   "ms_per_layer_step": round(step_s * 1e3, 3), "runs": step_runs,
                   "sample": f"one decode position at batch {decode_ids.shape[0]} through one layer, x12 layers"},
    }


def cpu_reference_times(extra: list, threads: int, budget_s: float) -> dict:
    """The reference's PyTorch formulas for each measured kernel row, on the host cores.

    Each is timed on a bounded sample of its configuration (median of up to
    five runs after one warmup, within ``budget_s`` per row) and scaled to the
    full configuration by the sample's share of the work; the samples have the
    configuration's shapes and distributions.
    """

    import torch
    import torch.nn.functional as F

    from oracle import herm_torch

    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(99)
    out = {}

    def median_ms(fn) -> float:
        return median_s(fn, 5, budget_s)[0] * 1000.0

    def seq_scan(a, b):  # the tests' sequential recurrence (test_dense_cuda.py:21-33)
        h = torch.zeros_like(a[:, 0])
        res = torch.empty_like(a)
        for t in range(a.shape[1]):
            h = a[:, t] * h + b[:, t]
            res[:, t] = h
        return res

    def hillis_steele(a, b):  # the model path, model/scan.py:17-30
        return herm_torch.window_scan(a, b, torch.zeros_like(a[:, 0]))

    if "1" in extra:
        a = torch.rand((4, 1024, 256), generator=g) * 0.199 + 0.8
        b = torch.randn((4, 1024, 256), generator=g)
        out["C1.affine_scan"] = {"ms": round(median_ms(lambda: seq_scan(a, b)), 3), "sample": "full C1, sequential loop",
                                 "ms_model_path": round(median_ms(lambda: hillis_steele(a, b)), 3)}
    if "2" in extra:
        from koemi_amd import workloads

        c = workloads.config2()
        x2, g2 = c.x.float(), c.gamma.float()

        def c2_step():  # layers.py:14-16 + F.silu; network.py:677-688; quantile admission
            F.silu(x2 * torch.rsqrt(x2.square().mean(dim=-1, keepdim=True) + 1e-6) * g2)
            nll = F.cross_entropy(c.logits, c.targets, reduction="none")
            s = torch.where(c.valid, 1.0 - torch.exp(-(nll / math.log(256))), torch.zeros(()))
            return s > torch.quantile(s, 0.9)

        out["C2.step"] = {"ms": round(median_ms(c2_step), 3), "sample": "full C2 step, fp32"}
    if "3" in extra:
        a = torch.sigmoid(torch.randn((1, 4096, 1024), generator=g) + 2.0)
        b = 0.5 * torch.randn((1, 4096, 1024), generator=g)
        out["C3.affine_scan"] = {"ms": round(32 * median_ms(lambda: seq_scan(a, b)), 3),
                                 "sample": "1 of the 32 sequences, sequential loop, x32",
                                 "ms_model_path": round(32 * median_ms(lambda: hillis_steele(a, b)), 3)}
        del a, b
        x = torch.randn((8192, 1024), generator=g).to(torch.bfloat16)
        gam = (1 + 0.02 * torch.randn((1024,), generator=g)).to(torch.bfloat16)

        def norm():  # core/rmsnorm_silu.py fallback formula (layers.py:14-16 + F.silu), fp32
            xf = x.float()
            return F.silu(xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + 1e-6) * gam.float()).to(x.dtype)

        out["C3.rmsnorm_silu"] = {"ms": round(16 * median_ms(norm), 3), "sample": "8192 of 131072 rows, x16"}
    if "4" in extra:
        T, D, H, E, K = C4_T, C4_D, C4_H, C4_E, C4_K
        tok = torch.randint(0, 256, (T,), generator=g)
        prev = torch.cat((torch.tensor([256]), tok[:-1]))
        valid = torch.ones((T,), dtype=torch.bool)

        def route():  # experts.py:30-38, 283-289 (int64)
            h = herm_torch.content_hash(tok, prev)
            e = (h.unsqueeze(-1) + torch.arange(K) * herm_torch.SLOT_OFFSET).remainder(E)
            return e.masked_fill(~valid.unsqueeze(-1), -1)

        out["C4.route_hash"] = {"ms": round(median_ms(route), 3), "sample": "full C4"}
        assign = route()
        ctx = torch.randn((T, D), generator=g).to(torch.bfloat16)

        def permute():  # experts.py:189-197: stable argsort by expert, gather rows
            keys = torch.where(assign >= 0, assign, torch.full_like(assign, E)).reshape(-1)
            order = torch.argsort(keys, stable=True)
            return ctx[order // K], order

        out["C4.permute"] = {"ms": round(median_ms(permute), 3), "sample": "full C4"}
        rows_e = 4096 // E  # a slice of the sorted pairs, equal per expert
        xs = torch.randn((E, rows_e, D), generator=g).to(torch.bfloat16)
        wg = (0.02 * torch.randn((E, H, D), generator=g)).to(torch.bfloat16)
        wv = (0.02 * torch.randn((E, H, D), generator=g)).to(torch.bfloat16)
        wo = (0.02 * torch.randn((E, D, H), generator=g)).to(torch.bfloat16)

        def ffn():  # GatedFeedForward per expert (layers.py:27-29), fp32 on the host
            for e in range(E):
                xe = xs[e].float()
                hgl = F.silu(xe @ wg[e].float().T) * (xe @ wv[e].float().T)
                _ = hgl @ wo[e].float().T

        out["C4.grouped_glu_ffn"] = {"ms": round(C4_PAIRS / 4096 * median_ms(ffn), 3),
                                     "sample": "4096 of 65536 pairs (256 per expert), fp32, x16"}
        del wg, wv, wo
        y = torch.randn((C4_PAIRS, D), generator=g).to(torch.bfloat16)
        idx = torch.arange(C4_PAIRS) // K

        def combine():  # moe_kernels.cu:201-229 semantics: sum of y / k per token
            acc = torch.zeros((T, D), dtype=torch.float32)
            acc.index_add_(0, idx, y.float() / K)
            return acc.to(torch.bfloat16)

        out["C4.combine"] = {"ms": round(median_ms(combine), 3), "sample": "full C4"}
    if "g" in extra:
        ug = torch.randn((8192, 1024), generator=g)
        lin_r, lin_c = torch.nn.Linear(1024, 1024), torch.nn.Linear(1024, 1024)

        def gates():  # BoundedRecurrentState.gates, model/memory.py:14-30
            with torch.no_grad():
                bounded = 2.0**-8 + ((1.0 - 2.0**-8) - 2.0**-8) * torch.sigmoid(lin_r(ug))
                return bounded, (1.0 - bounded) * torch.tanh(lin_c(ug))

        out["C3g.recurrent_gates"] = {"ms": round(16 * median_ms(gates), 3), "sample": "8192 of 131072 rows, x16"}
    if "5" in extra:
        b5, s5, l5, d5 = 8, 16, 128, 1024
        ck, cv = torch.randn((b5, s5, d5), generator=g), torch.randn((b5, s5, d5), generator=g)
        k5, v5, q5 = (torch.randn((b5, l5, d5), generator=g) for _ in range(3))
        cvalid, adm = torch.rand((b5, s5), generator=g) < 0.8, torch.rand((b5, l5), generator=g) < 0.1
        pos = torch.arange(l5)
        elig = torch.cat((cvalid.unsqueeze(1).expand(b5, l5, s5),
                          adm.unsqueeze(1) & (pos.unsqueeze(1) > pos.unsqueeze(0)).unsqueeze(0)), dim=-1)
        all_k, all_v = torch.cat((ck, k5), dim=1), torch.cat((cv, v5), dim=1)
        out["C5w.salient_read"] = {  # model/memory.py:405-429
            "ms": round(median_ms(lambda: herm_torch.masked_attention(all_k, all_v, q5, elig)), 3),
            "sample": "full C5 window"}
    return out


def traffic_probe() -> int:
    """Launch each HBM kernel at its configuration (and one device copy of known size)."""

    import torch

    from koemi_amd import core, dense, moe, think, workloads

    device = torch.device("cuda:0")
    src = torch.ones(COPY_BYTES // 4, device=device)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    c2 = workloads.config2()
    x, gamma = c2.x.to(device), c2.gamma.to(device)
    logits, targets, valid = c2.logits.to(device), c2.targets.to(device), c2.valid.to(device)
    for _ in range(3):
        core.rmsnorm_silu_forward(x, gamma, 1e-6)
        think.surprise_from_logits(logits, targets, valid)
    c3 = workloads.to_device(workloads.config3(), device)
    for _ in range(3):
        h = dense.scan_forward(c3.retention, c3.increment, c3.initial)
    hb = h.to(torch.bfloat16).view(-1, 1024)
    del c3, h
    g3 = workloads.config3(batch=1, seq=1, width=1024).gamma.to(device)
    for _ in range(3):
        core.rmsnorm_silu_forward(hb, g3, 1e-6)
    del hb
    c4 = workloads.to_device(workloads.config4(), device)
    a_l, w_l = moe.route_topk_learned(c4.router_logits, c4.valid, top_k=2)
    for _ in range(3):
        sc, rows, experts, offsets, sw = moe.permute_topk(c4.context, a_l, c4.valid, expert_count=16, pair_weights=w_l)
    for _ in range(3):
        moe.combine_topk(sc, rows, offsets, token_count=C4_T, top_k=2, pair_weights=sw)
    del c4, sc, rows, experts, offsets, sw
    # The C5 expert FFN of one layer over the prefill, as the bench times it:
    # hash-routed byte ids, the sorted bf16 context, one layer's weights
    # (N(0, 0.02)); TRAFFIC_GROUPS counts its three calls.
    from koemi_amd import herm

    g = torch.Generator(device=device).manual_seed(5)
    ids = torch.randint(0, 256, (C5_BATCH, C5_LEN), generator=g, device=device)
    valid5 = ids != herm.PAD_TOKEN_ID
    prev5 = torch.cat((torch.full_like(ids[:, :1], herm.PAD_TOKEN_ID), ids[:, :-1]), dim=1)
    assign5 = moe.route_topk_valid(ids, prev5, valid5, expert_count=C5_E, top_k=C5_K)
    ctx5 = torch.randn((C5_PREFILL_TOKENS, C5_WIDTH), generator=g, device=device).to(torch.bfloat16)
    sc5, _, experts5, offsets5 = moe.permute_topk(ctx5, assign5.reshape(-1, C5_K), valid5.reshape(-1),
                                                  expert_count=C5_E)
    shapes = ((C5_E, C5_HIDDEN, C5_WIDTH), (C5_E, C5_HIDDEN), (C5_E, C5_HIDDEN, C5_WIDTH), (C5_E, C5_HIDDEN),
              (C5_E, C5_WIDTH, C5_HIDDEN), (C5_E, C5_WIDTH))
    w5 = [(0.02 * torch.randn(shape, generator=g, device=device)).to(torch.bfloat16) for shape in shapes]
    torch.cuda.synchronize()
    for _ in range(3):
        moe.grouped_expert_mlp_inference(sc5, experts5, offsets5, *w5, validate=False)
    torch.cuda.synchronize()
    return 0


def summarize_pmc(fetch_dir: str, write_dir: str) -> int:
    """profiles/traffic.json from rocprofv3 counter_collection.csv files of FETCH_SIZE and WRITE_SIZE."""

    import csv

    def per_kernel(directory: str, counter: str) -> dict:
        rows = []
        for path in Path(directory).rglob("*counter_collection.csv"):
            with path.open() as fh:
                rows += [r for r in csv.DictReader(fh) if r["Counter_Name"] == counter]
        out = {}
        for r in rows:
            out.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return out

    fetch, write = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")

    def find(table: dict, fragments):
        vals = [v for name, vs in table.items() if any(f in name for f in fragments) for v in vs]
        return statistics.median(vals) if vals else None

    # The calibration copy is the largest device-to-device copy (hipMemcpy's blit kernel).
    copy_fetch = max(v for name, vs in fetch.items() if "copyBuffer" in name for v in vs)
    copy_write = max(v for name, vs in write.items() if "copyBuffer" in name for v in vs)
    fetch_scale = COPY_BYTES / (copy_fetch * 1024.0)
    write_scale = COPY_BYTES / (copy_write * 1024.0)
    result = {"_calibration": {"copy_bytes": COPY_BYTES, "copy_fetch_kib": copy_fetch, "copy_write_kib": copy_write,
                               "fetch_scale": round(fetch_scale, 4), "write_scale": round(write_scale, 4)}}
    for fragments, (key, algorithmic) in TRAFFIC_KERNELS.items():
        f, w = find(fetch, fragments), find(write, fragments)
        if f is None or w is None:
            continue
        read_b = f * 1024.0 * fetch_scale
        write_b = w * 1024.0 * write_scale
        result[key] = {"fetch_kib": f, "write_kib": w, "bytes_per_launch": round(read_b + write_b),
                       "algorithmic_bytes": algorithmic, "ratio": round((read_b + write_b) / algorithmic, 4)}
    for fragments, (key, calls, algorithmic) in TRAFFIC_GROUPS.items():
        f = sum(v for name, vs in fetch.items() if any(x in name for x in fragments) for v in vs)
        w = sum(v for name, vs in write.items() if any(x in name for x in fragments) for v in vs)
        if f == 0 or w == 0:
            continue
        read_b = f * 1024.0 * fetch_scale / calls
        write_b = w * 1024.0 * write_scale / calls
        result[key] = {"fetch_kib": round(f / calls, 1), "write_kib": round(w / calls, 1),
                       "bytes_per_launch": round(read_b + write_b), "algorithmic_bytes": algorithmic,
                       "ratio": round((read_b + write_b) / algorithmic, 4),
                       "note": f"sum over the {', '.join(fragments)} launches of one call"}
    out = ROOT / "profiles" / "traffic.json"
    out.write_text(json.dumps(result, indent=1) + "\n")
    print(json.dumps(result, indent=1))
    return 0


def window_by_window_rows(args, herm, params, settings, ids, start_states, kernels: dict):
    """The C5 prefill window by window (every layer of a window in one HIP
    graph, windows in turn) and as a wavefront over per-layer streams
    (bit-identical to it): rates into ``kernels``; returns its logits."""

    import torch

    log("C5: window-by-window graphed prefill (eager first window for the replay check)")
    eager_logits, _ = herm.stack_window(params, settings, ids[:, :C5_WINDOW].contiguous(),
                                        herm.initial_states(settings, C5_BATCH, ids.device))
    sequential, _, graph = herm.prefill_graphed(params, settings, ids, start_states)
    torch.cuda.synchronize()
    replay_vs_eager = float((sequential[:, :C5_WINDOW] - eager_logits).abs().max() / eager_logits.abs().max())
    assert replay_vs_eager < 1e-5, f"graph replay differs from the eager window: {replay_vs_eager:.3e}"
    assert torch.isfinite(sequential).all(), "non-finite prefill logits"
    seq_steps = 3
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(seq_steps):
        logits, _, graph = herm.prefill_graphed(params, settings, ids, start_states, graph)
    torch.cuda.synchronize()
    seq_ms = (time.perf_counter() - t0) * 1000.0 / seq_steps
    assert torch.equal(logits, sequential), "window-by-window prefill is not reproducible"
    kernels["C5.prefill_window_by_window"] = {"ms_per_step": round(seq_ms, 4),
                                              "tokens_per_s": round(C5_PREFILL_TOKENS / (seq_ms / 1000.0), 1),
                                              "replay_vs_eager_rel": replay_vs_eager,
                                              "note": "every layer of a window in one HIP graph, windows in turn"}
    del graph, logits, eager_logits

    log("C5: wavefront prefill (per-layer streams): capture and equality with the window-by-window prefill")
    wave = herm.WavefrontPrefill(params, settings, start_states, C5_BATCH, ids.device)
    logits = wave.run(ids)
    torch.cuda.synchronize()
    assert torch.equal(logits, sequential), "wavefront prefill differs from the window-by-window prefill"
    t0 = time.perf_counter()
    for _ in range(seq_steps):
        logits = wave.run(ids)
    torch.cuda.synchronize()
    wave_ms = (time.perf_counter() - t0) * 1000.0 / seq_steps
    kernels["C5.prefill_wavefront"] = {"ms_per_step": round(wave_ms, 4),
                                       "tokens_per_s": round(C5_PREFILL_TOKENS / (wave_ms / 1000.0), 1),
                                       "note": "window-by-window graphs of each layer on per-layer streams, "
                                               "bit-identical to the window-by-window prefill"}
    del wave, logits
    return sequential


class Timer:
    """Median per-launch GPU time of an operator: ``per_graph`` launches
    captured in one HIP graph (cycling over input sets), the graph replayed
    ``reps`` times with an event pair around each replay on the launch
    stream; every graph gets its own memory pool."""

    def __init__(self, torch, stream):
        self.torch = torch
        self.stream = stream

    def per_launch_ms(self, fns: list, per_graph: int, reps: int) -> float:
        torch = self.torch
        for fn in fns:  # eager warmup: libraries pick their kernels outside the capture
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(per_graph):
                fns[i % len(fns)]()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(reps):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(self.stream)
            g.replay()
            end.record(self.stream)
            end.synchronize()
            times.append(start.elapsed_time(end) / per_graph)
        del g
        return statistics.median(times)


def kernel_rows(args, extra: list, device, stream, timer, kernels: dict) -> None:
    """The per-kernel rows of the configurations in ``extra`` (1, 2, 3, 4, 5, g) into ``kernels``."""

    import torch

    from koemi_amd import core, dense, memory, moe, recurrent, think, workloads

    iters = args.kernel_iters

    # ---------------------------------------------------------------- C2 step
    if "2" in extra:
        log("C2: RMSNorm-SiLU + surprise + 0.9-quantile admission")
        per_set = C2_NORM_BYTES + C2_SURPRISE_BYTES + C2_ADMISSION_BYTES
        n_sets = max(2, math.ceil(2 * MALL_BYTES / per_set))
        sets = []
        for i in range(n_sets):
            c = workloads.config2(seed=1002 + i)
            sets.append({k: getattr(c, k).to(device) for k in ("x", "gamma", "logits", "targets", "valid")})
        for d in sets:
            s = think.surprise_from_logits(d["logits"], d["targets"], d["valid"])
            d["s"] = s
            d["want"] = tuple(t.clone() for t in (*core.rmsnorm_silu_forward(d["x"], d["gamma"], 1e-6), s,
                                                  *think.salience_admission(s, d["valid"], quantile=0.9)))

        def c2_step(d):
            y, inv = core.rmsnorm_silu_forward(d["x"], d["gamma"], 1e-6)
            s = think.surprise_from_logits(d["logits"], d["targets"], d["valid"])
            mask, tau = think.salience_admission(s, d["valid"], quantile=0.9)
            return y, inv, s, mask, tau

        # the step, replayed from one graph of 2 x n_sets steps; outputs compared with the eager ones
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs = [c2_step(sets[i % n_sets]) for i in range(2 * n_sets)]
        torch.cuda.synchronize()
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        for i, out in enumerate(outs):
            for got, want in zip(out, sets[i % n_sets]["want"]):
                assert torch.equal(got, want), "C2 graph replay differs from the eager step"
        reps = max(5, iters)
        times = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            g.replay()
            b.record(stream)
            b.synchronize()
            times.append(a.elapsed_time(b) / (2 * n_sets))
        step_ms = statistics.median(times)
        del g, outs
        c2_rows = {
            "rmsnorm_silu": ([lambda d=d: core.rmsnorm_silu_forward(d["x"], d["gamma"], 1e-6) for d in sets],
                             C2_NORM_BYTES),
            "surprise_rows": ([lambda d=d: think.surprise_from_logits(d["logits"], d["targets"], d["valid"])
                               for d in sets], C2_SURPRISE_BYTES),
            "quantile_admission": ([lambda d=d: think.salience_admission(d["s"], d["valid"], quantile=0.9)
                                    for d in sets], C2_ADMISSION_BYTES),
        }
        kernels["C2.step"] = {"ms": round(step_ms, 5), "tokens_per_s": round(C2_TOKENS / (step_ms / 1e3), 1),
                              "input_sets": n_sets}
        for name, (fns, nbytes) in c2_rows.items():
            ms = timer.per_launch_ms(fns, 2 * n_sets, reps)
            gbs = nbytes / ms / 1e6
            kernels[f"C2.{name}"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        del sets

    if "1" in extra:
        log("C1 scan")
        c1 = workloads.to_device(workloads.config1(), device)
        ms = timer.per_launch_ms([lambda: dense.scan_forward(c1.retention, c1.increment, c1.initial)], 20, iters)
        kernels["C1.affine_scan"] = {"ms": round(ms, 5), "GB/s": round(C1_SCAN_BYTES / ms / 1e6, 1),
                                     "frac_hbm": round(C1_SCAN_BYTES / ms / 1e6 / HBM_PEAK_GBS, 4),
                                     "note": "12.6 MB working set is launch-bound and fits the Infinity Cache"}
        del c1
    if "3" in extra:
        log("C3 scan + norm (generating 1.6 GB of inputs)")
        c3 = workloads.to_device(workloads.config3(), device)
        ms = timer.per_launch_ms([lambda: dense.scan_forward(c3.retention, c3.increment, c3.initial)], 4,
                                 max(5, iters // 2))
        gbs = C3_SCAN_BYTES / ms / 1e6
        kernels["C3.affine_scan"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                     "tokens_per_s": round(32 * 4096 / (ms / 1000.0))}
        h = dense.scan_forward(c3.retention, c3.increment, c3.initial).to(torch.bfloat16).view(-1, 1024)
        del c3
        hs = [h, h.clone()]  # two 268 MB inputs in turn: the second is not in the Infinity Cache after the first
        gamma = workloads.config3(batch=1, seq=1, width=1024).gamma.to(device)
        ms = timer.per_launch_ms([lambda x=x: core.rmsnorm_silu_forward(x, gamma, 1e-6) for x in hs], 8, iters)
        gbs = C3_NORM_BYTES / ms / 1e6
        kernels["C3.rmsnorm_silu"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                      "note": "two input copies alternate"}
        del h, hs
    if "4" in extra:
        log("C4 MoE (generating inputs)")
        c4 = workloads.to_device(workloads.config4(), device)
        ms = timer.per_launch_ms([lambda: moe.route_topk_valid(c4.token_ids, c4.previous_token_ids, c4.valid,
                                                               expert_count=16, top_k=2, validate=False)], 20, iters)
        kernels["C4.route_hash"] = {"ms": round(ms, 5), "GB/s": round(C4_ROUTE_BYTES / ms / 1e6, 1)}
        assign = moe.route_topk_valid(c4.token_ids, c4.previous_token_ids, c4.valid, expert_count=16, top_k=2)
        ctxs = [c4.context, c4.context.clone(), c4.context.clone()]  # 3 x 67 MB contexts + their 134 MB outputs
        ms = timer.per_launch_ms([lambda x=x: moe.permute_topk(x, assign, c4.valid, expert_count=16, validate=False)
                                  for x in ctxs], 6, iters)
        gbs = C4_PERMUTE_BYTES / ms / 1e6
        kernels["C4.permute"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                 "note": "three context copies in turn"}
        a_l, w_l = moe.route_topk_learned(c4.router_logits, c4.valid, top_k=2)
        sc, rows, experts, offsets, sw = moe.permute_topk(c4.context, a_l, c4.valid, expert_count=16, pair_weights=w_l)
        del ctxs
        weights = (c4.gate_weights, c4.gate_biases, c4.value_weights, c4.value_biases, c4.output_weights,
                   c4.output_biases)
        ms = timer.per_launch_ms([lambda: moe.grouped_expert_mlp_inference(sc, experts, offsets, *weights,
                                                                           validate=False)], 4, max(5, iters // 2))
        tflops = C4_GEMM_FLOP / ms / 1e9
        kernels["C4.grouped_glu_ffn"] = {"ms": round(ms, 5), "TFLOP/s": round(tflops, 1),
                                         "frac_mfma_bf16": round(tflops / BF16_PEAK_TFLOPS, 4)}
        ys = [moe.grouped_expert_mlp_inference(sc, experts, offsets, *weights, validate=False) for _ in range(2)]
        ms = timer.per_launch_ms([lambda y=y: moe.combine_topk(y, rows, offsets, token_count=C4_T, top_k=2,
                                                               pair_weights=sw, validate=False) for y in ys], 6, iters)
        gbs = C4_COMBINE_BYTES / ms / 1e6
        kernels["C4.combine"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                 "note": "two expert-output copies in turn"}
        # practical bf16 GEMM ceiling of the platform library at the same total shape
        a_mat = torch.randn((C4_PAIRS, C4_D), device=device, dtype=torch.bfloat16)
        b_mat = torch.randn((C4_D, 2 * C4_H), device=device, dtype=torch.bfloat16)
        ms = timer.per_launch_ms([lambda: torch.matmul(a_mat, b_mat)], 4, 10)
        kernels["hipblaslt_reference_gemm"] = {"shape": [C4_PAIRS, C4_D, 2 * C4_H],
                                               "TFLOP/s": round(2 * C4_PAIRS * C4_D * 2 * C4_H / ms / 1e9, 1)}
        del c4, sc, ys, a_mat, b_mat

    if "5" in extra:
        # One window's salient read at the C5 model shape (8 sequences, scan
        # window 128, 16 salient slots, width 1024, fp32), as network.py:350-358
        # issues it once per window.
        log("C5 window salient read")
        g5 = torch.Generator(device=device).manual_seed(1005)
        b5, s5, l5, d5 = 8, 16, 128, 1024
        r5 = lambda *shape: torch.randn(shape, generator=g5, device=device)
        ck, cv, k5, v5, q5 = r5(b5, s5, d5), r5(b5, s5, d5), r5(b5, l5, d5), r5(b5, l5, d5), r5(b5, l5, d5)
        cvalid = torch.rand((b5, s5), generator=g5, device=device) < 0.8
        adm5 = torch.rand((b5, l5), generator=g5, device=device) < 0.1
        ms = timer.per_launch_ms([lambda: memory.read_salient_window(ck, cv, cvalid, k5, v5, adm5, q5)], 20, iters)
        flop = 4 * b5 * l5 * (s5 + l5) * d5
        kernels["C5w.salient_read"] = {"ms": round(ms, 5), "TFLOP/s": round(flop / ms / 1e9, 2),
                                       "shape_b_l_s_d": [b5, l5, s5, d5]}
        del ck, cv, k5, v5, q5

    if "g" in extra:
        # The recurrent gates and the window scan at the C3 shape ([32, 4096, 1024]
        # fp32), the step before the C3 scan (network.py:306-310).
        log("C3g recurrent gates + scan (generating 0.5 GiB of inputs)")
        gg = torch.Generator(device=device).manual_seed(1006)
        ug = torch.randn((32, 4096, 1024), generator=gg, device=device)
        wts = [(1024 ** -0.5) * torch.randn(shape, generator=gg, device=device)
               for shape in ((1024, 1024), (1024,), (1024, 1024), (1024,))]
        vg = torch.ones((32, 4096), dtype=torch.bool, device=device)
        ms = timer.per_launch_ms([lambda: recurrent.recurrent_gates(ug, *wts, vg)], 2, max(3, iters // 4))
        kernels["C3g.recurrent_gates"] = {"ms": round(ms, 5), "TFLOP/s": round(C3G_FLOP / ms / 1e9, 1),
                                          "frac_mfma_fp32": round(C3G_FLOP / ms / 1e9 / FP32_PEAK_TFLOPS, 4)}
        ms = timer.per_launch_ms([lambda: recurrent.recurrent_scan(ug, *wts, vg)], 2, max(3, iters // 4))
        kernels["C3g.recurrent_scan"] = {"ms": round(ms, 5), "tokens_per_s": round(32 * 4096 / (ms / 1000.0)),
                                         "note": "the gate GEMMs, then the gates formed inside the affine scan"}
        # The same step for a bf16 window under autocast (the HERM block's case):
        # the gate projection on bf16 MFMA with the gates and the scan in its
        # epilogue, the pre-activations never in memory (koemi_gated_projection_scan).
        ub = ug.to(torch.bfloat16)
        del ug
        wb = torch.cat((wts[0], wts[2])).to(torch.bfloat16)
        bb = torch.cat((wts[1], wts[3])).to(torch.bfloat16)
        h0g = torch.zeros((32, 1024), device=device)
        gp_status = torch.zeros(1, device=device, dtype=torch.int32)  # a timed-out carry wait reports here
        ms = timer.per_launch_ms([lambda: recurrent.gated_projection_scan(ub, wb, bb, vg, h0g, with_bf16=True,
                                                                          status=gp_status)], 2, max(3, iters // 4))
        recurrent.check_gated_scan_status(gp_status)
        kernels["C3g.gated_projection_scan_bf16"] = {
            "ms": round(ms, 5), "TFLOP/s": round(C3G_FLOP / ms / 1e9, 1),
            "frac_mfma_bf16": round(C3G_FLOP / ms / 1e9 / BF16_PEAK_TFLOPS, 4),
            "note": "bf16 inputs and weights; fp32 states and their bf16 copy written; one kernel (+ its workspace clear)"}
        del ub, wb, bb, wts, vg



def decode_rows(herm, params, settings, c5, device, kernels: dict) -> None:
    """C5 greedy decode at batch 64: DecodeGraph steps, 3 untimed then
    C5_DECODE_STEPS timed, into kernels["C5.decode"]."""

    import torch

    log(f"C5: greedy decode, batch {C5_DECODE_BATCH}, {C5_DECODE_STEPS} steps")
    decode = herm.DecodeGraph(params, settings, c5.decode_ids.to(device),
                              herm.initial_states(settings, C5_DECODE_BATCH, device))
    for _ in range(3):
        decode.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(C5_DECODE_STEPS):
        decode.step()
    torch.cuda.synchronize()
    decode_s = time.perf_counter() - t0
    kernels["C5.decode"] = {"ms_per_step": round(decode_s * 1e3 / C5_DECODE_STEPS, 4),
                            "tokens_per_s": round(C5_DECODE_BATCH * C5_DECODE_STEPS / decode_s, 1),
                            "shape": "12 layers, batch 64, 256 greedy steps, PAD masked, one HIP graph per step"}


def read_floor() -> int:
    """The fastest plain read of the C2 surprise input (34,013,184 bytes) and of
    the C2 RMSNorm-SiLU input (33,554,432 bytes read of its 67 MB) over a
    sweep of launch shapes (16-byte loads, 1-8 per thread per pass, 256-1024
    threads per workgroup, 256 workgroups up to one pass over the data), six
    rotating input sets (204 MB, beyond the 256 MB Infinity Cache's reach for
    any one set between its uses), timed with HIP events over 120 launches
    after 12 untimed ones; the median of five such runs per shape."""

    import torch

    from koemi_amd import _native

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    stream = torch.cuda.current_stream(device)
    lib_stream = _native.stream_of(device)
    _native.load_library()
    out: dict = {}
    for name, nbytes in (("C2.surprise_rows_bytes", 34013184), ("C2.rmsnorm_silu_read_bytes", 33554432)):
        sets = [torch.empty(nbytes // 4, device=device, dtype=torch.float32).uniform_() for _ in range(6)]
        sink = torch.empty(2 ** 23, device=device, dtype=torch.float32)
        results = []
        n16 = nbytes // 16
        for unroll in (1, 2, 4, 8):
            for block in (256, 512, 1024):
                one_pass = -(-n16 // (block * unroll))
                for grid in sorted({256, 512, 1024, 2048, 4096, 8192, one_pass}):
                    if grid > one_pass or grid * block > sink.numel():
                        continue

                    def run(i, unroll=unroll, block=block, grid=grid):
                        _native.call("koemi_stream_read", sets[i % 6].data_ptr(), nbytes, unroll, block, grid,
                                     sink.data_ptr(), lib_stream)

                    for i in range(12):
                        run(i)
                    times = []
                    for _ in range(5):
                        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        start.record(stream)
                        for i in range(120):
                            run(i)
                        end.record(stream)
                        end.synchronize()
                        times.append(start.elapsed_time(end) / 120)
                    ms = sorted(times)[2]
                    results.append({"unroll": unroll, "block": block, "grid": grid, "us": round(ms * 1e3, 3),
                                    "GB/s": round(nbytes / ms / 1e6, 1), "frac_hbm": round(nbytes / ms / 1e6 / 8000, 4)})
        results.sort(key=lambda r: r["us"])
        out[name] = {"bytes": nbytes, "best": results, "shapes": len(results),
                     "one_pass_256x1": next(r for r in results if r["unroll"] == 1 and r["block"] == 256
                                            and r["grid"] == -(-n16 // 256))}
        del sets, sink
    print(json.dumps({"read_floor": out}), flush=True)
    return 0


def main() -> int:
    args = parse_args()
    if args.summarize_pmc:
        return summarize_pmc(*args.summarize_pmc)
    if args.traffic_probe:
        return traffic_probe()
    if args.read_floor:
        return read_floor()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures a single GPU: this build has no multi-GPU path and every box here has one GPU; "
              "run with --gpus 1", file=sys.stderr, flush=True)
        return 2

    import torch

    from koemi_amd import core, dense, herm, memory, moe, recurrent, think, workloads

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    stream = torch.cuda.current_stream(device)
    timer = Timer(torch, stream)
    kernels: dict = {}

    if args.rows_only:
        extra = [c for c in args.configs.split(",") if c.strip()]
        kernel_rows(args, extra, device, stream, timer, kernels)
        print(json.dumps({"kernels": kernels}), flush=True)
        return 0

    # ------------------------------------------------------------ headline C5
    log("C5: initialising the 12-layer stack")
    settings = herm.HermSettings()
    params = herm.prepare_stack(herm.init_stack(settings, 1005, device), settings, device)
    c5 = workloads.config5()
    ids = c5.prefill_ids.to(device)
    start_states = herm.initial_states(settings, C5_BATCH, device)

    if args.decode_only:
        decode_rows(herm, params, settings, c5, device, kernels)
        print(json.dumps({"kernels": kernels}), flush=True)
        return 0

    sequential = None
    if not args.headline_only:
        sequential = window_by_window_rows(args, herm, params, settings, ids, start_states, kernels)

    log("C5: sequence-parallel prefill (one HIP graph): capture and check against the window-by-window prefill")
    seq = herm.SequencePrefill(params, settings, start_states, ids)
    logits = seq.run(ids).clone()
    torch.cuda.synchronize()
    seq.check()  # the fused gate kernel's status word: no carry wait timed out
    assert torch.isfinite(logits).all(), "non-finite prefill logits"
    seq_rel = None
    if sequential is not None:
        seq_rel = float((logits - sequential).norm() / sequential.norm())
        assert seq_rel < 1e-2, f"sequence-parallel prefill differs from the window-by-window one: {seq_rel:.3e}"
    reference_logits = logits

    log(f"C5: {args.warmup} warmup + {args.steps} timed prefill steps")
    for _ in range(args.warmup):
        logits = seq.run(ids)
    torch.cuda.synchronize()
    start_ev, end_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start_ev.record(stream)
    for _ in range(args.steps):
        logits = seq.run(ids)
    end_ev.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start_ev.elapsed_time(end_ev)
    ms_per_step = max(wall * 1000.0, gpu_ms) / args.steps
    value = C5_PREFILL_TOKENS / (ms_per_step / 1000.0)
    seq.check()
    assert torch.equal(logits, reference_logits), "prefill steps are not reproducible"
    kernels["C5.prefill"] = {"ms_per_step": round(ms_per_step, 4), "tokens_per_s": round(value, 1),
                             "vs_window_by_window_rel": None if seq_rel is None else round(seq_rel, 6),
                             "schedule": "sequence-parallel: each layer over all 2048 positions (the windows' "
                                         "carried states from one scan, window rings and a windowed associative "
                                         "memory), the whole stack replayed from one HIP graph"}
    del seq, logits, sequential, reference_logits

    if not args.headline_only:
        decode_rows(herm, params, settings, c5, device, kernels)

    # --------------------------------------------- dominant kernel of C5 prefill
    # The expert FFN of one layer over the whole prefill at its exact shape:
    # the prefill ids routed by the hash (as every layer routes them), bf16
    # contexts, each layer's own weights in turn (two layers' experts, 403 MB,
    # do not fit the Infinity Cache, as the stack's twelve do not).
    log("C5: dominant kernel (the expert FFN of one layer over the prefill), live timing")
    valid5 = ids != herm.PAD_TOKEN_ID
    prev5 = torch.cat((torch.full_like(ids[:, :1], herm.PAD_TOKEN_ID), ids[:, :-1]), dim=1)
    assign5 = moe.route_topk_valid(ids, prev5, valid5, expert_count=C5_E, top_k=C5_K)
    ffn_sets = []
    for layer in (0, 1):
        ctx5 = torch.randn((C5_PREFILL_TOKENS, C5_WIDTH), device=device).to(torch.bfloat16)
        sc, rows, experts, offsets = moe.permute_topk(ctx5, assign5.reshape(-1, C5_K), valid5.reshape(-1),
                                                      expert_count=C5_E)
        p = params[layer]
        ffn_sets.append((sc, experts, offsets, p["gate_w"], p["gate_b"], p["up_w"], p["up_b"], p["down_w"],
                         p["down_b"]))
    ffn_ms = timer.per_launch_ms([lambda s=s: moe.grouped_expert_mlp_inference(*s, validate=False) for s in ffn_sets],
                                 4, max(10, args.kernel_iters))
    ffn_tflops = C5_FFN_FLOP / ffn_ms / 1e9
    kernels["C5.expert_ffn_layer"] = {"ms": round(ffn_ms, 5), "TFLOP/s": round(ffn_tflops, 1),
                                      "frac_mfma_bf16": round(ffn_tflops / BF16_PEAK_TFLOPS, 4),
                                      "pairs": C5_PAIRS, "flop": C5_FFN_FLOP}
    headline_roofline = {**roofline(ffn_tflops, BF16_PEAK_TFLOPS, "TFLOP/s", "mfma",
                                    load_traffic("C5.expert_ffn_layer")),
                         "kernel": "grouped expert GLU FFN of one C5 layer over the prefill: grouped_gemm_bf16_kernel "
                                   "launches of GEMM 1 (gate + value, SiLU-GLU epilogue) and GEMM 2 with the device "
                                   "tile schedule, split-K partial tiles and their fix-ups",
                         "algorithmic_flop": C5_FFN_FLOP, "avg_ms": round(ffn_ms, 5)}
    del ffn_sets
    extra = [c for c in args.configs.split(",") if c.strip()] if not args.headline_only else []
    kernel_rows(args, extra, device, stream, timer, kernels)

    # ------------------------------------------------------------ CPU baseline
    cpu_baseline = None
    extras = {}
    if not args.no_cpu_baseline:
        threads = len(os.sched_getaffinity(0))
        log(f"CPU baseline: torch block window on {threads} threads")
        cpu_baseline = cpu_stack_baseline(threads, c5.prefill_ids[:, :C5_WINDOW].contiguous(), c5.decode_ids)
        if extra:
            log("CPU reference formulas of the kernel rows")
            rows_cpu = cpu_reference_times(extra, threads, args.cpu_seconds)
            for key, row in rows_cpu.items():
                if key in kernels and "ms" in kernels[key]:
                    row["gpu_speedup"] = round(row["ms"] / kernels[key]["ms"], 1)
            extras["cpu_reference_rows"] = {"cores": threads, "rows": rows_cpu}

    result = {
        "metric": "HERM tokens/s on 1 MI355X (C5: 12-layer HERM stack, prefill 8 x 2048)",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "C5: random-initialised stack of 12 HERM blocks (width 1024, state 1024, 16 experts top-2 "
                        "hash-routed, local and salient rings of 16, byte vocabulary + PAD); step = prefill of "
                        "8 x 2048 seeded byte ids (windows of 128, state carried), computed sequence-parallel and "
                        "replayed from one HIP graph; decode = 256 greedy steps at batch 64",
            "tokens_per_step": C5_PREFILL_TOKENS,
            "decode_tokens_per_s": kernels.get("C5.decode", {}).get("tokens_per_s"),
            "compute": "bf16 projections and expert FFNs with fp32 accumulation; fp32 state, memories and "
                       "every other operation",
        },
        "roofline": headline_roofline,
        "cpu_baseline": cpu_baseline,
        "kernels": kernels,
        **extras,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
