#!/usr/bin/env python3
"""Benchmark of the MI355X HERM hot path (one GPU).

Headline ("C2"): one step = fused RMSNorm-SiLU of
x bf16 [32768, 512] + surprise of 32768 tokens from fp32 logits [32768, 256]
+ admission above the 0.9 quantile of the scores. ``value`` is HERM tokens/s
over K steps with every input resident in HBM. Each step reads a different
one of several input sets (>= 512 MiB in total) so that the 256 MiB Infinity
Cache cannot hold the working set; the step is captured once per input set in
a HIP graph and replayed (its three kernels are launch-bound at this size).

Also measured and reported (same JSON line, "kernels"): the C1/C3 affine scan,
the C3 RMSNorm-SiLU, the C4 MoE route/permute/grouped-GEMM/combine and one
window's salient read at the C5 model shape ("C5w"), each as
average kernel time from HIP events, GB/s or TFLOP/s, and the roofline fraction,
and the C5 end-to-end stack ("e": 12 random-initialised HERM blocks of width
1024, prefill 8 x 2048 byte ids, then 256 greedy decode steps at batch 64),
prefill and decode tokens/s from HIP-graph replays.
The CPU baseline is the oracle's single-threaded C port of the same C2 step
(and, as an extra, the reference's PyTorch formulas on all host cores).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import math
import os
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
C2_TOKENS = 16 * 2048

# Algorithmic bytes / FLOPs per launch.
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
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="1,3,4,5,g,e",
                    help="extra configurations to measure (comma list of 1,3,4,5,g,e; '' for none)")
    ap.add_argument("--kernel-iters", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run each HBM kernel a few times at its config plus a device copy of known size, for "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes (prints nothing else)")
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
COPY_BYTES = 512 * 2**20  # the calibration copy reads and writes this many bytes


def cpu_reference_times(extra: list, threads: int, budget_s: float) -> dict:
    """The reference's PyTorch formulas for each measured row, on the host cores.

    Each is timed on a bounded sample of its configuration (median of up to
    five runs after one warmup, within ``budget_s`` per row) and scaled to the
    full configuration by the sample's share of the work; the samples have the
    configuration's shapes and distributions.
    """

    import statistics

    import torch
    import torch.nn.functional as F

    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(99)
    out = {}

    def median_ms(fn) -> float:
        fn()
        times, t0 = [], time.perf_counter()
        while len(times) < 5 and (not times or time.perf_counter() - t0 < budget_s):
            t1 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t1)
        return statistics.median(times) * 1000.0

    def seq_scan(a, b):  # the tests' sequential recurrence (test_dense_cuda.py:21-33)
        h = torch.zeros_like(a[:, 0])
        res = torch.empty_like(a)
        for t in range(a.shape[1]):
            h = a[:, t] * h + b[:, t]
            res[:, t] = h
        return res

    def hillis_steele(a, b):  # the model path, model/scan.py:17-30
        coef, val, off, n = a, b, 1, a.shape[1]
        while off < n:
            sc = torch.cat((torch.ones_like(coef[:, :off]), coef[:, : n - off]), dim=1)
            sv = torch.cat((torch.zeros_like(val[:, :off]), val[:, : n - off]), dim=1)
            val = coef * sv + val
            coef = coef * sc
            off *= 2
        return val

    if "1" in extra:
        a = torch.rand((4, 1024, 256), generator=g) * 0.199 + 0.8
        b = torch.randn((4, 1024, 256), generator=g)
        out["C1.affine_scan"] = {"ms": round(median_ms(lambda: seq_scan(a, b)), 3), "sample": "full C1, sequential loop",
                                 "ms_model_path": round(median_ms(lambda: hillis_steele(a, b)), 3)}
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
            def mix(v):
                v = ((v >> 16) ^ v) * 0x45D9F3B % (1 << 32)
                v = ((v >> 16) ^ v) * 0x45D9F3B % (1 << 32)
                return (v >> 16) ^ v
            h = mix((tok * 1000003 + prev * 97409) % (1 << 32))
            e = torch.stack([(h + k * 0x9E3779B9) % E for k in range(K)], dim=-1)
            return torch.where(valid.unsqueeze(-1), e, torch.full_like(e, -1))

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

        def read():  # model/memory.py:405-429
            all_k, all_v = torch.cat((ck, k5), dim=1), torch.cat((cv, v5), dim=1)
            pos = torch.arange(l5)
            elig = torch.cat((cvalid.unsqueeze(1).expand(b5, l5, s5),
                              adm.unsqueeze(1) & (pos.unsqueeze(1) > pos.unsqueeze(0)).unsqueeze(0)), dim=-1)
            sc = torch.einsum("bsd,btd->bts", all_k, q5) / math.sqrt(d5)
            w = torch.softmax(sc.masked_fill(~elig, float("-inf")), dim=-1)
            w = torch.where(elig.any(dim=-1, keepdim=True), w, torch.zeros(()))
            return torch.einsum("bts,bsd->btd", w, all_v)

        out["C5w.salient_read"] = {"ms": round(median_ms(read), 3), "sample": "full C5 window"}
    if "e" in extra:
        # One block window (batch 8, 128 tokens, width 1024) with the float64
        # numpy restatement of forward_window, scaled to 16 windows x 12 layers.
        import numpy as np

        import oracle.herm as oherm
        from koemi_amd import herm

        settings = herm.HermSettings(layers=1)
        params = [{k: v.double().numpy() for k, v in p.items()} for p in herm.init_stack(settings, 1005)]
        cfg = settings.oracle_config()
        ids = np.random.default_rng(1005).integers(0, 256, (8, 128))
        state = oherm.initial_state(8, cfg)
        window_ms = median_ms(lambda: oherm.block_window(params[0], state, ids, cfg))
        out["C5.prefill"] = {"ms": round(window_ms * 16 * 12, 3),
                             "sample": "one layer x one window (8 x 128 tokens), numpy float64 block restatement, x192"}
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
    torch.cuda.synchronize()
    return 0


def summarize_pmc(fetch_dir: str, write_dir: str) -> int:
    """profiles/traffic.json from rocprofv3 counter_collection.csv files of FETCH_SIZE and WRITE_SIZE."""

    import csv
    import statistics

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
    out = ROOT / "profiles" / "traffic.json"
    out.write_text(json.dumps(result, indent=1) + "\n")
    print(json.dumps(result, indent=1))
    return 0


def main() -> int:
    args = parse_args()
    if args.summarize_pmc:
        return summarize_pmc(*args.summarize_pmc)
    if args.traffic_probe:
        return traffic_probe()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures a single GPU: this build has no multi-GPU path and every box has one GPU; "
              "run with --gpus 1", file=sys.stderr, flush=True)
        return 2

    import numpy as np
    import torch

    from koemi_amd import core, dense, memory, moe, recurrent, think, workloads

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    stream = torch.cuda.current_stream(device)

    def events_ms(fn, iters: int, warmup: int = 3) -> float:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(iters):
            fn()
        end.record(stream)
        end.synchronize()
        return start.elapsed_time(end) / iters

    # ------------------------------------------------------------- headline C2
    log("generating C2 input sets")
    per_set = C2_NORM_BYTES + C2_SURPRISE_BYTES + C2_ADMISSION_BYTES
    n_sets = max(2, math.ceil(512 * 2**20 / per_set))
    sets = []
    for i in range(n_sets):
        c = workloads.config2(seed=1002 + i)
        d = {
            "x": c.x.to(device), "gamma": c.gamma.to(device), "logits": c.logits.to(device),
            "targets": c.targets.to(device), "valid": c.valid.to(device),
        }
        sets.append(d)
    eps, q = 1e-6, 0.9

    def step_norm(d):
        return tuple(core.rmsnorm_silu_forward(d["x"], d["gamma"], eps))

    def step_surprise(d):
        s = think.surprise_from_logits(d["logits"], d["targets"], d["valid"])
        return (s, *think.salience_admission(s, d["valid"], quantile=q))

    def step(d):
        d["out"] = step_norm(d) + step_surprise(d)

    # eager reference outputs for the graph check
    for d in sets:
        step(d)
    torch.cuda.synchronize()
    eager = [tuple(t.clone() for t in d["out"]) for d in sets]

    # One graph holds `per_graph` consecutive steps (two passes over the input
    # sets) so that the host cost of a graph launch is amortized over many steps.
    # The RMSNorm-SiLU of a step does not depend on its surprise/admission
    # chain, so the graph holds the two as separate branches (captured from two
    # streams of default priority, joined at the end): the GPU may overlap the
    # gaps between one branch's kernels with the other's.
    per_graph = 2 * n_sets
    full_replays, remainder = divmod(args.steps, per_graph)
    log(f"capturing {per_graph}-step graphs")
    pool = torch.cuda.graph_pool_handle()
    branch = torch.cuda.Stream(device)

    keep_alive = []  # outputs of captured steps stay referenced, so no later capture reuses them

    def capture_steps(count: int):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=pool):
            main = torch.cuda.current_stream(device)
            branch.wait_stream(main)
            outs = []
            for i in range(count):
                d = sets[i % n_sets]
                with torch.cuda.stream(branch):
                    s_out = step_surprise(d)
                outs.append((d, step_norm(d) + s_out))
            main.wait_stream(branch)
        for d, out in outs:
            d["out"] = out
            keep_alive.append(out)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i in range(min(n_sets, count)):  # every replay must reproduce the eager outputs
            for got, want in zip(sets[i]["out"], eager[i]):
                assert torch.equal(got, want), "graph replay differs from the eager step"
        return g

    step_graph = capture_steps(per_graph) if full_replays else None
    tail_graph = capture_steps(remainder) if remainder else None

    for i in range(args.warmup):  # untimed warmup steps
        step(sets[i % n_sets])
    torch.cuda.synchronize()
    log(f"timing {args.steps} C2 steps")
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(full_replays):
        step_graph.replay()
    if tail_graph is not None:
        tail_graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(end)
    steps = args.steps
    ms_per_step = max(wall * 1000.0, gpu_ms) / steps
    value = C2_TOKENS / (ms_per_step / 1000.0)
    for i in range(min(n_sets, remainder if tail_graph is not None else per_graph)):
        for got, want in zip(sets[i]["out"], eager[i]):
            assert torch.equal(got, want), "graph replay differs from the eager step after timing"

    # Per-kernel times of the step: each kernel alone, `per_graph` launches per graph.
    def kernel_graph_ms(fn_for_set) -> float:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=pool):
            for i in range(per_graph):
                fn_for_set(sets[i % n_sets])
        torch.cuda.synchronize()
        reps = max(4, math.ceil(steps / per_graph))
        return events_ms(g.replay, reps, warmup=2) / per_graph

    log("timing C2 kernels")
    for d in sets:
        d["s"] = d["out"][2]
    c2_times = {
        "rmsnorm_silu": kernel_graph_ms(lambda d: core.rmsnorm_silu_forward(d["x"], d["gamma"], eps)),
        "surprise_rows": kernel_graph_ms(lambda d: think.surprise_from_logits(d["logits"], d["targets"], d["valid"])),
        "quantile_admission": kernel_graph_ms(lambda d: think.salience_admission(d["s"], d["valid"], quantile=q)),
    }
    c2_bytes = {"rmsnorm_silu": C2_NORM_BYTES, "surprise_rows": C2_SURPRISE_BYTES, "quantile_admission": C2_ADMISSION_BYTES}
    kernels = {}
    for name, ms in c2_times.items():
        gbs = c2_bytes[name] / (ms / 1000.0) / 1e9
        kernels[f"C2.{name}"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
    hbm_kernels = ("rmsnorm_silu", "surprise_rows")
    dominant = max(hbm_kernels, key=c2_times.get)
    dom_gbs = c2_bytes[dominant] / (c2_times[dominant] / 1000.0) / 1e9
    eager_ms = events_ms(lambda: step(sets[0]), 20)
    del step_graph, tail_graph, keep_alive
    for d in sets:
        d.pop("out", None)

    # ------------------------------------------------------------ other configs
    extra = [c for c in args.configs.split(",") if c.strip()]
    if "1" in extra:
        log("C1 scan")
        c1 = workloads.to_device(workloads.config1(), device)
        g1 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g1, pool=pool):
            for _ in range(20):
                dense.scan_forward(c1.retention, c1.increment, c1.initial)
        ms = events_ms(g1.replay, 10) / 20
        kernels["C1.affine_scan"] = {"ms": round(ms, 5), "GB/s": round(C1_SCAN_BYTES / ms / 1e6, 1),
                                     "frac_hbm": round(C1_SCAN_BYTES / ms / 1e6 / HBM_PEAK_GBS, 4),
                                     "note": "12.6 MB working set is launch-bound and fits the Infinity Cache"}
        del c1, g1
    if "3" in extra:
        log("C3 scan + norm (generating 1 GiB of inputs)")
        c3 = workloads.to_device(workloads.config3(), device)
        ms = events_ms(lambda: dense.scan_forward(c3.retention, c3.increment, c3.initial), args.kernel_iters)
        gbs = C3_SCAN_BYTES / ms / 1e6
        kernels["C3.affine_scan"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                     "tokens_per_s": round(32 * 4096 / (ms / 1000.0))}
        h = dense.scan_forward(c3.retention, c3.increment, c3.initial).to(torch.bfloat16).view(-1, 1024)
        del c3
        gamma = workloads.config3(batch=1, seq=1, width=1024).gamma.to(device)
        ms = events_ms(lambda: core.rmsnorm_silu_forward(h, gamma, 1e-6), args.kernel_iters)
        gbs = C3_NORM_BYTES / ms / 1e6
        kernels["C3.rmsnorm_silu"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        del h
    if "4" in extra:
        log("C4 MoE (generating inputs)")
        c4 = workloads.to_device(workloads.config4(), device)
        ms = events_ms(lambda: moe.route_topk_valid(c4.token_ids, c4.previous_token_ids, c4.valid, expert_count=16,
                                                    top_k=2, validate=False), args.kernel_iters)
        kernels["C4.route_hash"] = {"ms": round(ms, 5), "GB/s": round(C4_ROUTE_BYTES / ms / 1e6, 1)}
        a_l, w_l = moe.route_topk_learned(c4.router_logits, c4.valid, top_k=2)
        assign = moe.route_topk_valid(c4.token_ids, c4.previous_token_ids, c4.valid, expert_count=16, top_k=2)
        ms = events_ms(lambda: moe.permute_topk(c4.context, assign, c4.valid, expert_count=16, validate=False), args.kernel_iters)
        gbs = C4_PERMUTE_BYTES / ms / 1e6
        kernels["C4.permute"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        sc, rows, experts, offsets, sw = moe.permute_topk(c4.context, a_l, c4.valid, expert_count=16, pair_weights=w_l)
        weights = (c4.gate_weights, c4.gate_biases, c4.value_weights, c4.value_biases, c4.output_weights, c4.output_biases)
        ms = events_ms(lambda: moe.grouped_expert_mlp_inference(sc, experts, offsets, *weights, validate=False),
                       max(5, args.kernel_iters // 2))
        tflops = C4_GEMM_FLOP / ms / 1e9
        kernels["C4.grouped_glu_ffn"] = {"ms": round(ms, 5), "TFLOP/s": round(tflops, 1),
                                         "frac_mfma_bf16": round(tflops / BF16_PEAK_TFLOPS, 4)}
        y = moe.grouped_expert_mlp_inference(sc, experts, offsets, *weights, validate=False)
        ms = events_ms(lambda: moe.combine_topk(y, rows, offsets, token_count=C4_T, top_k=2, pair_weights=sw,
                                                validate=False), args.kernel_iters)
        gbs = C4_COMBINE_BYTES / ms / 1e6
        kernels["C4.combine"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        # practical bf16 GEMM ceiling of the platform library at the same total shape
        a_mat = torch.randn((C4_PAIRS, C4_D), device=device, dtype=torch.bfloat16)
        b_mat = torch.randn((C4_D, 2 * C4_H), device=device, dtype=torch.bfloat16)
        ms = events_ms(lambda: torch.matmul(a_mat, b_mat), 10)
        kernels["hipblaslt_reference_gemm"] = {"shape": [C4_PAIRS, C4_D, 2 * C4_H],
                                               "TFLOP/s": round(2 * C4_PAIRS * C4_D * 2 * C4_H / ms / 1e9, 1)}
        del c4, sc, y, a_mat, b_mat

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
        ms = events_ms(lambda: memory.read_salient_window(ck, cv, cvalid, k5, v5, adm5, q5), args.kernel_iters)
        flop = 4 * b5 * l5 * (s5 + l5) * d5
        nbytes = 4 * (4 * b5 * l5 * d5 + 2 * b5 * s5 * d5) + b5 * (s5 + l5)
        kernels["C5w.salient_read"] = {"ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1),
                                       "TFLOP/s": round(flop / ms / 1e9, 2), "shape_b_l_s_d": [b5, l5, s5, d5],
                                       "note": "HIP fp32-MFMA scores, softmax and weighted-sum kernels, eager launches"}
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
        ms = events_ms(lambda: recurrent.recurrent_gates(ug, *wts, vg), max(3, args.kernel_iters // 4))
        kernels["C3g.recurrent_gates"] = {"ms": round(ms, 5), "TFLOP/s": round(C3G_FLOP / ms / 1e9, 1),
                                          "frac_mfma_fp32": round(C3G_FLOP / ms / 1e9 / FP32_PEAK_TFLOPS, 4),
                                          "note": "two fp32 rocBLAS products + the HIP gate epilogue"}
        ms = events_ms(lambda: recurrent.recurrent_scan(ug, *wts, vg), max(3, args.kernel_iters // 4))
        kernels["C3g.recurrent_scan"] = {"ms": round(ms, 5), "tokens_per_s": round(32 * 4096 / (ms / 1000.0)),
                                         "note": "the two gate GEMMs, then one kernel forming the gates inside "
                                                 "the affine scan (network.py:306-310)"}
        del ug, wts, vg

    if "e" in extra:
        # C5 end to end: 12 HERM blocks, width 1024, 16 experts top-2, byte
        # vocabulary (+ PAD); prefill 8 x 2048 ids ~ U{0..255} in windows of 128,
        # then 256 greedy decode steps at batch 64 from the empty static state.
        log("C5 end-to-end stack (12 layers): graphed prefill and decode")
        from koemi_amd import herm

        settings = herm.HermSettings()
        params = herm.prepare_stack(herm.init_stack(settings, 1005, device), settings, device)
        ge = torch.Generator(device=device).manual_seed(1005)
        ids = torch.randint(0, 256, (8, 2048), generator=ge, device=device)
        start = herm.initial_states(settings, 8, device)
        logits, _, graph = herm.prefill_graphed(params, settings, ids, start)
        times = []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            logits, _, graph = herm.prefill_graphed(params, settings, ids, start, graph)
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        prefill_s = sorted(times)[1]
        assert torch.isfinite(logits).all()
        kernels["C5.prefill"] = {"ms": round(prefill_s * 1e3, 3), "tokens_per_s": round(ids.numel() / prefill_s),
                                 "shape": "12 layers x [8, 2048], windows of 128",
                                 "note": "bf16 projections (the reference's default GPU precision), fp32 state; "
                                         "each window replayed from one HIP graph"}
        del graph, logits, start
        dids = torch.randint(0, 256, (64, 1), generator=ge, device=device)
        decode = herm.DecodeGraph(params, settings, dids, herm.initial_states(settings, 64, device))
        for _ in range(3):
            decode.step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(256):
            decode.step()
        torch.cuda.synchronize()
        decode_s = time.perf_counter() - t0
        kernels["C5.decode"] = {"ms": round(decode_s * 1e3, 3), "ms_per_step": round(decode_s * 1e3 / 256, 4),
                                "tokens_per_s": round(64 * 256 / decode_s), "shape": "12 layers, batch 64, 256 steps",
                                "note": "greedy, padding id masked; each step replayed from one HIP graph"}
        del decode, params

    # ------------------------------------------------------------ CPU baseline
    cpu_baseline = None
    extras = {}
    if not args.no_cpu_baseline:
        import oracle

        log("CPU baseline (oracle C port, 1 thread)")
        c = workloads.config2()
        x32 = c.x.float().numpy()
        g32 = c.gamma.float().numpy()
        logits, targets, valid = c.logits.numpy(), c.targets.numpy(), c.valid.numpy()
        reps, t0 = 0, time.perf_counter()
        while True:
            oracle.rmsnorm_silu_f32(x32, g32, eps)
            s_cpu = oracle.surprise_rows(logits, targets, valid)
            oracle.admission(s_cpu, valid, q=q)
            reps += 1
            elapsed = time.perf_counter() - t0
            if elapsed >= args.cpu_seconds or reps >= 1000:
                break
        cpu_value = reps * C2_TOKENS / elapsed
        cpu_baseline = {"value": round(cpu_value, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
                        "sample": f"{reps} full C2 steps (32768 tokens each) with the oracle's C port, {elapsed:.1f} s"}
        # the reference's PyTorch formulas (its CPU fallback path) on all host cores
        import torch.nn.functional as F

        threads = len(os.sched_getaffinity(0))
        torch.set_num_threads(threads)
        x_t, g_t = c.x.float(), c.gamma.float()
        reps, t0 = 0, time.perf_counter()
        while True:
            F.silu(x_t * torch.rsqrt(x_t.square().mean(dim=-1, keepdim=True) + eps) * g_t)
            nll = F.cross_entropy(c.logits, c.targets, reduction="none")
            s_t = torch.where(c.valid, 1.0 - torch.exp(-(nll / math.log(256))), torch.zeros(()))
            s_t > torch.quantile(s_t, q)
            reps += 1
            elapsed = time.perf_counter() - t0
            if elapsed >= args.cpu_seconds / 2 or reps >= 1000:
                break
        extras["cpu_torch_reference_formulas"] = {"value": round(reps * C2_TOKENS / elapsed, 1), "unit": "tokens/s",
                                                  "cores": threads, "sample": f"{reps} C2 steps, fp32 torch CPU"}
        log("CPU reference formulas of the other rows")
        cpu_rows = cpu_reference_times(extra, threads, budget_s=args.cpu_seconds / 4)
        for key, row in cpu_rows.items():
            if key in kernels and "ms" in kernels[key]:
                row["gpu_speedup"] = round(row["ms"] / kernels[key]["ms"], 1)
        extras["cpu_reference_rows"] = {"cores": threads, "rows": cpu_rows}

    result = {
        "metric": "HERM tokens/s on 1 MI355X (C2: fused RMSNorm-SiLU + surprise + 0.9-quantile admission)",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "C2: RMSNorm-SiLU of x bf16 [32768,512] (eps 1e-6) + surprise from logits fp32 [32768,256] "
                        "+ admission above the 0.9 quantile; seeded inputs, rotated over "
                        f"{n_sets} HBM-resident sets (> Infinity Cache); step = RMSNorm-SiLU on one graph branch, surprise -> "
                        f"admission (partition + finish) on another (independent work), {per_graph} steps per HIP graph "
                        "replay",
            "tokens_per_step": C2_TOKENS,
            "compute": "bf16 activations, fp32 arithmetic in every kernel",
            "input_sets": n_sets,
        },
        "roofline": {**roofline(dom_gbs, HBM_PEAK_GBS, "GB/s", "hbm", load_traffic(f"C2.{dominant}")),
                     "kernel": f"C2.{dominant}", "algorithmic_bytes": c2_bytes[dominant],
                     "avg_ms": round(c2_times[dominant], 5)},
        "cpu_baseline": cpu_baseline,
        "eager_ms_per_step": round(eager_ms, 5),
        "kernels": kernels,
        **extras,
    }
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
