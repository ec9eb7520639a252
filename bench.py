#!/usr/bin/env python3
"""Benchmark of history-only PCP attention on one MI355X.

Default workload: 64 logical PCP ranks, 4096 current tokens attending a
131072-token paged FP8 (e4m3, per-tensor scale) history, 32 Q / 2 KV heads,
D 256, 512-token blocks, interleave 64, seeded random block table.  A step is
one launch of the gfx950 kernel over all ranks with every input resident in
HBM.  Prints one JSON line.

    python bench.py [--steps K] [--warmup W] [--workload NAME]

``value`` is model TFLOP/s (4 * Hq * Q * L_valid * D per step, the
reference's definition, README.md:167-171) from the wall time of the K timed
steps; ``roofline`` prices the kernel's own HIP-event duration against the
MI355X dense MFMA peak; ``cpu_baseline`` times the CPU ring model (the
oracle's restatement of reference.py:35-95) on a bounded sample of ranks.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "ms + TFLOP/s (% FP8 MFMA peak), Q=4K x 128K paged FP8 KV history, 1 GPU"
# HBM bytes per launch measured with rocprofv3 PMC counters (FETCH_SIZE and
# WRITE_SIZE, each calibrated on a copy kernel of known size).
TRAFFIC_FILE = ROOT / "profiles" / "pmc_traffic.txt"
# MI355X published dense MFMA peaks, TFLOP/s.
PEAK_TFLOPS = {"fp8_e4m3fn": 5000.0, "bfloat16": 2500.0}
HBM_PEAK_GBS = 8000.0


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[1])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=30)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--workload", default="full-fp8")
    parser.add_argument("--path", choices=("history", "cache-write", "current", "launch"), default="history",
                        help="history: the attention launch (the headline metric); cache-write: the KV-cache "
                             "producer filling the workload's page pool from BF16 K/V; current: causal attention "
                             "of the current tokens merged with the history output; launch: per-call latency of "
                             "the workload's history attention, eager calls against a replayed HIP graph")
    parser.add_argument("--seed", type=int, default=1234)
    parser.add_argument("--precision", choices=("auto", "fp8", "bf16"), default="auto",
                        help="MFMA precision of an e4m3 cache: auto (e4m3 MFMAs with the precision guard that "
                             "recomputes low-mass rows with BF16 MFMAs), fp8 (e4m3 only) or bf16")
    parser.add_argument("--exp2", choices=("fast", "exact"), default="fast",
                        help="e4m3 probabilities at head_dim 256: linear-mantissa exp2 (fast) or v_exp_f32 (exact)")
    parser.add_argument("--cpu-baseline-seconds", type=float, default=15.0,
                        help="approximate CPU time budget of the ring-model baseline sample")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--traffic-bytes", type=float, default=None,
                        help="HBM bytes per launch measured with rocprofv3 PMC counters (reported as roofline.traffic)")
    parser.add_argument("--copy-probe-mib", type=int, default=0,
                        help="instead of the benchmark, run --steps device-to-device copies of this many MiB "
                             "(a known-size kernel for calibrating FETCH_SIZE / WRITE_SIZE)")
    return parser.parse_args(argv)


def copy_probe(mib: int, steps: int) -> int:
    import torch

    device = torch.device("cuda", 0)
    src = torch.ones(mib * (1 << 20), dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": src.numel(), "steps": steps}), flush=True)
    return 0


def measured_traffic(workload: str):
    """(bytes, source) for ``workload`` from TRAFFIC_FILE, or (None, None)."""
    if not TRAFFIC_FILE.exists():
        return None, None
    for line in TRAFFIC_FILE.read_text().splitlines():
        fields = line.split()
        if len(fields) == 6 and not line.startswith("#") and fields[0] == workload:
            fetch = float(fields[2]) * 1024 * float(fields[3])
            write = float(fields[4]) * 1024 * float(fields[5])
            return fetch + write, f"{TRAFFIC_FILE.relative_to(ROOT)} ({fields[1]})"
    return None, None


def model_flops(cfg) -> float:
    return 4.0 * cfg.num_q_heads * cfg.current_len * cfg.actual_history_len * cfg.head_dim


def algorithmic_bytes(cfg) -> float:
    """Q in + O out + valid K/V + block table + valid lengths."""
    q = 2.0 * cfg.num_q_heads * cfg.current_len * cfg.head_dim
    kv = 2.0 * cfg.num_kv_heads * cfg.actual_history_len * cfg.head_dim * cfg.kv_element_size
    tables = 2 * 4.0 * cfg.num_pages
    return 2 * q + kv + tables


def cpu_baseline(problem, budget_s: float) -> dict:
    """Time the oracle's CPU ring model on the first k ranks and extrapolate."""
    import torch

    from aws_training_study_amd.pcp_attention.layout import shard_history, shard_query
    from oracle import pcp_oracle as orc

    cfg = problem.config
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    shape = orc.OracleShape.from_config(cfg)
    q_shards = shard_query(problem.inputs.q, cfg)
    k_shards, v_shards = shard_history(problem.inputs.k, problem.inputs.v, cfg)
    start = time.perf_counter()
    orc.ring_history_attention(q_shards[:1], k_shards, v_shards, shape)
    per_rank = time.perf_counter() - start
    ranks = 1
    extra = min(cfg.pcp_size - 1, int(max(0.0, budget_s - per_rank) / max(per_rank, 1e-9)))
    if extra > 0:
        start = time.perf_counter()
        orc.ring_history_attention(q_shards[1:1 + extra], k_shards, v_shards, shape)
        elapsed = time.perf_counter() - start
        per_rank = (per_rank + elapsed) / (1 + extra)
        ranks += extra
    full_s = per_rank * cfg.pcp_size
    return {
        "value": model_flops(cfg) / full_s / 1e12,
        "unit": "TFLOP/s",
        "ms": full_s * 1e3,
        "cores": threads,
        "kind": "port",
        "sample": (
            f"ring model (reference.py:35-95 loop order, FP32 torch on {threads} host threads) "
            f"over {ranks} of {cfg.pcp_size} ranks, full history each; every rank does identical "
            f"work, time extrapolated x{cfg.pcp_size / ranks:g}"
        ),
    }


def cache_write_bench(args) -> int:
    """KV-cache producer: quantise + scatter the workload's whole history into its page pool."""
    import torch

    from aws_training_study_amd.pcp_attention import KVCacheWriter, make_block_table, pack_page_pool, shard_history
    from aws_training_study_amd.pcp_attention.cache import device_per_tensor_scale
    from aws_training_study_amd.pcp_attention.inputs import make_raw_inputs, per_tensor_scale
    from aws_training_study_amd.pcp_attention.workloads import get_workload

    workload = get_workload(args.workload)
    cfg = workload.resolve(args.seed).with_overrides(backend="hip")
    if not cfg.is_history_aligned:
        raise SystemExit("cache-write bench expects a block-aligned workload")
    _, k, v = make_raw_inputs(cfg, args.seed)
    table = make_block_table(cfg, args.seed + 1)
    device = torch.device("cuda", 0)
    kd, vd, td = k.to(device), v.to(device), table.to(device)
    fp8 = cfg.kv_dtype == "fp8_e4m3fn"
    ks = device_per_tensor_scale(kd) if fp8 else 1.0
    vs = device_per_tensor_scale(vd) if fp8 else 1.0
    dtype = torch.float8_e4m3fn if fp8 else torch.bfloat16
    pool = torch.zeros((cfg.num_pages, cfg.page_elements), dtype=dtype, device=device)
    writer = KVCacheWriter(cfg)

    def step():
        writer(kd, vd, pool, td, k_scale=ks, v_scale=vs)

    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream(device)
    wall_s, kernel_ms = _timed(step, args.steps, stream)
    spread = _spread(step, min(args.steps, 20), stream)
    traffic, traffic_source = measured_traffic(f"{workload.name}/cache-write")
    elems = 2 * cfg.num_kv_heads * cfg.actual_history_len * cfg.head_dim
    algo = elems * 2 + elems * (1 if fp8 else 2) + 4 * cfg.num_pages  # read bf16, write pages, table
    ms_per_step = wall_s * 1e3 / args.steps
    result = {
        "metric": "KV-cache write GB/s (BF16 K/V -> paged pool, quantise + scatter), 1 GPU",
        "value": round(algo / (ms_per_step * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3" if fp8 else "bf16",
        "data": "synthetic (seeded N(0,1) BF16 K/V)",
        "config": {"workload": workload.name, "tokens": cfg.actual_history_len, "kv_heads": cfg.num_kv_heads,
                   "head_dim": cfg.head_dim, "pcp_ranks": cfg.pcp_size, "block_size": cfg.block_size,
                   "interleave": cfg.interleave_size, "kv_dtype": cfg.kv_dtype},
        "kernel_ms": _kernel_ms(kernel_ms, spread),
        "roofline": {"bound": "hbm", "achieved": round(algo / (kernel_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(algo / (kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_source, "algorithmic_bytes": algo},
    }
    if not args.no_cpu_baseline:
        threads = os.cpu_count() or 1
        torch.set_num_threads(threads)
        start = time.perf_counter()
        if fp8:
            kq = (k.float() / per_tensor_scale(float(k.float().abs().max()))).to(torch.float8_e4m3fn)
            vq = (v.float() / per_tensor_scale(float(v.float().abs().max()))).to(torch.float8_e4m3fn)
        else:
            kq, vq = k, v
        pack_page_pool(*shard_history(kq, vq, cfg), cfg, table)
        host_s = time.perf_counter() - start
        result["cpu_baseline"] = {
            "value": round(algo / host_s / 1e9, 2), "unit": "GB/s", "ms": round(host_s * 1e3, 1), "cores": threads,
            "kind": "port",
            "sample": "host chain of the reference (quantise, shard_history, pack_local_kv, place by block table) "
                      "over the whole history, torch CPU",
        }
    print(json.dumps(result), flush=True)
    return 0


def causal_flops(cfg) -> float:
    """4 * D per (query, visible key) pair; query g sees current keys 0..g."""
    return 2.0 * cfg.num_q_heads * cfg.head_dim * cfg.current_len * (cfg.current_len + 1)


def _timed(step, steps, stream):
    """The timed region: `steps` back-to-back steps between one pair of HIP
    events on `stream`, synchronised on both sides.  Returns wall seconds and
    the events' mean milliseconds per step.  (One event pair per step adds
    queue work to every step on ROCm: 0.161 instead of 0.154 ms per step on
    the 16-rank workload, 37.8 instead of 30.5 us on the 4-rank one.)"""
    import torch

    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    begin.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    return time.perf_counter() - t0, begin.elapsed_time(end) / steps


def _spread(step, steps, stream):
    """Per-step event times (sorted) from a pass after the timed region, each
    step between its own event pair: the spread of launch times, each
    including the per-pair event overhead."""
    import torch

    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for begin, end in events:
        begin.record(stream)
        step()
        end.record(stream)
    torch.cuda.synchronize()
    return sorted(b.elapsed_time(e) for b, e in events)


def _kernel_ms(mean_ms, spread):
    p90 = spread[max(0, (9 * len(spread) + 9) // 10 - 1)]
    return {"mean": round(mean_ms, 4), "per_step_min": round(spread[0], 4),
            "per_step_median": round(statistics.median(spread), 4), "per_step_p90": round(p90, 4)}


def current_bench(args) -> int:
    """Current-token step: causal attention among the current tokens, merged with a history result."""
    import torch

    from aws_training_study_amd.pcp_attention import CurrentAttentionKernel, PrefillAttention, stack_current_kv
    from aws_training_study_amd.pcp_attention.workloads import build_workload_problem, get_workload

    workload = get_workload(args.workload)
    problem = build_workload_problem(workload, args.seed)
    cfg = problem.config
    device = torch.device("cuda", 0)
    gpu = problem.to(device)
    g = torch.Generator().manual_seed(args.seed + 11)
    kv_shape = (cfg.num_kv_heads, cfg.current_len, cfg.head_dim)
    kc = torch.randn(kv_shape, generator=g, dtype=torch.bfloat16)
    vc = torch.randn(kv_shape, generator=g, dtype=torch.bfloat16)
    kv_cur = stack_current_kv(kc, vc).to(device)
    prefill = PrefillAttention(cfg)
    current = prefill.current
    hist_out, hist_lse = prefill.history(gpu.q_stacked, gpu.kv_pages, gpu.block_table,
                                         page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale,
                                         v_scale=problem.v_scale, return_lse=True)
    out = torch.empty_like(hist_out)

    def step():
        current(gpu.q_stacked, kv_cur, hist_out, hist_lse, out=out)

    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream(device)
    wall_s, kernel_ms = _timed(step, args.steps, stream)
    spread = _spread(step, min(args.steps, 20), stream)

    def prefill_step():
        prefill(gpu.q_stacked, gpu.kv_pages, gpu.block_table, kv_cur, page_valid_len=gpu.page_valid_len,
                k_scale=problem.k_scale, v_scale=problem.v_scale)

    prefill_step()
    _, prefill_ms = _timed(prefill_step, max(3, min(args.steps, 10)), stream)

    flops = causal_flops(cfg)
    ms_per_step = wall_s * 1e3 / args.steps
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    peak = PEAK_TFLOPS["bfloat16"]
    history_flops = model_flops(cfg)
    traffic, traffic_source = measured_traffic(f"{workload.name}/current")
    result = {
        "metric": "current-token causal attention + LSE merge TFLOP/s (BF16 MFMA), 1 GPU",
        "value": round(flops / (ms_per_step * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) BF16 Q and current K/V; history as the history bench)",
        "config": {"workload": workload.name, "pcp_ranks": cfg.pcp_size, "current_tokens": cfg.current_len,
                   "history_tokens": cfg.actual_history_len, "q_heads": cfg.num_q_heads,
                   "kv_heads": cfg.num_kv_heads, "head_dim": cfg.head_dim, "interleave": cfg.interleave_size},
        "kernel_ms": _kernel_ms(kernel_ms, spread),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4),
                     "traffic": round(traffic) if traffic is not None else None,
                     "traffic_source": traffic_source,
                     "algorithmic_bytes": 2.0 * (3 * cfg.num_q_heads * cfg.current_len * cfg.head_dim
                                                 + 2 * cfg.num_kv_heads * cfg.current_len * cfg.head_dim)
                     + 2 * 4.0 * cfg.num_q_heads * cfg.current_len},
        "prefill": {"ms": round(prefill_ms, 4),
                    "tflops": round((history_flops + flops) / (prefill_ms * 1e-3) / 1e12, 2),
                    "what": "history attention with lse + this step, in place"},
    }
    if not args.no_cpu_baseline:
        import torch.nn.functional as F

        threads = os.cpu_count() or 1
        torch.set_num_threads(threads)
        group = cfg.num_q_heads // cfg.num_kv_heads
        q = problem.inputs.q.float()
        kk = kc.float().repeat_interleave(group, dim=0)
        vv = vc.float().repeat_interleave(group, dim=0)
        start = time.perf_counter()
        F.scaled_dot_product_attention(q, kk, vv, is_causal=True, scale=cfg.softmax_scale)
        host_s = time.perf_counter() - start
        result["cpu_baseline"] = {
            "value": round(flops / host_s / 1e12, 4), "unit": "TFLOP/s", "ms": round(host_s * 1e3, 1),
            "cores": threads, "kind": "port",
            "sample": "the whole workload's causal current attention (no merge): torch float32 "
                      "scaled_dot_product_attention(is_causal=True) on the host",
        }
    print(json.dumps(result), flush=True)
    return 0


def launch_bench(args) -> int:
    """Per-call host-inclusive latency (call + synchronise) and back-to-back call rate, eager vs HIP graph."""
    import torch

    from aws_training_study_amd.pcp_attention import make_history_attention_kernel
    from aws_training_study_amd.pcp_attention.workloads import build_workload_problem, get_workload

    workload = get_workload(args.workload)
    problem = build_workload_problem(workload, args.seed)
    cfg = problem.config
    device = torch.device("cuda", 0)
    gpu = problem.to(device)
    kernel = make_history_attention_kernel(cfg)
    out = torch.empty_like(gpu.q_stacked)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale, out=out)

    def eager():
        kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, **kw)

    graphed = kernel.graphed(gpu.q_stacked, gpu.kv_pages, gpu.block_table, **kw)
    calls = max(args.steps, 50)

    def measure(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        lat = []
        for _ in range(calls):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            lat.append((time.perf_counter() - t0) * 1e3)
        lat.sort()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        torch.cuda.synchronize()
        rate_ms = (time.perf_counter() - t0) * 1e3 / calls
        return {"median_ms": round(statistics.median(lat), 4), "mean_ms": round(statistics.fmean(lat), 4),
                "p90_ms": round(lat[max(0, (9 * calls + 9) // 10 - 1)], 4), "back_to_back_ms": round(rate_ms, 4)}

    e, g = measure(eager), measure(graphed.replay)
    result = {
        "metric": "per-call latency ms (call + synchronise), history attention, eager vs HIP graph, 1 GPU",
        "value": g["median_ms"],
        "unit": "ms",
        "n_gpus": 1,
        "steps": calls,
        "warmup": args.warmup,
        "ms_per_step": g["median_ms"],
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3" if cfg.kv_dtype == "fp8_e4m3fn" else "bf16",
        "data": "synthetic (seeded, as the history bench)",
        "config": {"workload": workload.name, "pcp_ranks": cfg.pcp_size, "current_tokens": cfg.current_len,
                   "history_tokens": cfg.actual_history_len, "q_heads": cfg.num_q_heads,
                   "kv_heads": cfg.num_kv_heads, "head_dim": cfg.head_dim,
                   "splits": kernel.split_count(device, kernel.uses_bf16_mfma())},
        "eager": e,
        "graph": g,
    }
    print(json.dumps(result), flush=True)
    return 0


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(
            f"bench.py runs on one GPU only: the collapsed PCP path keeps every rank's pages in one "
            f"GPU's HBM and has no multi-GPU mode (asked for --gpus {args.gpus})",
            file=sys.stderr,
        )
        return 2
    if args.steps < 1 or args.warmup < 1:
        print("--steps and --warmup must be at least 1", file=sys.stderr)
        return 2
    if args.copy_probe_mib:
        return copy_probe(args.copy_probe_mib, args.steps)
    if args.path == "cache-write":
        return cache_write_bench(args)
    if args.path == "current":
        return current_bench(args)
    if args.path == "launch":
        return launch_bench(args)

    import torch

    from aws_training_study_amd.pcp_attention import make_history_attention_kernel
    from aws_training_study_amd.pcp_attention.workloads import build_workload_problem, get_workload

    workload = get_workload(args.workload)
    problem = build_workload_problem(workload, args.seed)
    cfg = problem.config
    device = torch.device("cuda", 0)
    gpu = problem.to(device)
    kernel = make_history_attention_kernel(cfg)
    out = torch.empty_like(gpu.q_stacked)

    def step():
        kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, page_valid_len=gpu.page_valid_len,
               k_scale=problem.k_scale, v_scale=problem.v_scale, out=out, precision=args.precision, exp2=args.exp2)

    for _ in range(args.warmup):
        step()

    # Timed region: exactly K steps, synchronised on both sides.
    stream = torch.cuda.current_stream(device)
    wall_s, kernel_ms = _timed(step, args.steps, stream)
    spread = _spread(step, min(args.steps, 20), stream)

    flops = model_flops(cfg)
    ms_per_step = wall_s * 1e3 / args.steps
    fp8 = not kernel.uses_bf16_mfma(args.precision)
    peak = PEAK_TFLOPS["fp8_e4m3fn" if fp8 else "bfloat16"]
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    traffic, traffic_source = (args.traffic_bytes, "--traffic-bytes") if args.traffic_bytes else \
        measured_traffic(workload.name)

    result = {
        "metric": METRIC if workload.name == "full-fp8" else
        f"ms + TFLOP/s (% {'FP8' if fp8 else 'BF16'} MFMA peak), {workload.name} history attention, 1 GPU",
        "value": round(flops / (ms_per_step * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3" if fp8 else "bf16",
        "data": "synthetic (seeded N(0,1) BF16 Q, K/V quantised to e4m3 with per-tensor amax/448 scales)" if fp8
        else "synthetic (seeded N(0,1) BF16 Q/K/V" + (", K with a per-channel factor in [0.5, 2])"
                                                      if workload.k_prescale == "per_channel" else ")"),
        "config": {
            "workload": workload.name,
            "pcp_ranks": cfg.pcp_size,
            "current_tokens": cfg.current_len,
            "history_tokens": cfg.actual_history_len,
            "q_heads": cfg.num_q_heads,
            "kv_heads": cfg.num_kv_heads,
            "head_dim": cfg.head_dim,
            "block_size": cfg.block_size,
            "interleave": cfg.interleave_size,
            "kv_dtype": cfg.kv_dtype,
            "mfma": "e4m3" if fp8 else "bf16",
            "exp2": (args.exp2 + (" (linear-mantissa e4m3 code)" if args.exp2 == "fast" else " (v_exp_f32)"))
            if fp8 and cfg.head_dim == 256 else "exact (v_exp_f32)",
            "precision_guard": kernel.guarded(args.precision),
            "splits": kernel.split_count(device, not fp8),
        },
        "pct_peak": round(100.0 * flops / (ms_per_step * 1e-3) / 1e12 / peak, 2),
        "kernel_ms": _kernel_ms(kernel_ms, spread),
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "algorithmic_bytes": algorithmic_bytes(cfg),
            "algorithmic_hbm_gbs": round(algorithmic_bytes(cfg) / (kernel_ms * 1e-3) / 1e9, 1),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(problem, args.cpu_baseline_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
