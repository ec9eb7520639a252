#!/usr/bin/env python3
"""Run history-only PCP attention on one MI355X with the gfx950 HIP backend.

Counterpart of the Trainium2 proof of concept's ``run_poc.py`` (run_poc.py:1-358):
same preset/override flags, ``--actual-history-len``/``--start-offset``,
``--seed``, ``--check`` and ``--benchmark-iterations``/``--benchmark-warmups``,
plus ``--backend hip``.  All logical PCP ranks run in one process and one
kernel launch; there is no torchrun, process group or device ring.

    python -m aws_training_study_amd.run_poc --backend hip --preset full --check sampled \
        --benchmark-iterations 30 --benchmark-warmups 3

``--backend cpu`` (the reference's CPU ring model) is not a runtime backend
here: that model is the test oracle (``oracle/pcp_oracle.py``), run by the
tests and by ``bench.py``'s CPU baseline.
"""

from __future__ import annotations

import argparse
import statistics
import sys
import time
from dataclasses import asdict, replace

from .pcp_attention.config import KV_DTYPES, PCPAttentionConfig, get_preset
from .pcp_attention.inputs import make_block_valid_mask, make_inputs, make_local_inputs

__all__ = ["make_block_valid_mask", "make_config", "make_inputs", "make_local_inputs", "main", "parse_args"]

MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3


def parse_args(argv=None) -> argparse.Namespace:
    parser = argparse.ArgumentParser()
    parser.add_argument("--backend", choices=("hip", "cpu"), default="hip")
    parser.add_argument("--preset", choices=("tiny", "full"), default="tiny")
    parser.add_argument("--pcp-size", type=int)
    parser.add_argument("--current-len", type=int)
    parser.add_argument("--max-history-len", type=int)
    parser.add_argument(
        "--actual-history-len",
        "--start-offset",
        dest="actual_history_len",
        type=int,
        help="runtime historical-token count; also the new-token start offset",
    )
    parser.add_argument("--block-size", type=int)
    parser.add_argument("--interleave-size", type=int)
    parser.add_argument("--num-q-heads", type=int)
    parser.add_argument("--num-kv-heads", type=int)
    parser.add_argument("--head-dim", type=int)
    parser.add_argument("--kv-dtype", choices=KV_DTYPES)
    parser.add_argument("--kv-scale", choices=("none", "per_tensor"), default="none",
                        help="FP8 K/V quantisation: direct cast (reference) or per-tensor amax/448 scale")
    parser.add_argument("--seed", type=int, default=1234)
    parser.add_argument("--check", choices=("full", "sampled", "none"), default="full")
    parser.add_argument("--benchmark-iterations", type=int, default=0)
    parser.add_argument("--benchmark-warmups", type=int, default=1)
    return parser.parse_args(argv)


def make_config(args: argparse.Namespace) -> PCPAttentionConfig:
    cfg = replace(get_preset(args.preset), backend="hip")
    names = (
        "pcp_size", "current_len", "max_history_len", "actual_history_len", "block_size",
        "interleave_size", "num_q_heads", "num_kv_heads", "head_dim", "kv_dtype",
    )
    overrides = {name: getattr(args, name) for name in names if getattr(args, name) is not None}
    return cfg.with_overrides(**overrides)


def run_hip(cfg: PCPAttentionConfig, seed: int, check: str, kv_scale: str, iterations: int, warmups: int) -> None:
    import torch

    from .pcp_attention.checks import dense_reference
    from .pcp_attention.kernel import make_history_attention_kernel
    from .pcp_attention.workloads import build_local_problem, build_paged_problem

    if iterations < 0 or warmups < 0:
        raise ValueError("benchmark iterations and warmups must be non-negative")
    if iterations and warmups == 0:
        raise ValueError("benchmark_warmups must be at least one so first-launch costs are untimed")
    if not torch.cuda.is_available():
        raise RuntimeError("--backend hip needs a visible MI355X GPU")
    device = torch.device("cuda", 0)
    if check == "none":
        # as the reference's unchecked runs (run_poc.py:221-222): every rank's
        # own seeded Q shard and local cache only, no global tensors
        problem = build_local_problem(cfg, seed)
    else:
        problem = build_paged_problem(cfg, seed, kv_scale=kv_scale if cfg.kv_dtype == "fp8_e4m3fn" else "none")
    gpu = problem.to(device)
    kernel = make_history_attention_kernel(cfg)

    def invoke(out=None):
        return kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, page_valid_len=gpu.page_valid_len,
                      k_scale=problem.k_scale, v_scale=problem.v_scale, out=out)

    out = invoke()
    torch.cuda.synchronize()
    if check != "none":
        expected = dense_reference(problem, device)
        actual = out.float()
        if check == "sampled":
            actual, expected = actual[:, :, :1], expected[:, :, :1]
        diff = (actual - expected).abs()
        max_abs, mean_abs = float(diff.max()), float(diff.mean())
        ok = max_abs <= MAX_ABS_TOL and mean_abs <= MEAN_ABS_TOL and bool(torch.isfinite(actual).all())
        print(f"HIP output {'OK' if ok else 'MISMATCH'}: max_abs_error={max_abs:.3e} mean_abs_error={mean_abs:.3e} "
              f"(bars {MAX_ABS_TOL:g} / {MEAN_ABS_TOL:g} vs float32 dense attention)", flush=True)
        if not ok:
            raise SystemExit(1)
    else:
        print("HIP run completed", flush=True)

    if iterations:
        # The reference's timing (run_poc.py:279-327): a host clock around
        # each call and its completion (a one-element device-to-host copy).
        for _ in range(warmups):
            invoke(out).reshape(-1)[:1].cpu()
        torch.cuda.synchronize()
        host_ms = []
        for _ in range(iterations):
            start = time.perf_counter()
            marker = invoke(out).reshape(-1)[:1].cpu()
            host_ms.append((time.perf_counter() - start) * 1e3)
            _ = marker[0].item()
        # Device time: the same calls back to back between one pair of HIP
        # events (an event pair per call would add queue work to each).
        stream = torch.cuda.current_stream(device)
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record(stream)
        for _ in range(iterations):
            invoke(out)
        end.record(stream)
        end.synchronize()
        device_ms = begin.elapsed_time(end) / iterations
        ordered = sorted(host_ms)
        p90 = ordered[max(0, (9 * len(ordered) + 9) // 10 - 1)]
        flops = 4.0 * cfg.num_q_heads * cfg.current_len * cfg.actual_history_len * cfg.head_dim
        fp8 = not kernel.uses_bf16_mfma()
        peak = 5000.0 if fp8 else 2500.0
        mean_ms = statistics.fmean(host_ms)
        print(
            "benchmark: mode=single_launch_all_ranks, "
            f"kv_dtype={cfg.kv_dtype}, iterations={iterations}, warmups={warmups}, "
            f"min_ms={min(host_ms):.3f}, median_ms={statistics.median(host_ms):.3f}, "
            f"mean_ms={mean_ms:.3f}, p90_ms={p90:.3f}, max_ms={max(host_ms):.3f}, "
            f"device_mean_ms={device_ms:.3f}, tflops={flops / device_ms / 1e9:.1f}, "
            f"pct_mfma_peak={100 * flops / device_ms / 1e9 / peak:.2f}, "
            f"global_current_tokens_per_s={cfg.current_len / (mean_ms / 1e3):.1f}",
            flush=True,
        )


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.backend == "cpu":
        raise SystemExit(
            "--backend cpu: the CPU ring model is this repository's test oracle (oracle/pcp_oracle.py), "
            "exercised by tests/ and timed by bench.py's cpu_baseline; run_poc drives the HIP kernel"
        )
    cfg = make_config(args)
    print("configuration:")
    for name, value in asdict(cfg).items():
        print(f"  {name}={value}")
    print(f"  local_q_len={cfg.local_q_len}")
    print(f"  actual_local_blocks={cfg.actual_local_blocks}")
    run_hip(cfg, args.seed, args.check, args.kv_scale, args.benchmark_iterations, args.benchmark_warmups)
    return 0


if __name__ == "__main__":
    sys.exit(main())
