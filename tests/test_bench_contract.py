"""The bench.py contract pieces that need no GPU: argument refusals, the
FLOP and byte accounting of the headline workload, the measured-traffic
lookup and the per-step spread summary."""

from __future__ import annotations

import bench
from aws_training_study_amd.pcp_attention.workloads import get_workload


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU only" in capsys.readouterr().err


def test_steps_and_warmup_must_be_positive():
    assert bench.main(["--steps", "0"]) == 2
    assert bench.main(["--warmup", "0"]) == 2


def test_headline_accounting():
    cfg = get_workload("full-fp8").resolve(1234)
    # 4 * Hq * Q * L * D: 32 heads, 4096 queries, 131072 keys, 256 dims
    assert bench.model_flops(cfg) == 4.0 * 32 * 4096 * 131072 * 256
    # Q in + O out (bf16) + e4m3 K and V of both KV heads + block table and valid lengths
    q = 2 * 32 * 4096 * 256
    kv = 2 * 2 * 131072 * 256
    assert bench.algorithmic_bytes(cfg) == 2 * q + kv + 2 * 4 * cfg.num_pages


def test_measured_traffic_reads_the_committed_pmc_line():
    for line in bench.TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("full-fp8 "):
            _, kernel, fetch, ffac, write, wfac = line.split()
            break
    traffic, source = bench.measured_traffic("full-fp8")
    assert traffic == float(fetch) * 1024 * float(ffac) + float(write) * 1024 * float(wfac)
    assert kernel in source
    assert bench.measured_traffic("no-such-workload") == (None, None)


def test_kernel_ms_summary():
    got = bench._kernel_ms(2.5, [1.0, 2.0, 3.0, 4.0])
    assert got == {"mean": 2.5, "per_step_min": 1.0, "per_step_median": 2.5, "per_step_p90": 4.0}
