"""The reference's runner on the HIP backend (run_poc.py:240-327 -> --backend hip).

`run_poc.main` with `--check full` and `--check sampled` compares the kernel
with float32 dense attention on the GPU (the reference's check,
run_poc.py:256-266, at this repository's 2e-2 / 2e-3 bar) and prints "HIP
output OK"; its benchmark prints the reference's statistics line.
`--check none` runs the memory-safe per-rank inputs (run_poc.py:107-134,
221-237); their output is checked here against the float64 oracle over
the same pages.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from aws_training_study_amd.pcp_attention import make_history_attention_kernel
from aws_training_study_amd.pcp_attention.config import get_preset
from aws_training_study_amd.pcp_attention.workloads import build_local_problem
from aws_training_study_amd.run_poc import main
from oracle import pcp_oracle as orc

from test_gpu_parity import MAX_ABS_TOL, MEAN_ABS_TOL

pytestmark = pytest.mark.gpu


def test_run_poc_tiny_check_full(cuda_device, capsys):
    print("case run_poc tiny --check full", flush=True)
    assert main(["--backend", "hip", "--preset", "tiny", "--check", "full"]) == 0
    out = capsys.readouterr().out
    assert "HIP output OK" in out, out


def test_run_poc_full_check_sampled_with_benchmark(cuda_device, capsys):
    print("case run_poc full --check sampled --benchmark-iterations 3", flush=True)
    assert main(["--backend", "hip", "--preset", "full", "--kv-scale", "per_tensor", "--check", "sampled",
                 "--benchmark-iterations", "3", "--benchmark-warmups", "1"]) == 0
    out = capsys.readouterr().out
    assert "HIP output OK" in out, out
    line = [l for l in out.splitlines() if l.startswith("benchmark:")]
    assert line and "device_mean_ms=" in line[0] and "global_current_tokens_per_s=" in line[0], out


def test_run_poc_check_none_runs_local_inputs(cuda_device, capsys):
    print("case run_poc tiny --check none", flush=True)
    assert main(["--backend", "hip", "--preset", "tiny", "--check", "none", "--benchmark-iterations", "2"]) == 0
    out = capsys.readouterr().out
    assert "HIP run completed" in out and "benchmark:" in out, out


@pytest.mark.parametrize("preset,overrides", [
    ("tiny", {}),
    ("tiny", {"max_history_len": 4096, "actual_history_len": 2048}),
    ("full", {"current_len": 1024, "pcp_size": 16, "max_history_len": 8192, "actual_history_len": 8192}),
])
def test_local_inputs_match_the_oracle(preset, overrides, cuda_device):
    cfg = get_preset(preset).with_overrides(backend="hip", **overrides)
    print(f"case local inputs {preset} {overrides}", flush=True)
    problem = build_local_problem(cfg, seed=1234)
    gpu = problem.to(cuda_device)
    out = make_history_attention_kernel(cfg)(gpu.q_stacked, gpu.kv_pages, gpu.block_table,
                                             page_valid_len=gpu.page_valid_len)
    torch.cuda.synchronize()
    shape = orc.OracleShape.from_config(cfg)
    pool = orc.decode_e4m3fn(problem.kv_pages.view(torch.uint8).numpy())
    q = orc.decode_bfloat16(problem.q_stacked.view(torch.int16).numpy().view(np.uint16))
    want = orc.paged_history_attention(q, pool, problem.block_table.numpy(), problem.page_valid_len.numpy(), shape)
    max_abs, mean_abs = orc.max_abs_and_mean_abs(out.float().cpu().numpy(), want)
    print(f"max_abs={max_abs:.3e} mean_abs={mean_abs:.3e}", flush=True)
    assert max_abs <= MAX_ABS_TOL and mean_abs <= MEAN_ABS_TOL
