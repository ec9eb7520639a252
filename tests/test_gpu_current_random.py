"""Seeded random configurations of the prefill step (history attention, then
the causal current-token step merged in place), against the float64 oracle
on every output row and its log-sum-exp.

Each case draws pcp size, interleave, current tokens per rank, heads, head
dim, cache dtype, history precision and a runtime history length from a
fixed seed; ``PCPA_RANDOM_CASES`` widens the sweep as for the history
kernel's.  Bars as in test_gpu_current.py (outputs 2e-2 / 2e-3; lse by the
MFMA precision of the history part), on every case: an e4m3 cache is drawn
with the guarded default, unguarded e4m3 MFMAs (only on histories of 2048
tokens or more, where no row's softmax rests on a few keys) or BF16 MFMAs.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from aws_training_study_amd.pcp_attention import PrefillAttention, stack_current_kv
from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig
from aws_training_study_amd.pcp_attention.workloads import build_paged_problem
from oracle import pcp_oracle as orc

from test_gpu_current import LSE_TOL
from test_gpu_parity import MAX_ABS_TOL, MEAN_ABS_TOL, _real_history

pytestmark = pytest.mark.gpu

CASES = int(os.environ.get("PCPA_RANDOM_CASES", "8"))


def _draw(i: int):
    rng = np.random.default_rng(5000 + i)
    for _ in range(200):
        pcp = int(rng.choice([1, 2, 3, 4, 8]))
        il = int(rng.choice([16, 32, 64]))
        local_q = il * int(rng.integers(1, 5))
        if (pcp * local_q) % 64:
            continue
        blk = int(rng.choice([64, 128, 256]))
        if blk % il:
            continue
        d = int(rng.choice([64, 128, 256]))
        hkv = int(rng.choice([1, 2]))
        group = int(rng.choice([1, 2, 4]))
        stride = pcp * il
        max_hist = stride * int(rng.integers(1, max(2, 4096 // stride) + 1))
        actual = int(rng.integers(0, max_hist + 1))
        kv_dtype = str(rng.choice(["fp8_e4m3fn", "bfloat16"]))
        try:
            cfg = PCPAttentionConfig(pcp_size=pcp, current_len=pcp * local_q, max_history_len=max_hist,
                                     actual_history_len=max(actual, 1), block_size=blk, interleave_size=il,
                                     num_q_heads=hkv * group, num_kv_heads=hkv, head_dim=d, kv_dtype=kv_dtype,
                                     backend="hip").validate()
        except ValueError:
            continue
        precision = str(rng.choice(["auto", "fp8", "bf16"])) if kv_dtype == "fp8_e4m3fn" else "auto"
        if precision == "fp8" and cfg.actual_history_len < 2048:
            precision = "auto"
        return cfg, kv_dtype, precision
    raise AssertionError("no valid configuration drawn")


@pytest.mark.parametrize("i", range(CASES))
def test_random_prefill(i, cuda_device):
    cfg, kv_dtype, precision = _draw(i)
    print(f"case {i}: pcp={cfg.pcp_size} il={cfg.interleave_size} local_q={cfg.local_q_len} blk={cfg.block_size} "
          f"Hq/Hkv={cfg.num_q_heads}/{cfg.num_kv_heads} D={cfg.head_dim} hist={cfg.actual_history_len}/"
          f"{cfg.max_history_len} {kv_dtype} {precision}", flush=True)
    problem = build_paged_problem(cfg, seed=6000 + i, kv_scale="per_tensor" if kv_dtype != "bfloat16" else "none")
    g = torch.Generator().manual_seed(7000 + i)
    shape = (cfg.num_kv_heads, cfg.current_len, cfg.head_dim)
    kc = torch.randn(shape, generator=g, dtype=torch.bfloat16)
    vc = torch.randn(shape, generator=g, dtype=torch.bfloat16)
    gpu = problem.to(cuda_device)
    prefill = PrefillAttention(cfg)
    kv_cur = stack_current_kv(kc, vc).to(cuda_device)
    out, lse = prefill(gpu.q_stacked, gpu.kv_pages, gpu.block_table, kv_cur, page_valid_len=gpu.page_valid_len,
                       k_scale=problem.k_scale, v_scale=problem.v_scale, precision=precision, return_lse=True)
    torch.cuda.synchronize()
    got, got_lse = out.float().cpu().numpy(), lse.cpu().numpy()
    assert np.isfinite(got).all() and np.isfinite(got_lse).all()
    q, k, v = _real_history(problem)
    eo, el = orc.expected_with_current(q, kc.double().numpy(), vc.double().numpy(), orc.OracleShape.from_config(cfg),
                                       k, v)
    max_abs, mean_abs = orc.max_abs_and_mean_abs(got, eo)
    lse_diff = np.abs(got_lse - el)
    print(f"  max_abs={max_abs:.3e} mean_abs={mean_abs:.3e} lse max={lse_diff.max():.3e} "
          f"mean={lse_diff.mean():.3e}", flush=True)
    mode = "bf16" if prefill.history.uses_bf16_mfma(precision) else "fp8"
    lse_max, lse_mean = LSE_TOL[mode]
    assert max_abs <= MAX_ABS_TOL and mean_abs <= MEAN_ABS_TOL
    assert lse_diff.max() <= lse_max and lse_diff.mean() <= lse_mean
