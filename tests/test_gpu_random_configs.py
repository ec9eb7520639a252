"""Seeded random configurations through every kernel variant, against the
float64 oracle on every output row.

Each case draws pcp size, interleave, block size, heads, head dim, cache
dtype, MFMA precision and a runtime history length (generally not aligned to
anything) from a fixed seed, so the set is the same on every run.  Bar:
max-abs <= 2e-2 and mean-abs <= 2e-3 for every case on BF16 MFMAs and under
``precision="auto"`` (e4m3 MFMAs with the precision guard).  Explicit
``precision="fp8"`` (no guard) over short histories can miss it: the e4m3
rounding of Q and P is not averaged away over few keys.  Such a case must
then match the e4m3 numerical model of its kernel (oracle/e4m3_model.py) to
within the output's bf16 rounding plus 5e-3 on at least 99% of the rows with
a probability mass of 64 or more, on the rest within one e4m3 code step of
one key (a score on a rounding tie, summed in another order by the MFMA:
random case 99 has such a key at an exact tie, and flipping its code in the
model leaves 9.6e-4), and in the mean; which shows the miss is the method's
rounding and nothing else.  Such a miss may only happen below 4096 history
tokens, and a case without a row of mass 64 must meet the bar under the
guard instead.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from aws_training_study_amd.pcp_attention import make_history_attention_kernel
from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig
from aws_training_study_amd.pcp_attention.workloads import build_paged_problem
from oracle import e4m3_model as em
from oracle import pcp_oracle as orc

from test_gpu_parity import MAX_ABS_TOL, MEAN_ABS_TOL, _real_history

pytestmark = pytest.mark.gpu

# PCPA_RANDOM_CASES widens the sweep (the same first 16 cases, then more).
CASES = int(os.environ.get("PCPA_RANDOM_CASES", "16"))


def _draw(i: int) -> tuple[PCPAttentionConfig, str, dict]:
    rng = np.random.default_rng(1000 + i)
    for _ in range(100):
        pcp = int(rng.choice([1, 2, 3, 4, 8]))
        il = int(rng.choice([16, 32, 64]))
        blk = int(rng.choice([64, 128, 256, 512]))
        if blk % il:
            continue
        d = int(rng.choice([64, 128, 256, 256]))
        hkv = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 2, 4, 8]))
        stride = pcp * il
        q_len = stride * int(rng.integers(1, max(2, 256 // stride) + 1))
        max_hist = stride * int(rng.integers(1, max(2, 8192 // stride) + 1))
        actual = int(rng.integers(1, max_hist + 1))
        kv_dtype = str(rng.choice(["fp8_e4m3fn", "fp8_e4m3fn", "bfloat16"]))
        try:
            cfg = PCPAttentionConfig(pcp_size=pcp, current_len=q_len, max_history_len=max_hist,
                                     actual_history_len=actual, block_size=blk, interleave_size=il,
                                     num_q_heads=hkv * group, num_kv_heads=hkv, head_dim=d, kv_dtype=kv_dtype,
                                     backend="hip").validate()
        except ValueError:
            continue
        precision = str(rng.choice(["auto", "fp8", "bf16"])) if kv_dtype == "fp8_e4m3fn" else "auto"
        kw = {"precision": precision}
        if precision != "bf16" and kv_dtype == "fp8_e4m3fn" and d == 256:
            kw["exp2"] = str(rng.choice(["fast", "exact"]))
            kw["splits"] = int(rng.choice([1, 1, 2, 3]))
        return cfg, kv_dtype, kw
    raise AssertionError("no valid configuration drawn")


@pytest.mark.parametrize("i", range(CASES))
def test_random_configuration(i, cuda_device):
    cfg, kv_dtype, kw = _draw(i)
    print(f"case {i}: pcp={cfg.pcp_size} il={cfg.interleave_size} blk={cfg.block_size} Hq/Hkv={cfg.num_q_heads}/"
          f"{cfg.num_kv_heads} D={cfg.head_dim} Q={cfg.current_len} hist={cfg.actual_history_len}/"
          f"{cfg.max_history_len} {kv_dtype} {kw}", flush=True)
    problem = build_paged_problem(cfg, seed=2000 + i, kv_scale="per_tensor" if kv_dtype != "bfloat16" else "none")
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    out = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, page_valid_len=gpu.page_valid_len,
                 k_scale=problem.k_scale, v_scale=problem.v_scale, **kw)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    q, k, v = _real_history(problem)
    exp = orc.expected_stacked(q, k, v, orc.OracleShape.from_config(cfg))
    max_abs, mean_abs = orc.max_abs_and_mean_abs(got, exp)
    print(f"  max_abs={max_abs:.3e} mean_abs={mean_abs:.3e}", flush=True)
    if max_abs <= MAX_ABS_TOL and mean_abs <= MEAN_ABS_TOL:
        return
    assert kw.get("precision") == "fp8", "BF16 or guarded path outside the bar"
    # the split count the call ran with (given, or the kernel's own choice)
    splits = kw["splits"] if "splits" in kw else kernel.split_count(cuda_device, False)
    model, _, mass = em.emulate_rows(problem.q_stacked.view(torch.int16).numpy().view(np.uint16),
                                     problem.kv_pages.view(torch.uint8).numpy(), problem.block_table.numpy(),
                                     problem.page_valid_len.numpy(), num_kv_heads=cfg.num_kv_heads,
                                     block_size=cfg.block_size, softmax_scale=cfg.softmax_scale,
                                     k_scale=problem.k_scale, v_scale=problem.v_scale,
                                     kernel="overlap" if cfg.head_dim == 256 else "tile",
                                     exp2=kw.get("exp2", "fast") if cfg.head_dim == 256 else "exact",
                                     splits=int(splits), return_mass=True)
    # Checked on rows with a probability mass of at least 64.  A score whose
    # e4m3 code lies on (or within the fp32 accumulation error of) a rounding
    # tie can round the other way in the MFMA's sum than in the model's exact
    # one; that one code step (at most 32, the e4m3 step above 256) moves the
    # output by up to 32 * 2 max|V| v_scale / l with l = 64 * mass.  Such rows
    # are rare; any other departure shows in every row or in the mean.
    rows_ok = mass >= 64
    ok = np.broadcast_to(rows_ok[..., None], got.shape)
    diff = np.abs(got - model)[ok]
    excess_row = (np.abs(got - model) - np.abs(model) * 2.0 ** -8).max(axis=-1)[rows_ok]
    vmax = float(np.abs(orc.E4M3FN_DECODE[problem.kv_pages.view(torch.uint8).numpy()]).max()) * problem.v_scale
    flip = 32.0 * 2.0 * vmax / (64.0 * mass[rows_ok])
    print(f"  e4m3 case outside the bar: vs e4m3 model on {rows_ok.mean():.2f} of the rows max={diff.max(initial=0):.3e} "
          f"excess={excess_row.max(initial=0):.3e}, rows over 5e-3: {(excess_row > 5e-3).sum()} of "
          f"{excess_row.size}", flush=True)
    # over long histories the e4m3 rounding averages away: a miss there is not
    # the method's
    assert cfg.actual_history_len < 4096, "e4m3 path outside the bar on a long history"
    if not rows_ok.any():
        # no row to hold against the model: the guarded call on the same
        # inputs must meet the bar instead
        auto = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, page_valid_len=gpu.page_valid_len,
                      k_scale=problem.k_scale, v_scale=problem.v_scale,
                      **{k: v for k, v in kw.items() if k != "precision"})
        torch.cuda.synchronize()
        a_max, a_mean = orc.max_abs_and_mean_abs(auto.float().cpu().numpy(), exp)
        print(f"  no row of mass >= 64; guarded: max_abs={a_max:.3e} mean_abs={a_mean:.3e}", flush=True)
        assert a_max <= MAX_ABS_TOL and a_mean <= MEAN_ABS_TOL
        return
    assert (excess_row > 5e-3).mean() <= 0.01
    assert (excess_row <= 5e-3 + flip).all()
    assert diff.mean() <= 2e-4 + np.abs(model[ok]).mean() * 2.0 ** -9
