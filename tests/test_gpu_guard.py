"""The e4m3 MFMA path's error envelope and its precision guard, on the GPU.

* ``precision="auto"`` (e4m3 MFMAs plus the guard) meets the bar (max-abs
  2e-2, mean-abs 2e-3 against float64 attention on the dequantised cache)
  where plain e4m3 MFMAs cannot: short runtime histories in a long bucket
  (given as page lengths and as the reference's mask) and peaked score
  distributions (Q scaled x2 and x3, K with a per-channel factor in [0.5, 2])
  at 8K and 131K keys, aligned and not, with either exp2 mode.
* ``precision="fp8"`` (no guard) matches the e4m3 numerical model
  (oracle/e4m3_model.py) tightly: its larger errors on such data are the
  method's rounding, not a kernel bug.  The same bound holds for the tile
  kernel's e4m3 path at head_dim 64 and 128.
* The guard recomputes exactly what the model says it should: rows whose
  model mass is far above the threshold keep the e4m3 result bit for bit,
  rows far below it get the BF16-MFMA result, and a dense fixup equals the
  BF16-MFMA kernel.
"""

from __future__ import annotations

import functools
from dataclasses import replace

import numpy as np
import pytest
import torch

from aws_training_study_amd import _native
from aws_training_study_amd.pcp_attention import make_history_attention_kernel
from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig
from aws_training_study_amd.pcp_attention.inputs import make_block_valid_mask
from aws_training_study_amd.pcp_attention.paging import page_valid_lengths
from aws_training_study_amd.pcp_attention.workloads import build_paged_problem, get_workload
from oracle import e4m3_model as em
from oracle import pcp_oracle as orc

from test_gpu_parity import MAX_ABS_TOL, MEAN_ABS_TOL

pytestmark = pytest.mark.gpu

FOUR = get_workload("four-chip-fp8").config   # 16 ranks, 8192-token history, D 256
FULL = get_workload("full-fp8").config        # 64 ranks, 131072-token history, D 256


@functools.lru_cache(maxsize=8)
def _problem(cfg: PCPAttentionConfig, k_prescale: str, seed: int, v_factor: float = 1.0):
    return build_paged_problem(cfg, seed, kv_scale="per_tensor", k_prescale=k_prescale, v_factor=v_factor)


def _thresholds(problem, page_valid_len, rows=None):
    """The guard's mass threshold of every KV head (of each listed row)."""
    cfg = problem.config
    thr = em.guard_thresholds(problem.kv_pages.view(torch.uint8).numpy(), problem.block_table.numpy(),
                              page_valid_len.cpu().numpy(), num_kv_heads=cfg.num_kv_heads,
                              block_size=cfg.block_size, head_dim=cfg.head_dim, v_scale=problem.v_scale)
    if rows is None:
        return thr
    return thr[np.asarray(rows)[:, 1] // (cfg.num_q_heads // cfg.num_kv_heads)]


def _sample(cfg, count, seed):
    rng = np.random.default_rng(seed)
    rows = np.stack([rng.integers(0, cfg.pcp_size, count), rng.integers(0, cfg.num_q_heads, count),
                     rng.integers(0, cfg.local_q_len, count)], axis=1)
    corners = np.array([[0, 0, 0], [cfg.pcp_size - 1, cfg.num_q_heads - 1, cfg.local_q_len - 1]])
    return np.concatenate([corners, rows])


def _paged_reference(problem, q_stacked, rows, page_valid_len, with_lse=False):
    """float64 attention of the listed rows over exactly the pages' valid
    prefixes (and each row's natural-log sum of exp(score))."""
    cfg = problem.config
    pool = orc.decode_e4m3fn(problem.kv_pages.view(torch.uint8).numpy()).reshape(
        -1, 2, cfg.num_kv_heads, cfg.block_size, cfg.head_dim)
    table = problem.block_table.numpy()
    lens = page_valid_len.cpu().numpy()
    keys, vals = [], []
    for r in range(cfg.pcp_size):
        for b in range(cfg.max_local_blocks):
            n = min(int(lens[r, b]), cfg.block_size)
            if n > 0:
                keys.append(pool[table[r, b], 0, :, :n])
                vals.append(pool[table[r, b], 1, :, :n])
    k = np.concatenate(keys, axis=1) * problem.k_scale
    v = np.concatenate(vals, axis=1) * problem.v_scale
    q = orc.decode_bfloat16(q_stacked.view(torch.int16).numpy().view(np.uint16))
    group = cfg.num_q_heads // cfg.num_kv_heads
    out = np.empty((len(rows), cfg.head_dim))
    lse = np.empty(len(rows))
    for i, (rank, qh, tok) in enumerate(rows):
        g = qh // group
        o, l = orc.attention_with_lse(q[rank, qh, tok][None, None, :], k[g:g + 1], v[g:g + 1], cfg.softmax_scale)
        out[i], lse[i] = o[0, 0], l[0, 0]
    return (out, lse) if with_lse else out


def _model(problem, q_stacked, rows, page_valid_len, kernel="overlap", exp2="fast", **kw):
    cfg = problem.config
    return em.emulate_rows(q_stacked.view(torch.int16).numpy().view(np.uint16),
                           problem.kv_pages.view(torch.uint8).numpy(), problem.block_table.numpy(),
                           page_valid_len.cpu().numpy(), num_kv_heads=cfg.num_kv_heads, block_size=cfg.block_size,
                           softmax_scale=cfg.softmax_scale, k_scale=problem.k_scale, v_scale=problem.v_scale,
                           kernel=kernel, exp2=exp2, rows=rows, **kw)


def _scaled_q(problem, factor):
    return problem.q_stacked if factor == 1 else (problem.q_stacked.float() * factor).to(torch.bfloat16)


def _pick(out, rows):
    got = out.float().cpu().numpy()
    return np.stack([got[r, h, t] for r, h, t in rows])


def _check_bar(got, want, label):
    max_abs, mean_abs = orc.max_abs_and_mean_abs(got, want)
    print(f"{label}: max_abs={max_abs:.3e} mean_abs={mean_abs:.3e}", flush=True)
    assert np.isfinite(got).all(), label
    assert max_abs <= MAX_ABS_TOL and mean_abs <= MEAN_ABS_TOL, label


def _check_model(got, model, mass, label):
    """The kernel against the model of its own arithmetic: a bf16 rounding of
    the output plus fp32 accumulation-order noise, on rows with a
    probability mass of at least 64.  (With fewer effective keys one e4m3
    code that the MFMA's fp32 accumulation rounds the other way moves the
    output by a large fraction of the key's weight; those rows are reported.)"""
    diff = np.abs(got - model)
    excess = diff - np.abs(model) * 2.0 ** -8
    ok = mass >= 64
    print(f"{label}: vs e4m3 model on {ok.sum()} of {len(ok)} rows max={diff[ok].max(initial=0):.3e} "
          f"excess over bf16 rounding={excess[ok].max(initial=0):.3e} mean={diff[ok].mean() if ok.any() else 0:.3e}; "
          f"low-mass rows max={diff[~ok].max(initial=0):.3e}", flush=True)
    if ok.any():
        assert excess[ok].max() <= 5e-3, label
        assert diff[ok].mean() <= 2e-4 + np.abs(model[ok]).mean() * 2.0 ** -9, label


# ---- short runtime histories in a long bucket (precision chosen from the runtime lengths)


@pytest.mark.parametrize("bucket", ["four-chip", "full"])
@pytest.mark.parametrize("tokens", [785, 1500, 4096])
def test_auto_on_short_runtime_history_page_lengths(bucket, tokens, cuda_device):
    cfg = FOUR if bucket == "four-chip" else FULL
    problem = _problem(cfg, "none", 41)
    lens = page_valid_lengths(replace(cfg, actual_history_len=tokens))
    print(f"case {bucket} bucket {cfg.max_history_len}, runtime {tokens} tokens (page_valid_len)", flush=True)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    out = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, page_valid_len=lens.to(cuda_device),
                 k_scale=problem.k_scale, v_scale=problem.v_scale)
    torch.cuda.synchronize()
    rows = _sample(cfg, 160, tokens)
    _check_bar(_pick(out, rows), _paged_reference(problem, problem.q_stacked, rows, lens),
               f"{bucket} runtime {tokens} auto")


@pytest.mark.parametrize("bucket,tokens", [("four-chip", 1024), ("four-chip", 4096), ("full", 4096), ("full", 8192)])
def test_auto_on_short_runtime_history_reference_mask(bucket, tokens, cuda_device):
    """The reference's mask form (run_poc.py:137-153) on the GPU: converted on
    the device, same result as the page-length form."""
    cfg = FOUR if bucket == "four-chip" else FULL
    problem = _problem(cfg, "none", 41)
    runtime = replace(cfg, actual_history_len=tokens)
    mask = make_block_valid_mask(runtime).to(cuda_device)
    print(f"case {bucket} bucket {cfg.max_history_len}, runtime {tokens} tokens (mask)", flush=True)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    out = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, mask, k_scale=problem.k_scale,
                 v_scale=problem.v_scale)
    lens = page_valid_lengths(runtime)
    ref_out = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, page_valid_len=lens.to(cuda_device),
                     k_scale=problem.k_scale, v_scale=problem.v_scale)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)
    rows = _sample(cfg, 160, tokens + 1)
    _check_bar(_pick(out, rows), _paged_reference(problem, problem.q_stacked, rows, lens),
               f"{bucket} runtime {tokens} mask auto")


# ---- peaked scores (e4m3 away from unit-normal data)

PEAKED = [("none", 2), ("none", 3), ("per_channel", 1), ("per_channel", 2), ("per_channel", 3)]


@pytest.mark.parametrize("k_prescale,q_factor", PEAKED)
@pytest.mark.parametrize("tokens,exp2", [(8192, "fast"), (8000, "exact"), (8000, "fast"), (8192, "exact")])
def test_peaked_scores_8k(k_prescale, q_factor, tokens, exp2, cuda_device):
    cfg = replace(FOUR, actual_history_len=tokens).validate()
    _peaked_case(cfg, k_prescale, q_factor, exp2, cuda_device, rows=192)


@pytest.mark.parametrize("k_prescale,q_factor", [("none", 2), ("none", 3), ("per_channel", 1), ("per_channel", 3)])
@pytest.mark.parametrize("tokens,exp2", [(131072, "fast"), (131000, "exact")])
def test_peaked_scores_131k(k_prescale, q_factor, tokens, exp2, cuda_device):
    cfg = replace(FULL, actual_history_len=tokens).validate()
    _peaked_case(cfg, k_prescale, q_factor, exp2, cuda_device, rows=48)


def _peaked_case(cfg, k_prescale, q_factor, exp2, device, rows):
    problem = _problem(cfg, k_prescale, 43)
    q = _scaled_q(problem, q_factor)
    label = f"L={cfg.actual_history_len} K {k_prescale} Q x{q_factor} exp2 {exp2}"
    print(f"case {label}", flush=True)
    gpu = problem.to(device)
    qd = q.to(device)
    kernel = make_history_attention_kernel(cfg)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale, exp2=exp2)
    auto = kernel(qd, gpu.kv_pages, gpu.block_table, **kw)
    fp8 = kernel(qd, gpu.kv_pages, gpu.block_table, precision="fp8", splits=1, **kw)
    torch.cuda.synchronize()
    sample = _sample(cfg, rows, cfg.actual_history_len + q_factor)
    ref = _paged_reference(problem, q, sample, problem.page_valid_len)
    model, _, mass = _model(problem, q, sample, problem.page_valid_len, exp2=exp2, return_mass=True)
    e4m3_max, e4m3_mean = orc.max_abs_and_mean_abs(_pick(fp8, sample), ref)
    print(f"{label}: e4m3 alone max_abs={e4m3_max:.3e} mean_abs={e4m3_mean:.3e}; rows below the guard mass "
          f"{(mass < _thresholds(problem, problem.page_valid_len, sample)).mean():.2f}", flush=True)
    _check_model(_pick(fp8, sample), model, mass, f"{label} fp8")
    _check_bar(_pick(auto, sample), ref, f"{label} auto")


# ---- V of a wider spread: the threshold grows with max_d Var(V)


@pytest.mark.parametrize("bucket", ["four-chip", "full"])
def test_auto_meets_the_bar_with_wide_v(bucket, cuda_device):
    """V ~ N(0, 16) (standard deviation 4): the rounding error of e4m3 Q
    and P grows 4x with it, past the bar on short and peaked rows; the guard's
    threshold (384 v_scale^2 max_d Var(V), ~16 x 384 here) recomputes those
    rows and the default call meets the bar at 8K and 131K keys."""
    cfg = FOUR if bucket == "four-chip" else FULL
    problem = _problem(cfg, "none", 48, 4.0)
    label = f"{bucket} L={cfg.actual_history_len} V x4"
    print(f"case {label}", flush=True)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale)
    auto = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, **kw)
    fp8 = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, precision="fp8", splits=1, **kw)
    torch.cuda.synchronize()
    sample = _sample(cfg, 96 if bucket == "four-chip" else 48, 48)
    ref = _paged_reference(problem, problem.q_stacked, sample, problem.page_valid_len)
    e4m3_max, e4m3_mean = orc.max_abs_and_mean_abs(_pick(fp8, sample), ref)
    thr = _thresholds(problem, problem.page_valid_len)
    print(f"{label}: thresholds {np.round(thr, 1)}; e4m3 alone max_abs={e4m3_max:.3e} mean_abs={e4m3_mean:.3e}",
          flush=True)
    assert 14 * 384 < thr.min() and thr.max() < 19 * 384
    _check_bar(_pick(auto, sample), ref, f"{label} auto")


@pytest.mark.parametrize("q_factor", [1.5, 2.0])
def test_guard_on_a_table_of_two_staging_chunks(q_factor, cuda_device):
    """2048 table entries (64 ranks x 32 pages of 64 tokens, 131072 keys):
    the V statistics stage the table in two chunks of 1024 entries.  V ~
    N(0, 4) (threshold ~4 x 384); Q x1.5 puts ~2% of the rows below it (a
    sparse fixup over ~20 groups, ~11 ranges each), Q x2 most (dense).
    Sampled rows above 1.25x the model's threshold keep the e4m3 pass's
    output bit for bit, rows below 0.8x get the BF16-MFMA result (to the
    rounding of the fixup's ranges), and the default call meets the bar."""
    cfg = replace(FULL, block_size=64).validate()
    assert cfg.pcp_size * cfg.max_local_blocks > 1024
    problem = _problem(cfg, "none", 49, 2.0)
    q = _scaled_q(problem, q_factor)
    print(f"case 2048 entries of 64 tokens, V x2, Q x{q_factor}", flush=True)
    gpu = problem.to(cuda_device)
    qd = q.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale)
    auto = kernel(qd, gpu.kv_pages, gpu.block_table, **kw)
    fp8 = kernel(qd, gpu.kv_pages, gpu.block_table, precision="fp8", splits=1, **kw)
    bf16 = kernel(qd, gpu.kv_pages, gpu.block_table, precision="bf16", splits=1, **kw)
    torch.cuda.synchronize()
    rows = _sample(cfg, 94, 49)
    _, _, mass = _model(problem, q, rows, problem.page_valid_len, return_mass=True)
    thr = _thresholds(problem, problem.page_valid_len, rows)
    kept, low = mass > 1.25 * thr, mass < 0.8 * thr
    print(f"thresholds {np.round(np.unique(thr), 1)}; rows kept {kept.sum()}, recomputed {low.sum()} of "
          f"{len(rows)}", flush=True)
    assert 3 * 384 < thr.min() and thr.max() < 5 * 384
    assert kept.sum() > 0 and low.sum() > 0
    a, f, b = _pick(auto, rows), _pick(fp8, rows), _pick(bf16, rows)
    assert np.array_equal(a[kept], f[kept])
    assert np.abs(a[low] - b[low]).max() <= 4e-3
    _check_bar(a, _paged_reference(problem, q, rows, problem.page_valid_len), f"2048 entries Q x{q_factor} auto")


# ---- the e4m3 log-sum-exp (the prefill merge's weights)


@pytest.mark.parametrize("q_factor,exp2,splits", [(1, "fast", 1), (1, "exact", 2), (2, "fast", 2), (2, "exact", 1)])
def test_fp8_lse_matches_model_and_auto_lse_meets_the_bar(q_factor, exp2, splits, cuda_device):
    """``precision="fp8"``: the lse equals the model's (which applies the same
    linear-mantissa bias correction, 0.03987 in ln) to fp32 noise plus the odd
    P code rounded the other way, on rows of mass >= 64.  ``"auto"``: rows
    whose mass is below the guard threshold - where the bias, a mean over
    evenly spread exponents, does not hold - carry the BF16 fixup's exact lse;
    every row is within 3e-2 (max) / 3e-3 (mean) of the float64 lse.  The
    residue is Q's rounding to e4m3, which grows with the scores: the model
    with exact Q is within 1.2e-3 of float64 at Q x1, with e4m3 Q 9.4e-3
    (x1) and 2.1e-2 (x2, rows above the guard mass)."""
    cfg = FOUR
    problem = _problem(cfg, "none", 47)
    q = _scaled_q(problem, q_factor)
    label = f"lse Q x{q_factor} exp2 {exp2} splits {splits}"
    print(f"case {label}", flush=True)
    gpu = problem.to(cuda_device)
    qd = q.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale, exp2=exp2,
              return_lse=True)
    _, lse8 = kernel(qd, gpu.kv_pages, gpu.block_table, precision="fp8", splits=splits, **kw)
    auto_out, lse_auto = kernel(qd, gpu.kv_pages, gpu.block_table, **kw)
    torch.cuda.synchronize()
    sample = _sample(cfg, 192, 47 + q_factor)
    _, model_lse, mass = _model(problem, q, sample, problem.page_valid_len, exp2=exp2, splits=splits,
                                return_mass=True)
    ref_out, ref_lse = _paged_reference(problem, q, sample, problem.page_valid_len, with_lse=True)
    got8 = np.array([float(lse8[r, h, t]) for r, h, t in sample])
    got_auto = np.array([float(lse_auto[r, h, t]) for r, h, t in sample])
    ok = mass >= 64
    diff = np.abs(got8 - model_lse)
    err8 = np.abs(got8 - ref_lse)
    err_auto = np.abs(got_auto - ref_lse)
    print(f"{label}: fp8 vs model on {ok.sum()} of {len(ok)} rows max={diff[ok].max(initial=0):.3e} "
          f"mean={diff[ok].mean() if ok.any() else 0:.3e}; fp8 vs float64 max={err8.max():.3e} "
          f"mean={err8.mean():.3e}; auto vs float64 max={err_auto.max():.3e} mean={err_auto.mean():.3e}", flush=True)
    if ok.any():
        assert diff[ok].max() <= 2e-3 and diff[ok].mean() <= 2e-4, label
    assert err_auto.max() <= 3e-2 and err_auto.mean() <= 3e-3, label
    _check_bar(_pick(auto_out, sample), ref_out, f"{label} auto output")


# ---- the tile kernel's e4m3 path (head_dim 64 / 128) against the model


@pytest.mark.parametrize("head_dim,tokens", [(64, 700), (128, 3000), (128, 8192)])
def test_tile_kernel_e4m3_matches_model(head_dim, tokens, cuda_device):
    cfg = PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=8192, actual_history_len=tokens,
                             block_size=256, interleave_size=64, num_q_heads=16, num_kv_heads=2, head_dim=head_dim,
                             backend="hip").validate()
    problem = _problem(cfg, "none", 44)
    print(f"case tile e4m3 D={head_dim} L={tokens}", flush=True)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale)
    fp8 = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, precision="fp8", splits=1, **kw)
    auto = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, **kw)
    torch.cuda.synchronize()
    rows = _sample(cfg, 256, tokens)
    model, _, mass = _model(problem, problem.q_stacked, rows, problem.page_valid_len, kernel="tile", exp2="exact",
                            return_mass=True)
    _check_model(_pick(fp8, rows), model, mass, f"tile D={head_dim} L={tokens} fp8")
    _check_bar(_pick(auto, rows), _paged_reference(problem, problem.q_stacked, rows, problem.page_valid_len),
               f"tile D={head_dim} L={tokens} auto")


@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_tile_kernel_guard_recomputes_the_low_mass_rows(head_dim, splits, cuda_device):
    """The tile kernel's e4m3 path on an 8K history: about a fifth of the rows
    fall below their KV head's threshold.  Rows whose model mass is above
    1.25x it keep the e4m3 pass's output bit for bit; rows below 0.8x get the
    BF16-MFMA result, to the rounding of the fixup's walk split into ranges
    and merged by guard_merge_kernel (whose lanes take the ranges in 32 or 16
    groups at head_dim 64 or 128).  splits 2: the split merge lists the rows."""
    cfg = PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=8192, actual_history_len=8192,
                             block_size=256, interleave_size=64, num_q_heads=16, num_kv_heads=2, head_dim=head_dim,
                             backend="hip").validate()
    problem = _problem(cfg, "none", 47)
    print(f"case tile guard D={head_dim} splits {splits}", flush=True)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale)
    q = gpu.q_stacked
    auto = kernel(q, gpu.kv_pages, gpu.block_table, splits=splits, **kw).float().cpu().numpy()
    fp8 = kernel(q, gpu.kv_pages, gpu.block_table, precision="fp8", splits=splits, **kw).float().cpu().numpy()
    bf16 = kernel(q, gpu.kv_pages, gpu.block_table, precision="bf16", splits=1, **kw).float().cpu().numpy()
    torch.cuda.synchronize()
    _, _, mass = _model(problem, problem.q_stacked, None, problem.page_valid_len, kernel="tile", exp2="exact",
                        splits=splits, return_mass=True)
    thr = _thresholds(problem, problem.page_valid_len)
    group = cfg.num_q_heads // cfg.num_kv_heads
    T = np.repeat(thr, group)[None, :, None]
    kept, low = mass > 1.25 * T, mass < 0.8 * T
    print(f"rows kept {kept.sum()}, recomputed {low.sum()} of {mass.size}", flush=True)
    assert kept.sum() > 0 and low.sum() > 0
    assert np.array_equal(auto[kept], fp8[kept])
    assert np.abs(auto[low] - bf16[low]).max() <= 2e-3
    assert np.abs(auto[low] - fp8[low]).max() > 0


# ---- what the guard recomputes


@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("q_factor,v_factor", [(1.2, 1.0), (1.0, 2.0)])
def test_guard_recomputes_exactly_the_low_mass_rows(q_factor, v_factor, splits, cuda_device):
    """On the 8K workload, Q x1.2 (unit V: threshold ~384) or V ~ N(0, 4)
    (threshold ~4 x 384): some rows fall below their KV head's threshold.
    Rows whose model mass is above 1.25x the model's threshold (oracle
    e4m3_model.guard_thresholds: 384 v_scale^2 max_d Var(V)) keep the e4m3
    pass's output bit for bit; rows below 0.8x get the BF16-MFMA result (to
    the rounding of the fixup's split walk).  splits 1: the row masses and
    the plan launch; 2: the split merge lists the rows."""
    cfg = FOUR
    problem = _problem(cfg, "none", 45, v_factor)
    q = _scaled_q(problem, q_factor)
    print(f"case Q x{q_factor} V x{v_factor} splits {splits}", flush=True)
    gpu = problem.to(cuda_device)
    qd = q.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale)
    auto = kernel(qd, gpu.kv_pages, gpu.block_table, splits=splits, **kw).float().cpu().numpy()
    fp8 = kernel(qd, gpu.kv_pages, gpu.block_table, precision="fp8", splits=splits, **kw).float().cpu().numpy()
    bf16 = kernel(qd, gpu.kv_pages, gpu.block_table, precision="bf16", splits=1, **kw).float().cpu().numpy()
    torch.cuda.synchronize()
    _, _, mass = _model(problem, q, None, problem.page_valid_len, splits=splits, return_mass=True)
    thr = _thresholds(problem, problem.page_valid_len)
    group = cfg.num_q_heads // cfg.num_kv_heads
    T = np.repeat(thr, group)[None, :, None]  # [pcp, Hq, local_q] broadcast
    kept, low = mass > 1.25 * T, mass < 0.8 * T
    print(f"rows kept {kept.sum()}, recomputed {low.sum()} of {mass.size}", flush=True)
    assert kept.sum() > 0 and low.sum() > 0
    assert np.array_equal(auto[kept], fp8[kept])
    assert np.abs(auto[low] - bf16[low]).max() <= 2e-3 * v_factor
    assert np.abs(auto[low] - fp8[low]).max() > 0


@pytest.mark.parametrize("splits", [1, 2])
def test_dense_fixup_equals_the_bf16_kernel(splits, cuda_device):
    """Q x4: every row is flagged, the plan goes dense (one pass per group of
    128 gathered rows), and the result is the one-pass BF16-MFMA kernel's,
    bit for bit, whatever order the rows were listed in (splits 2: by device
    atomics in the split merge)."""
    cfg = FOUR
    problem = _problem(cfg, "none", 46)
    q = _scaled_q(problem, 4).to(cuda_device)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale)
    auto, lse = kernel(q, gpu.kv_pages, gpu.block_table, return_lse=True, splits=splits, **kw)
    bf16, lse16 = kernel(q, gpu.kv_pages, gpu.block_table, precision="bf16", return_lse=True, splits=1, **kw)
    torch.cuda.synchronize()
    assert torch.equal(auto, bf16)
    assert torch.equal(lse, lse16)
    # and both against float64: scores this peaked raise the running max past
    # the lazy threshold mid-walk (O^T rescaled in place)
    sample = _sample(cfg, 96, 46)
    ref_out, ref_lse = _paged_reference(problem, q.cpu(), sample, problem.page_valid_len, with_lse=True)
    _check_bar(_pick(bf16, sample), ref_out, "Q x4 bf16")
    got_lse = np.array([float(lse16[r, h, t]) for r, h, t in sample])
    assert np.abs(got_lse - ref_lse).max() <= 1e-4
