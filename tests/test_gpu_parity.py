"""GPU parity of the gfx950 history attention kernel against the CPU oracle.

Bar (all workloads): max-abs error <= 2e-2 and mean-abs error <= 2e-3
versus float64 attention on the identical dequantised inputs.  Small
workloads are checked on every output row; the large ones on a seeded sample
of rows against the oracle, and on every row against a float32 torch
reference computed on the GPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from aws_training_study_amd.pcp_attention import make_history_attention_kernel
from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig
from aws_training_study_amd.pcp_attention.inputs import make_block_valid_mask
from aws_training_study_amd.pcp_attention.workloads import (
    build_paged_problem,
    build_workload_problem,
    get_workload,
)
from oracle import pcp_oracle as orc

MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3

pytestmark = pytest.mark.gpu


def _real_history(problem):
    """Dequantised global K/V as float64 numpy (the oracle's inputs)."""
    inputs = problem.inputs
    if inputs.k.dtype == torch.float8_e4m3fn:
        k = orc.decode_e4m3fn(inputs.k.view(torch.uint8).numpy()) * inputs.k_scale
        v = orc.decode_e4m3fn(inputs.v.view(torch.uint8).numpy()) * inputs.v_scale
    else:
        k = orc.decode_bfloat16(inputs.k.view(torch.int16).numpy().view(np.uint16))
        v = orc.decode_bfloat16(inputs.v.view(torch.int16).numpy().view(np.uint16))
    q = orc.decode_bfloat16(inputs.q.view(torch.int16).numpy().view(np.uint16))
    return q, k, v


def _run(problem, device, precision="auto", exp2="fast"):
    gpu = problem.to(device)
    kernel = make_history_attention_kernel(problem.config)
    out = kernel(
        gpu.q_stacked,
        gpu.kv_pages,
        gpu.block_table,
        page_valid_len=gpu.page_valid_len,
        k_scale=problem.k_scale,
        v_scale=problem.v_scale,
        precision=precision,
        exp2=exp2,
    )
    torch.cuda.synchronize()
    return out


def _sample_rows(shape, count, seed):
    rng = np.random.default_rng(seed)
    rows = np.stack(
        [
            rng.integers(0, shape.pcp_size, count),
            rng.integers(0, shape.num_q_heads, count),
            rng.integers(0, shape.local_q_len, count),
        ],
        axis=1,
    )
    corners = np.array(
        [
            [0, 0, 0],
            [shape.pcp_size - 1, shape.num_q_heads - 1, shape.local_q_len - 1],
            [0, shape.num_q_heads - 1, 0],
            [shape.pcp_size - 1, 0, shape.local_q_len - 1],
        ]
    )
    return np.concatenate([corners, rows])


def _assert_close(actual, expected, label):
    max_abs, mean_abs = orc.max_abs_and_mean_abs(actual, expected)
    print(f"{label}: max_abs={max_abs:.3e} mean_abs={mean_abs:.3e}", flush=True)
    assert np.isfinite(actual).all(), f"{label}: non-finite output"
    assert max_abs <= MAX_ABS_TOL, f"{label}: max_abs {max_abs:.3e} > {MAX_ABS_TOL}"
    assert mean_abs <= MEAN_ABS_TOL, f"{label}: mean_abs {mean_abs:.3e} > {MEAN_ABS_TOL}"


def _torch_dense_reference(problem, device, row_chunk=2048):
    """float32 dense attention of every stacked row on the GPU (independent of the kernel)."""
    cfg = problem.config
    q, k, v = (torch.from_numpy(x).to(device, torch.float32) for x in _real_history(problem))
    length = cfg.actual_history_len
    qs = problem.q_stacked.to(device).float()  # [pcp, Hq, Lq, D]
    out = torch.empty_like(qs)
    group = cfg.num_q_heads // cfg.num_kv_heads
    for g in range(cfg.num_kv_heads):
        kg = k[g, :length].contiguous()
        vg = v[g, :length].contiguous()
        rows = qs[:, g * group:(g + 1) * group].reshape(-1, cfg.head_dim)
        res = torch.empty_like(rows)
        for start in range(0, rows.shape[0], row_chunk):
            s = rows[start:start + row_chunk] @ kg.T * cfg.softmax_scale
            res[start:start + row_chunk] = torch.softmax(s, dim=-1) @ vg
        out[:, g * group:(g + 1) * group] = res.reshape(cfg.pcp_size, group, cfg.local_q_len, cfg.head_dim)
    return out


@pytest.mark.parametrize("name", ["tiny-gqa4-d64-bf16", "four-chip-fp8"])
def test_small_workloads_every_row(name, cuda_device):
    problem = build_workload_problem(name, seed=1234)
    print(f"case {name}: {problem.config}", flush=True)
    out = _run(problem, cuda_device).float().cpu().numpy()
    q, k, v = _real_history(problem)
    shape = orc.OracleShape.from_config(problem.config)
    _assert_close(out, orc.expected_stacked(q, k, v, shape), name)


@pytest.mark.parametrize("name", ["gqa8-d128-bf16", "full-fp8", "full-fp8-varlen", "full-bf16", "four-chip-q16k-fp8"])
def test_large_workloads(name, cuda_device):
    problem = build_workload_problem(name, seed=1234)
    print(f"case {name}: {problem.config}", flush=True)
    out = _run(problem, cuda_device)
    shape = orc.OracleShape.from_config(problem.config)
    rows = _sample_rows(shape, 96, seed=99)
    q, k, v = _real_history(problem)
    expected = orc.expected_rows(q, k, v, shape, rows)
    got = out.float().cpu().numpy()[rows[:, 0], rows[:, 1], rows[:, 2]]
    _assert_close(got, expected, f"{name} sampled rows vs oracle")
    ref = _torch_dense_reference(problem, cuda_device)
    _assert_close(out.float().cpu().numpy(), ref.cpu().numpy(), f"{name} every row vs fp32 torch")


def test_reference_mask_form_and_partial_blocks(cuda_device):
    """The reference's additive block mask (run_poc.py:137-153) gives the same result."""
    cfg = PCPAttentionConfig(
        pcp_size=4, current_len=256, max_history_len=4096, actual_history_len=1024,
        block_size=512, interleave_size=64, backend="hip",
    ).validate()
    problem = build_paged_problem(cfg, seed=7, kv_scale="per_tensor")
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    a = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, page_valid_len=gpu.page_valid_len,
               k_scale=problem.k_scale, v_scale=problem.v_scale)
    b = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, make_block_valid_mask(cfg),
               k_scale=problem.k_scale, v_scale=problem.v_scale)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    q, k, v = _real_history(problem)
    shape = orc.OracleShape.from_config(cfg)
    _assert_close(a.float().cpu().numpy(), orc.expected_stacked(q, k, v, shape), "partial-block tiny")


@pytest.mark.parametrize("actual", [64 * 4 * 3 + 17, 1000, 4096 - 1, 1])
def test_unaligned_history_lengths(actual, cuda_device):
    """Runtime lengths that end inside a chunk, a block or on the first token."""
    cfg = PCPAttentionConfig(
        pcp_size=4, current_len=256, max_history_len=4096, actual_history_len=actual,
        block_size=256, interleave_size=64, backend="hip",
    ).validate()
    problem = build_paged_problem(cfg, seed=actual, kv_scale="per_tensor")
    out = _run(problem, cuda_device).float().cpu().numpy()
    q, k, v = _real_history(problem)
    shape = orc.OracleShape.from_config(cfg)
    _assert_close(out, orc.expected_stacked(q, k, v, shape), f"unaligned actual={actual}")


@pytest.mark.parametrize("kv_dtype,head_dim", [("fp8_e4m3fn", 64), ("fp8_e4m3fn", 128), ("bfloat16", 256)])
def test_other_head_dims(kv_dtype, head_dim, cuda_device):
    cfg = PCPAttentionConfig(
        pcp_size=2, current_len=256, max_history_len=2048, actual_history_len=2048,
        block_size=128, interleave_size=64, num_q_heads=6, num_kv_heads=2, head_dim=head_dim,
        backend="hip", kv_dtype=kv_dtype,
    ).validate()
    problem = build_paged_problem(cfg, seed=head_dim, kv_scale="per_tensor" if kv_dtype != "bfloat16" else "none")
    out = _run(problem, cuda_device).float().cpu().numpy()
    q, k, v = _real_history(problem)
    shape = orc.OracleShape.from_config(cfg)
    _assert_close(out, orc.expected_stacked(q, k, v, shape), f"{kv_dtype} D={head_dim}")


def test_deterministic_and_page_order_invariant(cuda_device):
    """Same inputs give bit-identical output; a different page permutation moves data, not results."""
    problem = build_workload_problem("four-chip-fp8", seed=5)
    a = _run(problem, cuda_device)
    b = _run(problem, cuda_device)
    assert torch.equal(a, b)
    identity = build_paged_problem(problem.config, seed=5, kv_scale="per_tensor", shuffle_pages=False)
    assert not torch.equal(identity.block_table, problem.block_table)
    c = _run(identity, cuda_device)
    # Same pages visited in the same table order -> same arithmetic, same bits.
    assert torch.equal(a, c)


@pytest.mark.parametrize("precision", ["fp8", "bf16"])
@pytest.mark.parametrize("head_dim", [128, 256])
def test_fp8_cache_both_mfma_precisions(precision, head_dim, cuda_device):
    """An e4m3 cache through e4m3 MFMAs and through exactly widened BF16 MFMAs."""
    cfg = PCPAttentionConfig(
        pcp_size=8, current_len=512, max_history_len=8192, actual_history_len=8192, block_size=256,
        head_dim=head_dim, backend="hip",
    ).validate()
    problem = build_paged_problem(cfg, seed=head_dim + 1, kv_scale="per_tensor")
    kernel = make_history_attention_kernel(cfg)
    assert kernel.uses_bf16_mfma(precision) == (precision == "bf16")
    out = _run(problem, cuda_device, precision=precision).float().cpu().numpy()
    q, k, v = _real_history(problem)
    _assert_close(out, orc.expected_stacked(q, k, v, orc.OracleShape.from_config(cfg)),
                  f"fp8 cache, {precision} MFMA, D={head_dim}")


@pytest.mark.parametrize("exp2", ["fast", "exact"])
@pytest.mark.parametrize("actual", [8192, 5000])
def test_fp8_exp2_modes(exp2, actual, cuda_device):
    """Both ways of forming the e4m3 probabilities (D=256 e4m3 path) against the
    float64 oracle, aligned and with a partial last tile; the two results stay
    close to each other as well."""
    cfg = PCPAttentionConfig(
        pcp_size=8, current_len=512, max_history_len=8192, actual_history_len=actual, block_size=256,
        head_dim=256, backend="hip",
    ).validate()
    problem = build_paged_problem(cfg, seed=actual + 7, kv_scale="per_tensor")
    out = _run(problem, cuda_device, precision="fp8", exp2=exp2).float().cpu().numpy()
    q, k, v = _real_history(problem)
    _assert_close(out, orc.expected_stacked(q, k, v, orc.OracleShape.from_config(cfg)),
                  f"fp8 MFMA, exp2={exp2}, actual={actual}")
    other = _run(problem, cuda_device, precision="fp8", exp2="exact" if exp2 == "fast" else "fast")
    diff = np.abs(out - other.float().cpu().numpy())
    print(f"fast vs exact exp2: max_abs={diff.max():.3e} mean_abs={diff.mean():.3e}", flush=True)
    assert diff.max() <= MAX_ABS_TOL and diff.mean() <= MEAN_ABS_TOL


def test_per_rank_list_input(cuda_device):
    """The reference's per-rank Q list gives the stacked call's output, rank by rank."""
    problem = build_workload_problem("tiny-gqa4-d64-bf16", seed=9)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(problem.config)
    stacked = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, page_valid_len=gpu.page_valid_len)
    shards = [gpu.q_stacked[r] for r in range(problem.config.pcp_size)]
    listed = kernel(shards, gpu.kv_pages, gpu.block_table, page_valid_len=gpu.page_valid_len)
    torch.cuda.synchronize()
    assert torch.equal(listed, stacked)
    with pytest.raises(ValueError, match="per-rank Q shards"):
        kernel(shards[:-1], gpu.kv_pages, gpu.block_table)


@pytest.mark.parametrize("name", ["tiny-gqa4-d64-bf16", "four-chip-fp8"])
def test_per_rank_local_caches_equal_the_pool_form(name, cuda_device):
    """The NKI kernel's per-rank call form, kernel(q_ref, local_kv_ref,
    block_valid_mask_ref) with every rank's [max_local_blocks, payload]
    cache (kernel.py:84-118, run_poc.py:231-238), gives the pool form's
    output bit for bit: same pages in the same walk order, the pool here
    shuffled by a random block table."""
    problem = build_workload_problem(name, seed=10)
    cfg = problem.config
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    kw = dict(k_scale=problem.k_scale, v_scale=problem.v_scale)
    pooled = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, page_valid_len=gpu.page_valid_len, **kw)
    local_kv = [gpu.kv_pages.index_select(0, gpu.block_table[r].long()).contiguous() for r in range(cfg.pcp_size)]
    q_list = [gpu.q_stacked[r] for r in range(cfg.pcp_size)]
    mask = make_block_valid_mask(cfg).to(cuda_device)
    print(f"case {name}: per-rank caches, reference mask", flush=True)
    listed = kernel(q_list, local_kv, mask, **kw)
    again = kernel(q_list, local_kv, mask, **kw)  # the pool built once is reused
    torch.cuda.synchronize()
    assert torch.equal(listed, pooled) and torch.equal(again, pooled)


@pytest.mark.parametrize(
    "kv_dtype,head_dim,precision,splits",
    [
        ("fp8_e4m3fn", 256, "fp8", 1),
        ("fp8_e4m3fn", 256, "fp8", 3),
        ("fp8_e4m3fn", 128, "fp8", 1),
        ("fp8_e4m3fn", 256, "bf16", 1),
        ("bfloat16", 128, "auto", 1),
        # the tile kernel's split ranges over the same holes
        ("fp8_e4m3fn", 128, "fp8", 4),
        ("fp8_e4m3fn", 256, "bf16", 3),
        ("bfloat16", 128, "auto", 5),
    ],
)
def test_skipped_pages_holes_and_clamped_lengths(kv_dtype, head_dim, precision, splits, cuda_device):
    """Table entries outside [0, num_pages) and zero-length pages drop exactly their keys; lengths
    beyond the block count the whole block (C ABI contract), against the float64 paged oracle."""
    from test_oracle import _drop_pages

    cfg = PCPAttentionConfig(
        pcp_size=4, current_len=256, max_history_len=4096, actual_history_len=4096,
        block_size=256, interleave_size=64, num_q_heads=8, head_dim=head_dim, backend="hip", kv_dtype=kv_dtype,
    ).validate()
    print(f"case {kv_dtype} D={head_dim} precision={precision} splits={splits}", flush=True)
    problem = build_paged_problem(cfg, seed=13, kv_scale="per_tensor" if kv_dtype != "bfloat16" else "none")
    shape = orc.OracleShape.from_config(cfg)
    table, valid, kept = _drop_pages(problem, shape)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(cfg)
    out = kernel(gpu.q_stacked, gpu.kv_pages, torch.from_numpy(table).to(cuda_device),
                 page_valid_len=torch.from_numpy(valid).to(cuda_device), k_scale=problem.k_scale,
                 v_scale=problem.v_scale, precision=precision, splits=splits)
    torch.cuda.synchronize()
    q, k, v = _real_history(problem)
    qs = np.stack(orc.shard_query(q, shape))
    expected = np.stack([orc.dense_history_attention(qs[r], k[:, kept], v[:, kept], shape.softmax_scale)
                         for r in range(shape.pcp_size)])
    _assert_close(out.float().cpu().numpy(), expected, f"{kv_dtype} D={head_dim} {precision} dropped pages")
