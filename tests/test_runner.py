"""Runner helpers (reference tests/test_runner.py:7-22, run_poc.py:81-169)."""

import numpy as np
import pytest
import torch

from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig, get_preset
from aws_training_study_amd.run_poc import main, make_block_valid_mask, make_inputs, make_local_inputs, parse_args
from aws_training_study_amd.pcp_attention.inputs import make_scaled_inputs
from oracle import pcp_oracle as orc


def test_partial_block_valid_mask():
    cfg = get_preset("tiny").with_overrides(actual_history_len=1024)
    mask = make_block_valid_mask(cfg)
    assert mask.shape == (1, 4, 1, 128)
    assert mask.dtype == torch.bfloat16
    assert torch.all(mask[0, :2] == 0)
    assert torch.all(mask[0, 2:] == -9984)


def test_local_kv_inputs_use_final_fp8_storage():
    _, k, v = make_local_inputs(get_preset("tiny"), seed=1234, rank=0)
    assert k.dtype == torch.float8_e4m3fn
    assert v.dtype == torch.float8_e4m3fn


@pytest.mark.parametrize("actual", [512, 1024, 1536, 2048])
def test_block_mask_matches_oracle(actual):
    cfg = get_preset("tiny").with_overrides(max_history_len=4096, actual_history_len=actual)
    np.testing.assert_array_equal(
        make_block_valid_mask(cfg).float().numpy(), orc.block_valid_mask(orc.OracleShape.from_config(cfg))
    )


def test_make_inputs_draw_order():
    """One generator draws Q, then K, then V as BF16 N(0,1); K/V cast to e4m3 (run_poc.py:81-104)."""
    cfg = get_preset("tiny")
    q, k, v = make_inputs(cfg, seed=77)
    g = torch.Generator().manual_seed(77)
    q2 = torch.randn(32, 256, 256, generator=g, dtype=torch.bfloat16)
    k2 = torch.randn(2, 2048, 256, generator=g, dtype=torch.bfloat16)
    v2 = torch.randn(2, 2048, 256, generator=g, dtype=torch.bfloat16)
    assert torch.equal(q, q2)
    assert torch.equal(k.view(torch.uint8), k2.to(torch.float8_e4m3fn).view(torch.uint8))
    assert torch.equal(v.view(torch.uint8), v2.to(torch.float8_e4m3fn).view(torch.uint8))
    # The scaled variant draws the same normals first.
    scaled = make_scaled_inputs(cfg, seed=77)
    assert torch.equal(scaled.q, q) and torch.equal(scaled.k.view(torch.uint8), k.view(torch.uint8))


def test_per_tensor_scale_roundtrip():
    cfg = get_preset("tiny")
    scaled = make_scaled_inputs(cfg, seed=5, kv_scale="per_tensor")
    ref = make_scaled_inputs(cfg, seed=5)
    g = torch.Generator().manual_seed(5)
    torch.randn(32, 256, 256, generator=g, dtype=torch.bfloat16)
    k_bf16 = torch.randn(2, 2048, 256, generator=g, dtype=torch.bfloat16)
    assert scaled.k_scale == pytest.approx(float(k_bf16.float().abs().max()) / 448.0)
    deq = scaled.k.float() * scaled.k_scale
    rel = ((deq - k_bf16.float()).abs() / k_bf16.float().abs().clamp_min(1e-3)).max()
    assert rel <= 2 ** -4 + 1e-6  # round-to-nearest e4m3: half an ulp of 3 mantissa bits
    assert float(scaled.k.float().abs().max()) <= 448.0
    assert ref.k_scale == 1.0


def test_run_poc_cpu_backend_points_to_oracle():
    with pytest.raises(SystemExit, match="CPU ring model"):
        main(["--backend", "cpu", "--preset", "tiny"])


def test_run_poc_args():
    args = parse_args(["--backend", "hip", "--preset", "full", "--start-offset", "65536", "--kv-dtype", "fp8_e4m3fn"])
    assert args.actual_history_len == 65536 and args.backend == "hip"


def test_local_problem_is_the_per_rank_draws_packed_into_pages():
    """--check none inputs: rank r's own seeded Q shard and local cache
    (seed + 104729 * r, run_poc.py:107-134), padded to max_local_blocks with
    zero pages (run_poc.py:231-237) and placed by the block table."""
    from aws_training_study_amd.pcp_attention.kernel import pack_local_kv
    from aws_training_study_amd.pcp_attention.workloads import build_local_problem

    cfg = get_preset("tiny").with_overrides(backend="hip", max_history_len=4096, actual_history_len=2048)
    problem = build_local_problem(cfg, seed=9)
    assert cfg.actual_local_blocks == 1 and cfg.max_local_blocks == 2
    table = problem.block_table
    for rank in range(cfg.pcp_size):
        q, k, v = make_local_inputs(cfg, seed=9, rank=rank)
        assert torch.equal(problem.q_stacked[rank], q)
        assert torch.equal(problem.kv_pages[int(table[rank, 0])].view(torch.uint8),
                           pack_local_kv(k, v)[0].view(torch.uint8))
        assert not bool(problem.kv_pages[int(table[rank, 1])].view(torch.uint8).any())
    # every rank's 512 valid tokens in its first block, none in the padding
    assert problem.page_valid_len.tolist() == [[512, 0]] * cfg.pcp_size
    assert problem.k_scale == problem.v_scale == 1.0
    # the oracle over those pages is ordinary attention over every rank's cache
    shape = orc.OracleShape.from_config(cfg)
    pool = orc.decode_e4m3fn(problem.kv_pages.view(torch.uint8).numpy())
    q = orc.decode_bfloat16(problem.q_stacked.view(torch.int16).numpy().view(np.uint16))
    out = orc.paged_history_attention(q, pool, table.numpy(), problem.page_valid_len.numpy(), shape)
    keys = np.concatenate([pool[int(table[r, 0])].reshape(2, 2, 512, 256)[0] for r in range(4)], axis=1)
    vals = np.concatenate([pool[int(table[r, 0])].reshape(2, 2, 512, 256)[1] for r in range(4)], axis=1)
    want = orc.dense_history_attention(q[1], keys, vals, shape.softmax_scale)
    np.testing.assert_allclose(out[1], want, rtol=0, atol=1e-12)


def test_local_problem_needs_an_aligned_history():
    from aws_training_study_amd.pcp_attention.workloads import build_local_problem

    cfg = get_preset("tiny").with_overrides(backend="hip", actual_history_len=1000)
    with pytest.raises(ValueError, match="multiple of pcp_size"):
        build_local_problem(cfg, seed=1)
