"""Paged pool, block table and per-page validity (host side, no GPU)."""

import numpy as np
import pytest
import torch

from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig, get_preset
from aws_training_study_amd.pcp_attention.inputs import make_block_valid_mask
from aws_training_study_amd.pcp_attention.kernel import pack_local_kv
from aws_training_study_amd.pcp_attention.layout import shard_history
from aws_training_study_amd.pcp_attention.paging import (
    check_block_table,
    make_block_table,
    pack_page_pool,
    page_valid_lengths,
    valid_lengths_from_block_mask,
)
from aws_training_study_amd.pcp_attention.workloads import WORKLOADS, build_paged_problem
from oracle import pcp_oracle as orc


def _cfg(**kw):
    base = dict(pcp_size=4, current_len=256, max_history_len=4096, actual_history_len=4096, block_size=256,
                head_dim=64, backend="hip")
    base.update(kw)
    return PCPAttentionConfig(**base).validate()


@pytest.mark.parametrize("actual", [1, 63, 64, 65, 255, 256, 1000, 2048, 4095, 4096])
def test_page_valid_lengths_match_oracle(actual):
    cfg = _cfg(actual_history_len=actual)
    ours = page_valid_lengths(cfg)
    assert ours.dtype == torch.int32 and ours.shape == (4, cfg.max_local_blocks)
    np.testing.assert_array_equal(ours.numpy(), orc.page_valid_lengths(orc.OracleShape.from_config(cfg)))
    assert int(ours.sum()) == actual


@pytest.mark.parametrize("actual", [512, 1024, 1536, 2048])
def test_reference_mask_converts_to_valid_lengths(actual):
    cfg = get_preset("tiny").with_overrides(max_history_len=4096, actual_history_len=actual)
    hip_cfg = cfg.with_overrides(backend="hip")
    converted = valid_lengths_from_block_mask(make_block_valid_mask(cfg), hip_cfg)
    assert torch.equal(converted, page_valid_lengths(hip_cfg))


def test_mask_conversion_rejects_non_prefix_masks():
    cfg = get_preset("tiny").with_overrides(backend="hip")
    mask = make_block_valid_mask(cfg).clone()
    mask[0, 1, 0, 3] = -9984
    with pytest.raises(ValueError, match="prefix"):
        valid_lengths_from_block_mask(mask, cfg)
    mask = make_block_valid_mask(cfg).clone()
    mask[0, 0, 0, 0] = -1.0
    with pytest.raises(ValueError, match="0 \\(valid\\)"):
        valid_lengths_from_block_mask(mask, cfg)
    with pytest.raises(ValueError, match="shape"):
        valid_lengths_from_block_mask(mask[:, :2], cfg)


def test_block_table_is_a_seeded_permutation():
    cfg = _cfg()
    a, b = make_block_table(cfg, 5), make_block_table(cfg, 5)
    assert torch.equal(a, b) and a.dtype == torch.int32
    assert sorted(a.reshape(-1).tolist()) == list(range(cfg.num_pages))
    assert not torch.equal(a, make_block_table(cfg, 6))
    with pytest.raises(ValueError, match="lie in"):
        check_block_table(torch.full_like(a, cfg.num_pages), cfg, cfg.num_pages)
    dup = a.clone()
    dup[0, 0] = dup[0, 1]
    with pytest.raises(ValueError, match="same page"):
        check_block_table(dup, cfg, cfg.num_pages)


def test_pool_rows_are_packed_blocks():
    cfg = _cfg(actual_history_len=2048)  # ranks hold 2 of 4 blocks; the rest are zero pages
    g = torch.Generator().manual_seed(0)
    k = torch.randn(2, 2048, 64, generator=g).to(torch.float8_e4m3fn)
    v = torch.randn(2, 2048, 64, generator=g).to(torch.float8_e4m3fn)
    k_shards, v_shards = shard_history(k, v, cfg)
    table = make_block_table(cfg, 9)
    pool = pack_page_pool(k_shards, v_shards, cfg, table)
    assert pool.shape == (cfg.num_pages, cfg.page_elements) and pool.dtype == torch.float8_e4m3fn
    for r in range(4):
        packed = pack_local_kv(k_shards[r], v_shards[r])
        for b in range(cfg.max_local_blocks):
            row = pool[table[r, b]].view(torch.uint8)
            if b < packed.shape[0]:
                assert torch.equal(row, packed[b].view(torch.uint8))
            else:
                assert int(row.count_nonzero()) == 0


@pytest.mark.parametrize("name", sorted(WORKLOADS))
def test_workload_configs_are_valid(name):
    w = WORKLOADS[name]
    cfg = w.resolve(1234)
    assert cfg.backend == "hip"
    if w.random_history_len:
        assert cfg.max_history_len // 2 <= cfg.actual_history_len < cfg.max_history_len
        assert cfg.actual_history_len == w.resolve(1234).actual_history_len


def test_four_chip_problem_layout():
    problem = build_paged_problem(WORKLOADS["four-chip-fp8"].config, seed=1, kv_scale="per_tensor")
    cfg = problem.config
    assert problem.q_stacked.shape == (16, 32, 64, 256)
    assert problem.kv_pages.shape == (16, 2 * 2 * 512 * 256)
    assert 0 < problem.k_scale < 1 and 0 < problem.v_scale < 1
    assert torch.equal(problem.page_valid_len, torch.full((16, 1), 512, dtype=torch.int32))
