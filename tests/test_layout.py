"""Striped layout: reference known answers (tests/test_layout.py:12-40), closed form
(README.md:22-29), bit-exactness against the oracle, and properties."""

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig, get_preset
from aws_training_study_amd.pcp_attention.layout import (
    gather_history,
    global_positions_for_rank,
    owner_and_local_position,
    shard_history,
    shard_history_bucket,
    shard_query,
    stacked_query,
)
from oracle import pcp_oracle as orc


def test_owner_round_trip():
    pcp_size, interleave = 4, 64
    for rank in range(pcp_size):
        positions = global_positions_for_rank(2048, rank, pcp_size, interleave)
        for local_position, global_position in enumerate(positions.tolist()):
            assert owner_and_local_position(global_position, pcp_size, interleave) == (rank, local_position)


def test_history_shard_and_gather_are_inverse():
    cfg = get_preset("tiny")
    shape = (cfg.num_kv_heads, cfg.actual_history_len, cfg.head_dim)
    k = torch.arange(int(np.prod(shape)), dtype=torch.float32).reshape(shape)
    k_shards, v_shards = shard_history(k, -k, cfg)
    torch.testing.assert_close(gather_history(k_shards, cfg), k)
    torch.testing.assert_close(gather_history(v_shards, cfg), -k)


def test_partial_cache_block_shard_and_gather_are_inverse():
    cfg = get_preset("tiny").with_overrides(actual_history_len=1024)
    shape = (cfg.num_kv_heads, cfg.actual_history_len, cfg.head_dim)
    k = torch.arange(int(np.prod(shape)), dtype=torch.float32).reshape(shape)
    k_shards, _ = shard_history(k, -k, cfg)
    assert k_shards[0].shape[0] == 1
    assert torch.count_nonzero(k_shards[0][:, :, 256:, :]) == 0
    torch.testing.assert_close(gather_history(k_shards, cfg), k)


def test_owner_known_answer_table():
    """pcp 3, interleave 2, worked by hand from chunk = p // 2, owner = chunk % 3,
    local = (chunk // 3) * 2 + p % 2."""
    owners = [0, 0, 1, 1, 2, 2, 0, 0, 1, 1, 2, 2, 0, 0]
    locals_ = [0, 1, 0, 1, 0, 1, 2, 3, 2, 3, 2, 3, 4, 5]
    for p, (owner, local) in enumerate(zip(owners, locals_)):
        assert owner_and_local_position(p, 3, 2) == (owner, local)
        assert orc.owner_and_local_position(p, 3, 2) == (owner, local)
    assert global_positions_for_rank(12, 1, 3, 2).tolist() == [2, 3, 8, 9]
    assert global_positions_for_rank(12, 2, 3, 2).tolist() == [4, 5, 10, 11]


@settings(max_examples=60, deadline=None)
@given(pcp=st.integers(1, 9), il=st.integers(1, 17), rounds=st.integers(1, 6))
def test_positions_partition_and_invert(pcp, il, rounds):
    total = pcp * il * rounds
    seen = np.zeros(total, dtype=np.int64)
    for rank in range(pcp):
        ours = global_positions_for_rank(total, rank, pcp, il)
        assert ours.dtype == torch.int64
        np.testing.assert_array_equal(ours.numpy(), orc.global_positions(total, rank, pcp, il))
        assert torch.all(ours[1:] > ours[:-1])  # strictly increasing in local order
        seen[ours.numpy()] += 1
        for local, p in enumerate(ours.tolist()):
            assert owner_and_local_position(p, pcp, il) == (rank, local)
    assert np.all(seen == 1)


def test_layout_rejects_bad_arguments():
    with pytest.raises(ValueError, match="outside"):
        global_positions_for_rank(128, 4, 4, 16)
    with pytest.raises(ValueError, match="divide evenly"):
        global_positions_for_rank(100, 0, 4, 16)
    cfg = get_preset("tiny")
    with pytest.raises(ValueError, match="expected Q shape"):
        shard_query(torch.zeros(1, 2, 3), cfg)
    with pytest.raises(ValueError, match="expected K/V shape"):
        shard_history(torch.zeros(1, 2, 3), torch.zeros(1, 2, 3), cfg)
    with pytest.raises(ValueError, match="expected 4 shards"):
        gather_history([torch.zeros(1)], cfg)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
def test_shards_bit_exact_vs_oracle(dtype):
    cfg = PCPAttentionConfig(
        pcp_size=3, current_len=96, max_history_len=1536, actual_history_len=1152,
        block_size=256, interleave_size=32, num_q_heads=4, num_kv_heads=2, head_dim=64, backend="hip",
    ).validate()
    g = torch.Generator().manual_seed(3)
    q = torch.randn(4, 96, 64, generator=g).to(dtype)
    k = torch.randn(2, 1152, 64, generator=g).to(dtype)
    v = torch.randn(2, 1152, 64, generator=g).to(dtype)
    byte_views = {torch.float8_e4m3fn: torch.uint8, torch.bfloat16: torch.int16}
    view = (lambda t: t.view(byte_views[dtype])) if dtype in byte_views else (lambda t: t)
    shape = orc.OracleShape.from_config(cfg)
    for ours, theirs in zip(shard_query(q, cfg), orc.shard_query(view(q).numpy(), shape)):
        np.testing.assert_array_equal(view(ours).numpy(), theirs)
    stacked = stacked_query(q, cfg)
    assert stacked.shape == (3, 4, 32, 64)
    assert torch.equal(view(stacked), view(torch.stack(shard_query(q, cfg))))
    k_shards, v_shards = shard_history(k, v, cfg)
    ok = orc.shard_history(view(k).numpy(), shape, 1152)
    ov = orc.shard_history(view(v).numpy(), shape, 1152)
    for a, b, c, d in zip(k_shards, ok, v_shards, ov):
        assert a.dtype == dtype and a.is_contiguous()
        np.testing.assert_array_equal(view(a).numpy(), b)
        np.testing.assert_array_equal(view(c).numpy(), d)
    np.testing.assert_array_equal(view(gather_history(k_shards, cfg)).numpy(), orc.gather_history(ok, shape, 1152))
    np.testing.assert_array_equal(view(gather_history(k_shards, cfg)).numpy(), view(k).numpy())


def test_bucket_shard_covers_max_history():
    cfg = PCPAttentionConfig(
        pcp_size=4, current_len=256, max_history_len=4096, actual_history_len=1000, block_size=256,
        backend="hip",
    ).validate()
    k = torch.arange(2 * 4096, dtype=torch.float32).reshape(2, 4096, 1).expand(2, 4096, 256).contiguous()
    k_shards, _ = shard_history_bucket(k, k, cfg)
    assert len(k_shards) == 4 and k_shards[0].shape == (cfg.max_local_blocks, 2, 256, 256)
    for rank, shard in enumerate(k_shards):
        tokens = shard.transpose(0, 1).reshape(2, -1, 256)[0, :, 0]
        expected = torch.from_numpy(orc.global_positions(4096, rank, 4, 64)).float()
        assert torch.equal(tokens, expected)
