"""Page payload format (reference tests/test_kernel_pack.py:6-28, kernel.py:17-29)."""

import numpy as np
import pytest
import torch

from aws_training_study_amd.pcp_attention.kernel import pack_local_kv
from oracle import pcp_oracle as orc


def test_pack_local_kv_order():
    k = torch.arange(2 * 2 * 4 * 8).reshape(2, 2, 4, 8)
    v = -k
    packed = pack_local_kv(k, v)
    restored = packed.reshape(2, 2, 2, 4, 8)
    torch.testing.assert_close(restored[:, 0], k)
    torch.testing.assert_close(restored[:, 1], v)


def test_pack_local_kv_preserves_fp8_storage():
    k = torch.randn(1, 2, 4, 8, dtype=torch.bfloat16).to(torch.float8_e4m3fn)
    v = torch.randn(1, 2, 4, 8, dtype=torch.bfloat16).to(torch.float8_e4m3fn)
    packed = pack_local_kv(k, v)
    assert packed.dtype == torch.float8_e4m3fn
    assert packed.element_size() == 1
    restored = packed.reshape(1, 2, 2, 4, 8)
    torch.testing.assert_close(restored[:, 0].float(), k.float())
    torch.testing.assert_close(restored[:, 1].float(), v.float())


def test_pack_matches_oracle_bytes():
    g = torch.Generator().manual_seed(11)
    k = torch.randn(3, 2, 16, 32, generator=g).to(torch.float8_e4m3fn)
    v = torch.randn(3, 2, 16, 32, generator=g).to(torch.float8_e4m3fn)
    ours = pack_local_kv(k, v)
    assert ours.shape == (3, 2 * 2 * 16 * 32) and ours.is_contiguous()
    theirs = orc.pack_local_kv(k.view(torch.uint8).numpy(), v.view(torch.uint8).numpy())
    np.testing.assert_array_equal(ours.view(torch.uint8).numpy(), theirs)


def test_pack_rejects_mismatched_shapes():
    with pytest.raises(ValueError, match="equal"):
        pack_local_kv(torch.zeros(1, 2, 4, 8), torch.zeros(1, 2, 4, 4))
    with pytest.raises(ValueError, match="equal"):
        pack_local_kv(torch.zeros(2, 4, 8), torch.zeros(2, 4, 8))


def test_per_rank_local_caches_become_a_pool():
    """The NKI kernel's per-rank caches (run_poc.py:231-238: pack_local_kv of
    each rank's shard, zero-padded to max_local_blocks) become one pool in
    which rank r's block b is page r * max_local_blocks + b; the pool is built
    once per set of unchanged tensors."""
    import torch

    from aws_training_study_amd.pcp_attention import make_history_attention_kernel
    from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig
    from aws_training_study_amd.pcp_attention.layout import shard_history

    cfg = PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=4096, actual_history_len=2048,
                             block_size=256, interleave_size=64, num_q_heads=8, num_kv_heads=2, head_dim=64,
                             kv_dtype="bfloat16", backend="hip").validate()
    g = torch.Generator().manual_seed(5)
    k = torch.randn(2, cfg.actual_history_len, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(2, cfg.actual_history_len, 64, generator=g).to(torch.bfloat16)
    local = []
    for ks, vs in zip(*shard_history(k, v, cfg)):
        packed = pack_local_kv(ks, vs)
        padded = torch.zeros(cfg.max_local_blocks, packed.shape[1], dtype=packed.dtype)
        padded[: packed.shape[0]] = packed
        local.append(padded)
    kernel = make_history_attention_kernel(cfg)
    pool, table = kernel.pool_from_local_caches(local)
    assert pool.shape == (cfg.pcp_size * cfg.max_local_blocks, cfg.page_elements)
    for r in range(cfg.pcp_size):
        for b in range(cfg.max_local_blocks):
            assert int(table[r, b]) == r * cfg.max_local_blocks + b
            assert torch.equal(pool[int(table[r, b])], local[r][b])
    assert kernel.pool_from_local_caches(local)[0] is pool  # reused
    local[1][0, 0] = 7.0  # an in-place torch write: built again
    pool2, _ = kernel.pool_from_local_caches(local)
    assert pool2 is not pool and float(pool2[cfg.max_local_blocks, 0]) == 7.0
    with pytest.raises(ValueError, match="per-rank caches"):
        kernel.pool_from_local_caches(local[:-1])
    with pytest.raises(ValueError, match="rank 2's cache"):
        kernel.pool_from_local_caches(local[:2] + [local[2][:-1].contiguous()] + local[3:])
