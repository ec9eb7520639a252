"""Paged KV pool for the collapsed (single-GPU) PCP history.

The Trainium2 proof of concept keeps one contiguous cache per rank,
``[blocks, Hkv, block_size, D]`` (layout.py:89-94), packs it per block with
``pack_local_kv`` (kernel.py:17-29) and rotates blocks around a device ring
(kernel.py:276-293).  On one GPU every rank's packed blocks live in one pool
``[num_pages, 2 * Hkv * block_size * D]`` and a block table maps
``(rank, local block)`` to a physical page.  A runtime history shorter than
the compiled bucket is described per page by the number of valid leading
tokens, which is the reference's additive bias (run_poc.py:137-153) in
compact form: a rank's valid tokens are always a prefix of its local
sequence, because its global positions increase with the local position.
"""

from __future__ import annotations

import torch

from .config import PCPAttentionConfig

# Additive bias the reference uses for a padded key (run_poc.py:143).
MASKED_SCORE_BIAS = -9984.0


def make_block_table(config: PCPAttentionConfig, seed: int) -> torch.Tensor:
    """Seeded random ``(rank, local block) -> page`` permutation, int32 ``[pcp, blocks]``."""
    generator = torch.Generator().manual_seed(seed)
    pages = torch.randperm(config.num_pages, generator=generator)
    return pages.to(torch.int32).reshape(config.pcp_size, config.max_local_blocks)


def identity_block_table(config: PCPAttentionConfig) -> torch.Tensor:
    """Rank-major contiguous pages: page ``rank * blocks + block``."""
    return torch.arange(config.num_pages, dtype=torch.int32).reshape(
        config.pcp_size, config.max_local_blocks
    )


def check_block_table(block_table: torch.Tensor, config: PCPAttentionConfig, num_pages: int) -> None:
    """Raise ``ValueError`` unless ``block_table`` maps every slot to a distinct page."""
    expected = (config.pcp_size, config.max_local_blocks)
    if tuple(block_table.shape) != expected:
        raise ValueError(f"expected block_table shape {expected}, got {tuple(block_table.shape)}")
    table = block_table.detach().to("cpu", torch.int64).reshape(-1)
    if table.numel() and (int(table.min()) < 0 or int(table.max()) >= num_pages):
        raise ValueError(f"block_table entries must lie in [0, {num_pages})")
    if torch.unique(table).numel() != table.numel():
        raise ValueError("block_table maps two cache blocks to the same page")


def page_valid_lengths(config: PCPAttentionConfig) -> torch.Tensor:
    """Valid leading tokens of every ``(rank, local block)``, int32 ``[pcp, blocks]``.

    Token ``p`` of the history is valid iff ``p < actual_history_len``.  For a
    history that is a multiple of ``pcp_size * interleave_size`` this equals
    the reference's mask (run_poc.py:137-153) on every rank.
    """
    lengths = torch.tensor(
        [config.local_history_len_for_rank(rank) for rank in range(config.pcp_size)],
        dtype=torch.int64,
    )
    starts = torch.arange(config.max_local_blocks, dtype=torch.int64) * config.block_size
    valid = (lengths[:, None] - starts[None, :]).clamp(0, config.block_size)
    return valid.to(torch.int32)


def valid_lengths_from_block_mask(mask: torch.Tensor, config: PCPAttentionConfig) -> torch.Tensor:
    """Convert the reference's additive bias mask to per-page valid lengths.

    ``mask`` is ``[max_local_blocks, block_size / 128, 1, 128]`` with 0 for a
    valid key and ``-9984`` for a padded one (run_poc.py:137-153); it applies
    to every rank.  Only prefix masks of those two values are representable,
    which is every mask the reference builds.

    A CPU mask is converted on the host and its values are checked
    (``ValueError`` otherwise).  A GPU mask is converted by a HIP kernel on
    the current stream, with no host synchronisation (so the call can be
    captured in a HIP graph): each block's length is the number of leading
    keys with a zero bias, and the values are not checked.
    """
    kv_tiles = config.block_size // 128
    expected = (config.max_local_blocks, kv_tiles, 1, 128)
    if config.block_size % 128 or tuple(mask.shape) != expected:
        raise ValueError(f"expected block_valid_mask shape {expected}, got {tuple(mask.shape)}")
    if mask.is_cuda:
        return _device_valid_lengths(mask, config)
    bias = mask.detach().to("cpu", torch.float32).reshape(config.max_local_blocks, config.block_size)
    valid = bias == 0
    if not bool(torch.all(valid | (bias <= MASKED_SCORE_BIAS))):
        raise ValueError("block_valid_mask values must be 0 (valid) or <= -9984 (masked)")
    counts = valid.sum(dim=1)
    prefix = torch.arange(config.block_size)[None, :] < counts[:, None]
    if not bool(torch.all(prefix == valid)):
        raise ValueError("block_valid_mask must mark a prefix of every cache block as valid")
    return counts.to(torch.int32)[None, :].expand(config.pcp_size, -1).contiguous()


def _device_valid_lengths(mask: torch.Tensor, config: PCPAttentionConfig) -> torch.Tensor:
    from .. import _native

    if mask.dtype != torch.bfloat16:
        raise ValueError(f"a GPU block_valid_mask must be bfloat16, got {mask.dtype}")
    mask = mask.contiguous()
    lengths = torch.empty((config.pcp_size, config.max_local_blocks), dtype=torch.int32, device=mask.device)
    lib = _native.load_library()
    with torch.cuda.device(mask.device):
        status = lib.pcpa_block_mask_valid_len(mask.data_ptr(), config.pcp_size, config.max_local_blocks,
                                               config.block_size, lengths.data_ptr(),
                                               torch.cuda.current_stream(mask.device).cuda_stream)
    _native.check(status)
    return lengths


def pack_page_pool(
    k_shards: list[torch.Tensor],
    v_shards: list[torch.Tensor],
    config: PCPAttentionConfig,
    block_table: torch.Tensor,
) -> torch.Tensor:
    """Scatter every rank's packed cache blocks into one page pool.

    ``k_shards[r]``/``v_shards[r]`` are ``[blocks_r, Hkv, block_size, D]``
    (``shard_history`` output) with ``blocks_r <= max_local_blocks``; blocks
    a rank does not hold become zero pages, as the reference pads its local
    cache to ``max_local_blocks`` (run_poc.py:232-237).
    """
    from .kernel import pack_local_kv

    if len(k_shards) != config.pcp_size or len(v_shards) != config.pcp_size:
        raise ValueError(f"expected {config.pcp_size} K and V shards")
    check_block_table(block_table, config, config.num_pages)
    dtype = k_shards[0].dtype
    pool = torch.zeros((config.num_pages, config.page_elements), dtype=dtype, device=k_shards[0].device)
    table = block_table.to("cpu", torch.int64)
    for rank in range(config.pcp_size):
        packed = pack_local_kv(k_shards[rank], v_shards[rank])
        blocks = packed.shape[0]
        if blocks > config.max_local_blocks:
            raise ValueError(f"rank {rank} holds {blocks} blocks > max_local_blocks")
        pool[table[rank, :blocks].to(pool.device)] = packed
    return pool
