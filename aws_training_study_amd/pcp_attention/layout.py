"""Striped token ownership and host-side shard/gather helpers.

Same functions, argument meaning and errors as ``pcp_attention/layout.py`` of
the Trainium2 proof of concept (layout.py:10-132).  Ownership follows the
closed form of README.md:22-29: global position ``p`` lies in chunk
``p // interleave_size``; chunks are dealt round-robin to ranks, so the owner
is ``chunk % pcp_size`` and the local position is
``(chunk // pcp_size) * interleave_size + p % interleave_size``.

Added for the collapsed single-GPU path: ``stacked_query`` (all ranks' Q
shards as one ``[pcp, Hq, local_q, D]`` tensor) and ``shard_history_bucket``
(sharding at ``max_history_len`` for histories that are not a multiple of the
rank stride).
"""

from __future__ import annotations

from dataclasses import replace

import torch

from .config import PCPAttentionConfig


def _storage_view(tensor: torch.Tensor) -> torch.Tensor:
    """Byte view of 1-byte float tensors, whose dtype lacks CPU index kernels."""
    if tensor.element_size() == 1 and tensor.dtype.is_floating_point:
        return tensor.view(torch.uint8)
    return tensor


def owner_and_local_position(
    global_position: int, pcp_size: int, interleave_size: int
) -> tuple[int, int]:
    """Return ``(owner_rank, local_position)`` of one global token position."""
    chunk = global_position // interleave_size
    round_index = chunk // pcp_size
    return chunk - round_index * pcp_size, round_index * interleave_size + (
        global_position - chunk * interleave_size
    )


def global_positions_for_rank(
    total_len: int, rank: int, pcp_size: int, interleave_size: int
) -> torch.Tensor:
    """Global positions of ``rank``'s local tokens, in local order (int64)."""
    if not 0 <= rank < pcp_size:
        raise ValueError(f"rank {rank} is outside [0, {pcp_size})")
    if total_len % (pcp_size * interleave_size):
        raise ValueError("total_len must divide evenly across striped ranks")
    local = torch.arange(total_len // pcp_size, dtype=torch.int64)
    chunk_round = torch.div(local, interleave_size, rounding_mode="floor")
    within = local - chunk_round * interleave_size
    return (chunk_round * pcp_size + rank) * interleave_size + within


def _position_table(total_len: int, pcp_size: int, interleave_size: int) -> torch.Tensor:
    """``[pcp, total_len / pcp]`` table of every rank's global positions."""
    return torch.stack(
        [
            global_positions_for_rank(total_len, rank, pcp_size, interleave_size)
            for rank in range(pcp_size)
        ]
    )


def shard_query(q: torch.Tensor, config: PCPAttentionConfig) -> list[torch.Tensor]:
    """Shard global ``[Hq, current_len, D]`` Q by striped ownership.

    The current tokens start at global position ``actual_history_len``; the
    history is a whole number of rank strides in the original layout, so the
    current segment is dealt to ranks from rank 0 (layout.py:34-51).
    """
    config.validate()
    expected = (config.num_q_heads, config.current_len, config.head_dim)
    if tuple(q.shape) != expected:
        raise ValueError(f"expected Q shape {expected}, got {tuple(q.shape)}")
    table = _position_table(config.current_len, config.pcp_size, config.interleave_size)
    return [q.index_select(1, table[rank].to(q.device)) for rank in range(config.pcp_size)]


def stacked_query(q: torch.Tensor, config: PCPAttentionConfig) -> torch.Tensor:
    """All ranks' Q shards as one contiguous ``[pcp, Hq, local_q, D]`` tensor.

    Equal to ``torch.stack(shard_query(q, config))``, built with one gather.
    """
    config.validate()
    expected = (config.num_q_heads, config.current_len, config.head_dim)
    if tuple(q.shape) != expected:
        raise ValueError(f"expected Q shape {expected}, got {tuple(q.shape)}")
    table = _position_table(config.current_len, config.pcp_size, config.interleave_size)
    gathered = q.index_select(1, table.reshape(-1).to(q.device))
    return (
        gathered.reshape(config.num_q_heads, config.pcp_size, config.local_q_len, config.head_dim)
        .permute(1, 0, 2, 3)
        .contiguous()
    )


def _to_cache_blocks(
    tensor: torch.Tensor, positions: torch.Tensor, config: PCPAttentionConfig
) -> torch.Tensor:
    """Gather one rank's tokens into zero-padded ``[blocks, Hkv, block, D]``."""
    blocks = config.actual_local_blocks
    cache = torch.zeros(
        (config.num_kv_heads, blocks * config.block_size, config.head_dim),
        dtype=tensor.dtype,
        device=tensor.device,
    )
    cache[:, : positions.numel(), :] = tensor.index_select(1, positions.to(tensor.device))
    return (
        cache.reshape(config.num_kv_heads, blocks, config.block_size, config.head_dim)
        .transpose(0, 1)
        .contiguous()
    )


def shard_history(
    k: torch.Tensor, v: torch.Tensor, config: PCPAttentionConfig
) -> tuple[list[torch.Tensor], list[torch.Tensor]]:
    """Shard global ``[Hkv, actual_history_len, D]`` K/V into per-rank caches.

    Each rank's shard is ``[actual_local_blocks, Hkv, block_size, D]``; the
    tail of its last block is zero padding (layout.py:54-98).
    """
    config.validate()
    expected = (config.num_kv_heads, config.actual_history_len, config.head_dim)
    if tuple(k.shape) != expected or tuple(v.shape) != expected:
        raise ValueError(
            f"expected K/V shape {expected}, got {tuple(k.shape)} and {tuple(v.shape)}"
        )
    k_shards: list[torch.Tensor] = []
    v_shards: list[torch.Tensor] = []
    for rank in range(config.pcp_size):
        positions = global_positions_for_rank(
            config.actual_history_len, rank, config.pcp_size, config.interleave_size
        )
        k_shards.append(_to_cache_blocks(k, positions, config))
        v_shards.append(_to_cache_blocks(v, positions, config))
    return k_shards, v_shards


def shard_history_bucket(
    k: torch.Tensor, v: torch.Tensor, config: PCPAttentionConfig
) -> tuple[list[torch.Tensor], list[torch.Tensor]]:
    """Shard a history allocated at the ``max_history_len`` bucket.

    ``k``/``v`` are ``[Hkv, max_history_len, D]``; positions at or beyond
    ``actual_history_len`` are cache slots that the runtime mask hides.  Every
    rank receives ``max_local_blocks`` blocks.
    """
    bucket = replace(config, actual_history_len=config.max_history_len)
    return shard_history(k, v, bucket)


def gather_history(shards: list[torch.Tensor], config: PCPAttentionConfig) -> torch.Tensor:
    """Invert ``shard_history`` for one of K or V (layout.py:101-132)."""
    config.validate()
    if len(shards) != config.pcp_size:
        raise ValueError(f"expected {config.pcp_size} shards, got {len(shards)}")
    expected = (
        config.actual_local_blocks,
        config.num_kv_heads,
        config.block_size,
        config.head_dim,
    )
    sample = shards[0]
    result = torch.empty(
        (config.num_kv_heads, config.actual_history_len, config.head_dim),
        dtype=sample.dtype,
        device=sample.device,
    )
    for rank, shard in enumerate(shards):
        if tuple(shard.shape) != expected:
            raise ValueError(f"rank {rank}: expected {expected}, got {tuple(shard.shape)}")
        positions = global_positions_for_rank(
            config.actual_history_len, rank, config.pcp_size, config.interleave_size
        ).to(shard.device)
        tokens = shard.transpose(0, 1).reshape(config.num_kv_heads, -1, config.head_dim)
        _storage_view(result).index_copy_(
            1, positions, _storage_view(tokens[:, : positions.numel(), :])
        )
    return result
