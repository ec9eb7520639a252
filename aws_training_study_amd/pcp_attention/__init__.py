"""History-only PCP attention: config, striped layout and the gfx950 kernel entry.

Same exported names as ``pcp_attention/__init__.py`` of the Trainium2 proof
of concept (``__init__.py:3-15``) minus the CPU executable specification,
which in this repository is test infrastructure (``oracle/``), plus the
kernel entry points, the paged-pool helpers, the KV-cache producer and the
current-token step.
"""

from .cache import KVCacheWriter, PageAllocator, absmax, append_history, build_page_pool
from .config import PCPAttentionConfig, get_preset
from .current import CurrentAttentionKernel, PrefillAttention, stack_current_kv
from .kernel import make_history_attention_kernel, pack_local_kv, wrap_for_native_torch
from .launch import GraphedLaunch
from .layout import (
    gather_history,
    global_positions_for_rank,
    owner_and_local_position,
    shard_history,
    shard_history_bucket,
    shard_query,
    stacked_query,
)
from .paging import make_block_table, pack_page_pool, page_valid_lengths, valid_lengths_from_block_mask

__all__ = [
    "CurrentAttentionKernel",
    "GraphedLaunch",
    "KVCacheWriter",
    "PCPAttentionConfig",
    "PageAllocator",
    "absmax",
    "append_history",
    "build_page_pool",
    "gather_history",
    "get_preset",
    "global_positions_for_rank",
    "make_block_table",
    "make_history_attention_kernel",
    "owner_and_local_position",
    "pack_local_kv",
    "pack_page_pool",
    "page_valid_lengths",
    "PrefillAttention",
    "shard_history",
    "shard_history_bucket",
    "shard_query",
    "stack_current_kv",
    "stacked_query",
    "valid_lengths_from_block_mask",
    "wrap_for_native_torch",
]
