"""Named workloads and the paged problem they expand to.

Each workload is a config plus input options.  ``PagedProblem`` carries
everything one kernel call needs (stacked Q, page pool, block table, per-page
valid lengths, scales) next to the global tensors it was built from.

Workloads (sizes are global; "ranks" are logical PCP ranks on one GPU):

``tiny-gqa4-d64-bf16``  4 ranks, 8 Q / 2 KV heads, D 64, 256 current and 2048
    history tokens, 128-token blocks, interleave 16, BF16 KV, K * 1/sqrt(D).
``four-chip-fp8``       16 ranks, 32 Q / 2 KV heads, D 256, 1024 current and
    8192 history tokens, 512-token blocks, interleave 64, FP8 KV with
    per-tensor scales (the reference's 4-chip shape, README.md:93-102).
``full-fp8``            64 ranks, 4096 current and 131072 history tokens,
    otherwise as ``four-chip-fp8`` (the reference's ``full`` preset,
    README.md:180-188).
``full-fp8-varlen``     ``full-fp8`` with the 131072-token bucket and a runtime
    history drawn in [65536, 131072) (generally not page aligned).
``gqa8-d128-bf16``      16 ranks, 64 Q / 8 KV heads, D 128, 2048 current and
    32768 history tokens, 256-token blocks, BF16 KV, K with a per-channel
    factor in [0.5, 2].
``full-bf16``           ``full-fp8`` with a BF16 cache (the reference's BF16-KV
    run of the full shape, README.md:191-199).
``four-chip-q4k-fp8``, ``four-chip-q8k-fp8``, ``four-chip-q16k-fp8``
    ``four-chip-fp8`` with 4096, 8192 and 16384 current tokens (the
    reference's Q sweep at an 8192-token history, README.md:156-165).
"""

from __future__ import annotations

from dataclasses import dataclass, replace

import torch

from .config import PCPAttentionConfig
from .inputs import HistoryInputs, make_local_inputs, make_scaled_inputs
from .layout import shard_history, shard_history_bucket, stacked_query
from .paging import make_block_table, pack_page_pool, page_valid_lengths


@dataclass(frozen=True)
class Workload:
    name: str
    config: PCPAttentionConfig
    kv_scale: str = "none"
    k_prescale: str = "none"
    random_history_len: bool = False

    def resolve(self, seed: int) -> PCPAttentionConfig:
        """The config with its runtime history length for ``seed``."""
        if not self.random_history_len:
            return self.config
        generator = torch.Generator().manual_seed(seed + 3)
        low = self.config.max_history_len // 2
        length = int(torch.randint(low, self.config.max_history_len, (1,), generator=generator))
        return replace(self.config, actual_history_len=length).validate()


def _hip(**kwargs) -> PCPAttentionConfig:
    return PCPAttentionConfig(backend="hip", **kwargs).validate()


WORKLOADS: dict[str, Workload] = {
    "tiny-gqa4-d64-bf16": Workload(
        "tiny-gqa4-d64-bf16",
        _hip(
            pcp_size=4, current_len=256, max_history_len=2048, actual_history_len=2048,
            block_size=128, interleave_size=16, num_q_heads=8, num_kv_heads=2, head_dim=64,
            alignment=256, kv_dtype="bfloat16",
        ),
        k_prescale="inv_sqrt_d",
    ),
    "four-chip-fp8": Workload(
        "four-chip-fp8",
        _hip(pcp_size=16, current_len=1024, max_history_len=8192, actual_history_len=8192),
        kv_scale="per_tensor",
    ),
    "full-fp8": Workload(
        "full-fp8",
        _hip(pcp_size=64, current_len=4096, max_history_len=131072, actual_history_len=131072),
        kv_scale="per_tensor",
    ),
    "full-fp8-varlen": Workload(
        "full-fp8-varlen",
        _hip(pcp_size=64, current_len=4096, max_history_len=131072, actual_history_len=131072),
        kv_scale="per_tensor",
        random_history_len=True,
    ),
    "full-bf16": Workload(
        "full-bf16",
        _hip(pcp_size=64, current_len=4096, max_history_len=131072, actual_history_len=131072,
             kv_dtype="bfloat16"),
    ),
    **{
        f"four-chip-q{q // 1024}k-fp8": Workload(
            f"four-chip-q{q // 1024}k-fp8",
            _hip(pcp_size=16, current_len=q, max_history_len=8192, actual_history_len=8192),
            kv_scale="per_tensor",
        )
        for q in (4096, 8192, 16384)
    },
    "gqa8-d128-bf16": Workload(
        "gqa8-d128-bf16",
        _hip(
            pcp_size=16, current_len=2048, max_history_len=32768, actual_history_len=32768,
            block_size=256, interleave_size=64, num_q_heads=64, num_kv_heads=8, head_dim=128,
            kv_dtype="bfloat16",
        ),
        k_prescale="per_channel",
    ),
}


def get_workload(name: str) -> Workload:
    try:
        return WORKLOADS[name]
    except KeyError as exc:
        raise ValueError(f"unknown workload {name!r}; choose one of: {', '.join(WORKLOADS)}") from exc


@dataclass
class PagedProblem:
    """One kernel call's inputs plus the global tensors they came from."""

    config: PCPAttentionConfig
    inputs: HistoryInputs
    q_stacked: torch.Tensor      # [pcp, Hq, local_q, D] bf16
    kv_pages: torch.Tensor       # [num_pages, page_elements]
    block_table: torch.Tensor    # [pcp, max_local_blocks] int32
    page_valid_len: torch.Tensor  # [pcp, max_local_blocks] int32

    @property
    def k_scale(self) -> float:
        return self.inputs.k_scale

    @property
    def v_scale(self) -> float:
        return self.inputs.v_scale

    def to(self, device) -> "PagedProblem":
        return PagedProblem(
            self.config,
            self.inputs,
            self.q_stacked.to(device),
            self.kv_pages.to(device),
            self.block_table.to(device),
            self.page_valid_len.to(device),
        )


def build_paged_problem(
    config: PCPAttentionConfig,
    seed: int,
    *,
    kv_scale: str = "none",
    k_prescale: str = "none",
    shuffle_pages: bool = True,
    v_factor: float = 1.0,
) -> PagedProblem:
    """Generate inputs, shard them by striped ownership and page them."""
    inputs = make_scaled_inputs(config, seed, kv_scale=kv_scale, k_prescale=k_prescale, v_factor=v_factor)
    if config.is_history_aligned:
        k_shards, v_shards = shard_history(inputs.k, inputs.v, config)
    else:
        k_shards, v_shards = shard_history_bucket(inputs.k, inputs.v, config)
    if shuffle_pages:
        table = make_block_table(config, seed + 1)
    else:
        table = torch.arange(config.num_pages, dtype=torch.int32).reshape(config.pcp_size, config.max_local_blocks)
    pool = pack_page_pool(k_shards, v_shards, config, table)
    return PagedProblem(config, inputs, stacked_query(inputs.q, config), pool, table, page_valid_lengths(config))


def build_workload_problem(workload: Workload | str, seed: int) -> PagedProblem:
    if isinstance(workload, str):
        workload = get_workload(workload)
    config = workload.resolve(seed)
    return build_paged_problem(config, seed, kv_scale=workload.kv_scale, k_prescale=workload.k_prescale)


def build_local_problem(config: PCPAttentionConfig, seed: int, *, shuffle_pages: bool = True) -> PagedProblem:
    """The memory-safe per-rank inputs of the reference's unchecked runs.

    Every rank draws only its own Q shard and local cache with seed
    ``seed + 104729 * rank`` (``make_local_inputs``, run_poc.py:107-134),
    the cache padded with zero blocks to ``max_local_blocks`` and valid up to
    ``actual_local_history_len`` per rank, as the reference's runner does
    (run_poc.py:221-237).  No global tensor exists: ``inputs`` carries only
    the (unit) scales, and the problem has no dense reference.
    """
    if not config.is_history_aligned:
        raise ValueError("per-rank local inputs need a history that is a multiple of pcp_size * interleave_size")
    q_shards, k_shards, v_shards = [], [], []
    for rank in range(config.pcp_size):
        q, k, v = make_local_inputs(config, seed, rank)
        q_shards.append(q)
        k_shards.append(k)
        v_shards.append(v)
    if shuffle_pages:
        table = make_block_table(config, seed + 1)
    else:
        table = torch.arange(config.num_pages, dtype=torch.int32).reshape(config.pcp_size, config.max_local_blocks)
    pool = pack_page_pool(k_shards, v_shards, config, table)
    inputs = HistoryInputs(config, None, None, None, 1.0, 1.0)
    return PagedProblem(config, inputs, torch.stack(q_shards), pool, table, page_valid_lengths(config))
