"""Static and runtime configuration for history-only PCP attention.

Mirrors ``pcp_attention/config.py`` of the Trainium2 proof of concept
(config.py:9-139): the same frozen dataclass fields, derived properties,
``with_overrides``/``validate``/``get_preset`` and the same ``ValueError``
messages.  Two fields are added, both with defaults that keep the original
behaviour:

``backend``
    Selects the validation profile.  ``"neuron"`` applies every rule of the
    original ``validate()`` (config.py:64-107), including the NKI/TensorE tile
    rules.  ``"hip"`` applies the generic rules plus the limits of the MI355X
    HIP kernel; it drops the TensorE tile rules (``head_dim % 128``,
    ``block_size % 128``, the LNC head split, the 128-token Q tile) and accepts
    an ``actual_history_len`` that is not a multiple of
    ``pcp_size * interleave_size`` (the history is then sharded at the
    ``max_history_len`` bucket and masked per token).
``kv_dtype``
    Storage type of the paged K/V cache: ``"fp8_e4m3fn"`` (the original's only
    type, run_poc.py:96,103) or ``"bfloat16"``.
"""

from __future__ import annotations

from dataclasses import dataclass, replace
from math import ceil, sqrt

BACKENDS = ("neuron", "hip")
KV_DTYPES = ("fp8_e4m3fn", "bfloat16")

# Shapes the gfx950 kernel is specialised for.
HIP_HEAD_DIMS = (64, 128, 256)
# Keys are consumed in 64-token tiles; a cache block holds whole tiles.
HIP_BLOCK_MULTIPLE = 64


@dataclass(frozen=True)
class PCPAttentionConfig:
    """Configuration shared by layout, kernel entry, runner and bench.

    ``actual_history_len`` is the runtime history length; every other field
    is static for a compiled/launched kernel shape.
    """

    pcp_size: int
    current_len: int
    max_history_len: int
    actual_history_len: int
    block_size: int = 512
    interleave_size: int = 64
    num_q_heads: int = 32
    num_kv_heads: int = 2
    head_dim: int = 256
    lnc: int = 2
    alignment: int = 4096
    backend: str = "neuron"
    kv_dtype: str = "fp8_e4m3fn"

    # ---- derived shapes (config.py:29-59) ---------------------------------
    @property
    def softmax_scale(self) -> float:
        return 1.0 / sqrt(self.head_dim)

    @property
    def q_heads_per_kv_head(self) -> int:
        return self.num_q_heads // self.num_kv_heads

    @property
    def local_q_len(self) -> int:
        return self.current_len // self.pcp_size

    @property
    def max_local_history_len(self) -> int:
        return self.max_history_len // self.pcp_size

    @property
    def actual_local_history_len(self) -> int:
        """Valid history tokens held by rank 0, the rank holding the most.

        For a history length that is a multiple of ``pcp_size *
        interleave_size`` every rank holds ``actual_history_len / pcp_size``
        tokens, which is the original definition (config.py:45-47).
        """
        return self.local_history_len_for_rank(0)

    @property
    def max_local_blocks(self) -> int:
        return ceil(self.max_local_history_len / self.block_size)

    @property
    def actual_local_blocks(self) -> int:
        return ceil(self.actual_local_history_len / self.block_size)

    @property
    def rank_stride(self) -> int:
        return self.pcp_size * self.interleave_size

    @property
    def is_history_aligned(self) -> bool:
        return self.actual_history_len % self.rank_stride == 0

    @property
    def kv_element_size(self) -> int:
        return 1 if self.kv_dtype == "fp8_e4m3fn" else 2

    @property
    def num_pages(self) -> int:
        """Pages in the collapsed pool: every rank's ``max_local_blocks``."""
        return self.pcp_size * self.max_local_blocks

    @property
    def page_elements(self) -> int:
        """Elements of one packed page row (kernel.py:17-29 payload)."""
        return 2 * self.num_kv_heads * self.block_size * self.head_dim

    def local_history_len_for_rank(self, rank: int) -> int:
        """Number of history positions ``p < actual_history_len`` owned by ``rank``.

        Ownership is striped in ``interleave_size`` chunks (layout.py:10-16):
        each full round of ``pcp_size`` chunks gives every rank
        ``interleave_size`` tokens, and the tail of ``rem`` tokens is dealt to
        ranks in order, ``interleave_size`` at a time.
        """
        if not 0 <= rank < self.pcp_size:
            raise ValueError(f"rank {rank} is outside [0, {self.pcp_size})")
        rounds, rem = divmod(self.actual_history_len, self.rank_stride)
        tail = min(max(rem - rank * self.interleave_size, 0), self.interleave_size)
        return rounds * self.interleave_size + tail

    def with_overrides(self, **kwargs) -> "PCPAttentionConfig":
        return replace(self, **kwargs).validate()

    # ---- validation (config.py:64-107) ------------------------------------
    def validate(self) -> "PCPAttentionConfig":
        if self.backend not in BACKENDS:
            raise ValueError(f"backend must be one of {BACKENDS}, got {self.backend!r}")
        if self.kv_dtype not in KV_DTYPES:
            raise ValueError(f"kv_dtype must be one of {KV_DTYPES}, got {self.kv_dtype!r}")
        positive = {
            "pcp_size": self.pcp_size,
            "current_len": self.current_len,
            "max_history_len": self.max_history_len,
            "actual_history_len": self.actual_history_len,
            "block_size": self.block_size,
            "interleave_size": self.interleave_size,
            "num_q_heads": self.num_q_heads,
            "num_kv_heads": self.num_kv_heads,
            "head_dim": self.head_dim,
            "lnc": self.lnc,
        }
        for name, value in positive.items():
            if value <= 0:
                raise ValueError(f"{name} must be positive, got {value}")
        if self.actual_history_len > self.max_history_len:
            raise ValueError("actual_history_len must not exceed max_history_len")
        if self.num_q_heads % self.num_kv_heads:
            raise ValueError("num_q_heads must be divisible by num_kv_heads")
        if self.backend == "neuron":
            self._validate_neuron_tiles()
        else:
            self._validate_hip_kernel()
        if self.block_size % self.interleave_size:
            raise ValueError("block_size must be divisible by interleave_size")
        striped = [("current_len", self.current_len), ("max_history_len", self.max_history_len)]
        if self.backend == "neuron":
            striped.append(("actual_history_len", self.actual_history_len))
        for name, value in striped:
            if value % self.rank_stride:
                raise ValueError(
                    f"{name} must be divisible by pcp_size * interleave_size "
                    f"({self.rank_stride}), got {value}"
                )
        if self.backend == "neuron" and self.local_q_len > 128 and self.local_q_len % 128:
            raise ValueError(
                "local_q_len values above 128 must be divisible by the "
                "128-token NKI Q tile"
            )
        return self

    def _validate_neuron_tiles(self) -> None:
        if self.num_q_heads % self.lnc or self.num_kv_heads % self.lnc:
            raise ValueError("Q and KV heads must divide evenly across LNC cores")
        if self.head_dim % 128:
            raise ValueError("head_dim must be a multiple of the TensorE K tile (128)")
        if self.block_size % 128:
            raise ValueError("block_size must be a multiple of the KV tile (128)")

    def _validate_hip_kernel(self) -> None:
        if self.head_dim not in HIP_HEAD_DIMS:
            raise ValueError(
                f"head_dim must be one of {HIP_HEAD_DIMS} for the HIP kernel, got {self.head_dim}"
            )
        if self.block_size % HIP_BLOCK_MULTIPLE:
            raise ValueError(
                f"block_size must be a multiple of the {HIP_BLOCK_MULTIPLE}-token HIP key tile, "
                f"got {self.block_size}"
            )


_PRESETS = {
    # One local KV block per rank with the Qwen head dimensions (config.py:112-120).
    "tiny": PCPAttentionConfig(
        pcp_size=4,
        current_len=256,
        max_history_len=2048,
        actual_history_len=2048,
        block_size=512,
        interleave_size=64,
        alignment=256,
    ),
    # The 64-rank full-machine layout (config.py:122-130).
    "full": PCPAttentionConfig(
        pcp_size=64,
        current_len=4096,
        max_history_len=131072,
        actual_history_len=131072,
        block_size=512,
        interleave_size=64,
        alignment=4096,
    ),
}


def get_preset(name: str) -> PCPAttentionConfig:
    try:
        return _PRESETS[name].validate()
    except KeyError as exc:
        choices = ", ".join(sorted(_PRESETS))
        raise ValueError(f"unknown preset {name!r}; choose one of: {choices}") from exc
