"""Seeded synthetic inputs and the reference-form runtime mask.

``make_inputs``, ``make_local_inputs`` and ``make_block_valid_mask`` keep the
behaviour of run_poc.py:81-153: one CPU generator seeded with ``seed`` draws
Q, then K, then V as BF16 N(0, 1); K/V are stored in the config's
``kv_dtype`` (the reference always casts to FP8 e4m3 without a scale).

``make_scaled_inputs`` adds what the reference lacks, drawing the same Q, K,
V first so that reference-compatible tensors are unchanged: per-tensor FP8
scales (``amax / 448``), a K pre-scale (``1/sqrt(D)`` or a per-channel
factor in ``[0.5, 2]`` from a generator seeded ``seed + 2``), and histories
allocated at the ``max_history_len`` bucket when the runtime length is not a
multiple of the rank stride.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import sqrt

import torch

from .config import PCPAttentionConfig
from .paging import MASKED_SCORE_BIAS

FP8_E4M3_MAX = 448.0
KV_SCALE_MODES = ("none", "per_tensor")
K_PRESCALE_MODES = ("none", "inv_sqrt_d", "per_channel")


def _storage_dtype(config: PCPAttentionConfig) -> torch.dtype:
    return torch.float8_e4m3fn if config.kv_dtype == "fp8_e4m3fn" else torch.bfloat16


def generated_history_len(config: PCPAttentionConfig) -> int:
    """History tokens drawn: the runtime length, or the bucket if unaligned."""
    return config.actual_history_len if config.is_history_aligned else config.max_history_len


def make_inputs(cfg: PCPAttentionConfig, seed: int):
    """Global ``q [Hq, Q, D]`` BF16 and ``k``/``v`` ``[Hkv, L, D]`` in ``kv_dtype``."""
    generator = torch.Generator().manual_seed(seed)
    length = generated_history_len(cfg)
    q = torch.randn(cfg.num_q_heads, cfg.current_len, cfg.head_dim, generator=generator, dtype=torch.bfloat16)
    k = torch.randn(cfg.num_kv_heads, length, cfg.head_dim, generator=generator, dtype=torch.bfloat16)
    v = torch.randn(cfg.num_kv_heads, length, cfg.head_dim, generator=generator, dtype=torch.bfloat16)
    storage = _storage_dtype(cfg)
    return q, k.to(storage), v.to(storage)


def make_local_inputs(cfg: PCPAttentionConfig, seed: int, rank: int):
    """One rank's Q shard and ``[blocks, Hkv, block, D]`` K/V cache only.

    The per-rank seed is ``seed + 104729 * rank`` (run_poc.py:107-134).
    """
    generator = torch.Generator().manual_seed(seed + 104729 * rank)
    q = torch.randn(cfg.num_q_heads, cfg.local_q_len, cfg.head_dim, generator=generator, dtype=torch.bfloat16)
    cache_shape = (cfg.actual_local_blocks, cfg.num_kv_heads, cfg.block_size, cfg.head_dim)
    storage = _storage_dtype(cfg)
    k = torch.randn(*cache_shape, generator=generator, dtype=torch.bfloat16).to(storage)
    v = torch.randn(*cache_shape, generator=generator, dtype=torch.bfloat16).to(storage)
    return q, k, v


def make_block_valid_mask(cfg: PCPAttentionConfig) -> torch.Tensor:
    """Additive BF16 score bias ``[max_local_blocks, block/128, 1, 128]``.

    0 marks a valid key and -9984 a padded one; every rank holds
    ``actual_local_history_len`` valid tokens (run_poc.py:137-153).
    """
    if cfg.block_size % 128:
        raise ValueError("the block mask form needs block_size to be a multiple of 128")
    kv_tiles = cfg.block_size // 128
    key_index = torch.arange(cfg.max_local_blocks * cfg.block_size).reshape(cfg.max_local_blocks, kv_tiles, 1, 128)
    bias = torch.where(
        key_index < cfg.actual_local_history_len,
        torch.tensor(0.0),
        torch.tensor(MASKED_SCORE_BIAS),
    )
    return bias.to(torch.bfloat16)


@dataclass
class HistoryInputs:
    """Global inputs with per-tensor dequantisation scales.

    ``q`` is ``[Hq, current_len, D]`` BF16; ``k``/``v`` are ``[Hkv, L, D]`` in
    the storage dtype, ``L = generated_history_len(config)``.  The real
    values are ``k.float() * k_scale`` and ``v.float() * v_scale``.
    """

    config: PCPAttentionConfig
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    k_scale: float
    v_scale: float


def _quantize_per_tensor(x: torch.Tensor) -> tuple[torch.Tensor, float]:
    values = x.float()
    scale = per_tensor_scale(float(values.abs().max()))
    return (values / scale).to(torch.float8_e4m3fn), scale


def make_raw_inputs(cfg: PCPAttentionConfig, seed: int, *, k_prescale: str = "none", v_factor: float = 1.0):
    """BF16 ``q [Hq, Q, D]``, ``k``/``v`` ``[Hkv, L, D]`` before any FP8 quantisation.

    Same draws as ``make_scaled_inputs`` (and, without a pre-scale, as
    ``make_inputs``) up to the storage cast; this is what a KV-cache producer
    quantises.  ``v_factor`` multiplies V (V ~ N(0, v_factor^2)).
    """
    if k_prescale not in K_PRESCALE_MODES:
        raise ValueError(f"k_prescale must be one of {K_PRESCALE_MODES}, got {k_prescale!r}")
    generator = torch.Generator().manual_seed(seed)
    length = generated_history_len(cfg)
    q = torch.randn(cfg.num_q_heads, cfg.current_len, cfg.head_dim, generator=generator, dtype=torch.bfloat16)
    k = torch.randn(cfg.num_kv_heads, length, cfg.head_dim, generator=generator, dtype=torch.bfloat16)
    v = torch.randn(cfg.num_kv_heads, length, cfg.head_dim, generator=generator, dtype=torch.bfloat16)
    if k_prescale == "inv_sqrt_d":
        k = (k.float() * (1.0 / sqrt(cfg.head_dim))).to(torch.bfloat16)
    elif k_prescale == "per_channel":
        channel = torch.Generator().manual_seed(seed + 2)
        factor = torch.rand(cfg.num_kv_heads, 1, cfg.head_dim, generator=channel) * 1.5 + 0.5
        k = (k.float() * factor).to(torch.bfloat16)
    if v_factor != 1.0:
        v = (v.float() * v_factor).to(torch.bfloat16)
    return q, k, v


def per_tensor_scale(amax: float) -> float:
    """The per-tensor e4m3 scale for a tensor whose largest magnitude is ``amax``."""
    return amax / FP8_E4M3_MAX if amax > 0 else 1.0


def make_scaled_inputs(
    cfg: PCPAttentionConfig,
    seed: int,
    *,
    kv_scale: str = "none",
    k_prescale: str = "none",
    v_factor: float = 1.0,
) -> HistoryInputs:
    if kv_scale not in KV_SCALE_MODES:
        raise ValueError(f"kv_scale must be one of {KV_SCALE_MODES}, got {kv_scale!r}")
    q, k, v = make_raw_inputs(cfg, seed, k_prescale=k_prescale, v_factor=v_factor)
    k_scale = v_scale = 1.0
    if cfg.kv_dtype == "fp8_e4m3fn":
        if kv_scale == "per_tensor":
            k, k_scale = _quantize_per_tensor(k)
            v, v_scale = _quantize_per_tensor(v)
        else:
            k, v = k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn)
    elif kv_scale != "none":
        raise ValueError("per-tensor KV scales apply to FP8 storage only")
    return HistoryInputs(cfg, q, k, v, k_scale, v_scale)
