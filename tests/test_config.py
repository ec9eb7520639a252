"""Config maths and validation (reference tests/test_config.py:6-44, config.py:29-107)."""

import pytest

from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig, get_preset
from oracle.pcp_oracle import OracleShape


def test_full_shape_math():
    cfg = get_preset("full")
    assert cfg.local_q_len == 64
    assert cfg.actual_local_history_len == 2048
    assert cfg.actual_local_blocks == 4
    assert cfg.softmax_scale == 1 / 16


def test_rejects_unequal_striped_shards():
    with pytest.raises(ValueError, match=r"pcp_size \* interleave_size"):
        get_preset("tiny").with_overrides(current_len=320)


def test_partial_last_local_cache_block():
    cfg = get_preset("tiny").with_overrides(max_history_len=2048, actual_history_len=1024)
    assert cfg.actual_local_history_len == 256
    assert cfg.actual_local_blocks == 1


def test_accepts_multiple_local_q_tiles():
    cfg = get_preset("full").with_overrides(
        pcp_size=16, current_len=4096, max_history_len=8192, actual_history_len=8192
    )
    assert cfg.local_q_len == 256


def test_rejects_partial_local_q_tile_above_128():
    with pytest.raises(ValueError, match="128-token NKI Q tile"):
        get_preset("full").with_overrides(pcp_size=16, current_len=3072)


@pytest.mark.parametrize(
    "overrides,message",
    [
        (dict(pcp_size=0), "pcp_size must be positive"),
        (dict(actual_history_len=4096), "must not exceed max_history_len"),
        (dict(num_q_heads=3, num_kv_heads=2), "divisible by num_kv_heads"),
        (dict(num_q_heads=6, num_kv_heads=3), "divide evenly across LNC cores"),
        (dict(head_dim=64), "TensorE K tile"),
        (dict(block_size=192, interleave_size=64), "KV tile"),
        (dict(block_size=512, interleave_size=384), "divisible by interleave_size"),
        (dict(actual_history_len=1024 + 256 * 0 + 128), "actual_history_len must be divisible"),
    ],
)
def test_reference_validation_messages(overrides, message):
    """Every rule of config.py:64-107 keeps its message under the default profile."""
    with pytest.raises(ValueError, match=message):
        get_preset("tiny").with_overrides(**overrides)


def test_hip_profile_drops_tensor_engine_rules():
    base = dict(pcp_size=4, current_len=256, max_history_len=2048, actual_history_len=2048, backend="hip")
    cfg = PCPAttentionConfig(head_dim=64, block_size=128, interleave_size=16, num_q_heads=8, **base).validate()
    assert cfg.local_q_len == 64
    # A 192-token local Q (rejected by the NKI tile rule) is fine for the HIP kernel.
    PCPAttentionConfig(**{**base, "pcp_size": 16, "current_len": 3072, "max_history_len": 8192, "actual_history_len": 8192}).validate()
    # Unaligned runtime history lengths are accepted (bucketed + masked).
    cfg = PCPAttentionConfig(**{**base, "actual_history_len": 1000}).validate()
    assert not cfg.is_history_aligned
    with pytest.raises(ValueError, match="head_dim must be one of"):
        PCPAttentionConfig(head_dim=96, **base).validate()
    with pytest.raises(ValueError, match="64-token HIP key tile"):
        PCPAttentionConfig(block_size=96, interleave_size=32, **base).validate()
    with pytest.raises(ValueError, match=r"current_len must be divisible"):
        PCPAttentionConfig(**{**base, "current_len": 320}).validate()
    with pytest.raises(ValueError, match="backend must be one of"):
        PCPAttentionConfig(**{**base, "backend": "cuda"}).validate()
    with pytest.raises(ValueError, match="kv_dtype must be one of"):
        PCPAttentionConfig(kv_dtype="fp16", **base).validate()


def test_unknown_preset():
    with pytest.raises(ValueError, match="unknown preset 'huge'; choose one of: full, tiny"):
        get_preset("huge")


@pytest.mark.parametrize("actual", [1, 63, 64, 65, 1000, 2047, 2048, 4095, 4096])
@pytest.mark.parametrize("pcp,il", [(4, 64), (3, 16), (8, 8)])
def test_rank_history_len_matches_brute_force(actual, pcp, il):
    """Per-rank valid counts equal a count of owner_and_local_position over p < actual."""
    from oracle.pcp_oracle import owner_and_local_position

    max_len = pcp * il * ((4096 + pcp * il - 1) // (pcp * il))
    cfg = PCPAttentionConfig(
        pcp_size=pcp, current_len=pcp * il, max_history_len=max_len, actual_history_len=actual,
        block_size=64 * il, interleave_size=il, backend="hip", head_dim=64,
    ).validate()
    counts = [0] * pcp
    for p in range(actual):
        counts[owner_and_local_position(p, pcp, il)[0]] += 1
    assert [cfg.local_history_len_for_rank(r) for r in range(pcp)] == counts


@pytest.mark.parametrize("name", ["tiny", "full"])
def test_derived_shapes_match_oracle(name):
    cfg = get_preset(name)
    shape = OracleShape.from_config(cfg)
    assert cfg.softmax_scale == shape.softmax_scale
    assert cfg.q_heads_per_kv_head == shape.group
    assert cfg.local_q_len == shape.local_q_len
    assert cfg.max_local_history_len == shape.max_local_history_len
    assert cfg.actual_local_history_len == shape.actual_local_history_len
    assert cfg.max_local_blocks == shape.max_local_blocks
    assert cfg.actual_local_blocks == shape.actual_local_blocks
    assert cfg.rank_stride == cfg.pcp_size * cfg.interleave_size
