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
