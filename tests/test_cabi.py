"""C ABI of libpcp_attention_hip.so without a GPU: the library loads, exports every
symbol include/pcp_attention_hip.h declares, and rejects bad parameters before
any HIP call."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from aws_training_study_amd import _native
from aws_training_study_amd.pcp_attention import make_history_attention_kernel
from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig

HEADER = Path(__file__).resolve().parents[1] / "include" / "pcp_attention_hip.h"


@pytest.fixture(scope="module")
def lib():
    if not _native.library_path().exists():
        pytest.fail("libpcp_attention_hip.so is not built; run __graft_entry__.build()")
    return _native.load_library()


def _declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int32_t|int64_t|const char\*)\s+(pcpa_\w+)\s*\(", text, re.M)))


def test_header_declares_what_python_binds():
    assert _declared_functions() == sorted(_native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name


def test_status_codes_match_header(lib):
    text = HEADER.read_text()
    codes = {name: int(value) for name, value in re.findall(r"#define (PCPA_(?:OK|ERR_\w+))\s+\(?(-?\d+)\)?", text)}
    assert codes["PCPA_OK"] == 0
    for name, value in codes.items():
        assert _native.STATUS_NAMES[value] == name
        assert lib.pcpa_status_string(value).decode() != "unknown status"
    assert lib.pcpa_abi_version() == _native.ABI_VERSION
    assert f"#define PCPA_ABI_VERSION {_native.ABI_VERSION}" in text


def test_params_struct_layout():
    text = HEADER.read_text()
    body = re.search(r"typedef struct pcpa_params \{(.*?)\} pcpa_params;", text, re.S).group(1)
    fields = re.findall(r"(?:int32_t|uint32_t|float)\s+(\w+);", body)
    assert fields == [name for name, _ in _native.PcpaParams._fields_]
    assert ctypes.sizeof(_native.PcpaParams) == 4 * len(fields)


def _good_params(**kw):
    p = dict(abi_version=_native.ABI_VERSION, pcp_size=4, num_q_heads=8, num_kv_heads=2, head_dim=64, local_q_len=64,
             block_size=128, max_local_blocks=4, num_pages=16, q_dtype=1, kv_dtype=1, out_dtype=1,
             softmax_scale=0.125, k_scale=1.0, v_scale=1.0, flags=0)
    p.update(kw)
    return _native.PcpaParams(**p)


@pytest.mark.parametrize(
    "change,status",
    [
        ({}, 0),
        ({"abi_version": _native.ABI_VERSION - 1}, -2),
        ({"pcp_size": 0}, -3),
        ({"num_q_heads": 7}, -3),
        ({"flags": 1}, 0),
        ({"flags": 2}, 0),
        ({"flags": 3}, 0),
        ({"flags": 4}, 0),
        ({"flags": 8}, 0),
        ({"flags": 15}, 0),
        ({"flags": 16}, 0),
        ({"flags": 27}, 0),
        ({"flags": 20}, -3),   # the guard asked for and refused at once
        ({"flags": 32}, -3),
        ({"q_dtype": 2}, -4),
        ({"kv_dtype": 9}, -4),
        ({"head_dim": 96}, -5),
        ({"block_size": 96}, -5),
        ({"softmax_scale": 0.0}, -9),
        ({"v_scale": float("nan")}, -9),
        ({"pcp_size": 1 << 20, "local_q_len": 1 << 12}, -8),
    ],
)
def test_check_params(lib, change, status):
    assert lib.pcpa_check_params(ctypes.byref(_good_params(**change))) == status


def test_launch_rejects_null_and_misaligned_pointers_without_a_gpu(lib):
    p = _good_params()
    assert lib.pcpa_history_attention(None, 16, 16, 16, 16, 16, None) == -1
    assert lib.pcpa_history_attention(ctypes.byref(p), None, 16, 16, 16, 16, None) == -1
    assert lib.pcpa_history_attention(ctypes.byref(p), 16, 16, 16, 16, 0, None) == -1
    assert lib.pcpa_history_attention(ctypes.byref(p), 8, 16, 16, 16, 16, None) == -6
    assert lib.pcpa_history_attention(ctypes.byref(p), 16, 16, 2, 16, 16, None) == -6
    bad = _good_params(head_dim=96)
    assert lib.pcpa_history_attention(ctypes.byref(bad), 16, 16, 16, 16, 16, None) == -5


def test_python_entry_validates_before_launch():
    with pytest.raises(ValueError, match="head_dim must be one of"):
        make_history_attention_kernel(PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=2048,
                                                         actual_history_len=2048, head_dim=384))
    kernel = make_history_attention_kernel(PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=2048,
                                                              actual_history_len=2048, backend="hip"))
    q = torch.zeros(4, 32, 64, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        kernel(q, torch.zeros(4, 10), torch.zeros(4, 1, dtype=torch.int32))


def test_split_workspace_size_from_python():
    cfg = PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=2048, actual_history_len=2048,
                             backend="hip")
    kernel = make_history_attention_kernel(cfg)
    rows = cfg.pcp_size * cfg.num_q_heads * cfg.local_q_len
    # e4m3 MFMAs at head_dim 256: fp16 partial output, fp32 log-sum-exp and
    # reference max per row and split
    assert kernel.split_workspace_bytes(3) == 3 * rows * (cfg.head_dim * 2 + 8)
    bf16 = make_history_attention_kernel(PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=2048,
                                                            actual_history_len=2048, backend="hip",
                                                            kv_dtype="bfloat16"))
    assert bf16.split_workspace_bytes(3) == 3 * rows * (cfg.head_dim + 2) * 4
    assert kernel.workspace_bytes(1, precision="fp8") == 0
    # the precision guard needs its thresholds, plan (row counts and a list
    # slot per row) and fixup partials even for one pass, and the same
    # beside a split call's partials
    guard = kernel.workspace_bytes(1, precision="auto")
    assert guard >= 4 * (4 + rows) + cfg.num_kv_heads * cfg.head_dim // 16 * 4
    assert kernel.workspace_bytes(3, precision="auto") == kernel.split_workspace_bytes(3) + guard
    with pytest.raises(_native.PcpaError, match="BAD_SHAPE"):
        kernel.split_workspace_bytes(_native.MAX_SPLITS + 1)


def test_cache_write_validates_without_a_gpu(lib):
    """pcpa_kv_cache_write / pcpa_absmax_bf16 argument errors come back before any HIP call."""
    p = _good_params()  # pcp 4, Hkv 2, D 64, block 128, 4 local blocks: 512 local slots per rank
    w = lib.pcpa_kv_cache_write
    assert w(None, 16, 0, 8, 16, 16, 16, 16, None, None) == -1
    assert w(ctypes.byref(p), 16, 0, 8, None, 16, 16, 16, None, None) == -1
    assert w(ctypes.byref(p), 16, 0, 8, 16, 16, None, 16, None, None) == -1
    assert w(ctypes.byref(p), 0, 0, 8, 16, 16, 16, 16, None, None) == -3      # interleave
    assert w(ctypes.byref(p), 16, -1, 8, 16, 16, 16, 16, None, None) == -3    # first_pos
    assert w(ctypes.byref(p), 16, 0, -1, 16, 16, 16, 16, None, None) == -3    # num_tokens
    assert w(ctypes.byref(p), 16, 0, 8, 8, 16, 16, 16, None, None) == -6      # k alignment
    assert w(ctypes.byref(p), 16, 0, 8, 16, 16, 2, 16, None, None) == -6      # table alignment
    assert w(ctypes.byref(p), 16, 0, 0, 16, 16, 16, 16, None, None) == 0      # nothing to write
    # capacity: 4 ranks x 512 slots = global positions [0, 2048)
    assert w(ctypes.byref(p), 16, 2040, 9, 16, 16, 16, 16, None, None) == -3
    assert w(ctypes.byref(_good_params(head_dim=96)), 16, 0, 8, 16, 16, 16, 16, None, None) == -5
    assert lib.pcpa_absmax_bf16(None, 8, 16, None) == -1
    assert lib.pcpa_absmax_bf16(16, -1, 16, None) == -3
    assert lib.pcpa_absmax_bf16(8, 8, 16, None) == -6


def test_lse_and_current_entries_validate_without_a_gpu(lib):
    """pcpa_history_attention_lse / pcpa_current_attention argument errors come back before any HIP call."""
    p = _good_params()  # pcp 4 x local_q 64 = 256 current tokens
    h = lib.pcpa_history_attention_lse
    assert h(None, 16, 16, 16, 16, 16, None, None) == -1
    assert h(ctypes.byref(p), 16, 16, 16, 16, 16, 2, None) == -6       # lse alignment
    assert h(ctypes.byref(_good_params(head_dim=96)), 16, 16, 16, 16, 16, None, None) == -5
    c = lib.pcpa_current_attention
    assert c(None, 16, 16, 16, None, None, 16, None, None) == -1
    assert c(ctypes.byref(p), 16, None, 16, None, None, 16, None, None) == -1   # q
    assert c(ctypes.byref(p), 16, 16, None, None, None, 16, None, None) == -1   # kv_current
    assert c(ctypes.byref(p), 16, 16, 16, 16, None, 16, None, None) == -1       # hist_out without hist_lse
    assert c(ctypes.byref(p), 16, 16, 16, None, 16, 16, None, None) == -1       # hist_lse without hist_out
    assert c(ctypes.byref(_good_params(kv_dtype=2)), 16, 16, 16, None, None, 16, None, None) == -4
    assert c(ctypes.byref(p), 0, 16, 16, None, None, 16, None, None) == -3      # interleave
    assert c(ctypes.byref(p), 48, 16, 16, None, None, 16, None, None) == -3     # local_q % interleave
    assert c(ctypes.byref(_good_params(local_q_len=8)), 8, 16, 16, None, None, 16, None, None) == -5  # 32 tokens
    assert c(ctypes.byref(p), 16, 8, 16, None, None, 16, None, None) == -6      # q alignment
    assert c(ctypes.byref(p), 16, 16, 16, 16, 2, 16, None, None) == -6          # hist_lse alignment
    assert c(ctypes.byref(p), 16, 16, 16, None, None, 16, 2, None) == -6        # lse alignment


@pytest.mark.parametrize("workload,bf16_mfma,expected", [
    ("four-chip-fp8", False, 2),        # 128 overlap workgroups of 256 rows for 256 CUs
    ("full-fp8", False, 1),             # 512 already fill the GPU
    ("four-chip-fp8", True, 1),         # BF16 MFMAs at head_dim 256: 256 tile workgroups, one per CU
    ("tiny-gqa4-d64-bf16", True, 8),    # 16 tile workgroups; 32 tiles, at least 4 per split
    ("gqa8-d128-bf16", True, 1),        # 1024 tile workgroups
])
def test_auto_split_counts(workload, bf16_mfma, expected):
    from aws_training_study_amd.pcp_attention.workloads import get_workload

    kernel = make_history_attention_kernel(get_workload(workload).resolve(1234).with_overrides(backend="hip"))
    assert kernel.auto_splits(bf16_mfma, cus=256) == expected
    # never more splits than table entries, and none for a history of a few tiles
    short = make_history_attention_kernel(PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=2048,
                                                             actual_history_len=200, backend="hip"))
    assert short.auto_splits(True, cus=256) == 1


def test_split_entry_validates_without_a_gpu(lib):
    """pcpa_split_workspace_bytes / pcpa_history_attention_split errors come back before any HIP call."""
    # unguarded e4m3 MFMAs, 4 ranks x 8 heads x 64 tokens = 2048 rows: fp16
    # partials of O / l, fp32 log-sum-exp and reference max per row and split
    p = _good_params(kv_dtype=2, head_dim=256, flags=16)
    size = lib.pcpa_split_workspace_bytes(ctypes.byref(p), 3)
    assert size == 3 * 2048 * (256 * 2 + 8)
    assert lib.pcpa_split_workspace_bytes(ctypes.byref(p), 1) == 0
    assert lib.pcpa_split_workspace_bytes(ctypes.byref(p), 0) == -3
    assert lib.pcpa_split_workspace_bytes(ctypes.byref(p), 65) == -3
    assert lib.pcpa_split_workspace_bytes(ctypes.byref(_good_params(abi_version=1)), 2) == -2
    size = lib.pcpa_split_workspace_bytes(ctypes.byref(p), 2)
    f = lib.pcpa_history_attention_split
    assert f(ctypes.byref(p), 2, 16, 16, 16, 16, 16, None, None, size, None) == -10         # workspace
    assert f(ctypes.byref(p), 2, 16, 16, 16, 16, 16, None, 16, size - 16, None) == -10      # too small
    assert f(ctypes.byref(p), 2, 16, 16, 16, 16, 16, None, 8, size, None) == -6             # alignment
    assert f(ctypes.byref(p), 2, 16, 16, 16, 16, 16, 2, 16, size, None) == -6               # lse alignment
    # BF16 caches and BF16 MFMAs split too (tile kernel): their sizes are checked the same way
    for other in (_good_params(head_dim=128), _good_params(kv_dtype=2, head_dim=256, flags=1)):
        need = lib.pcpa_split_workspace_bytes(ctypes.byref(other), 4)
        assert need == 4 * 2048 * (other.head_dim + 2) * 4
        assert f(ctypes.byref(other), 4, 16, 16, 16, 16, 16, None, 16, need - 16, None) == -10
    # the guard (the default on an e4m3 cache, or asked for): it needs its
    # workspace through the split entry; the one-pass entries take none (the
    # library's guard scratch) and check every argument before using it
    for g in (_good_params(kv_dtype=2, head_dim=256), _good_params(kv_dtype=2, head_dim=256, flags=4)):
        assert lib.pcpa_split_workspace_bytes(ctypes.byref(g), 1) > 0
        assert f(ctypes.byref(g), 1, 16, 16, 16, 16, 16, None, None, 0, None) == -10
        assert lib.pcpa_history_attention(ctypes.byref(g), 16, 16, 16, 16, 0, None) == -1
        assert lib.pcpa_history_attention(ctypes.byref(g), 8, 16, 16, 16, 16, None) == -6
        assert lib.pcpa_history_attention_lse(ctypes.byref(g), 16, 16, 16, 16, 16, 2, None) == -6
    # the guard's buffers of a launch beyond the guard scratch: that launch
    # runs BF16 MFMAs instead, so its one-pass size is what matters
    big = _good_params(kv_dtype=2, head_dim=256, pcp_size=2048, local_q_len=256)
    assert lib.pcpa_split_workspace_bytes(ctypes.byref(big), 1) > _native.GUARD_SCRATCH_BYTES
    # an int64 block table must be 8-byte aligned
    t = _good_params(flags=8)
    assert lib.pcpa_history_attention(ctypes.byref(t), 16, 16, 20, 16, 16, None) == -6


def test_paging_entries_validate_without_a_gpu(lib):
    """pcpa_block_mask_valid_len / pcpa_page_alloc errors come back before any HIP call."""
    m = lib.pcpa_block_mask_valid_len
    assert m(None, 4, 4, 128, 16, None) == -1
    assert m(16, 4, 4, 128, None, None) == -1
    assert m(16, 0, 4, 128, 16, None) == -3
    assert m(16, 4, 4, 64, 16, None) == -3      # the mask form needs 128-key tiles
    assert m(17, 4, 4, 128, 16, None) == -6
    assert m(16, 4, 4, 128, 18, None) == -6
    a = lib.pcpa_page_alloc
    p = _good_params()  # 4 ranks x 4 blocks x 128 slots: positions [0, 2048)
    assert a(None, 16, 0, 8, 16, 16, 16, None) == -1
    assert a(ctypes.byref(p), 16, 0, 8, None, 16, 16, None) == -1
    assert a(ctypes.byref(p), 16, 0, 8, 16, None, 16, None) == -1
    assert a(ctypes.byref(p), 16, 0, 8, 16, 16, None, None) == -1
    assert a(ctypes.byref(p), 0, 0, 8, 16, 16, 16, None) == -3
    assert a(ctypes.byref(p), 16, -1, 8, 16, 16, 16, None) == -3
    assert a(ctypes.byref(p), 16, 0, 8, 18, 16, 16, None) == -6
    assert a(ctypes.byref(_good_params(flags=8)), 16, 0, 8, 20, 16, 16, None) == -6
    assert a(ctypes.byref(p), 16, 2040, 9, 16, 16, 16, None) == -3   # past the cache's capacity
    assert a(ctypes.byref(p), 16, 0, 0, 16, 16, 16, None) == 0       # nothing to place
