"""ctypes binding of the gfx950 C-ABI library ``libpcp_attention_hip.so``.

The library is built in-tree (``aws_training_study_amd/_lib``) by
``aws_training_study_amd.build_native.build()``.  Nothing here falls back to
another implementation: a missing or stale library raises ``RuntimeError``.
The C declarations live in ``include/pcp_attention_hip.h``.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "_lib"
LIB_NAME = "libpcp_attention_hip.so"

ABI_VERSION = 3

PCPA_OK = 0
STATUS_NAMES = {
    0: "PCPA_OK",
    -1: "PCPA_ERR_NULL_POINTER",
    -2: "PCPA_ERR_ABI_VERSION",
    -3: "PCPA_ERR_BAD_SHAPE",
    -4: "PCPA_ERR_BAD_DTYPE",
    -5: "PCPA_ERR_UNSUPPORTED",
    -6: "PCPA_ERR_MISALIGNED",
    -7: "PCPA_ERR_LAUNCH",
    -8: "PCPA_ERR_TOO_LARGE",
    -9: "PCPA_ERR_BAD_SCALE",
    -10: "PCPA_ERR_WORKSPACE",
    -11: "PCPA_ERR_SCRATCH",
}

DTYPE_BF16 = 1
DTYPE_FP8_E4M3FN = 2

FLAG_BF16_MFMA = 1
FLAG_EXACT_EXP2 = 2
FLAG_PRECISION_GUARD = 4
FLAG_TABLE_INT64 = 8
FLAG_E4M3_UNGUARDED = 16
# Rows whose probability mass sum_k 2^(x_k - m) is below this are recomputed
# with BF16 MFMAs by the precision guard (PCPA_GUARD_MIN_MASS), which runs on
# every e4m3-MFMA launch without FLAG_E4M3_UNGUARDED.
GUARD_MIN_MASS = 384.0

MAX_SPLITS = 64
# Device scratch of pcpa_history_attention_noalloc, per GPU (bytes).
NOALLOC_SCRATCH_BYTES = 80 << 20
# Guard scratch of pcpa_history_attention / _lse, per GPU (bytes).
GUARD_SCRATCH_BYTES = 48 << 20

# Every symbol the header declares; the CPU test suite checks they resolve.
EXPORTED_SYMBOLS = (
    "pcpa_abi_version",
    "pcpa_status_string",
    "pcpa_check_params",
    "pcpa_history_attention",
    "pcpa_history_attention_lse",
    "pcpa_history_attention_split",
    "pcpa_history_attention_noalloc",
    "pcpa_split_workspace_bytes",
    "pcpa_current_attention",
    "pcpa_kv_cache_write",
    "pcpa_absmax_bf16",
    "pcpa_block_mask_valid_len",
    "pcpa_page_alloc",
)


class PcpaParams(ctypes.Structure):
    """Mirror of ``pcpa_params`` (include/pcp_attention_hip.h)."""

    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("pcp_size", ctypes.c_int32),
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("local_q_len", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("max_local_blocks", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("q_dtype", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("k_scale", ctypes.c_float),
        ("v_scale", ctypes.c_float),
        ("flags", ctypes.c_uint32),
    ]


class PcpaError(RuntimeError):
    """A non-zero status returned by the C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


_lib: ctypes.CDLL | None = None


def library_path() -> Path:
    return LIB_DIR / LIB_NAME


def load_library() -> ctypes.CDLL:
    """Load the in-tree library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"HIP extension {path} is missing; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` "
            "(or aws_training_study_amd.build_native.build())"
        )
    lib = ctypes.CDLL(os.fspath(path))
    lib.pcpa_abi_version.restype = ctypes.c_int32
    lib.pcpa_abi_version.argtypes = []
    lib.pcpa_status_string.restype = ctypes.c_char_p
    lib.pcpa_status_string.argtypes = [ctypes.c_int32]
    lib.pcpa_check_params.restype = ctypes.c_int32
    lib.pcpa_check_params.argtypes = [ctypes.POINTER(PcpaParams)]
    lib.pcpa_history_attention.restype = ctypes.c_int32
    lib.pcpa_history_attention.argtypes = [
        ctypes.POINTER(PcpaParams),
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
    ]
    lib.pcpa_history_attention_lse.restype = ctypes.c_int32
    lib.pcpa_history_attention_lse.argtypes = [ctypes.POINTER(PcpaParams)] + [ctypes.c_void_p] * 7
    lib.pcpa_split_workspace_bytes.restype = ctypes.c_int64
    lib.pcpa_split_workspace_bytes.argtypes = [ctypes.POINTER(PcpaParams), ctypes.c_int32]
    lib.pcpa_history_attention_split.restype = ctypes.c_int32
    lib.pcpa_history_attention_split.argtypes = (
        [ctypes.POINTER(PcpaParams), ctypes.c_int32] + [ctypes.c_void_p] * 7 + [ctypes.c_int64, ctypes.c_void_p])
    lib.pcpa_history_attention_noalloc.restype = ctypes.c_int32
    lib.pcpa_history_attention_noalloc.argtypes = [ctypes.POINTER(PcpaParams), ctypes.c_int32] + [ctypes.c_void_p] * 7
    lib.pcpa_current_attention.restype = ctypes.c_int32
    lib.pcpa_current_attention.argtypes = [ctypes.POINTER(PcpaParams), ctypes.c_int32] + [ctypes.c_void_p] * 7
    lib.pcpa_kv_cache_write.restype = ctypes.c_int32
    lib.pcpa_kv_cache_write.argtypes = [
        ctypes.POINTER(PcpaParams),
        ctypes.c_int32,
        ctypes.c_int64,
        ctypes.c_int32,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
        ctypes.c_void_p,
    ]
    lib.pcpa_absmax_bf16.restype = ctypes.c_int32
    lib.pcpa_absmax_bf16.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    lib.pcpa_block_mask_valid_len.restype = ctypes.c_int32
    lib.pcpa_block_mask_valid_len.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                              ctypes.c_void_p, ctypes.c_void_p]
    lib.pcpa_page_alloc.restype = ctypes.c_int32
    lib.pcpa_page_alloc.argtypes = [ctypes.POINTER(PcpaParams), ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                    ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    version = lib.pcpa_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def status_string(status: int) -> str:
    return load_library().pcpa_status_string(status).decode()


def check(status: int) -> None:
    if status != PCPA_OK:
        raise PcpaError(status, status_string(status))
