"""On-GPU KV-cache producer: the step before history attention.

The reference builds its cache on the host: ``shard_history``
(layout.py:54-98) places each history token on its owner rank at its local
position, K/V are cast to FP8 e4m3 (run_poc.py:96-103) and ``pack_local_kv``
(kernel.py:17-29) packs each rank's blocks into page rows, which the block
table then places in the pool (``paging.pack_page_pool``).  ``KVCacheWriter``
does all of it in one HIP launch for a range of global positions, so the
same call fills a whole history or appends tokens to it; e4m3 pools get
``round_e4m3(x / scale)`` bit for bit as torch's cast computes it.
"""

from __future__ import annotations

import ctypes
from dataclasses import replace
from typing import Optional

from .config import PCPAttentionConfig
from .inputs import per_tensor_scale
from .kernel import _KV_DTYPE_CODES, _torch_kv_dtype


def absmax(x):
    """max |x| of a contiguous BF16 GPU tensor, as a 0-d float32 GPU tensor (HIP reduction)."""
    import torch

    from .. import _native

    if not x.is_cuda or x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("absmax expects a contiguous bfloat16 GPU tensor")
    lib = _native.load_library()
    out = torch.empty((), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        status = lib.pcpa_absmax_bf16(x.data_ptr(), x.numel(), out.data_ptr(),
                                      torch.cuda.current_stream(x.device).cuda_stream)
    _native.check(status)
    return out


def device_per_tensor_scale(x) -> float:
    """``per_tensor_scale`` of a GPU tensor (one device reduction, one sync)."""
    return per_tensor_scale(float(absmax(x)))


class KVCacheWriter:
    """Writes history K/V into a page pool (``pack_local_kv`` rows) on the GPU.

    ``writer(k, v, kv_pages, block_table, *, first_pos=0, k_scale=1.0,
    v_scale=1.0, page_valid_len=None)``: ``k``/``v`` are contiguous BF16
    ``[Hkv, n, D]`` GPU tensors holding the tokens at global positions
    ``first_pos .. first_pos + n - 1``; ``kv_pages`` is the config's
    ``[num_pages, page_elements]`` pool; ``block_table`` int32 or int64
    ``[pcp, max_local_blocks]`` (entries outside ``[0, num_pages)`` are not
    written).  An e4m3 pool stores ``x / scale`` rounded to e4m3;
    a BF16 pool stores ``x``.  ``page_valid_len`` (int32, optional) is
    raised to cover every written token.  Asynchronous on the current stream.
    """

    def __init__(self, config: PCPAttentionConfig):
        from .. import _native

        self.config = replace(config, backend="hip").validate()
        self._native = _native
        self._lib = _native.load_library()
        cfg = self.config
        self._static = dict(
            abi_version=_native.ABI_VERSION,
            pcp_size=cfg.pcp_size,
            num_q_heads=cfg.num_q_heads,
            num_kv_heads=cfg.num_kv_heads,
            head_dim=cfg.head_dim,
            local_q_len=cfg.local_q_len,
            block_size=cfg.block_size,
            max_local_blocks=cfg.max_local_blocks,
            q_dtype=_native.DTYPE_BF16,
            kv_dtype=_KV_DTYPE_CODES[cfg.kv_dtype],
            out_dtype=_native.DTYPE_BF16,
            softmax_scale=cfg.softmax_scale,
            flags=0,
        )

    def __call__(self, k, v, kv_pages, block_table, *, first_pos: int = 0, k_scale: float = 1.0,
                 v_scale: float = 1.0, page_valid_len: Optional[object] = None) -> None:
        import torch

        cfg = self.config
        shape = (cfg.num_kv_heads, k.shape[1] if k.ndim == 3 else -1, cfg.head_dim)
        for name, t in (("k", k), ("v", v)):
            if (t.ndim != 3 or tuple(t.shape) != shape or t.dtype != torch.bfloat16 or not t.is_contiguous()
                    or not t.is_cuda):
                raise ValueError(f"{name} must be a contiguous bfloat16 GPU tensor {shape}, got "
                                 f"{t.dtype} {tuple(t.shape)}")
        if (kv_pages.ndim != 2 or kv_pages.shape[1] != cfg.page_elements
                or kv_pages.dtype != _torch_kv_dtype(cfg.kv_dtype) or not kv_pages.is_contiguous()):
            raise ValueError(f"kv_pages must be a contiguous {cfg.kv_dtype} [num_pages, {cfg.page_elements}] pool")
        table_shape = (cfg.pcp_size, cfg.max_local_blocks)
        for name, t, dtypes in (("block_table", block_table, (torch.int32, torch.int64)),
                                ("page_valid_len", page_valid_len, (torch.int32,))):
            if t is None:
                continue
            if tuple(t.shape) != table_shape or t.dtype not in dtypes or not t.is_contiguous() or not t.is_cuda:
                raise ValueError(f"{name} must be a contiguous {' or '.join(str(d) for d in dtypes)} GPU tensor "
                                 f"{table_shape}")
        for name, t in (("v", v), ("kv_pages", kv_pages), ("block_table", block_table),
                        ("page_valid_len", page_valid_len)):
            if t is not None and t.device != k.device:
                raise ValueError(f"{name} is on {t.device}, k on {k.device}: all tensors must share one GPU")
        if k.shape[1] >= 2**31 or not 0 <= int(first_pos) < 2**63:
            raise ValueError("num_tokens must be below 2^31 and first_pos non-negative")
        params = self._native.PcpaParams(num_pages=kv_pages.shape[0], k_scale=float(k_scale),
                                         v_scale=float(v_scale), **self._static)
        if block_table.dtype == torch.int64:
            params.flags |= self._native.FLAG_TABLE_INT64
        with torch.cuda.device(k.device):
            status = self._lib.pcpa_kv_cache_write(
                ctypes.byref(params), cfg.interleave_size, int(first_pos), k.shape[1], k.data_ptr(),
                v.data_ptr(), block_table.data_ptr(), kv_pages.data_ptr(),
                None if page_valid_len is None else page_valid_len.data_ptr(),
                torch.cuda.current_stream(k.device).cuda_stream)
        self._native.check(status)


def build_page_pool(config: PCPAttentionConfig, k, v, block_table, *, kv_scale: str = "per_tensor"):
    """A fresh zeroed pool holding history tokens ``0 .. k.shape[1] - 1``.

    Returns ``(pool, k_scale, v_scale, page_valid_len)``; e4m3 pools use
    per-tensor scales ``amax / 448`` (``kv_scale="per_tensor"``) or none.
    The GPU counterpart of ``pack_page_pool(shard_history(...))``.
    """
    import torch

    cfg = replace(config, backend="hip").validate()
    if kv_scale not in ("per_tensor", "none"):
        raise ValueError(f"kv_scale must be 'per_tensor' or 'none', got {kv_scale!r}")
    k_scale = v_scale = 1.0
    if cfg.kv_dtype == "fp8_e4m3fn" and kv_scale == "per_tensor":
        # both reductions queued, then one synchronisation for the two scales
        amax_k, amax_v = torch.stack([absmax(k), absmax(v)]).tolist()
        k_scale, v_scale = per_tensor_scale(amax_k), per_tensor_scale(amax_v)
    pool = torch.zeros((cfg.num_pages, cfg.page_elements), dtype=_torch_kv_dtype(cfg.kv_dtype), device=k.device)
    valid = torch.zeros((cfg.pcp_size, cfg.max_local_blocks), dtype=torch.int32, device=k.device)
    table = block_table.to(device=k.device, dtype=torch.int32).contiguous()
    KVCacheWriter(cfg)(k, v, pool, table, k_scale=k_scale, v_scale=v_scale, page_valid_len=valid)
    return pool, k_scale, v_scale, valid


class PageAllocator:
    """Free-page stack on the GPU for block tables filled as history grows.

    The reference places every rank's blocks into a padded local cache on
    the host (run_poc.py:231-237, layout.py:54-98).  Here pages of one pool
    are handed out on the device: ``allocate(first_pos, num_tokens,
    block_table)`` gives every cache block that the positions reach and
    whose table entry is negative a page from the top of the stack, in
    (rank, block) order, without a host round trip (``pcpa_page_alloc``).
    ``free_count`` (a 0-d int32 GPU tensor) is the stack height; a block that
    finds the stack empty keeps its negative entry and its tokens are not
    written.  Initially pages are handed out in ascending order.
    """

    def __init__(self, config: PCPAttentionConfig, device, num_pages: Optional[int] = None):
        import torch

        from .. import _native

        self.config = replace(config, backend="hip").validate()
        self.num_pages = self.config.num_pages if num_pages is None else int(num_pages)
        self._native = _native
        self._lib = _native.load_library()
        # the top of the stack is the last element: page 0 is handed out first
        self.free_pages = torch.arange(self.num_pages - 1, -1, -1, dtype=torch.int32, device=device)
        self.free_count = torch.tensor(self.num_pages, dtype=torch.int32, device=device)
        self._params = self._native.PcpaParams(
            abi_version=_native.ABI_VERSION, pcp_size=self.config.pcp_size, num_q_heads=self.config.num_q_heads,
            num_kv_heads=self.config.num_kv_heads, head_dim=self.config.head_dim,
            local_q_len=self.config.local_q_len, block_size=self.config.block_size,
            max_local_blocks=self.config.max_local_blocks, num_pages=self.num_pages, q_dtype=_native.DTYPE_BF16,
            kv_dtype=_KV_DTYPE_CODES[self.config.kv_dtype], out_dtype=_native.DTYPE_BF16,
            softmax_scale=self.config.softmax_scale, k_scale=1.0, v_scale=1.0, flags=0)

    def empty_table(self, dtype=None):
        """A block table with no page assigned (every entry -1)."""
        import torch

        cfg = self.config
        return torch.full((cfg.pcp_size, cfg.max_local_blocks), -1, dtype=dtype or torch.int32,
                          device=self.free_pages.device)

    def allocate(self, first_pos: int, num_tokens: int, block_table) -> None:
        """Assign pages to the blocks that positions [first_pos, first_pos + num_tokens) reach (asynchronous)."""
        import torch

        cfg = self.config
        if (tuple(block_table.shape) != (cfg.pcp_size, cfg.max_local_blocks)
                or block_table.dtype not in (torch.int32, torch.int64) or not block_table.is_contiguous()
                or block_table.device != self.free_pages.device):
            raise ValueError("block_table must be a contiguous int32/int64 tensor "
                             f"{(cfg.pcp_size, cfg.max_local_blocks)} on {self.free_pages.device}")
        flags = self._native.FLAG_TABLE_INT64 if block_table.dtype == torch.int64 else 0
        params = self._native.PcpaParams.from_buffer_copy(self._params)
        params.flags = flags
        with torch.cuda.device(block_table.device):
            status = self._lib.pcpa_page_alloc(
                ctypes.byref(params), cfg.interleave_size, int(first_pos), int(num_tokens), block_table.data_ptr(),
                self.free_pages.data_ptr(), self.free_count.data_ptr(),
                torch.cuda.current_stream(block_table.device).cuda_stream)
        self._native.check(status)


def append_history(writer: KVCacheWriter, allocator: PageAllocator, k, v, kv_pages, block_table, page_valid_len, *,
                   first_pos: int, k_scale: float = 1.0, v_scale: float = 1.0) -> None:
    """Append tokens ``first_pos ..`` to a paged history: pages for the blocks
    they reach (``allocator``), then quantise and write them (``writer``),
    raising ``page_valid_len``.  Two launches on the current stream."""
    allocator.allocate(first_pos, k.shape[1], block_table)
    writer(k, v, kv_pages, block_table, first_pos=first_pos, k_scale=k_scale, v_scale=v_scale,
           page_valid_len=page_valid_len)
