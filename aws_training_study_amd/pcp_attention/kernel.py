"""HIP (gfx950) implementation of history-only PCP attention.

Same public names as ``pcp_attention/kernel.py`` of the Trainium2 proof of
concept: ``pack_local_kv`` (kernel.py:17-29), ``make_history_attention_kernel``
(kernel.py:32-556) and ``wrap_for_native_torch`` (kernel.py:559-564).  The
device code is a hand-written gfx950 kernel in
``aws_training_study_amd/csrc/pcp_attention_hip.hip`` reached through its C
ABI (``include/pcp_attention_hip.h``) with ctypes; there is no other
execution path, and a missing library raises.

Difference in calling convention: the reference kernel runs once per
logical rank and circulates KV blocks around a device ring.  Here one call
takes every rank's Q stacked as ``[pcp, Hq, local_q, D]`` plus the paged pool
of every rank's packed KV blocks and a block table, and returns every rank's
output ``[pcp, Hq, local_q, D]`` (``out[r]`` is the reference's rank-``r``
output).
"""

from __future__ import annotations

import ctypes
from dataclasses import replace
from typing import Any

from .config import PCPAttentionConfig


def pack_local_kv(k: Any, v: Any) -> Any:
    """Pack ``[blocks, Hkv, block_size, D]`` K and V into one row per block.

    Row ``b`` holds all of block ``b``'s K followed by all of its V, so it
    reshapes to ``[2, Hkv, block_size, D]``.  The dtype is kept (FP8 stays one
    byte per element).
    """
    import torch

    if k.shape != v.shape or k.ndim != 4:
        raise ValueError("K and V must have equal [blocks, Hkv, block, D] shapes")
    blocks = k.shape[0]
    packed = torch.empty((blocks, 2, *k.shape[1:]), dtype=k.dtype, device=k.device)
    packed[:, 0] = k
    packed[:, 1] = v
    return packed.reshape(blocks, -1)


_KV_DTYPE_CODES = {"fp8_e4m3fn": 2, "bfloat16": 1}

PRECISIONS = ("auto", "fp8", "bf16")
EXP2_MODES = ("fast", "exact")


def _torch_kv_dtype(name: str):
    import torch

    return {"fp8_e4m3fn": torch.float8_e4m3fn, "bfloat16": torch.bfloat16}[name]


class HistoryAttentionKernel:
    """Callable launching the gfx950 history attention kernel.

    ``kernel(q, kv_pages, block_table, block_valid_mask=None, *,
    page_valid_len=None, k_scale=1.0, v_scale=1.0, out=None) -> out``

    * ``q``: ``[pcp, Hq, local_q, D]`` bfloat16 on the GPU (every rank's Q
      shard, ``layout.stacked_query``), or the reference's per-rank list of
      ``[Hq, local_q, D]`` shards (stacked here).  ``out[r]`` is rank r's
      output; ``list(out)`` gives the per-rank list.
    * ``kv_pages``: ``[num_pages, 2 * Hkv * block_size * D]`` in the config's
      ``kv_dtype``; row ``p`` is a ``pack_local_kv`` row.  Or the reference's
      per-rank caches: a list of ``pcp`` ``[max_local_blocks, payload]``
      tensors (``pool_from_local_caches``), with no block table; the third
      positional argument is then the reference's ``block_valid_mask``, as in
      the NKI kernel's ``(q_ref, local_kv_ref, block_valid_mask_ref)``.
    * ``block_table``: int ``[pcp, max_local_blocks]`` page of each cache block.
    * validity: ``page_valid_len`` (int ``[pcp, max_local_blocks]``), or the
      reference's ``block_valid_mask`` (run_poc.py:137-153, shared by all
      ranks; a GPU mask is converted on the GPU, a CPU mask on the host with
      its values checked), or neither, in which case the config's
      ``actual_history_len`` decides.
    * ``block_table``: int32 or int64 (read as is by the kernels; entries
      outside ``[0, num_pages)`` are empty pages).
    * ``k_scale``/``v_scale``: per-tensor dequantisation scales of K and V.
    * ``precision``: for an e4m3 cache, ``"fp8"`` runs both GEMMs as e4m3
      MFMAs (Q and P rounded to e4m3), ``"bf16"`` as BF16 MFMAs on the exactly
      widened cache, and ``"auto"`` (default) runs e4m3 MFMAs with the
      precision guard: every row whose probability mass
      ``sum_k 2^(x_k - m)`` is below its KV head's threshold
      ``_native.GUARD_MIN_MASS * v_scale^2 * max_d Var(V[h, :, d])`` - few
      valid keys, a peaked score distribution or a wide V, where the e4m3
      rounding of Q and P is not averaged away - is recomputed on the
      device with BF16 MFMAs (a later launch whose workgroups exit at once
      when they hold no such row).  The decision is made per row on the GPU
      from the runtime lengths and data; nothing is read back to the host.
    * ``exp2``: how the e4m3 MFMA path at head_dim 256 forms the e4m3
      probabilities.  ``"fast"`` (default) writes the e4m3 code of 2^x
      directly, interpolating the exponential linearly between powers of two
      (at most 6.1% high before the e4m3 rounding, a +-3% shape error after
      normalisation); ``"exact"`` rounds ``v_exp_f32``.  Other paths always
      use ``v_exp_f32``.

    * ``splits``: cut the history into this many ranges of table entries run
      by separate workgroups and merged by log-sum-exp; ``"auto"`` splits
      only when the (row tile, KV head) workgroups would leave CUs idle,
      judged from the runtime history when its lengths are host tensors
      (``page_valid_len`` or ``block_valid_mask`` on the CPU, or neither
      given), else from the config's ``actual_history_len``.
      Split partials and the guard's row flags go to ``workspace`` (a uint8
      GPU tensor of ``workspace_bytes(splits, precision)`` bytes) or, if
      none is given, to a workspace the kernel object keeps per (device,
      current stream): calls on one stream run in order, calls on other
      streams get workspaces of their own.
    * ``return_lse``: also return each row's log-sum-exp (float32
      ``[pcp, Hq, local_q]``, natural log of the sum of ``exp(score)`` over
      the valid history keys, ``-inf`` for none) - the input of a merge with
      the current tokens (``current.CurrentAttentionKernel``).  The call then
      returns ``(out, lse)``.

    The launch is asynchronous on the current torch stream.
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
        status = self._lib.pcpa_check_params(ctypes.byref(self._params(cfg.num_pages, 1.0, 1.0)))
        if status != _native.PCPA_OK:
            raise ValueError(f"configuration rejected by the HIP kernel: {_native.status_string(status)}")
        self._default_valid = None
        # per-call host work kept small (a 14 us launch pair is otherwise host
        # bound): launch parameters, split counts and shapes are cached
        self._call_params = {}
        self._splits = {}
        self._ws_sizes = {}
        self._split_ws = {}
        self._local_pools = {}
        self._q_shape = (cfg.pcp_size, cfg.num_q_heads, cfg.local_q_len, cfg.head_dim)
        self._table_shape = (cfg.pcp_size, cfg.max_local_blocks)
        self._modes = {p: (self.uses_bf16_mfma(p), self.guarded(p)) for p in PRECISIONS}

    def _params(self, num_pages: int, k_scale: float, v_scale: float):
        return self._native.PcpaParams(
            num_pages=num_pages, k_scale=float(k_scale), v_scale=float(v_scale), **self._static
        )

    def uses_bf16_mfma(self, precision: str = "auto") -> bool:
        """Whether a call with ``precision`` runs its (first) pass on BF16 MFMAs."""
        return self.config.kv_dtype != "fp8_e4m3fn" or precision == "bf16"

    def guarded(self, precision: str = "auto") -> bool:
        """Whether a call with ``precision`` runs the precision guard (e4m3 cache, ``"auto"``)."""
        return self.config.kv_dtype == "fp8_e4m3fn" and precision == "auto"

    def default_page_valid_len(self, device) -> Any:
        from .paging import page_valid_lengths

        if self._default_valid is None or self._default_valid.device != device:
            self._default_valid = page_valid_lengths(self.config).to(device)
        return self._default_valid

    def _resolve_lengths(self, device, page_valid_len, block_valid_mask):
        """(int32 page_valid_len on ``device``, valid tokens if known on the host else None)."""
        import torch

        from .paging import valid_lengths_from_block_mask

        cfg = self.config
        table_shape = self._table_shape
        if page_valid_len is not None and block_valid_mask is not None:
            raise ValueError("pass either page_valid_len or block_valid_mask, not both")
        if page_valid_len is None and block_valid_mask is None:
            return self.default_page_valid_len(device), cfg.actual_history_len
        if page_valid_len is None:
            # a GPU mask is converted on the GPU (no host round trip)
            page_valid_len = valid_lengths_from_block_mask(block_valid_mask, cfg)
        if page_valid_len.shape != table_shape:
            raise ValueError(f"page_valid_len must be {table_shape}, got {tuple(page_valid_len.shape)}")
        tokens = None
        if not page_valid_len.is_cuda:
            tokens = int(page_valid_len.to(torch.int64).clamp(0, cfg.block_size).sum())
        if page_valid_len.dtype != torch.int32 or page_valid_len.device != device or not page_valid_len.is_contiguous():
            page_valid_len = page_valid_len.to(device=device, dtype=torch.int32).contiguous()
        return page_valid_len, tokens

    def __call__(
        self,
        q,
        kv_pages,
        block_table=None,
        block_valid_mask=None,
        *,
        page_valid_len=None,
        k_scale: float = 1.0,
        v_scale: float = 1.0,
        out=None,
        precision: str = "auto",
        exp2: str = "fast",
        return_lse: bool = False,
        splits="auto",
        workspace=None,
    ):
        import torch

        cfg = self.config
        if precision not in PRECISIONS:
            raise ValueError(f"precision must be one of {PRECISIONS}, got {precision!r}")
        if exp2 not in EXP2_MODES:
            raise ValueError(f"exp2 must be one of {EXP2_MODES}, got {exp2!r}")
        if isinstance(q, (list, tuple)):
            # the reference's per-rank form: one [Hq, local_q, D] shard per rank
            if len(q) != cfg.pcp_size:
                raise ValueError(f"expected {cfg.pcp_size} per-rank Q shards, got {len(q)}")
            q = torch.stack(list(q))
        if not q.is_cuda:
            raise ValueError("q must be a GPU tensor")
        device = q.device
        if isinstance(kv_pages, (list, tuple)):
            # the reference's per-rank caches: kernel(q_list, local_kv_list, mask)
            if block_table is not None and block_table.is_floating_point():
                if block_valid_mask is not None:
                    raise ValueError("pass the block-valid mask once")
                block_table, block_valid_mask = None, block_table
            if block_table is not None:
                raise ValueError("a per-rank cache list brings its own block table (rank r's block b is page "
                                 "r * max_local_blocks + b); pass a pool to use another")
            kv_pages, block_table = self.pool_from_local_caches(kv_pages, device)
        elif block_table is None:
            raise ValueError("block_table is required with a page pool")
        q_shape = self._q_shape
        if q.shape != q_shape or q.dtype != torch.bfloat16 or not q.is_contiguous():
            raise ValueError(f"q must be contiguous bfloat16 {q_shape}, got {q.dtype} {tuple(q.shape)}")
        kv_dtype = _torch_kv_dtype(cfg.kv_dtype)
        if (
            kv_pages.ndim != 2
            or kv_pages.shape[1] != cfg.page_elements
            or kv_pages.dtype != kv_dtype
            or not kv_pages.is_contiguous()
            or kv_pages.device != device
        ):
            raise ValueError(
                f"kv_pages must be contiguous {kv_dtype} [num_pages, {cfg.page_elements}] on {device}, "
                f"got {kv_pages.dtype} {tuple(kv_pages.shape)} on {kv_pages.device}"
            )
        num_pages = kv_pages.shape[0]
        table_shape = self._table_shape
        if block_table.shape != table_shape:
            raise ValueError(f"block_table must be {table_shape}, got {tuple(block_table.shape)}")
        if (block_table.dtype not in (torch.int32, torch.int64) or block_table.device != device
                or not block_table.is_contiguous()):
            block_table = block_table.to(device=device, dtype=torch.int32).contiguous()
        table64 = block_table.dtype == torch.int64
        page_valid_len, tokens = self._resolve_lengths(device, page_valid_len, block_valid_mask)
        if out is None:
            out = torch.empty(q_shape, dtype=torch.bfloat16, device=device)
        elif out.shape != q_shape or out.dtype != torch.bfloat16 or not out.is_contiguous() or out.device != device:
            raise ValueError(f"out must be contiguous bfloat16 {q_shape} on {device}")
        lse = None
        if return_lse:
            lse = torch.empty(q_shape[:3], dtype=torch.float32, device=device)
        bf16_mfma, guard = self._modes[precision]
        # scales by value (a tensor or numpy scalar is read here, not kept)
        if type(k_scale) is not float:
            k_scale = float(k_scale)
        if type(v_scale) is not float:
            v_scale = float(v_scale)
        key = (num_pages, k_scale, v_scale, precision, exp2, table64)
        params = self._call_params.get(key)
        if params is None:
            params = self._params(num_pages, k_scale, v_scale)
            if bf16_mfma:
                params.flags |= self._native.FLAG_BF16_MFMA
            if exp2 == "exact":
                params.flags |= self._native.FLAG_EXACT_EXP2
            if guard:
                params.flags |= self._native.FLAG_PRECISION_GUARD
            elif not bf16_mfma:
                params.flags |= self._native.FLAG_E4M3_UNGUARDED
            if table64:
                params.flags |= self._native.FLAG_TABLE_INT64
            if len(self._call_params) >= 64:
                self._call_params.clear()
            self._call_params[key] = params
        if splits == "auto":
            skey = (device, bf16_mfma, tokens)
            n_split = self._splits.get(skey)
            if n_split is None:
                if len(self._splits) >= 64:
                    self._splits.clear()
                n_split = self._splits[skey] = self.split_count(device, bf16_mfma, tokens)
        else:
            n_split = int(splits)
        if n_split > 1 or guard:
            size = self.workspace_bytes(n_split, precision)
            if workspace is None:
                workspace = self._workspace(size, device, _current_raw_stream(device))
            elif workspace.dtype != torch.uint8 or workspace.device != device or not workspace.is_contiguous():
                raise ValueError(f"workspace must be a contiguous uint8 tensor on {device}")
            status = _on_device(device, self._lib.pcpa_history_attention_split, params, n_split, q.data_ptr(),
                                kv_pages.data_ptr(), block_table.data_ptr(), page_valid_len.data_ptr(),
                                out.data_ptr(), None if lse is None else lse.data_ptr(), workspace.data_ptr(),
                                workspace.numel())
        else:
            status = _on_device(device, self._lib.pcpa_history_attention_lse, params, q.data_ptr(),
                                kv_pages.data_ptr(), block_table.data_ptr(), page_valid_len.data_ptr(),
                                out.data_ptr(), None if lse is None else lse.data_ptr())
        if status:
            self._native.check(status)
        return (out, lse) if return_lse else out

    def pool_from_local_caches(self, local_kv, device=None):
        """(pool, identity block table) of the reference's per-rank caches.

        ``local_kv``: one ``[max_local_blocks, 2 * Hkv * block_size * D]``
        tensor per rank, ``pack_local_kv`` rows padded to ``max_local_blocks``
        as run_poc.py:231-238 builds them (the NKI kernel's ``local_kv_ref``,
        kernel.py:84-118).  The pool holds rank r's block b as page
        ``r * max_local_blocks + b``.  It is built once and reused while the
        same tensors come back unchanged (same storage, same torch version
        counter: an in-place torch write to one of them builds it again;
        writes that bypass torch are not seen).
        """
        import torch

        cfg = self.config
        if len(local_kv) != cfg.pcp_size:
            raise ValueError(f"expected {cfg.pcp_size} per-rank caches, got {len(local_kv)}")
        kv_dtype = _torch_kv_dtype(cfg.kv_dtype)
        shape = (cfg.max_local_blocks, cfg.page_elements)
        device = local_kv[0].device if device is None else device
        for r, t in enumerate(local_kv):
            if tuple(t.shape) != shape or t.dtype != kv_dtype or t.device != device or not t.is_contiguous():
                raise ValueError(f"rank {r}'s cache must be contiguous {kv_dtype} {shape} on {device}, "
                                 f"got {t.dtype} {tuple(t.shape)} on {t.device}")
        key = (device, tuple((t.data_ptr(), t._version) for t in local_kv))
        hit = self._local_pools.get(key)
        if hit is not None:
            return hit
        pool = torch.cat(list(local_kv), dim=0)
        table = torch.arange(cfg.pcp_size * cfg.max_local_blocks, dtype=torch.int32, device=device).reshape(
            cfg.pcp_size, cfg.max_local_blocks)
        self._local_pools.clear()  # the last set of caches only
        self._local_pools[key] = (pool, table)
        return pool, table

    def graphed(self, q, kv_pages, block_table, block_valid_mask=None, *, warmup: int = 1, **kwargs):
        """This call captured into a HIP graph (``launch.GraphedLaunch``).

        The output buffer (``out=``, allocated here if not given) and the
        log-sum-exp (``return_lse=True``) are fixed; ``replay()`` recomputes
        them from the current contents of the same input tensors (a GPU
        ``block_valid_mask`` is converted to page lengths inside the graph).
        A split or guarded call gets a workspace of its own, held by the
        graph, so replays do not share it with eager calls or other graphs.
        """
        import torch

        from .launch import GraphedLaunch

        if isinstance(kv_pages, (list, tuple)):
            raise ValueError("graphed() takes a page pool and block table (pool_from_local_caches builds them "
                             "from per-rank caches; a graph replays against that pool)")
        if kwargs.get("out") is None:
            kwargs["out"] = torch.empty_like(q)
        if kwargs.get("workspace") is None:
            kwargs["workspace"] = self.graph_workspace(q.device, kwargs.get("precision", "auto"),
                                                       kwargs.get("splits", "auto"))
        # host-side lengths and tables move to the GPU once, outside the graph
        if block_valid_mask is not None and not block_valid_mask.is_cuda:
            from .paging import valid_lengths_from_block_mask

            kwargs["page_valid_len"] = valid_lengths_from_block_mask(block_valid_mask, self.config)
            block_valid_mask = None
        if kwargs.get("page_valid_len") is not None:
            kwargs["page_valid_len"] = kwargs["page_valid_len"].to(device=q.device, dtype=torch.int32).contiguous()
        if not block_table.is_cuda or block_table.dtype not in (torch.int32, torch.int64):
            block_table = block_table.to(device=q.device, dtype=torch.int32).contiguous()
        return GraphedLaunch(lambda: self(q, kv_pages, block_table, block_valid_mask, **kwargs), warmup=warmup)

    # Query rows per workgroup and workgroups per CU: the e4m3 head_dim-256
    # kernel takes 256 rows and a whole CU; the tile kernel 128 rows, two
    # per CU (one for BF16 MFMAs at head_dim 256).
    ROWS_PER_WORKGROUP = {"overlap": 256, "tile": 128}
    # A split should still walk at least this many 64-key tiles (measured on
    # the MI355X: the overlap kernel's deeper pipeline needs longer ranges).
    MIN_TILES_PER_SPLIT = {"overlap": 16, "tile": 4}

    def split_count(self, device, bf16_mfma: bool, tokens=None) -> int:
        """History splits for ``splits="auto"`` on ``device`` (``auto_splits``)."""
        import torch

        return self.auto_splits(bf16_mfma, torch.cuda.get_device_properties(device).multi_processor_count, tokens)

    def auto_splits(self, bf16_mfma: bool, cus: int, tokens=None) -> int:
        """Enough (row tile, KV head, split) workgroups to fill the workgroup
        slots of ``cus`` CUs, each split still walking ``MIN_TILES_PER_SPLIT``
        tiles of the ``tokens`` valid history tokens (default: the config's
        ``actual_history_len``) and holding a table entry; 1 when the row
        tiles already fill the GPU."""
        cfg = self.config
        overlap = not bf16_mfma and cfg.kv_dtype == "fp8_e4m3fn" and cfg.head_dim == 256
        kind = "overlap" if overlap else "tile"
        per_cu = 1 if overlap or (bf16_mfma and cfg.head_dim == 256) else 2
        rows_per_head = cfg.pcp_size * cfg.local_q_len * (cfg.num_q_heads // cfg.num_kv_heads)
        items = -(-rows_per_head // self.ROWS_PER_WORKGROUP[kind]) * cfg.num_kv_heads
        slots = cus * per_cu
        if items >= slots:
            return 1
        tiles = -(-(cfg.actual_history_len if tokens is None else tokens) // 64)
        entries = cfg.pcp_size * cfg.max_local_blocks
        return max(1, min(self._native.MAX_SPLITS, entries, -(-slots // items),
                          tiles // self.MIN_TILES_PER_SPLIT[kind]))

    def workspace_bytes(self, n_split: int, precision: str = "auto") -> int:
        """Bytes of the workspace of a call with ``n_split`` splits and ``precision``."""
        key = (int(n_split), self.guarded(precision), self.uses_bf16_mfma(precision))
        size = self._ws_sizes.get(key)
        if size is None:
            params = self._params(self.config.num_pages, 1.0, 1.0)
            if key[1]:
                params.flags |= self._native.FLAG_PRECISION_GUARD
            elif key[2]:
                params.flags |= self._native.FLAG_BF16_MFMA
            else:
                params.flags |= self._native.FLAG_E4M3_UNGUARDED
            size = self._lib.pcpa_split_workspace_bytes(ctypes.byref(params), key[0])
            if size < 0:
                self._native.check(int(size))
            size = self._ws_sizes[key] = int(size)
        return size

    def split_workspace_bytes(self, n_split: int) -> int:
        """Bytes of the split partials of a call with ``n_split`` splits (no guard)."""
        return self.workspace_bytes(n_split, precision="fp8")

    def graph_workspace(self, device, precision="auto", splits="auto"):
        """A new workspace for a call that ``precision``/``splits`` would split or guard, else ``None``."""
        import torch

        n_split = self.split_count(device, self.uses_bf16_mfma(precision)) if splits == "auto" else int(splits)
        size = self.workspace_bytes(n_split, precision)
        if size <= 0:
            return None
        return torch.empty(size, dtype=torch.uint8, device=device)

    def _workspace(self, size: int, device, stream: int):
        """The workspace this object keeps for calls on (``device``, ``stream``).

        Calls on one stream run in order, so they can share one; calls on
        different streams may overlap on the GPU, so each stream gets its own
        (a guarded call's thresholds, plan and fixup partials, or a split
        call's partials, must not be rewritten by another call in flight).
        """
        import torch

        key = (device, stream)
        ws = self._split_ws.get(key)
        if ws is None or ws.numel() < size:
            if ws is None and len(self._split_ws) >= 16:
                self._split_ws.clear()
            ws = torch.empty(max(size, 16), dtype=torch.uint8, device=device)
            self._split_ws[key] = ws
        return ws


def _current_raw_stream(device) -> int:
    """Raw handle of torch's current stream on ``device``."""
    import torch

    raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw_stream is not None:
        return raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _on_device(device, fn, *args):
    """``fn(*args, stream)`` with ``device`` current and its current torch
    stream (raw handle) last: the launch is queued where torch would queue
    work on that device.  Switches the current device only when it differs
    (a switch and the stream object cost microseconds a small launch does not
    take on the GPU)."""
    import torch

    index = device.index
    raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if torch.cuda.current_device() == index:
        stream = raw_stream(index) if raw_stream else torch.cuda.current_stream(device).cuda_stream
        return fn(*args, stream)
    with torch.cuda.device(device):
        return fn(*args, torch.cuda.current_stream(device).cuda_stream)


def make_history_attention_kernel(config: PCPAttentionConfig) -> HistoryAttentionKernel:
    """Build the gfx950 kernel callable for ``config``.

    Raises ``ValueError`` for shapes the HIP kernel does not support (the
    reference raises for shapes its NKI kernel does not, kernel.py:42-51).
    """
    return HistoryAttentionKernel(config)


def wrap_for_native_torch(config: PCPAttentionConfig) -> HistoryAttentionKernel:
    """Torch-callable kernel; the HIP callable already takes torch tensors."""
    return make_history_attention_kernel(config)
