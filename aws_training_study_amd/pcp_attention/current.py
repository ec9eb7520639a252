"""Current-token causal attention and its merge with the history: the step after it.

The reference computes history-only attention; its current tokens do not
attend to one another yet (README.md:17-18).  ``CurrentAttentionKernel``
adds that step on the GPU with the standard causal rule: the query at global
current position ``g`` sees the current keys ``0..g``.  Given the history
output and log-sum-exp of ``HistoryAttentionKernel(..., return_lse=True)``,
the same launch merges the two by log-sum-exp, so the result is softmax
attention over the history keys and the causal current keys together.
``PrefillAttention`` chains the two launches.

Current K/V are BF16 in global token order, ``[2, Hkv, current_len, D]``
(``stack_current_kv``); queries are every rank's striped shard as for the
history kernel (``layout.stacked_query``).
"""

from __future__ import annotations

import ctypes
from dataclasses import replace

from .config import PCPAttentionConfig
from .kernel import HistoryAttentionKernel


def stack_current_kv(k, v):
    """``[2, Hkv, current_len, D]`` from current K and V ``[Hkv, current_len, D]`` (global order)."""
    import torch

    if k.shape != v.shape or k.ndim != 3:
        raise ValueError(f"k and v must both be [Hkv, current_len, D], got {tuple(k.shape)} and {tuple(v.shape)}")
    return torch.stack((k, v)).to(torch.bfloat16).contiguous()


class CurrentAttentionKernel:
    """Causal attention of the current tokens, optionally merged with the history.

    ``kernel(q, kv_current, hist_out=None, hist_lse=None, *, out=None,
    return_lse=False)``

    * ``q``: ``[pcp, Hq, local_q, D]`` bfloat16 GPU tensor (``stacked_query``).
    * ``kv_current``: ``[2, Hkv, current_len, D]`` bfloat16, K then V of the
      current tokens in global order; ``current_len`` must be a multiple of 64.
    * ``hist_out``/``hist_lse``: both or neither - the history attention's
      output and log-sum-exp for the same ``q``; with them the output covers
      history and current keys.  ``out`` may be ``hist_out`` (in place).
    * ``return_lse``: also return the float32 ``[pcp, Hq, local_q]``
      log-sum-exp of the keys the output covers.

    Asynchronous on the current torch stream.
    """

    def __init__(self, config: PCPAttentionConfig):
        from .. import _native

        self.config = replace(config, backend="hip", kv_dtype="bfloat16").validate()
        cfg = self.config
        if cfg.current_len % 64:
            raise ValueError(f"current_len must be a multiple of 64 for the HIP kernel, got {cfg.current_len}")
        self._native = _native
        self._lib = _native.load_library()
        self._static = dict(
            abi_version=_native.ABI_VERSION,
            pcp_size=cfg.pcp_size,
            num_q_heads=cfg.num_q_heads,
            num_kv_heads=cfg.num_kv_heads,
            head_dim=cfg.head_dim,
            local_q_len=cfg.local_q_len,
            block_size=cfg.block_size,
            max_local_blocks=cfg.max_local_blocks,
            num_pages=cfg.num_pages,
            q_dtype=_native.DTYPE_BF16,
            kv_dtype=_native.DTYPE_BF16,
            out_dtype=_native.DTYPE_BF16,
            softmax_scale=cfg.softmax_scale,
            k_scale=1.0,
            v_scale=1.0,
            flags=0,
        )
        # the launch parameters never change: built once, read by every call
        self._launch_params = _native.PcpaParams(**self._static)
        status = self._lib.pcpa_check_params(ctypes.byref(self._launch_params))
        if status != _native.PCPA_OK:
            raise ValueError(f"configuration rejected by the HIP kernel: {_native.status_string(status)}")

    def __call__(self, q, kv_current, hist_out=None, hist_lse=None, *, out=None, return_lse: bool = False):
        import torch

        cfg = self.config
        if not q.is_cuda:
            raise ValueError("q must be a GPU tensor")
        device = q.device
        q_shape = (cfg.pcp_size, cfg.num_q_heads, cfg.local_q_len, cfg.head_dim)
        kv_shape = (2, cfg.num_kv_heads, cfg.current_len, cfg.head_dim)
        lse_shape = q_shape[:3]

        def check(name, t, shape, dtype):
            if t is None:
                return
            if tuple(t.shape) != shape or t.dtype != dtype or not t.is_contiguous() or t.device != device:
                raise ValueError(f"{name} must be contiguous {dtype} {shape} on {device}, "
                                 f"got {t.dtype} {tuple(t.shape)} on {t.device}")

        check("q", q, q_shape, torch.bfloat16)
        check("kv_current", kv_current, kv_shape, torch.bfloat16)
        if (hist_out is None) != (hist_lse is None):
            raise ValueError("pass both hist_out and hist_lse, or neither")
        check("hist_out", hist_out, q_shape, torch.bfloat16)
        check("hist_lse", hist_lse, lse_shape, torch.float32)
        if out is None:
            out = torch.empty(q_shape, dtype=torch.bfloat16, device=device)
        check("out", out, q_shape, torch.bfloat16)
        lse = torch.empty(lse_shape, dtype=torch.float32, device=device) if return_lse else None
        with torch.cuda.device(device):
            status = self._lib.pcpa_current_attention(
                ctypes.byref(self._launch_params),
                cfg.interleave_size,
                q.data_ptr(),
                kv_current.data_ptr(),
                None if hist_out is None else hist_out.data_ptr(),
                None if hist_lse is None else hist_lse.data_ptr(),
                out.data_ptr(),
                None if lse is None else lse.data_ptr(),
                torch.cuda.current_stream(device).cuda_stream,
            )
        self._native.check(status)
        return (out, lse) if return_lse else out


class PrefillAttention:
    """History attention followed by the causal current-token step, merged in place.

    ``prefill(q, kv_pages, block_table, kv_current, *, page_valid_len=None,
    k_scale=1.0, v_scale=1.0, precision="auto", exp2="fast",
    return_lse=False, workspace=None)`` - two launches on the current
    stream; the output buffer of the first is updated in place by the
    second (``workspace``: the history's split workspace, as for
    ``HistoryAttentionKernel``).
    """

    def __init__(self, config: PCPAttentionConfig):
        self.history = HistoryAttentionKernel(config)
        self.current = CurrentAttentionKernel(config)
        self.config = self.history.config

    def graphed(self, q, kv_pages, block_table, kv_current, *, warmup: int = 1, **kwargs):
        """Both launches captured into one HIP graph (``launch.GraphedLaunch``),
        with a split workspace of the graph's own when the history is split."""
        from .launch import GraphedLaunch

        if kwargs.get("workspace") is None:
            kwargs["workspace"] = self.history.graph_workspace(q.device, kwargs.get("precision", "auto"))
        return GraphedLaunch(lambda: self(q, kv_pages, block_table, kv_current, **kwargs), warmup=warmup)

    def __call__(self, q, kv_pages, block_table, kv_current, block_valid_mask=None, *, page_valid_len=None,
                 k_scale: float = 1.0, v_scale: float = 1.0, precision: str = "auto", exp2: str = "fast",
                 return_lse: bool = False, workspace=None):
        out, lse = self.history(q, kv_pages, block_table, block_valid_mask, page_valid_len=page_valid_len,
                                k_scale=k_scale, v_scale=v_scale, precision=precision, exp2=exp2,
                                return_lse=True, workspace=workspace)
        return self.current(q, kv_current, out, lse, out=out, return_lse=return_lse)
