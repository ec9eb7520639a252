"""Float32 dense attention on the GPU with torch, for ``run_poc --check``.

This is a verification aid only (the reference's runner checks its device
output against dense attention, run_poc.py:256-266); the kernel output is
never produced by it.
"""

from __future__ import annotations

import torch

from .workloads import PagedProblem


def dequantised_history(problem: PagedProblem, device) -> tuple[torch.Tensor, torch.Tensor]:
    inputs = problem.inputs
    if inputs.k is None:
        raise ValueError("a problem built from per-rank local inputs has no global history to check against")
    k = inputs.k.to(device).float() * inputs.k_scale
    v = inputs.v.to(device).float() * inputs.v_scale
    return k, v


@torch.no_grad()
def dense_reference(problem: PagedProblem, device, row_chunk: int = 2048) -> torch.Tensor:
    """``[pcp, Hq, local_q, D]`` float32: softmax(q k^T * scale) v over valid history."""
    cfg = problem.config
    k, v = dequantised_history(problem, device)
    length = cfg.actual_history_len
    qs = problem.q_stacked.to(device).float()
    out = torch.empty_like(qs)
    group = cfg.num_q_heads // cfg.num_kv_heads
    for g in range(cfg.num_kv_heads):
        kg = k[g, :length].contiguous()
        vg = v[g, :length].contiguous()
        rows = qs[:, g * group:(g + 1) * group].reshape(-1, cfg.head_dim)
        res = torch.empty_like(rows)
        for start in range(0, rows.shape[0], row_chunk):
            scores = rows[start:start + row_chunk] @ kg.T * cfg.softmax_scale
            res[start:start + row_chunk] = torch.softmax(scores, dim=-1) @ vg
        out[:, g * group:(g + 1) * group] = res.reshape(cfg.pcp_size, group, cfg.local_q_len, cfg.head_dim)
    return out
