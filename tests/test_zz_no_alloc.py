"""pcpa_history_attention_noalloc: the workspace-taking history entry point
with its workspace in the library's fixed device scratch.

Called through the C ABI, it must give pcpa_history_attention_split's output
and log-sum-exp bit for bit (same kernels, same inputs) on two calls in a
row, the second with a smaller input, and reject a launch that needs more
than PCPA_NOALLOC_SCRATCH_BYTES.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from aws_training_study_amd import _native
from aws_training_study_amd.pcp_attention import make_history_attention_kernel
from aws_training_study_amd.pcp_attention.config import PCPAttentionConfig
from aws_training_study_amd.pcp_attention.workloads import build_paged_problem, build_workload_problem

pytestmark = pytest.mark.gpu


def _params(kernel, problem, flags):
    params = kernel._params(problem.kv_pages.shape[0], problem.k_scale, problem.v_scale)
    params.flags = flags
    return params


def _both(problem, flags, splits, device):
    """(split entry point's out, lse), (no-alloc entry point's out, lse)."""
    lib = _native.load_library()
    kernel = make_history_attention_kernel(problem.config)
    gpu = problem.to(device)
    params = _params(kernel, problem, flags)
    need = lib.pcpa_split_workspace_bytes(ctypes.byref(params), splits)
    assert 0 < need <= _native.NOALLOC_SCRATCH_BYTES
    stream = torch.cuda.current_stream(device).cuda_stream
    results = []
    for noalloc in (False, True):
        out = torch.full_like(gpu.q_stacked, float("nan"))
        lse = torch.full(gpu.q_stacked.shape[:3], float("nan"), dtype=torch.float32, device=device)
        args = (gpu.q_stacked.data_ptr(), gpu.kv_pages.data_ptr(), gpu.block_table.data_ptr(),
                gpu.page_valid_len.data_ptr(), out.data_ptr(), lse.data_ptr())
        if noalloc:
            status = lib.pcpa_history_attention_noalloc(ctypes.byref(params), splits, *args, stream)
        else:
            ws = torch.empty(need, dtype=torch.uint8, device=device)
            status = lib.pcpa_history_attention_split(ctypes.byref(params), splits, *args, ws.data_ptr(), need, stream)
        _native.check(status)
        torch.cuda.synchronize()
        results.append((out, lse))
    return results


def test_noalloc_equals_the_workspace_entry_point_on_a_large_then_a_smaller_launch(cuda_device):
    # 1) 16 ranks, 8192-token e4m3 history, 2 history splits, flags 0 (e4m3
    # MFMAs with the precision guard): 34 MB of fp16 partials and 34 MB of
    # the guard's fixup partials
    big = build_workload_problem("four-chip-fp8", seed=61)
    print("case four-chip-fp8, e4m3 MFMAs with the guard, 2 splits", flush=True)
    (ref_out, ref_lse), (out, lse) = _both(big, 0, 2, cuda_device)
    assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)
    assert not torch.isnan(out.float()).any()
    # 2) a smaller launch after it: 4 ranks, D=128, guarded, 3 splits (the
    # scratch keeps the first call's contents; nothing of it may leak in)
    cfg = PCPAttentionConfig(pcp_size=4, current_len=256, max_history_len=4096, actual_history_len=3000,
                             block_size=256, interleave_size=64, num_q_heads=16, num_kv_heads=2, head_dim=128,
                             backend="hip").validate()
    small = build_paged_problem(cfg, seed=62, kv_scale="per_tensor")
    print("case 4 ranks D=128, guard, 3 splits", flush=True)
    (ref_out, ref_lse), (out, lse) = _both(small, _native.FLAG_PRECISION_GUARD, 3, cuda_device)
    assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)
    assert not torch.isnan(out.float()).any()


def test_noalloc_rejects_a_launch_beyond_its_scratch(cuda_device):
    """16 ranks with 8 splits and the guard: more than the fixed scratch."""
    problem = build_workload_problem("four-chip-fp8", seed=63)
    lib = _native.load_library()
    kernel = make_history_attention_kernel(problem.config)
    params = _params(kernel, problem, _native.FLAG_PRECISION_GUARD)
    assert lib.pcpa_split_workspace_bytes(ctypes.byref(params), 8) > _native.NOALLOC_SCRATCH_BYTES
    gpu = problem.to(cuda_device)
    out = torch.empty_like(gpu.q_stacked)
    status = lib.pcpa_history_attention_noalloc(
        ctypes.byref(params), 8, gpu.q_stacked.data_ptr(), gpu.kv_pages.data_ptr(), gpu.block_table.data_ptr(),
        gpu.page_valid_len.data_ptr(), out.data_ptr(), None, torch.cuda.current_stream(cuda_device).cuda_stream)
    assert status == -11  # PCPA_ERR_SCRATCH, before any launch
