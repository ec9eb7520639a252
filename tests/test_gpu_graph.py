"""HIP-graph launch path: a captured call replays to the eager call's bits.

Each case replays the graph several times with eager work and
synchronisations in between, checks every replay against the eager result,
then changes the inputs in place and checks again.
"""

from __future__ import annotations

import pytest
import torch

from aws_training_study_amd.pcp_attention import (
    PrefillAttention,
    make_history_attention_kernel,
    stack_current_kv,
)
from aws_training_study_amd.pcp_attention.workloads import build_workload_problem

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["tiny-gqa4-d64-bf16", "four-chip-fp8"])
def test_graphed_history_replays_exactly(name, cuda_device):
    problem = build_workload_problem(name, seed=41)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(problem.config)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale)
    q = gpu.q_stacked.clone()
    graphed = kernel.graphed(q, gpu.kv_pages, gpu.block_table, **kw)
    print(f"case {name}: splits={kernel.split_count(cuda_device, kernel.uses_bf16_mfma())}", flush=True)
    eager = kernel(q, gpu.kv_pages, gpu.block_table, **kw)
    scratch = torch.randn(1 << 20, device=cuda_device)
    for i in range(3):
        out = graphed.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager call"
        scratch.mul_(1.0001).add_(1.0)  # eager work between replays
        torch.cuda.synchronize()
    q.copy_(torch.flip(gpu.q_stacked, dims=[2]))  # new inputs, same tensor
    eager2 = kernel(q, gpu.kv_pages, gpu.block_table, **kw)
    out = graphed.replay()
    torch.cuda.synchronize()
    assert not torch.equal(eager2, eager)
    assert torch.equal(out, eager2)


def test_graphed_prefill_replays_exactly(cuda_device):
    problem = build_workload_problem("four-chip-fp8", seed=42)
    cfg = problem.config
    gpu = problem.to(cuda_device)
    g = torch.Generator().manual_seed(43)
    shape = (cfg.num_kv_heads, cfg.current_len, cfg.head_dim)
    kv_cur = stack_current_kv(torch.randn(shape, generator=g).bfloat16(), torch.randn(shape, generator=g).bfloat16())
    kv_cur = kv_cur.to(cuda_device)
    prefill = PrefillAttention(cfg)
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale)
    graphed = prefill.graphed(gpu.q_stacked, gpu.kv_pages, gpu.block_table, kv_cur, **kw)
    eager = prefill(gpu.q_stacked, gpu.kv_pages, gpu.block_table, kv_cur, **kw)
    for i in range(3):
        out = graphed.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"prefill replay {i} differs from the eager call"


def test_graph_keeps_its_split_workspace(cuda_device):
    """A split graph holds its own workspace: eager calls that grow or use the
    kernel's kept workspace in between leave its replays unchanged."""
    problem = build_workload_problem("four-chip-fp8", seed=44)
    gpu = problem.to(cuda_device)
    kernel = make_history_attention_kernel(problem.config)
    n_split = kernel.split_count(cuda_device, kernel.uses_bf16_mfma())
    print(f"case four-chip-fp8: auto splits={n_split}", flush=True)
    assert n_split > 1
    kw = dict(page_valid_len=gpu.page_valid_len, k_scale=problem.k_scale, v_scale=problem.v_scale)
    graphed = kernel.graphed(gpu.q_stacked, gpu.kv_pages, gpu.block_table, **kw)
    eager = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, **kw)
    # more splits: the kept workspace is replaced by a larger one
    wider = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, splits=2 * n_split, **kw)
    out = graphed.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    assert (wider.float() - eager.float()).abs().max().item() < 2e-2  # same attention, another split
    # a caller-provided workspace gives the kept one's bits
    ws = torch.empty(kernel.workspace_bytes(n_split), dtype=torch.uint8, device=cuda_device)
    own = kernel(gpu.q_stacked, gpu.kv_pages, gpu.block_table, workspace=ws, **kw)
    torch.cuda.synchronize()
    assert torch.equal(own, eager)
