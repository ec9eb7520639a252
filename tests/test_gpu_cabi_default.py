"""The drop-in C entry points with flags = 0 on an e4m3 cache meet the bar.

``pcpa_history_attention`` and ``pcpa_history_attention_lse`` are what a
reference-side binding calls in place of kernel.py:32-556.  With no flag
set, an e4m3 cache runs e4m3 MFMAs with the precision guard, its buffers in
the library's guard scratch.  Called through ctypes and through the plain C
caller (csrc/abi_example.c), on the two kinds of data where unguarded e4m3
MFMAs miss max-abs 2e-2 / mean-abs 2e-3 against float64 attention:

* the 64-rank, 131072-token bucket with a 785-token runtime history;
* 8192 keys with a per-channel K factor in [0.5, 2] and Q scaled x3.

Their output also equals the Python wrapper's guarded call (same kernels,
workspace of its own) bit for bit, and two guarded calls queued on two
streams at once give the results they give one after the other (the library
orders the calls that share its guard scratch).
"""

from __future__ import annotations

import ctypes
import subprocess
from dataclasses import replace

import numpy as np
import pytest
import torch

from aws_training_study_amd import _native
from aws_training_study_amd.build_native import EXAMPLE
from aws_training_study_amd.pcp_attention import make_history_attention_kernel
from aws_training_study_amd.pcp_attention.paging import page_valid_lengths

from test_gpu_guard import FOUR, FULL, _check_bar, _paged_reference, _pick, _problem, _sample, _scaled_q

pytestmark = pytest.mark.gpu


def _case(name):
    """(problem, Q, page_valid_len on the host) of a named case."""
    if name == "full-bucket-785":
        problem = _problem(FULL, "none", 41)
        return problem, problem.q_stacked, page_valid_lengths(replace(FULL, actual_history_len=785))
    cfg = replace(FOUR, actual_history_len=8192).validate()
    problem = _problem(cfg, "per_channel", 43)
    return problem, _scaled_q(problem, 3), problem.page_valid_len


CASES = ["full-bucket-785", "8k-per-channel-q3"]


def _plain_call(lib, params, gpu_args, out, lse, stream):
    q, kv, table, lens = gpu_args
    if lse is None:
        return lib.pcpa_history_attention(ctypes.byref(params), q.data_ptr(), kv.data_ptr(), table.data_ptr(),
                                          lens.data_ptr(), out.data_ptr(), stream)
    return lib.pcpa_history_attention_lse(ctypes.byref(params), q.data_ptr(), kv.data_ptr(), table.data_ptr(),
                                          lens.data_ptr(), out.data_ptr(), lse.data_ptr(), stream)


@pytest.mark.parametrize("name", CASES)
def test_default_flags_meet_the_bar_through_ctypes(name, cuda_device):
    problem, q, lens = _case(name)
    cfg = problem.config
    lib = _native.load_library()
    kernel = make_history_attention_kernel(cfg)
    params = kernel._params(problem.kv_pages.shape[0], problem.k_scale, problem.v_scale)
    assert params.flags == 0
    gpu = problem.to(cuda_device)
    args = (q.to(cuda_device), gpu.kv_pages, gpu.block_table, lens.to(device=cuda_device, dtype=torch.int32))
    stream = torch.cuda.current_stream(cuda_device).cuda_stream
    out = torch.full_like(args[0], float("nan"))
    out_l = torch.full_like(args[0], float("nan"))
    lse = torch.full(args[0].shape[:3], float("nan"), dtype=torch.float32, device=cuda_device)
    print(f"case {name}: pcpa_history_attention, pcpa_history_attention_lse (flags 0)", flush=True)
    _native.check(_plain_call(lib, params, args, out, None, stream))
    _native.check(_plain_call(lib, params, args, out_l, lse, stream))
    py_out, py_lse = kernel(args[0], gpu.kv_pages, gpu.block_table, page_valid_len=args[3], k_scale=problem.k_scale,
                            v_scale=problem.v_scale, splits=1, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out_l)
    assert torch.equal(out, py_out) and torch.equal(lse, py_lse)
    rows = _sample(cfg, 192, 7)
    ref = _paged_reference(problem, q, rows, lens)
    _check_bar(_pick(out, rows), ref, f"{name} pcpa_history_attention flags 0")


def test_guard_scratch_calls_on_two_streams_are_ordered(cuda_device):
    """Both cases queued on two streams without waiting: each result equals
    the one it gives alone (the second call's kernels would otherwise rewrite
    the first call's row flags, lists and partials in the shared scratch)."""
    lib = _native.load_library()
    runs = []
    for name in CASES:
        problem, q, lens = _case(name)
        kernel = make_history_attention_kernel(problem.config)
        params = kernel._params(problem.kv_pages.shape[0], problem.k_scale, problem.v_scale)
        gpu = problem.to(cuda_device)
        args = (q.to(cuda_device), gpu.kv_pages, gpu.block_table, lens.to(device=cuda_device, dtype=torch.int32))
        runs.append((params, args))
    alone = []
    stream = torch.cuda.current_stream(cuda_device).cuda_stream
    for params, args in runs:
        out = torch.empty_like(args[0])
        _native.check(_plain_call(lib, params, args, out, None, stream))
        alone.append(out)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(cuda_device), torch.cuda.Stream(cuda_device)]
    outs = [torch.empty_like(args[0]) for _, args in runs]
    torch.cuda.synchronize()
    print("case two streams, guard scratch shared", flush=True)
    for rep in range(3):
        for (params, args), out, s in zip(runs, outs, streams):
            _native.check(_plain_call(lib, params, args, out, None, s.cuda_stream))
        torch.cuda.synchronize()
        for got, want in zip(outs, alone):
            assert torch.equal(got, want), f"repetition {rep}"


@pytest.mark.parametrize("name", CASES)
def test_default_flags_meet_the_bar_through_the_c_caller(name, tmp_path, cuda_device):
    """csrc/abi_example.c fills pcpa_params with flags 0, copies the tensors
    itself and calls pcpa_history_attention_lse."""
    if not EXAMPLE.exists():
        pytest.fail("abi_example is not built; run __graft_entry__.build()")
    problem, q, lens = _case(name)
    cfg = problem.config
    kernel = make_history_attention_kernel(cfg)
    params = kernel._params(problem.kv_pages.shape[0], problem.k_scale, problem.v_scale)
    (tmp_path / "params.bin").write_bytes(bytes(params))
    (tmp_path / "q.bin").write_bytes(q.contiguous().view(torch.int16).numpy().tobytes())
    (tmp_path / "kv.bin").write_bytes(problem.kv_pages.contiguous().view(torch.uint8).numpy().tobytes())
    (tmp_path / "table.bin").write_bytes(problem.block_table.to(torch.int32).contiguous().numpy().tobytes())
    (tmp_path / "lens.bin").write_bytes(lens.to(torch.int32).contiguous().numpy().tobytes())
    print(f"case {name}: abi_example run (flags 0)", flush=True)
    res = subprocess.run([str(EXAMPLE), "run", str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(res.stdout.strip(), flush=True)
    assert res.returncode == 0, res.stderr + res.stdout
    shape = (cfg.pcp_size, cfg.num_q_heads, cfg.local_q_len, cfg.head_dim)
    out_c = torch.from_numpy(np.frombuffer((tmp_path / "out.bin").read_bytes(), dtype=np.int16).reshape(shape).copy())
    out_c = out_c.view(torch.bfloat16)
    gpu = problem.to(cuda_device)
    py_out = kernel(q.to(cuda_device), gpu.kv_pages, gpu.block_table,
                    page_valid_len=lens.to(device=cuda_device, dtype=torch.int32), k_scale=problem.k_scale,
                    v_scale=problem.v_scale, splits=1)
    torch.cuda.synchronize()
    assert torch.equal(out_c, py_out.cpu()), "C caller and Python outputs differ"
    rows = _sample(cfg, 192, 8)
    _check_bar(_pick(out_c, rows), _paged_reference(problem, q, rows, lens), f"{name} abi_example flags 0")
