"""Properties of the compiled gfx950 device code (CPU only: hipcc cross-compiles).

* No attention kernel spills to scratch, except the BF16 head_dim-256 tile
  kernels (eight waves in key-split pairs, 256 registers a wave), whose few
  spills (values the epilogue needs from the prologue) must stay outside
  every loop: a Q fragment reloaded from scratch inside the walk cost 30% on
  the MI355X (8.87 against 6.8 ms on the full 64-rank workload; the reload's
  vmcnt wait also waits for every LDS-DMA in flight).
* No LDS read writes a register that an MFMA issued before it is still
  going to write.  The transposing V reads and the score-operand reads are
  inline asm, invisible to the compiler's hazard checks; the kernels keep
  every MFMA result allocated until it is read (an empty asm tie), and this
  scan of the assembly checks that no read lands in a pending destination
  (the failure once gave NaN outputs).
* m0 belongs to the LDS-DMA helpers alone.  Their inline asm writes m0 (the
  LDS destination of global_load_lds_dwordx4) and lists it as clobbered; the
  compiler treats m0 as reserved and does not save a value of its own across
  the asm (it warns).  That is only safe while no code the compiler
  generates uses m0: in every kernel, each instruction naming m0 must be the
  helper's `s_mov_b32 m0, s<n>` directly followed by `s_nop 0` and the
  `global_load_lds_dwordx4` it feeds, every LDS-DMA must be preceded by that
  pair, and no instruction that reads m0 implicitly (LDS-DMA of another
  form, relative moves, messages, GWS / append / consume, LDS-direct or
  parameter loads) may appear.
"""

from __future__ import annotations

import os
import re
import subprocess

import pytest

from aws_training_study_amd import build_native

ATTENTION = re.compile(r"history_fwd_(kernel|overlap)")


@pytest.fixture(scope="module")
def device_code(tmp_path_factory):
    out = tmp_path_factory.mktemp("devcode") / "pcpa.s"
    cmd = [build_native.hipcc(), f"--offload-arch={build_native.OFFLOAD_ARCH}", "-O3", "-std=c++17",
           f"-I{build_native.INCLUDE_DIR}", *build_native.DEVICE_FLAGS, "--cuda-device-only", "-S",
           "-Rpass-analysis=kernel-resource-usage", *[os.fspath(s) for s in build_native.SOURCES], "-o",
           os.fspath(out)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    assert result.returncode == 0, result.stderr[-2000:]
    usage, current = {}, None
    for line in result.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            current = usage.setdefault(m.group(1), {})
            continue
        m = re.search(r"remark:\s+([A-Za-z ]+?)(?: \[[^\]]*\])?: (\d+) \[", line)
        if m and current is not None:
            current[m.group(1).strip()] = int(m.group(2))
    asm = out.read_text()
    bodies = {}
    for m in re.finditer(r"^(_Z\S+):", asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        bodies[m.group(1)] = asm[m.end():end].splitlines()
    return usage, bodies


def _attention_kernels(usage):
    names = [n for n in usage if ATTENTION.search(n)]
    assert len(names) >= 20, names  # every instantiation the C ABI launches
    return names


def _is_pair_tile(name):
    # history_fwd_kernel<256, STORE8, FP8 = false, ...>: the key-split pair mode
    return re.search(r"history_fwd_kernelILi256ELb[01]ELb0E", name) is not None


def _is_split_overlap(name):
    # history_fwd_overlap<D, FAST, LSE, SPLIT = true>
    return "history_fwd_overlap" in name and name.endswith("ELb1EEEvNS_7FwdArgsE")


def _scratch_ops(lines):
    """(scratch instructions, of which inside a loop) per the assembler's loop comments."""
    in_loop, total, looped = False, 0, 0
    for line in lines:
        if line.startswith(".LBB") or line.startswith("; %bb"):
            in_loop = "in Loop" in line or "Loop Header" in line
        if re.match(r"\s*scratch_", line):
            total += 1
            looped += in_loop
    return total, looped


def test_attention_kernels_do_not_spill(device_code):
    usage, _ = device_code
    split = [n for n in _attention_kernels(usage) if _is_split_overlap(n)]
    assert len(split) == 2, split  # the split instantiations (fast and exact exp2) are covered too
    pair = [n for n in _attention_kernels(usage) if _is_pair_tile(n)]
    assert len(pair) == 6, pair  # BF16 and widened caches: one pass, split, guard fixup, current step
    for name in _attention_kernels(usage):
        limit = 128 if _is_pair_tile(name) else 0
        assert 0 <= usage[name].get("ScratchSize", -1) <= limit, (name, usage[name])
        assert usage[name].get("SGPRs Spill", -1) == 0, (name, usage[name])
        if not limit:
            assert usage[name].get("VGPRs Spill", -1) == 0, (name, usage[name])


def test_no_scratch_access_inside_any_loop(device_code):
    usage, bodies = device_code
    for name in _attention_kernels(usage):
        total, looped = _scratch_ops(bodies[name])
        assert looped == 0, f"{name}: {looped} of {total} scratch accesses inside a loop"


def _regs(token):
    """Vector or accumulation registers a token names, as (file, index) pairs."""
    m = re.match(r"([va])\[(\d+):(\d+)\]", token)
    if m:
        return {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", token)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _pending_destination_reads(lines):
    """LDS reads whose destination overlaps an MFMA destination not yet read.

    Straight-line scan: an MFMA's destination is pending from its issue until
    a non-LDS-read instruction names one of its registers (the first reader
    or writer waits for the result), or control flow (label or branch)."""
    found = []
    code = [l.strip() for l in lines if l.strip() and not l.strip().startswith(";")]
    for i, line in enumerate(code):
        if not line.startswith("v_mfma"):
            continue
        dst = _regs(line.split(None, 1)[1].split(",")[0].strip())
        for later in code[i + 1:i + 400]:
            if later.startswith((".LBB", "s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
                break
            if later.startswith("ds_read"):
                if _regs(later.split(None, 1)[1].split(",")[0].strip()) & dst:
                    found.append((line, later))
                continue
            if any(_regs(t) & dst for t in re.findall(r"[va]\[\d+:\d+\]|[va]\d+", later)):
                break
    return found


def test_no_lds_read_into_a_pending_mfma_destination(device_code):
    usage, bodies = device_code
    for name in _attention_kernels(usage):
        hits = _pending_destination_reads(bodies[name])
        assert not hits, f"{name}: {hits[:3]}"


def test_the_scan_finds_a_planted_hazard():
    """The scan itself: an LDS read into the destination of an MFMA whose
    result nothing has read yet is reported; after a reader it is not."""
    planted = ["v_mfma_f32_32x32x64_f8f6f4 v[16:31], v[0:7], v[8:15], 0",
               "ds_read_b64_tr_b8 v[20:21], v40 offset:0"]
    assert _pending_destination_reads(planted)
    safe = ["v_mfma_f32_32x32x64_f8f6f4 v[16:31], v[0:7], v[8:15], 0",
            "v_add_f32_e32 v50, v16, v17",
            "ds_read_b64_tr_b8 v[20:21], v40 offset:0"]
    assert not _pending_destination_reads(safe)


# Instructions that read m0 without naming it (gfx9 ISA): LDS-DMA loads,
# relative register moves, messages, GWS / append / consume, LDS-direct and
# interpolation loads.
_IMPLICIT_M0 = re.compile(r"^(buffer_load\S*\s.*\blds\b|global_load_lds\S*|s_movrel\S*|v_movrel\S*|s_sendmsg\S*|"
                          r"ds_gws\S*|ds_append|ds_consume|ds_read_addtid\S*|ds_write_addtid\S*|"
                          r"v_interp\S*|lds_direct\S*|lds_param\S*)")


def _m0_misuse(lines):
    """Instructions that break the m0 rule above, with the reason."""
    code = [l.strip() for l in lines if l.strip() and not l.strip().startswith((";", "."))]
    found = []
    helper_loads = set()
    for i, line in enumerate(code):
        names_m0 = re.search(r"\bm0\b", line) is not None
        if names_m0:
            if not re.fullmatch(r"s_mov_b32 m0, s\d+", line):
                found.append(("m0 named outside the helper", line))
                continue
            if code[i + 1:i + 2] != ["s_nop 0"] or not code[i + 2].startswith("global_load_lds_dwordx4"):
                found.append(("m0 write not followed by s_nop 0 and its LDS-DMA", line))
                continue
            helper_loads.add(i + 2)
    for i, line in enumerate(code):
        if _IMPLICIT_M0.match(line) and i not in helper_loads:
            found.append(("implicit m0 reader outside the helper", line))
    return found


def test_m0_is_written_and_read_only_by_the_lds_dma_helpers(device_code):
    _, bodies = device_code
    dma = 0
    for name, lines in bodies.items():
        hits = _m0_misuse(lines)
        assert not hits, f"{name}: {hits[:3]}"
        dma += sum(1 for l in lines if l.strip().startswith("global_load_lds_dwordx4"))
    assert dma > 0  # the kernels do use the helpers


def test_the_m0_scan_finds_planted_misuse():
    good = ["s_mov_b32 m0, s12", "s_nop 0", "global_load_lds_dwordx4 v3, s[4:5] offset:1024"]
    assert not _m0_misuse(good)
    assert not _m0_misuse(good + ["buffer_load_dword v1, off, s[0:3], 0"])  # no lds: no m0
    # a compiler-made m0 value, an LDS-DMA without the helper's write, a
    # relative move and an append that read m0 implicitly
    for planted in (["s_mov_b32 m0, -1"] + good,
                    good + ["s_add_u32 m0, s1, 0x400"],
                    good + ["global_load_lds_dwordx4 v3, s[4:5] offset:2048"],
                    good + ["s_movrels_b32 s0, s8"],
                    good + ["ds_append v1 offset:4"],
                    good + ["buffer_load_dword v1, off, s[0:3], 0 lds"],
                    ["s_mov_b32 m0, s12", "v_add_f32_e32 v1, v2, v3", "global_load_lds_dwordx4 v3, s[4:5]"]):
        assert _m0_misuse(planted), planted
