"""Build the gfx950 HIP library in-tree with hipcc.

``python -m aws_training_study_amd.build_native`` compiles
``csrc/pcp_attention_hip.hip`` (which includes the kernel headers in
``csrc/``) into ``_lib/libpcp_attention_hip.so``.  hipcc cross-compiles for
gfx950 without a GPU present.  Then gcc builds ``csrc/abi_example.c``, a
plain C caller of the library, into ``_lib/abi_example``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
SOURCES = [PACKAGE_DIR / "csrc" / "pcp_attention_hip.hip"]
INCLUDE_DIR = REPO_ROOT / "include"
OUTPUT = PACKAGE_DIR / "_lib" / "libpcp_attention_hip.so"
EXAMPLE_SOURCE = PACKAGE_DIR / "csrc" / "abi_example.c"
EXAMPLE = PACKAGE_DIR / "_lib" / "abi_example"
OFFLOAD_ARCH = "gfx950"

# Packed FP32 VALU forms are disabled for all device code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.exists():
        return os.fspath(candidate)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build the HIP library")
    return found


def compile_command(output: Path = OUTPUT) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={OFFLOAD_ARCH}",
        "-O3",
        "-std=c++17",
        "-shared",
        "-fPIC",
        f"-I{INCLUDE_DIR}",
        *DEVICE_FLAGS,
        *[os.fspath(s) for s in SOURCES],
        "-o",
        os.fspath(output),
    ]


def example_command(output: Path = EXAMPLE) -> list[str]:
    """gcc line of the C caller: the header, the HIP runtime's C API, the
    library beside it (rpath $ORIGIN)."""
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return [
        "gcc",
        "-O2",
        "-std=c11",
        "-Wall",
        "-Werror",
        "-D__HIP_PLATFORM_AMD__",
        f"-I{INCLUDE_DIR}",
        f"-I{rocm}/include",
        os.fspath(EXAMPLE_SOURCE),
        f"-L{OUTPUT.parent}",
        "-lpcp_attention_hip",
        f"-L{rocm}/lib",
        "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{rocm}/lib",
        "-o",
        os.fspath(output),
    ]


def build_example(verbose: bool = False) -> Path:
    """Compile the C caller against the built library."""
    cmd = example_command()
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"gcc failed ({result.returncode}):\n{result.stderr}")
    return EXAMPLE


def build(verbose: bool = False) -> Path:
    """Compile the library; always recompiles. Returns the output path."""
    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = compile_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{stderr}")
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)
    os.replace(tmp, OUTPUT)
    build_example(verbose)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
