"""Writes input_hashes.json: SHA-256 of the synthetic inputs this repository
draws for two workloads (the reference's draw order: one seeded CPU
generator, Q then K then V).  A drift detector for torch's CPU generator and
the input code, not a pin of the reference (which holds no golden files).

    python tests/golden/make_input_hashes.py
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

CASES = [("tiny-gqa4-d64-bf16", 1234), ("four-chip-fp8", 1234)]


def digests(name: str, seed: int) -> dict:
    import torch

    from aws_training_study_amd.pcp_attention.workloads import build_workload_problem

    problem = build_workload_problem(name, seed)
    tensors = {"q": problem.inputs.q, "k": problem.inputs.k, "v": problem.inputs.v,
               "block_table": problem.block_table, "page_valid_len": problem.page_valid_len}
    out = {}
    for key, t in tensors.items():
        raw = t.contiguous().view(torch.uint8)
        out[key] = {"shape": list(t.shape), "dtype": str(t.dtype).replace("torch.", ""),
                    "sha256": hashlib.sha256(raw.numpy().tobytes()).hexdigest()}
    out["k_scale"] = float(problem.k_scale)
    out["v_scale"] = float(problem.v_scale)
    return out


def main() -> None:
    import torch

    data = {"torch": torch.__version__.split("+")[0],
            "cases": {f"{n}/{s}": digests(n, s) for n, s in CASES}}
    (HERE / "input_hashes.json").write_text(json.dumps(data, indent=1) + "\n")


if __name__ == "__main__":
    main()
