"""Committed fixtures under tests/golden: the hand-worked owner table and
the SHA-256 drift detector of this repository's synthetic inputs."""

from __future__ import annotations

import importlib.util
import json
from pathlib import Path

import pytest
import torch

from aws_training_study_amd.pcp_attention.layout import global_positions_for_rank, owner_and_local_position
from oracle import pcp_oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_owner_table_fixture():
    t = json.loads((GOLDEN / "owner_pcp3_il2.json").read_text())
    pcp, il = t["pcp_size"], t["interleave_size"]
    for p, (owner, local) in enumerate(zip(t["owners"], t["locals"])):
        assert owner_and_local_position(p, pcp, il) == (owner, local)
        assert orc.owner_and_local_position(p, pcp, il) == (owner, local)
    for rank, positions in t["rank_positions_total_12"].items():
        assert global_positions_for_rank(12, int(rank), pcp, il).tolist() == positions
        assert orc.global_positions(12, int(rank), pcp, il).tolist() == positions


def test_input_hashes_fixture():
    data = json.loads((GOLDEN / "input_hashes.json").read_text())
    if torch.__version__.split("+")[0] != data["torch"]:
        pytest.skip(f"fixture written with torch {data['torch']}; the CPU generator may differ")
    spec = importlib.util.spec_from_file_location("make_input_hashes", GOLDEN / "make_input_hashes.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    for key, expected in data["cases"].items():
        name, seed = key.rsplit("/", 1)
        assert mod.digests(name, int(seed)) == expected, f"synthetic inputs of {key} changed"
