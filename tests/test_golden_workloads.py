"""The input generators against the reference's own outputs
(tests/golden/reference_workloads.json, written from the reference's
sparsebench/workloads.py by tests/golden/make_workloads_vectors.py): every
routing case and router score the benchmarks and tests draw must be the
reference's, bit for bit, so both sides run on identical inputs.
"""
from __future__ import annotations

import json
import pathlib

import pytest
import torch

from sparsebench_amd.workloads import router_scores, routing_case

G = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_workloads.json").read_text())


@pytest.mark.parametrize("case", G["routing_case"], ids=lambda c: f"{c['name']}-{c['num_tokens']}x{c['num_experts']}")
def test_routing_case_matches_the_reference(case) -> None:
    got = routing_case(case["name"], case["num_tokens"], case["num_experts"], case["seed"])
    assert got.dtype == torch.int64
    assert got.tolist() == case["expert_idx"]


@pytest.mark.parametrize("case", G["router_scores"], ids=lambda c: f"{c['name']}-{c['num_tokens']}x{c['num_experts']}")
def test_router_scores_match_the_reference_bit_for_bit(case) -> None:
    got = router_scores(case["name"], case["num_tokens"], case["num_experts"], case["seed"])
    assert got.dtype == torch.float32
    assert got.contiguous().view(torch.int32).reshape(-1).tolist() == case["fp32_bits"]


def test_fixture_covers_every_reference_routing_name() -> None:
    assert {c["name"] for c in G["routing_case"]} == {"random", "skewed", "two_experts_only", "empty_middle", "zipf"}
