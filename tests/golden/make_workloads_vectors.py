"""Writes tests/golden/reference_workloads.json: outputs of the reference's
input generators (sparsebench/workloads.py:12-36 routing_case, 39-52
router_scores) on small seeded cases, as data.

Run in a container that holds the reference checkout (not on the GPU box, and
not by the test suite, which reads only the JSON this writes):

    python tests/golden/make_workloads_vectors.py /path/to/reference

The reference module is loaded from its file (it imports only torch), so
neither its package nor this repository's `sparsebench` shim is imported.
Integer picks are stored as lists; fp32 scores as their IEEE-754 bit
patterns, so the comparison is exact.
"""
from __future__ import annotations

import importlib.util
import json
import pathlib
import sys

import torch

CASES = [  # (num_tokens, num_experts, seed)
    (7, 5, 0),
    (64, 16, 3),
    (33, 130, 11),
]
SCORE_CASES = [(6, 5, 0), (17, 64, 4)]


def main(reference: str) -> None:
    path = pathlib.Path(reference) / "sparsebench" / "workloads.py"
    spec = importlib.util.spec_from_file_location("reference_workloads", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out: dict = {
        "about": ("Outputs of the reference's input generators (saransh-debugs/SparseBench "
                  "sparsebench/workloads.py: routing_case 12-36, router_scores 39-52) on small seeded cases, "
                  "written by tests/golden/make_workloads_vectors.py. Scores are fp32 bit patterns."),
        "torch": torch.__version__,
        "routing_case": [],
        "router_scores": [],
    }
    for name in mod.CASE_NAMES:
        for t, e, seed in CASES:
            idx = mod.routing_case(name, t, e, seed)
            out["routing_case"].append({"name": name, "num_tokens": t, "num_experts": e, "seed": seed,
                                        "expert_idx": idx.tolist()})
    for name in ("uniform", "zipf"):
        for t, e, seed in SCORE_CASES:
            s = mod.router_scores(name, t, e, seed).contiguous()
            bits = s.view(torch.int32).reshape(-1).tolist()
            out["router_scores"].append({"name": name, "num_tokens": t, "num_experts": e, "seed": seed,
                                         "fp32_bits": bits})
    dst = pathlib.Path(__file__).with_name("reference_workloads.json")
    dst.write_text(json.dumps(out, separators=(",", ":")) + "\n")
    print("wrote", dst, dst.stat().st_size, "bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
