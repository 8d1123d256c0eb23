"""The reference tests' known answers (tests/golden/reference_known_answers.json)
against the CPU oracle, and against the HIP path on the GPU."""

import json
import pathlib

import numpy as np
import pytest
import torch

from oracle.moe_ref import route
from oracle.token_rounding_ref import round_counts as round_counts_ref
from oracle.token_rounding_ref import token_rounding as token_rounding_ref
from oracle.topology_ref import build_layout, device_layout

G = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def hand_worked_scores() -> np.ndarray:
    s0 = np.asarray(G["token_rounding_hand_worked"]["scores_expert0"], dtype=np.float32)
    return np.stack([s0, np.float32(1) - s0], axis=1)


def kept_by_expert(token, expert) -> dict[str, list[int]]:
    out: dict[str, list[int]] = {}
    for t, e in zip(np.asarray(token).tolist(), np.asarray(expert).tolist()):
        out.setdefault(str(e), []).append(t)
    return {e: sorted(v) for e, v in out.items()}


# ---------------------------------------------------------------- oracle ---

def test_oracle_routing_bad_ids() -> None:
    c = G["routing_bad_ids"]
    lay = device_layout(np.asarray(c["expert_idx"]), c["num_experts"], c["ffn_dim"], c["block_size"])
    assert lay.copy_row.tolist() == c["expected_copy_row"]
    assert int(lay.tokens_per_expert.sum()) == c["expected_tokens_placed"]
    assert lay.error == c["expected_error"]


def test_oracle_exact_multiple() -> None:
    c = G["exact_multiple_no_padding"]
    lay = build_layout(np.asarray(c["expert_idx"]), c["num_experts"], c["ffn_dim"], c["block_size"])
    assert lay.num_rows == c["expected_num_rows"]
    assert int((lay.row_token < 0).sum()) == c["expected_padding_rows"]


def test_oracle_route() -> None:
    c = G["route_top2"]
    idx, w = route(torch.tensor(c["logits"]), k=c["k"])
    assert idx.tolist() == c["expected_idx"]
    torch.testing.assert_close(w.sum(-1), torch.ones(len(c["logits"])))


def test_oracle_round_counts_and_hand_worked_rounding() -> None:
    c = G["round_counts"]
    assert round_counts_ref(np.asarray(c["counts"]), c["tile"], c["max_count"]).tolist() == c["expected"]
    h = G["token_rounding_hand_worked"]
    a = token_rounding_ref(hand_worked_scores(), h["k"], h["tile"])
    assert kept_by_expert(a.token, a.expert) == h["expected_tokens_of_expert"]
    assert np.allclose(a.weight, h["expected_weight"])


# ------------------------------------------------------------------- GPU ---

@pytest.mark.gpu
def test_gpu_routing_bad_ids() -> None:
    from sparsebench_amd.routing import route_device

    c = G["routing_bad_ids"]
    dev = route_device(torch.tensor(c["expert_idx"]).cuda(), c["num_experts"], c["ffn_dim"], c["block_size"])
    assert dev.copy_row.tolist() == c["expected_copy_row"]
    assert int(dev.tokens_per_expert.sum()) == c["expected_tokens_placed"]
    assert int(dev.error) == c["expected_error"]
    with pytest.raises(ValueError, match="outside"):
        dev.to_topology()


@pytest.mark.gpu
def test_gpu_exact_multiple() -> None:
    from sparsebench_amd.routing import build_topology_cuda

    c = G["exact_multiple_no_padding"]
    topo = build_topology_cuda(torch.tensor(c["expert_idx"]).cuda(), c["num_experts"], c["ffn_dim"], c["block_size"])
    assert topo.num_rows == c["expected_num_rows"]
    assert int((topo.row_token < 0).sum()) == c["expected_padding_rows"]


@pytest.mark.gpu
def test_gpu_router_known_answers() -> None:
    from sparsebench_amd.token_rounding import token_rounding, top_k_assignments

    c = G["route_top2"]
    logits = torch.tensor(c["logits"])
    a = top_k_assignments(torch.softmax(logits, dim=-1).cuda(), c["k"])
    assert a.expert.view(-1, c["k"]).tolist() == c["expected_idx"]
    h = G["token_rounding_hand_worked"]
    r = token_rounding(torch.from_numpy(hand_worked_scores()).cuda(), h["k"], h["tile"])
    assert kept_by_expert(r.token.cpu(), r.expert.cpu()) == h["expected_tokens_of_expert"]
    assert torch.allclose(r.weight.cpu(), torch.full_like(r.weight.cpu(), h["expected_weight"]))
