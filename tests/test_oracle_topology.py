"""Pins the layout oracle (oracle/topology_ref.py) before anything is checked against it.

- a hand-worked known answer, and the reference's own known answers
  (tests/test_topology.py:61-66, tests/test_routing.py:111-120 in the reference)
- agreement with an independent brute-force construction on small inputs
- the layout invariants of the reference's tests/test_topology.py:8-45
- the worst-case / past-the-end conventions of csrc/routing.cu:162-193, 248-249
- the golden vectors under tests/golden/
"""

import numpy as np
import pytest

from oracle.topology_ref import brute_force_layout, build_layout, device_layout, worst_case_sizes
from sparsebench_amd.workloads import CASE_NAMES, routing_case

FIELDS = ("tokens_per_expert", "padded_offsets", "row_token", "copy_row", "row_block_expert", "row_offsets",
          "col_indices")


def assert_same(a, b) -> None:
    for f in FIELDS:
        x, y = getattr(a, f), getattr(b, f)
        assert x.dtype == np.int32 and y.dtype == np.int32, f
        np.testing.assert_array_equal(x, y, err_msg=f)


def check_invariants(lay, expert_idx: np.ndarray) -> None:
    bs, num_experts = lay.block_size, lay.num_experts
    num_tokens, k = expert_idx.shape
    flat = expert_idx.reshape(-1).astype(np.int64)
    counts = lay.tokens_per_expert.astype(np.int64)
    offsets = lay.padded_offsets.astype(np.int64)
    row_token = lay.row_token.astype(np.int64)
    copy_row = lay.copy_row.astype(np.int64)
    np.testing.assert_array_equal(counts, np.bincount(flat, minlength=num_experts))
    sizes = np.diff(offsets)
    assert offsets[0] == 0
    assert np.all(sizes % bs == 0) and np.all(sizes >= counts) and np.all(sizes - counts < bs)
    assert np.all(sizes[counts == 0] == 0)
    assert np.unique(copy_row).size == num_tokens * k
    assert np.all(copy_row >= offsets[flat]) and np.all(copy_row < offsets[flat] + counts[flat])
    np.testing.assert_array_equal(row_token[copy_row], np.arange(num_tokens * k) // k)
    assert int((row_token < 0).sum()) == lay.num_rows - num_tokens * k
    for e in range(num_experts):  # stable: rows follow copy order inside an expert
        rows = copy_row[flat == e]
        assert np.all(rows[1:] > rows[:-1])
    rbe = lay.row_block_expert.astype(np.int64)
    starts = np.arange(rbe.size) * bs
    assert np.all(starts >= offsets[rbe]) and np.all(starts + bs <= offsets[rbe + 1])
    assert np.all(np.diff(lay.row_offsets) == lay.ffn_blocks)
    cols = lay.col_indices.reshape(rbe.size, lay.ffn_blocks)
    np.testing.assert_array_equal(cols, rbe[:, None] * lay.ffn_blocks + np.arange(lay.ffn_blocks))


def test_hand_worked_example() -> None:
    # copies c = t*2 + j: [1, 0, 1, 2, 0, 1]; block size 2, 4 experts, F = 8 (4 column blocks)
    idx = np.array([[1, 0], [1, 2], [0, 1]])
    lay = build_layout(idx, num_experts=4, ffn_dim=8, block_size=2)
    np.testing.assert_array_equal(lay.tokens_per_expert, [2, 3, 1, 0])
    np.testing.assert_array_equal(lay.padded_offsets, [0, 2, 6, 8, 8])
    np.testing.assert_array_equal(lay.copy_row, [2, 0, 3, 6, 1, 4])
    np.testing.assert_array_equal(lay.row_token, [0, 2, 0, 1, 2, -1, 1, -1])
    np.testing.assert_array_equal(lay.row_block_expert, [0, 1, 1, 2])
    np.testing.assert_array_equal(lay.row_offsets, [0, 4, 8, 12, 16])
    np.testing.assert_array_equal(lay.col_indices, [0, 1, 2, 3, 4, 5, 6, 7, 4, 5, 6, 7, 8, 9, 10, 11])


def test_exact_multiple_has_no_padding() -> None:
    lay = build_layout(np.tile([[0, 1]], (8, 1)), num_experts=4, ffn_dim=8, block_size=4)
    assert lay.num_rows == 16 and int((lay.row_token < 0).sum()) == 0


def test_bad_ids_are_skipped_and_flagged() -> None:
    # Known answer of the reference's tests/test_routing.py:111-120.
    lay = device_layout(np.array([[0, 1], [2, 8], [-1, 3]]), 8, 32, 16)
    assert lay.error == 1
    assert int(lay.tokens_per_expert.sum()) == 4
    assert lay.copy_row.tolist() == [0, 16, 32, -1, -1, 48]


@pytest.mark.parametrize("case", CASE_NAMES)
@pytest.mark.parametrize("num_experts", [2, 8, 64])
@pytest.mark.parametrize("block_size", [4, 16, 128])
@pytest.mark.parametrize("num_tokens", [1, 13, 129, 300])
def test_matches_brute_force(case: str, num_experts: int, block_size: int, num_tokens: int) -> None:
    idx = routing_case(case, num_tokens, num_experts).numpy()
    lay = build_layout(idx, num_experts, 2 * block_size, block_size)
    assert_same(lay, brute_force_layout(idx, num_experts, 2 * block_size, block_size))
    check_invariants(lay, idx)


@pytest.mark.parametrize("k", [1, 2, 4])
def test_any_k_matches_brute_force(k: int) -> None:
    idx = routing_case("random", 77, 16, seed=3, k=k).numpy()
    lay = build_layout(idx, 16, 32, 16)
    assert_same(lay, brute_force_layout(idx, 16, 32, 16))
    check_invariants(lay, idx)


@pytest.mark.parametrize("case", CASE_NAMES)
def test_device_layout_past_the_end(case: str) -> None:
    idx = routing_case(case, 100, 8).numpy()
    dev = device_layout(idx, 8, 32, 16)
    trimmed = build_layout(idx, 8, 32, 16)
    max_rb, max_rows = worst_case_sizes(idx.size, 8, 32, 16)
    nrows, nrb = trimmed.num_rows, trimmed.num_row_blocks
    assert dev.row_token.size == max_rows and dev.row_block_expert.size == max_rb
    assert dev.row_offsets.size == max_rb + 1 and dev.col_indices.size == max_rb * 2
    np.testing.assert_array_equal(dev.row_token[:nrows], trimmed.row_token)
    assert np.all(dev.row_token[nrows:] == -1)
    assert np.all(dev.row_block_expert[nrb:] == -1)
    assert np.all(dev.col_indices[nrb * 2:] == -1)
    assert np.all(dev.row_offsets[nrb:] == nrb * 2)
    np.testing.assert_array_equal(dev.copy_row, trimmed.copy_row)
    assert dev.error == 0


def test_valid_tokens_equals_truncated_input() -> None:
    idx = routing_case("zipf", 500, 16, seed=4).numpy()
    dev = device_layout(idx, 16, 256, 128, valid_tokens=123)
    ref = build_layout(idx[:123], 16, 256, 128)
    np.testing.assert_array_equal(dev.copy_row[: 123 * 2], ref.copy_row)
    assert np.all(dev.copy_row[123 * 2:] == -1)
    np.testing.assert_array_equal(dev.row_token[: ref.num_rows], ref.row_token)
    np.testing.assert_array_equal(dev.tokens_per_expert, ref.tokens_per_expert)
    np.testing.assert_array_equal(dev.padded_offsets, ref.padded_offsets)
    assert dev.error == 0


def test_int32_matches_int64() -> None:
    idx = routing_case("random", 50, 8).numpy()
    assert_same(build_layout(idx, 8, 32, 16), build_layout(idx.astype(np.int32), 8, 32, 16))


@pytest.mark.parametrize(
    ("idx", "kwargs", "error"),
    [
        (np.zeros((0, 2), dtype=np.int64), {}, ValueError),
        (np.zeros(4, dtype=np.int64), {}, ValueError),
        (np.zeros((4, 2)), {}, TypeError),
        (np.array([[0, 8]]), {}, ValueError),
        (np.array([[-1, 0]]), {}, ValueError),
        (np.array([[0, 1]]), {"ffn_dim": 10}, ValueError),
        (np.array([[0, 1]]), {"block_size": 0}, ValueError),
    ],
)
def test_rejects_bad_input(idx, kwargs, error) -> None:
    args = {"num_experts": 8, "ffn_dim": 8, "block_size": 4} | kwargs
    with pytest.raises(error):
        build_layout(idx, **args)
