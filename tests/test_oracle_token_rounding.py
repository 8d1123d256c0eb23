"""Pins of the token-rounding oracle (oracle/token_rounding_ref.py), on the CPU.

Known answers and properties are the reference's own tests
(tests/test_token_rounding.py:13-83); the brute force ranks by counting,
with no sort, on small inputs with many ties.
"""

import numpy as np
import pytest
import torch

from oracle.moe_ref import moe_assigned_reference, moe_reference
from oracle.token_rounding_ref import (
    brute_force_keep,
    keep_mask,
    round_counts,
    routing_change,
    token_rounding,
    top_k,
    top_k_assignments,
)
from sparsebench_amd.workloads import router_scores


def test_round_counts_nearest_ties_down() -> None:
    # tests/test_token_rounding.py:13-16 (reference)
    counts = np.array([0, 1, 63, 64, 65, 128, 191, 192, 200])
    expected = np.array([0, 0, 0, 0, 128, 128, 128, 128, 256])
    assert np.array_equal(round_counts(counts, 128, 10_000), expected)


def test_round_counts_cap() -> None:
    # Never more than the largest multiple of the tile that fits in T.
    assert np.array_equal(round_counts(np.array([300, 250]), 128, 260), np.array([256, 256]))


def test_hand_worked_case() -> None:
    # tests/test_token_rounding.py:19-33 (reference): 8 tokens, 2 experts,
    # k = 1, tile 4; expert 0 has 5 picks -> 4 (drops token 4), expert 1 has
    # 3 -> 4 (adds token 4, its best non-pick).
    s0 = np.array([0.9, 0.8, 0.7, 0.6, 0.55, 0.1, 0.2, 0.3], dtype=np.float32)
    scores = np.stack([s0, 1 - s0], axis=1)
    a = token_rounding(scores, k=1, tile=4)
    kept = set(zip(a.token.tolist(), a.expert.tolist()))
    assert {t for t, e in kept if e == 0} == {0, 1, 2, 3}
    assert {t for t, e in kept if e == 1} == {4, 5, 6, 7}
    assert np.allclose(a.weight, 1.0)


@pytest.mark.parametrize("name", ["uniform", "zipf"])
@pytest.mark.parametrize(("num_tokens", "num_experts", "k"), [(4096, 64, 2), (2000, 8, 2), (3000, 16, 4)])
def test_properties(name: str, num_tokens: int, num_experts: int, k: int) -> None:
    # tests/test_token_rounding.py:36-83 (reference)
    tile = 128
    scores = router_scores(name, num_tokens, num_experts).numpy()
    rounded = token_rounding(scores, k, tile)
    plain = top_k_assignments(scores, k)
    before = np.bincount(plain.expert, minlength=num_experts)
    after = np.bincount(rounded.expert, minlength=num_experts)
    assert np.all(after % tile == 0)
    assert np.all(np.abs(after - before) <= tile // 2)

    picked = np.zeros((num_tokens, num_experts), dtype=bool)
    picked[plain.token, plain.expert] = True
    kept = np.zeros_like(picked)
    kept[rounded.token, rounded.expert] = True
    for e in range(num_experts):
        col = scores[:, e]
        if after[e] <= before[e]:
            assert not (kept[:, e] & ~picked[:, e]).any()
            if kept[:, e].any() and (picked[:, e] & ~kept[:, e]).any():
                assert col[kept[:, e]].min() >= col[picked[:, e] & ~kept[:, e]].max()
        else:
            assert np.array_equal(kept[:, e] & picked[:, e], picked[:, e])
            added, rest = kept[:, e] & ~picked[:, e], ~kept[:, e]
            if rest.any():
                assert col[added].min() >= col[rest].max()

    sums = np.zeros(num_tokens, dtype=np.float64)
    np.add.at(sums, rounded.token, rounded.weight)
    has = np.zeros(num_tokens, dtype=bool)
    has[rounded.token] = True
    np.testing.assert_allclose(sums[has], 1.0, rtol=1e-5)

    again = token_rounding(scores, k, tile)
    assert np.array_equal(again.token, rounded.token) and np.array_equal(again.expert, rounded.expert)
    # (token, expert) order, like nonzero()
    order = rounded.token * num_experts + rounded.expert
    assert np.all(np.diff(order) > 0)
    stats = routing_change(scores, k, rounded, tile)
    assert 0 <= stats["topk_picks_dropped_pct"] <= 100


def tie_heavy_scores(num_tokens: int, num_experts: int, levels: int, seed: int) -> np.ndarray:
    """Scores on a coarse grid: many exact ties, in picks and in columns."""
    rng = np.random.default_rng(seed)
    return (rng.integers(0, levels, size=(num_tokens, num_experts)) / levels).astype(np.float32)


@pytest.mark.parametrize(("num_tokens", "num_experts", "k", "tile", "levels"),
                         [(40, 6, 2, 4, 5), (33, 3, 1, 8, 3), (64, 8, 3, 16, 7), (25, 5, 2, 4, 1000)])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_keep_matches_brute_force(num_tokens, num_experts, k, tile, levels, seed) -> None:
    scores = tie_heavy_scores(num_tokens, num_experts, levels, seed)
    keep, target = keep_mask(scores, k, tile)
    assert np.array_equal(keep, brute_force_keep(scores, k, tile))
    assert np.array_equal(keep.sum(axis=0), target)


def test_top_k_matches_sorting_by_hand() -> None:
    scores = tie_heavy_scores(50, 7, 4, 3)
    top_s, top_i = top_k(scores, 3)
    for t in range(50):
        ranked = sorted(range(7), key=lambda e: (-scores[t, e], e))[:3]
        assert top_i[t].tolist() == ranked
        assert top_s[t].tolist() == [scores[t, e] for e in ranked]


def test_top_k_weights_sum_to_one() -> None:
    scores = router_scores("zipf", 300, 16).numpy()
    a = top_k_assignments(scores, 4)
    np.testing.assert_allclose(a.weight.reshape(300, 4).sum(axis=1), 1.0, rtol=1e-6)
    assert np.array_equal(a.token, np.repeat(np.arange(300), 4))


def test_assigned_reference_equals_loop_reference_on_top_k() -> None:
    # A top-k list through the assigned layer == the top-k layer.
    g = torch.Generator().manual_seed(0)
    t, e, d, f, k = 64, 6, 32, 48, 2
    x = torch.randn(t, d, generator=g)
    w1 = torch.randn(e, d, f, generator=g) / d**0.5
    w2 = torch.randn(e, f, d, generator=g) / f**0.5
    idx = torch.rand(t, e, generator=g).topk(k, dim=1).indices
    w = torch.softmax(torch.randn(t, k, generator=g), dim=1)
    token = torch.arange(t).repeat_interleave(k)
    got = moe_assigned_reference(x, token, idx.reshape(-1), w.reshape(-1), w1, w2)
    torch.testing.assert_close(got, moe_reference(x, idx, w, w1, w2), rtol=1e-5, atol=1e-5)


def test_assigned_reference_token_without_copies_is_zero() -> None:
    g = torch.Generator().manual_seed(1)
    x = torch.randn(5, 16, generator=g)
    w1, w2 = torch.randn(3, 16, 16, generator=g), torch.randn(3, 16, 16, generator=g)
    out = moe_assigned_reference(x, [1, 2, 2, 4], [0, 1, 2, 0], [1.0, 0.5, 0.5, 1.0], w1, w2)
    assert torch.all(out[0] == 0) and torch.all(out[3] == 0)
