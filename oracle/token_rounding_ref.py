"""TEST INFRASTRUCTURE ONLY: CPU restatement of the reference's router side
(sparsebench/token_rounding.py) in numpy. Only tests/, __graft_entry__.smoke()
and bench.py's CPU-baseline leg may import this module; the product path
never does.

Each function follows the reference file:line it names. Pinned by
tests/test_oracle_token_rounding.py against:
  - the reference tests' known answers (tests/test_token_rounding.py:13-16
    for round_counts, :18-33 for the hand-worked 8-token case);
  - the reference tests' properties (tests/test_token_rounding.py:36-83):
    every count a multiple of the tile, each expert moved by at most half a
    tile, rounded-down experts keep only their best picks, rounded-up
    experts add the best non-picks, weights sum to 1, determinism;
  - a brute force from the definition of the rank (count the tokens that
    rank above), independent of any sort, on small inputs.

Tie rules: top-k picks the lower expert index among equal scores (torch's
topk leaves this unspecified; with continuous scores ties do not occur), and
within an expert's column equal shifted scores rank by token index (the
reference's stable sort, token_rounding.py:73).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class Assignments:
    """A routing as a flat list: copy c sends token[c] to expert[c] with weight[c]."""

    token: np.ndarray  # [N] int64
    expert: np.ndarray  # [N] int64
    weight: np.ndarray  # [N] float32


def top_k(scores: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """(top_s, top_i) [T, k], descending, equal scores to the lower index (scores.topk at token_rounding.py:42)."""
    scores = np.asarray(scores, dtype=np.float32)
    order = np.argsort(-scores, axis=1, kind="stable")[:, :k]
    return np.take_along_axis(scores, order, axis=1), order.astype(np.int64)


def _sequential_row_sum(values: np.ndarray) -> np.ndarray:
    """fp32 sum of each row, added left to right from 0."""
    total = np.zeros(values.shape[0], dtype=np.float32)
    for j in range(values.shape[1]):
        total = (total + values[:, j]).astype(np.float32)
    return total


def top_k_assignments(scores: np.ndarray, k: int) -> Assignments:
    """Plain top-k as a list; weight = picked score / sum of the picks (token_rounding.py:39-46)."""
    top_s, top_i = top_k(scores, k)
    num_tokens = top_s.shape[0]
    token = np.repeat(np.arange(num_tokens, dtype=np.int64), k)
    weight = (top_s / _sequential_row_sum(top_s)[:, None]).astype(np.float32).reshape(-1)
    return Assignments(token, top_i.reshape(-1), weight)


def round_counts(counts: np.ndarray, tile: int, max_count: int) -> np.ndarray:
    """Nearest multiple of `tile`, ties down, at most max_count // tile * tile (token_rounding.py:49-55)."""
    counts = np.asarray(counts, dtype=np.int64)
    low = counts // tile * tile
    high = low + tile * (counts % tile > 0)
    rounded = np.where(high - counts < counts - low, high, low)
    return np.minimum(rounded, max_count // tile * tile)


def shifted_scores(scores: np.ndarray, top_s: np.ndarray, top_i: np.ndarray) -> np.ndarray:
    """Picks keep their score, every other entry drops by 1, in fp32 (token_rounding.py:67-70)."""
    shifted = (np.asarray(scores, dtype=np.float32) - np.float32(1.0)).astype(np.float32)
    np.put_along_axis(shifted, top_i, top_s, axis=1)
    return shifted


def keep_mask(scores: np.ndarray, k: int, tile: int) -> tuple[np.ndarray, np.ndarray]:
    """(keep [T, E] bool, target [E]) of token rounding (token_rounding.py:61-76)."""
    scores = np.asarray(scores, dtype=np.float32)
    num_tokens, num_experts = scores.shape
    top_s, top_i = top_k(scores, k)
    counts = np.bincount(top_i.reshape(-1), minlength=num_experts)
    target = round_counts(counts, tile, num_tokens)
    shifted = shifted_scores(scores, top_s, top_i)
    order = np.argsort(-shifted, axis=0, kind="stable")  # descending, equal values in token order
    rank = np.empty_like(order)
    rank[order, np.arange(num_experts)[None, :]] = np.arange(num_tokens)[:, None]
    return rank < target[None, :], target


def token_rounding(scores: np.ndarray, k: int, tile: int = 128) -> Assignments:
    """Every expert's count rounded to a multiple of `tile` (token_rounding.py:58-81).

    The list is in (token, expert) order (nonzero of the keep mask); weights
    are the kept scores over each token's kept total, summed in list order.
    """
    scores = np.asarray(scores, dtype=np.float32)
    keep, _ = keep_mask(scores, k, tile)
    token, expert = np.nonzero(keep)
    raw = scores[token, expert]
    total = np.zeros(scores.shape[0], dtype=np.float32)
    np.add.at(total, token, raw)  # unbuffered: added in list order
    with np.errstate(invalid="ignore"):  # a token whose kept scores are all 0: 0/0, as in torch
        weight = (raw / total[token]).astype(np.float32)
    return Assignments(token.astype(np.int64), expert.astype(np.int64), weight)


def brute_force_keep(scores: np.ndarray, k: int, tile: int) -> np.ndarray:
    """keep[t, e] by the definition of the rank, no sort: fewer than target[e]
    tokens rank above t in column e (a higher shifted score, or the same
    score and a lower token index). O(T^2 E): small inputs only."""
    scores = np.asarray(scores, dtype=np.float32)
    num_tokens, num_experts = scores.shape
    picks = [set() for _ in range(num_tokens)]
    for t in range(num_tokens):
        row = [(-float(scores[t, e]), e) for e in range(num_experts)]
        for _, e in sorted(row)[:k]:
            picks[t].add(e)
    counts = [sum(e in picks[t] for t in range(num_tokens)) for e in range(num_experts)]
    cap = num_tokens // tile * tile
    keep = np.zeros((num_tokens, num_experts), dtype=bool)
    for e in range(num_experts):
        f = counts[e]
        low, high = f // tile * tile, (f // tile + (f % tile > 0)) * tile
        target = min(high if high - f < f - low else low, cap)
        col = [np.float32(scores[t, e]) if e in picks[t] else np.float32(scores[t, e]) - np.float32(1.0)
               for t in range(num_tokens)]
        for t in range(num_tokens):
            above = sum(1 for u in range(num_tokens) if col[u] > col[t] or (col[u] == col[t] and u < t))
            keep[t, e] = above < target
    return keep


def routing_change(scores: np.ndarray, k: int, rounded: Assignments, tile: int = 128) -> dict[str, float]:
    """How far `rounded` is from plain top-k (token_rounding.py:84-103)."""
    scores = np.asarray(scores, dtype=np.float32)
    num_tokens, num_experts = scores.shape
    _, top_i = top_k(scores, k)
    picked = np.zeros_like(scores, dtype=bool)
    np.put_along_axis(picked, top_i, True, axis=1)
    kept = np.zeros_like(picked)
    kept[rounded.token, rounded.expert] = True
    counts = picked.sum(axis=0)
    padded = ((counts + tile - 1) // tile * tile).sum()
    per_token = kept.sum(axis=1)
    return {
        "topk_padding_pct": 100 * float((padded - counts.sum()) / padded),
        "topk_picks_dropped_pct": 100 * float((picked & ~kept).sum() / picked.sum()),
        "assignments_added_pct": 100 * float((kept & ~picked).sum() / picked.sum()),
        "tokens_with_0_experts_pct": 100 * float((per_token == 0).mean()),
        "tokens_with_more_than_k_pct": 100 * float((per_token > k).mean()),
        "topk_score_mass_kept_pct": 100 * float(scores[picked & kept].sum() / scores[picked].sum()),
    }

