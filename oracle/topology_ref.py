"""Block-sparse layout oracle (numpy, integer-exact). TEST INFRASTRUCTURE ONLY.

Restates the algorithm of the reference's sparsebench/topology.py:53-118
(stable counting sort of copies by expert, padding to block_size, BSR with
every row block holding its expert's ffn_blocks column blocks) and the
device-side conventions of csrc/routing.cu: bad expert ids are skipped and
flagged (routing.cu:44-51, 125-132, 157-158), and the worst-case buffers are
marked past the real end (routing.cu:162-193, 248-249).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Layout:
    """All arrays int32 numpy. Worst-case-sized when built by device_layout."""

    block_size: int
    num_experts: int
    ffn_blocks: int
    tokens_per_expert: np.ndarray
    padded_offsets: np.ndarray
    row_token: np.ndarray
    copy_row: np.ndarray
    row_block_expert: np.ndarray
    row_offsets: np.ndarray
    col_indices: np.ndarray
    error: int = 0

    FIELDS = ("tokens_per_expert", "padded_offsets", "row_token", "copy_row",
              "row_block_expert", "row_offsets", "col_indices")

    @property
    def num_rows(self) -> int:
        return int(self.padded_offsets[-1])

    @property
    def num_row_blocks(self) -> int:
        return self.num_rows // self.block_size


def worst_case_sizes(num_copies: int, num_experts: int, ffn_dim: int, block_size: int) -> tuple[int, int]:
    """(max_row_blocks, max_rows): every expert wastes block_size - 1 rows (routing.cu:213-216)."""
    max_row_blocks = (num_copies + num_experts * (block_size - 1)) // block_size
    return max_row_blocks, max_row_blocks * block_size


def _validate(expert_idx: np.ndarray, num_experts: int, ffn_dim: int, block_size: int) -> None:
    # The checks of topology.py:57-67 (ValueError / TypeError).
    if expert_idx.ndim != 2 or expert_idx.shape[0] == 0 or expert_idx.shape[1] == 0:
        raise ValueError(f"expert_idx must be [T, k] with T, k > 0, got {tuple(expert_idx.shape)}")
    if expert_idx.dtype not in (np.int32, np.int64):
        raise TypeError(f"expert_idx must be int32 or int64, got {expert_idx.dtype}")
    if num_experts <= 0 or block_size <= 0:
        raise ValueError("num_experts and block_size must be positive")
    if ffn_dim <= 0 or ffn_dim % block_size != 0:
        raise ValueError(f"ffn_dim ({ffn_dim}) must be a positive multiple of block_size ({block_size})")


def _core(flat: np.ndarray, k: int, num_experts: int, block_size: int, ffn_dim: int, keep: np.ndarray):
    """Layout of the copies where keep is True, the others skipped."""
    counts = np.bincount(flat[keep], minlength=num_experts).astype(np.int64)
    padded = (counts + block_size - 1) // block_size * block_size
    padded_offsets = np.concatenate(([0], np.cumsum(padded))).astype(np.int64)
    # Kept copies in (expert, copy index) order: a stable sort by expert.
    key = np.where(keep, flat, num_experts)
    order = np.argsort(key, kind="stable")[: int(keep.sum())]
    sorted_expert = flat[order]
    first_of_expert = np.cumsum(counts) - counts
    rank = np.arange(order.size) - first_of_expert[sorted_expert]
    dest = padded_offsets[sorted_expert] + rank
    copy_row = np.full(flat.size, -1, dtype=np.int64)
    copy_row[order] = dest
    num_rows = int(padded_offsets[-1])
    row_token = np.full(num_rows, -1, dtype=np.int64)
    row_token[dest] = order // k
    ffn_blocks = ffn_dim // block_size
    row_block_expert = np.repeat(np.arange(num_experts), padded // block_size)
    row_offsets = np.arange(row_block_expert.size + 1) * ffn_blocks
    col_indices = (row_block_expert[:, None] * ffn_blocks + np.arange(ffn_blocks)).reshape(-1)
    return counts, padded_offsets, row_token, copy_row, row_block_expert, row_offsets, col_indices


def build_layout(expert_idx: np.ndarray, num_experts: int, ffn_dim: int, block_size: int) -> Layout:
    """Trimmed layout; raises like topology.py:build_topology on bad input."""
    expert_idx = np.asarray(expert_idx)
    _validate(expert_idx, num_experts, ffn_dim, block_size)
    lo, hi = int(expert_idx.min()), int(expert_idx.max())
    if lo < 0 or hi >= num_experts:
        raise ValueError(f"expert ids must be in [0, {num_experts}), got range [{lo}, {hi}]")
    flat = expert_idx.reshape(-1).astype(np.int64)
    parts = _core(flat, expert_idx.shape[1], num_experts, block_size, ffn_dim, np.ones(flat.size, dtype=bool))
    if int(parts[1][-1]) * ffn_dim >= 2**31:
        raise ValueError("problem too large for int32 indexing")
    return Layout(block_size, num_experts, ffn_dim // block_size, *(p.astype(np.int32) for p in parts))


def device_layout(
    expert_idx: np.ndarray, num_experts: int, ffn_dim: int, block_size: int, valid_tokens: int | None = None
) -> Layout:
    """The worst-case buffers of build_topology_cuda (routing.cu:197-281), every element.

    Bad ids are skipped (copy_row = -1, not counted) and set error = 1;
    with valid_tokens = T', copies of tokens >= T' are skipped without error.
    Past the real end: row_token = -1, row_block_expert = -1,
    col_indices = -1, row_offsets flat at num_row_blocks * ffn_blocks.
    """
    expert_idx = np.asarray(expert_idx)
    _validate(expert_idx, num_experts, ffn_dim, block_size)
    num_tokens, k = expert_idx.shape
    flat = expert_idx.reshape(-1).astype(np.int64)
    in_range = (flat >= 0) & (flat < num_experts)
    live = np.ones(flat.size, dtype=bool)
    if valid_tokens is not None:
        live = np.arange(flat.size) // k < valid_tokens
    keep = in_range & live
    error = int(np.any(live & ~in_range))
    counts, offsets, row_token, copy_row, rbe, row_offsets, cols = _core(
        np.where(in_range, flat, 0), k, num_experts, block_size, ffn_dim, keep
    )
    ffn_blocks = ffn_dim // block_size
    max_rb, max_rows = worst_case_sizes(flat.size, num_experts, ffn_dim, block_size)
    nrb = rbe.size

    def pad(a: np.ndarray, size: int, fill: int) -> np.ndarray:
        out = np.full(size, fill, dtype=np.int64)
        out[: a.size] = a
        return out

    return Layout(
        block_size, num_experts, ffn_blocks,
        counts.astype(np.int32), offsets.astype(np.int32),
        pad(row_token, max_rows, -1).astype(np.int32),
        copy_row.astype(np.int32),
        pad(rbe, max_rb, -1).astype(np.int32),
        pad(row_offsets, max_rb + 1, nrb * ffn_blocks).astype(np.int32),
        pad(cols, max_rb * ffn_blocks, -1).astype(np.int32),
        error,
    )


def brute_force_layout(expert_idx, num_experts: int, ffn_dim: int, block_size: int) -> Layout:
    """The same layout by direct construction with Python loops (tiny inputs only).

    Walks experts in order and, inside each, copies in index order, handing
    out consecutive rows, then pads the group with -1 rows. Shares no code
    with build_layout: it pins it.
    """
    rows_idx = [list(map(int, r)) for r in np.asarray(expert_idx)]
    k = len(rows_idx[0])
    flat = [e for r in rows_idx for e in r]
    ffn_blocks = ffn_dim // block_size
    copy_row = [-1] * len(flat)
    row_token: list[int] = []
    offsets = [0]
    counts = []
    rbe: list[int] = []
    for e in range(num_experts):
        mine = [c for c, ee in enumerate(flat) if ee == e]
        counts.append(len(mine))
        for c in mine:
            copy_row[c] = len(row_token)
            row_token.append(c // k)
        while len(row_token) % block_size:
            row_token.append(-1)
        rbe += [e] * ((len(row_token) - offsets[-1]) // block_size)
        offsets.append(len(row_token))
    row_offsets = [r * ffn_blocks for r in range(len(rbe) + 1)]
    cols = [e * ffn_blocks + j for e in rbe for j in range(ffn_blocks)]
    a = lambda v: np.asarray(v, dtype=np.int32)  # noqa: E731
    return Layout(block_size, num_experts, ffn_blocks, a(counts), a(offsets), a(row_token), a(copy_row),
                  a(rbe), a(row_offsets), a(cols))


def row_block_of_nnz(layout: Layout) -> np.ndarray:
    """Row block of each non-zero block, [nnz]."""
    counts = np.diff(layout.row_offsets.astype(np.int64))
    return np.repeat(np.arange(counts.size), counts)
