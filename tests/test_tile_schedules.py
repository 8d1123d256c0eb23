"""The layer kernels' tile schedules, restated on the CPU: every tile of a
stage is handed to exactly one workgroup of the grid the host launches.

A workgroup that finds no tile returns, so a grid bound that is too small,
or a mapping that hands one tile to two workgroups, would leave output rows
unwritten or written twice without any error on the GPU. These tests walk
every workgroup id of the launched grid through the mappings of
csrc/common.hpp (split_tail, split_tail_slack), csrc/expert_chunks.hpp
(balanced_chunk_tile, pair_counts, first_pair_unit_at, find_pair_unit) and
csrc/experts.hip (sdd_pair_kernel, pair_units_per_xcd) over many layouts.
"""
from __future__ import annotations

import numpy as np
import pytest

XCD = 8
BS = 128
PAIR_COST, SINGLE_COST = 10, 7


def split_tail(bid: int, tiles: int, cus_per_xcd: int) -> tuple[int, int]:
    per, rem = divmod(tiles, XCD)
    x, q = bid % XCD, bid // XCD
    n = per + (1 if x < rem else 0)
    start = x * (per + 1) if x < rem else rem * (per + 1) + (x - rem) * per
    r = n % cus_per_xcd if cus_per_xcd > 0 else 0
    split = r if (r > 0 and 2 * r <= cus_per_xcd) else 0
    whole = n - split
    if q < whole:
        return start + q, -1
    if q < whole + 2 * split:
        return start + whole + (q - whole) // 2, (q - whole) % 2
    return tiles, -1


def split_tail_slack(cus: int) -> int:
    return XCD * (cus // XCD // 2 + 1)


def balanced_chunk_tile(bid: int, chunks: int, slices: int):
    x, q = bid % XCD, bid // XCD
    rows, rem = divmod(chunks, XCD)
    pos = XCD - 1 - x if rows & 1 else x
    n = rows + (1 if pos < rem else 0)
    if n == 0 or q >= n * slices:
        return None
    j = q % n
    return XCD * j + (XCD - 1 - x if j & 1 else x), q // n


def pair_units_per_xcd(units: int) -> int:
    return (units * PAIR_COST // XCD + PAIR_COST) // SINGLE_COST + 1


def first_pair_unit_at(counts: list[int], target: int) -> tuple[int, int]:
    """(pairs, singles) before the first unit whose cost start is >= target."""
    cost_before = pairs_before = singles_before = 0
    for n in counts:
        rb = -(-n // BS) if n > 0 else 0
        p, s = rb >> 1, rb & 1
        cost = p * PAIR_COST + s * SINGLE_COST
        if target < cost_before + cost:
            off = target - cost_before
            i = 0 if off <= 0 else (-(-off // PAIR_COST) if off <= p * PAIR_COST else p + 1)
            return pairs_before + min(i, p), singles_before + (1 if i > p else 0)
        cost_before += cost
        pairs_before += p
        singles_before += s
    return pairs_before, singles_before


def pair_unit_rows(counts: list[int], single: bool, k: int) -> tuple[int, int]:
    """Padded rows [row0, row0 + 128 * blocks) of pair k or single k (each kind in expert order)."""
    off = 0
    for n in counts:
        rb = -(-n // BS) if n > 0 else 0
        mine = rb & 1 if single else rb >> 1
        if k < mine:
            first_rb = rb - 1 if single else 2 * k
            return off + first_rb * BS, BS if single else 2 * BS
        k -= mine
        off += rb * BS
    raise AssertionError("unit past the layout")


def pair_kernel_tiles(counts: list[int], max_row_blocks: int, slices: int) -> list[tuple[int, int]]:
    """(first padded row, slice) of every tile sdd_pair_kernel computes, over its whole grid."""
    live_rb = sum(-(-n // BS) for n in counts if n > 0)
    pairs = sum((-(-n // BS) >> 1) for n in counts if n > 0)
    singles = sum((-(-n // BS) & 1) for n in counts if n > 0)
    cost = pairs * PAIR_COST + singles * SINGLE_COST
    grid = XCD * pair_units_per_xcd(max_row_blocks) * slices
    tiles = []
    for bid in range(grid):
        q, x = divmod(bid, XCD)
        if q >= pair_units_per_xcd(live_rb) * slices:
            continue
        lo = first_pair_unit_at(counts, (cost * x + XCD - 1) // XCD)
        hi = (pairs, singles) if x == XCD - 1 else first_pair_unit_at(counts, (cost * (x + 1) + XCD - 1) // XCD)
        u, sl = divmod(q, slices)
        np_, ns = hi[0] - lo[0], hi[1] - lo[1]
        if u >= np_ + ns:
            continue
        single = u >= np_
        row0, nrows = pair_unit_rows(counts, single, lo[1] + u - np_ if single else lo[0] + u)
        tiles.extend((r, sl) for r in range(row0 // BS, (row0 + nrows) // BS))
    return tiles


def layouts():
    rng = np.random.default_rng(7)
    out = []
    for e in (1, 3, 8, 24, 64, 130, 300):
        for t in (1, 37, 500, 4096, 16384):
            k = min(2, e)
            idx = np.stack([rng.choice(e, size=k, replace=False) for _ in range(min(t, 3000))])
            out.append(np.bincount(idx.ravel(), minlength=e).tolist())
            w = 1.0 / (np.arange(1, e + 1) ** 1.2)
            z = rng.choice(e, size=t * k, p=w / w.sum())
            out.append(np.bincount(z, minlength=e).tolist())
    out.append([0] * 10 + [5000] + [0] * 5)  # one live expert among empty ones
    out.append([128, 129, 255, 256, 257, 383, 384, 1, 0, 640])  # row-block edges
    return out


@pytest.mark.parametrize("slices", [1, 3, 8])
def test_pair_kernel_covers_every_live_row_block_once(slices: int) -> None:
    for counts in layouts():
        copies = sum(counts)
        e = len(counts)
        max_rb = (copies + e * (BS - 1)) // BS  # the routing's worst-case sizing
        tiles = pair_kernel_tiles(counts, max_rb, slices)
        live_rb = sum(-(-n // BS) for n in counts if n > 0)
        assert sorted(tiles) == [(r, s) for r in range(live_rb) for s in range(slices)], counts


def test_pair_units_per_xcd_bounds_each_xcds_range() -> None:
    for counts in layouts():
        live_rb = sum(-(-n // BS) for n in counts if n > 0)
        pairs = sum((-(-n // BS) >> 1) for n in counts if n > 0)
        singles = sum((-(-n // BS) & 1) for n in counts if n > 0)
        cost = pairs * PAIR_COST + singles * SINGLE_COST
        ranges = [first_pair_unit_at(counts, (cost * x + XCD - 1) // XCD) for x in range(XCD)] + [(pairs, singles)]
        for x in range(XCD):
            n = (ranges[x + 1][0] - ranges[x][0]) + (ranges[x + 1][1] - ranges[x][1])
            assert 0 <= n <= pair_units_per_xcd(live_rb), (counts, x)


@pytest.mark.parametrize("slices", [1, 2, 8, 28])
def test_balanced_deal_hands_out_every_chunk_slice_once(slices: int) -> None:
    for chunks in list(range(0, 70)) + [130, 255, 256, 257, 1000]:
        grid = XCD * (-(-chunks // XCD)) * slices  # the kernels' grids hold at least this many
        seen = [balanced_chunk_tile(b, chunks, slices) for b in range(grid + 3 * XCD)]
        got = sorted(t for t in seen if t is not None)
        assert got == [(c, s) for c in range(chunks) for s in range(slices)], chunks


@pytest.mark.parametrize("cus", [256, 304, 80])
def test_split_tail_covers_every_tile_once(cus: int) -> None:
    for tiles in list(range(0, 200)) + [511, 512, 513, 848, 987, 1316, 1932]:
        halves: dict[int, list[int]] = {}
        for b in range(tiles + split_tail_slack(cus)):
            t, h = split_tail(b, tiles, cus // XCD)
            if t < tiles:
                halves.setdefault(t, []).append(h)
        assert sorted(halves) == list(range(tiles)), tiles
        assert all(v == [-1] or sorted(v) == [0, 1] for v in halves.values()), tiles
