"""The layer kernels' tile schedules on the CPU: every tile of a stage is
handed to exactly one workgroup of the grid the host launches.

A workgroup that finds no tile returns, so a grid bound that is too small,
or a mapping that hands one tile to two workgroups, would leave output rows
unwritten or written twice without any error on the GPU. These tests walk
every workgroup id of the launched grid through the mappings the kernels
call: csrc/common.hpp (xcd_remap, split_tail, split_tail_slack, tile_coords)
and csrc/expert_chunks.hpp (balanced_chunk_tile, lpt_group_tile,
pair_units_per_xcd, pair_tile_for) are __host__ __device__ functions, compiled for the CPU into
the tool library's shims (csrc/schedule_shims.hip), so what is checked here
is the compiled code, not a restatement of it. What each workgroup must
cover is stated independently below (the live row blocks, each kind of pair
unit in expert order).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from sparsebench_amd import _lib

XCD = 8
BS = 128


@pytest.fixture(scope="module")
def sched():
    path = _lib.LIB_PATH.with_name("libsparsebench_probe.so")
    if not path.exists():
        from sparsebench_amd.build import build

        build()
    _lib.lib()  # torch's HIP runtime first
    h = ctypes.CDLL(str(path))
    ip = ctypes.POINTER(ctypes.c_int)
    i = ctypes.c_int
    for name, res, args in [
        ("sbt_xcd_remap", i, [i, i]),
        ("sbt_split_tail", None, [i, i, i, ip, ip]),
        ("sbt_split_tail_slack", ctypes.c_int64, [i]),
        ("sbt_tile_coords", None, [i, i, i, i, ip, ip]),
        ("sbt_balanced_chunk_tile", i, [i, i, i, ip, ip]),
        ("sbt_pair_units_per_xcd", i, [i]),
        ("sbt_pair_tile_for", i, [i, i, i, i, i, ip, ip, ip, ip]),
        ("sbt_lpt_group_tile", None, [i, i, i, ctypes.c_uint32, ip, ip]),
    ]:
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


def split_tail(sched, bid: int, tiles: int, cus_per_xcd: int) -> tuple[int, int]:
    t, hf = ctypes.c_int(), ctypes.c_int()
    sched.sbt_split_tail(bid, tiles, cus_per_xcd, ctypes.byref(t), ctypes.byref(hf))
    return t.value, hf.value


def balanced_chunk_tile(sched, bid: int, chunks: int, slices: int):
    r, s = ctypes.c_int(), ctypes.c_int()
    if not sched.sbt_balanced_chunk_tile(bid, chunks, slices, ctypes.byref(r), ctypes.byref(s)):
        return None
    return r.value, s.value


def pair_unit_rows(counts: list[int], single: bool, k: int) -> tuple[int, int]:
    """Padded rows [row0, row0 + 128 * blocks) of pair k or single k (each
    kind in expert order): the units find_pair_unit numbers."""
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


def pair_kernel_tiles(sched, counts: list[int], max_row_blocks: int, slices: int,
                      cus: int = 32) -> list[tuple[int, int, int]]:
    """(row block, slice, half) of every tile sdd_pair_kernel computes over its whole grid (the
    launch's size: each XCD's units x slices plus half its CUs); half -1 is the whole slice."""
    live_rb = sum(-(-n // BS) for n in counts if n > 0)
    pairs = sum((-(-n // BS) >> 1) for n in counts if n > 0)
    singles = sum((-(-n // BS) & 1) for n in counts if n > 0)
    grid = XCD * (sched.sbt_pair_units_per_xcd(max_row_blocks) * slices + cus // 2)
    single, k, sl, half = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    tiles = []
    for bid in range(grid):
        if bid // XCD >= sched.sbt_pair_units_per_xcd(live_rb) * slices + cus // 2:
            continue  # the kernel's first exit test
        if not sched.sbt_pair_tile_for(bid, pairs, singles, slices, cus, ctypes.byref(single), ctypes.byref(k),
                                       ctypes.byref(sl), ctypes.byref(half)):
            continue
        row0, nrows = pair_unit_rows(counts, bool(single.value), k.value)
        assert half.value == -1 or (single.value and nrows == BS), "only singles are split"
        tiles.extend((r, sl.value, half.value) for r in range(row0 // BS, (row0 + nrows) // BS))
    # Workgroups past the launched grid would be lost: none may have work.
    for bid in range(grid, grid + 3 * XCD):
        assert not sched.sbt_pair_tile_for(bid, pairs, singles, slices, cus, ctypes.byref(single), ctypes.byref(k),
                                           ctypes.byref(sl), ctypes.byref(half))
    return tiles


def covered_once(tiles: list[tuple[int, int, int]]) -> list[tuple[int, int]]:
    """(row block, slice) pairs, each once, from whole tiles or both halves; fails on any overlap."""
    seen: dict[tuple[int, int], list[int]] = {}
    for r, s, h in tiles:
        seen.setdefault((r, s), []).append(h)
    assert all(v == [-1] or sorted(v) == [0, 1] for v in seen.values()), seen
    return sorted(seen)


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
@pytest.mark.parametrize("cus", [32, 38, 10])
def test_pair_kernel_covers_every_live_row_block_once(sched, slices: int, cus: int) -> None:
    for counts in layouts():
        copies = sum(counts)
        e = len(counts)
        max_rb = (copies + e * (BS - 1)) // BS  # the routing's worst-case sizing
        tiles = pair_kernel_tiles(sched, counts, max_rb, slices, cus)
        live_rb = sum(-(-n // BS) for n in counts if n > 0)
        assert covered_once(tiles) == [(r, s) for r in range(live_rb) for s in range(slices)], counts


def test_pair_kernel_splits_only_a_short_last_round_of_singles(sched) -> None:
    # Per XCD: n tiles on `cus` CUs, r = n % cus in the last round; split iff
    # those r tiles are all singles and 2r CUs are free for their halves: cus
    # less the pair tiles still running from the round before.
    single, k, sl, half = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    for pairs, singles, slices, cus in [(0, 330 // 3, 3, 32), (114, 101, 3, 32), (16, 20, 3, 32), (0, 5, 3, 32),
                                        (80, 8, 3, 32), (0, 64, 1, 32), (7, 300, 2, 38), (10, 122, 3, 32),
                                        (1, 109, 3, 32), (100, 180, 3, 32)]:
        for x in range(XCD):
            np_ = pairs * (x + 1) // XCD - pairs * x // XCD
            ns = singles * (x + 1) // XCD - singles * x // XCD
            n = (np_ + ns) * slices
            r = n % cus
            whole = n - r
            busy = max(0, np_ * slices - (whole - cus)) if whole >= cus else 0
            split = r > 0 and 2 * r <= cus - busy and whole >= np_ * slices
            halves = 0
            for q in range(n + cus):
                if sched.sbt_pair_tile_for(q * XCD + x, pairs, singles, slices, cus, ctypes.byref(single),
                                           ctypes.byref(k), ctypes.byref(sl), ctypes.byref(half)):
                    halves += half.value >= 0
            assert halves == (2 * r if split else 0), (pairs, singles, slices, cus, x)


def test_pair_kernel_xcds_share_each_kind_evenly(sched) -> None:
    # Each XCD's pairs and singles are within one unit of an eighth of each kind.
    single, k, sl, half = ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    for pairs, singles in [(114, 101), (0, 7), (5, 0), (31, 1), (1000, 3)]:
        units = [set() for _ in range(XCD)]
        for bid in range(XCD * (sched.sbt_pair_units_per_xcd(pairs + singles) + 16)):
            if sched.sbt_pair_tile_for(bid, pairs, singles, 1, 32, ctypes.byref(single), ctypes.byref(k),
                                       ctypes.byref(sl), ctypes.byref(half)):
                units[bid % XCD].add((single.value, k.value))
        per = [[sum(1 for kind, _ in u if kind == c) for c in (0, 1)] for u in units]
        assert sum(p for p, _ in per) == pairs and sum(s for _, s in per) == singles
        assert max(p for p, _ in per) - min(p for p, _ in per) <= 1
        assert max(s for _, s in per) - min(s for _, s in per) <= 1


@pytest.mark.parametrize("slices", [1, 2, 8, 28])
def test_balanced_deal_hands_out_every_chunk_slice_once(sched, slices: int) -> None:
    for chunks in list(range(0, 70)) + [130, 255, 256, 257, 1000]:
        grid = XCD * (-(-chunks // XCD)) * slices  # the kernels' grids hold at least this many
        seen = [balanced_chunk_tile(sched, b, chunks, slices) for b in range(grid + 3 * XCD)]
        got = sorted(t for t in seen if t is not None)
        assert got == [(c, s) for c in range(chunks) for s in range(slices)], chunks


@pytest.mark.parametrize("cus", [256, 304, 80])
def test_split_tail_covers_every_tile_once(sched, cus: int) -> None:
    for tiles in list(range(0, 200)) + [511, 512, 513, 848, 987, 1316, 1932]:
        halves: dict[int, list[int]] = {}
        for b in range(tiles + sched.sbt_split_tail_slack(cus)):
            t, h = split_tail(sched, b, tiles, cus // XCD)
            if t < tiles:
                halves.setdefault(t, []).append(h)
        assert sorted(halves) == list(range(tiles)), tiles
        assert all(v == [-1] or sorted(v) == [0, 1] for v in halves.values()), tiles


def test_xcd_remap_is_a_permutation_of_the_live_tiles(sched) -> None:
    for live in list(range(0, 100)) + [256, 511, 512, 1316]:
        got = sorted(sched.sbt_xcd_remap(b, live) for b in range(live))
        assert got == list(range(live)), live
        # each XCD (bid % 8) gets one contiguous range
        for x in range(XCD):
            mine = sorted(sched.sbt_xcd_remap(b, live) for b in range(x, live, XCD))
            assert mine == list(range(mine[0], mine[0] + len(mine))) if mine else True


def test_tile_coords_cover_the_live_grid_once(sched) -> None:
    rb, sl = ctypes.c_int(), ctypes.c_int()
    for live_rb in (1, 5, 8, 13, 64, 92):
        for slices in (1, 2, 4, 8):
            got = set()
            for t in range(live_rb * slices):
                sched.sbt_tile_coords(t, live_rb, slices, 8, ctypes.byref(rb), ctypes.byref(sl))
                got.add((rb.value, sl.value))
            assert got == {(r, s) for r in range(live_rb) for s in range(slices)}, (live_rb, slices)


def test_lpt_group_tile_runs_big_chunks_first_and_covers_the_group_once(sched) -> None:
    # Each group of G chunks x slices is handed out once, the chunks of `big`
    # (all their slices) before the others.
    pos, sl = ctypes.c_int(), ctypes.c_int()
    rng = np.random.default_rng(3)
    for g in (1, 2, 4, 5, 8, 13, 32):
        for slices in (1, 3, 16, 28):
            for big in {0, (1 << g) - 1 if g < 32 else 0xFFFFFFFF, int(rng.integers(0, 1 << min(g, 31)))}:
                order = []
                for local in range(g * slices):
                    sched.sbt_lpt_group_tile(local, g, slices, big, ctypes.byref(pos), ctypes.byref(sl))
                    order.append((pos.value, sl.value))
                assert sorted(order) == [(p, s) for p in range(g) for s in range(slices)], (g, slices, big)
                nb = bin(big & ((1 << g) - 1)).count("1")
                assert all((big >> p) & 1 for p, _ in order[:nb * slices]), (g, slices, big)
