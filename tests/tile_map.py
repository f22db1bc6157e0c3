"""Host restatement of the grouped GEMM's workgroup -> tile mapping, used by
the tests to pick whole output tiles (XCD range boundaries, tail tiles, the
uneven block split of a run) for comparison with the oracle.

It follows the expert-aligned, XCD-aware order of the kernel: tiles run-major
over runs of consecutive align blocks with one expert, n-tiles in groups of 4
inside a run (row-tile-major within a group), each XCD taking one contiguous
range of tile ids, and a run's blocks split as evenly as possible over its row
tiles, larger tiles last.  The result is only a choice of which outputs to
check: every check compares outputs with the oracle, so a restatement that
drifted from the kernel would check other outputs, not pass wrong ones.  The
restatement itself is held to covering every (position, n-tile) of the sorted
order exactly once (tests/test_host.py)."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

XCDS = 8
GROUP = 4  # n-tiles per group inside a run


@dataclass(frozen=True)
class TileInfo:
    t: int            # tile id in the expert-major order
    xcd: int          # XCD range holding t
    j: int            # n-tile (256 columns: two 128-column scale groups)
    pos0: int         # sorted position of tile row 0
    rows: int         # rows of the run inside the tile (a multiple of the align block)
    expert: int       # expert id of the run (-1: not local)
    run_blocks: int   # blocks of the run
    units: int        # row tiles of the run
    u: int            # this tile's row tile within the run


def runs_of(eids: np.ndarray) -> list[tuple[int, int]]:
    """(first block, block count) of every run of equal expert ids."""
    out = []
    b = 0
    n = eids.size
    while b < n:
        e = eids[b]
        c = 1
        while b + c < n and eids[b + c] == e:
            c += 1
        out.append((b, c))
        b += c
    return out


COL_MAJOR_K = 8192  # plain launches with K >= this order a group column-major


def tile_map(eids: np.ndarray, ntpp: int, bma: int, tile_m: int, n_tiles: int,
             col_major: bool = False) -> list[TileInfo]:
    """Every active tile of one launch (idle tile ids are left out).
    ``col_major``: the group order of plain launches with K >= COL_MAJOR_K."""
    n_blocks = ntpp // bma
    eids = np.asarray(eids[:n_blocks])
    total = n_blocks * n_tiles
    per_xcd = (total + XCDS - 1) // XCDS
    ub = tile_m // bma
    tiles = []
    for b0, run in runs_of(eids):
        units = (run + ub - 1) // ub
        base, n_short = run // units, units - run % units
        for in_run in range(units * n_tiles):
            gj0 = in_run // (GROUP * units) * GROUP
            gsz = min(n_tiles - gj0, GROUP)
            in_grp = in_run - gj0 * units
            j = gj0 + (in_grp // units if col_major else in_grp % gsz)
            u = in_grp % units if col_major else in_grp // gsz
            b = b0 + (u * base if u < n_short else n_short * base + (u - n_short) * (base + 1))
            rows = (base if u < n_short else base + 1) * bma
            t = b0 * n_tiles + in_run
            tiles.append(TileInfo(t, t // per_xcd, j, b * bma, rows, int(eids[b0]), run, units, u))
    return tiles


def pick_tiles(tiles: list[TileInfo], sorted_ids: np.ndarray, S: int, tail_rows: int = 64) -> dict[str, TileInfo]:
    """Named tiles worth checking whole: the first and last active tile of each
    XCD range, a tile short enough for the tail body, both parts of a run
    split unevenly over its row tiles (the smaller first part -- one block
    when a 3-block run is split 1 + 2 -- and the larger last part), a tile of
    an expert with a single row tile (16- and 32-row launches load its
    weights with the non-temporal hint), a 256-row tile whose valid rows fit
    the 128-row body but not the 64-row one, and the first row tile (first
    n-tile) and last row tile (last n-tile) of the expert with the most
    blocks."""
    out: dict[str, TileInfo] = {}
    by_xcd: dict[int, list[TileInfo]] = {}
    for ti in tiles:
        by_xcd.setdefault(ti.xcd, []).append(ti)
    for x, lst in sorted(by_xcd.items()):
        lst = sorted(lst, key=lambda a: a.t)
        out[f"xcd{x}_first"] = lst[0]
        out[f"xcd{x}_last"] = lst[-1]

    def nvalid(ti: TileInfo) -> int:
        return int((sorted_ids[ti.pos0:ti.pos0 + ti.rows] < S).sum())

    for ti in tiles:
        if ti.expert >= 0 and "tail" not in out and 0 < nvalid(ti) <= tail_rows and ti.rows > tail_rows:
            out["tail"] = ti
        if ti.expert >= 0 and "short_of_split" not in out and ti.units > 1 and ti.run_blocks % ti.units \
                and ti.u == 0:
            out["short_of_split"] = ti
        if ti.expert >= 0 and "long_of_split" not in out and ti.units > 1 and ti.run_blocks % ti.units \
                and ti.u == ti.units - 1:
            out["long_of_split"] = ti
        if ti.expert >= 0 and "single_row_tile" not in out and ti.units == 1:
            out["single_row_tile"] = ti
        if ti.expert >= 0 and "body128_of_256" not in out and ti.rows > 128 and tail_rows < nvalid(ti) <= 128:
            out["body128_of_256"] = ti
    live = [ti for ti in tiles if ti.expert >= 0]
    if live:
        hot = max(live, key=lambda a: (a.run_blocks, -a.t))
        n_tiles = max(ti.j for ti in tiles) + 1
        run_tiles = [ti for ti in live if ti.expert == hot.expert and ti.run_blocks == hot.run_blocks]
        first = [ti for ti in run_tiles if ti.u == 0 and ti.j == 0]
        last = [ti for ti in run_tiles if ti.u == ti.units - 1 and ti.j == n_tiles - 1]
        if first:
            out["hot_first"] = first[0]
        if last:
            out["hot_last"] = last[0]
    return out


def tile_positions(ti: TileInfo, sorted_ids: np.ndarray, S: int) -> np.ndarray:
    """Sorted positions of the tile that hold slots."""
    p = np.arange(ti.pos0, ti.pos0 + ti.rows)
    return p[sorted_ids[p] < S]
