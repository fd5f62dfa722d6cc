"""The cell-block search's failure lists (torchbvh_amd/csrc/knn.hip,
grid_append / grid_sublist / grid_chunk_start / grid_layout): a CPU model of
the launch grids' index arithmetic, checked for the two properties the
kernels rely on, over many call sizes:

* no sub-list can overflow: the launch positions a sub-list can receive (the
  tiles of one XCD share with one residue of the local tile index) fit its
  `seg` entries, and the second list's sub-list receives only entries of the
  first's same sub-list;
* the next stage reads every entry a sub-list can hold: the work-groups that
  read a sub-list (the same grid as the pass) cover chunks 0 .. seg / 64 - 1
  of it, each once.

The model follows the kernels' integer arithmetic; what it checks is the
capacity and coverage that arithmetic must provide, for every tile count
from 1 to 3000 and a few large ones."""

from __future__ import annotations

from collections import Counter

import pytest

WAVE = 64          # kKnnBlock: one wave per work-group, one launch position per lane
XCDS = 8           # kXcds
SUBLISTS = 64      # kGridSubLists


def grid_for(total_q: int) -> int:
    tiles = (total_q + WAVE - 1) // WAVE
    return (tiles + XCDS - 1) // XCDS * XCDS  # launch_grid_dk / launch_dk


def seg_entries(total_q: int) -> int:
    tiles = (total_q + WAVE - 1) // WAVE
    per_xcd = (tiles + XCDS - 1) // XCDS
    return (per_xcd + SUBLISTS - 1) // SUBLISTS * WAVE  # grid_layout


def sublist(b: int) -> int:
    return (b % XCDS) * SUBLISTS + (b // XCDS) % SUBLISTS


def chunk_start(b: int) -> int:
    return (b // XCDS // SUBLISTS) * WAVE


def tile_of(b: int, grid: int) -> int:
    per_xcd = grid // XCDS
    return (b % XCDS) * per_xcd + b // XCDS  # the pass's tile map


def check(total_q: int) -> None:
    grid = grid_for(total_q)
    seg = seg_entries(total_q)
    # Producers (pass 1): each work-group's valid launch positions can all fail.
    cap = Counter()
    for b in range(grid):
        t = tile_of(b, grid)
        valid = max(0, min(WAVE, total_q - t * WAVE))
        cap[sublist(b)] += valid
    assert all(c <= seg for c in cap.values()), (total_q, max(cap.values()), seg)
    # Every launch position belongs to exactly one producer.
    assert sum(cap.values()) == total_q
    # Consumers (pass 2 and the fallback traversal: the same grid) read chunks of
    # the sub-list; the chunks a sub-list's readers take are 0, 1, ... once each
    # and reach every entry it can hold.
    chunks = {}
    for b in range(grid):
        chunks.setdefault(sublist(b), []).append(chunk_start(b))
    for s, c in cap.items():
        got = sorted(chunks.get(s, []))
        assert got == [i * WAVE for i in range(len(got))], (total_q, s)
        assert len(got) * WAVE >= c, (total_q, s, len(got), c)
        assert got[-1] + WAVE <= seg if got else c == 0


@pytest.mark.parametrize("tiles", list(range(1, 3001, 7)) + [2999, 3000])
def test_lists_capacity_and_coverage(tiles):
    for extra in (0, 1, 63):
        total_q = max(1, tiles * WAVE - extra)
        check(total_q)


@pytest.mark.parametrize("total_q", [1 << 17, (1 << 17) + 4099, 1 << 20, (1 << 22) + 777, 6_888_960])
def test_lists_at_bench_sizes(total_q):
    check(total_q)
