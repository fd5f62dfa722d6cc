"""CPU restatement of the segmented radix sort's index arithmetic
(torchbvh_amd/csrc/sort.hip: tile_count_kernel, tile_scan_kernel,
scatter_kernel), term by term, to show that its two memory guards never
bind: the LDS staging position `at` (clamped to kSortTile - 1) is a
bijection onto [0, count) of each tile, and the segment-relative output row
`rel` (skipped when >= n) is a bijection onto [0, n) of each segment, for
any keys, segment sizes and surplus tiles.  The composed passes equal
numpy's stable argsort per segment (the CUB contract the sort replaces,
bvh_build.cu:580-594).  The build's tree pass reads this sort's output as
its permutation, which is why its index clamp (build.hip, tree_pass_kernel)
never binds either."""

from __future__ import annotations

import numpy as np
import pytest

TILE = 4096      # kSortTile
THREADS = 512    # kThreads
WAVE = 64        # kWave
ITEMS = TILE // THREADS  # kItems: keys per thread
RADIX = 256      # kRadix


def plan(sizes):
    """Segments' first rows, tile counts and first tiles; the launch's tile
    count tiles_bound = ceil(total / TILE) + S (tbvh_internal.hpp)."""
    starts = np.concatenate([[0], np.cumsum(sizes)[:-1]]).astype(np.int64)
    tiles = [(n + TILE - 1) // TILE for n in sizes]
    tile_first = np.concatenate([[0], np.cumsum(tiles)[:-1]]).astype(np.int64)
    bound = (int(sum(sizes)) + TILE - 1) // TILE + len(sizes)
    assert sum(tiles) < bound  # at least one surplus tile past the last segment
    return starts, tiles, tile_first, bound


def one_pass(keys, vals, sizes, shift):
    starts, tiles, tile_first, bound = plan(sizes)
    # tile_count_kernel: digit counts per tile, digit-major; surplus tiles 0.
    hist = np.zeros((RADIX, bound), np.int64)
    for s, n in enumerate(sizes):
        for lt in range(tiles[s]):
            row0 = starts[s] + lt * TILE
            count = min(TILE, n - lt * TILE)
            d = (keys[row0:row0 + count] >> shift) & (RADIX - 1)
            hist[:, tile_first[s] + lt] = np.bincount(d, minlength=RADIX)
    # tile_scan_kernel: exclusive scan along all tiles, per digit.
    scan = np.cumsum(hist, axis=1) - hist
    out_k = np.full(keys.shape, -1, np.int64)
    out_v = np.full(vals.shape, -1, np.int64)
    for s, n in enumerate(sizes):
        first = tile_first[s]
        for lt in range(tiles[s]):
            t = first + lt
            row0 = starts[s] + lt * TILE
            count = min(TILE, n - lt * TILE)
            k = keys[row0:row0 + count]
            v = vals[row0:row0 + count]
            digit = (k >> shift) & (RADIX - 1)
            pos = np.arange(count)
            wave = pos // (WAVE * ITEMS)  # pos = wave * WAVE * ITEMS + i * WAVE + lane
            # Per-wave LDS counters: rank[i] = prior count of the digit in
            # this wave + peers in lower lanes of the same ballot, i.e. the
            # same-digit keys earlier in the wave (pos order within a wave
            # is (i, lane) order).
            group = wave * RADIX + digit
            order = np.argsort(group, kind="stable")
            sorted_groups = group[order]
            first_of_group = np.searchsorted(sorted_groups, sorted_groups, side="left")
            rank = np.empty(count, np.int64)
            rank[order] = np.arange(count) - first_of_group
            # s_cnt[w][d] after the conversion loop: the digit's count in
            # waves before w; s_start[d]: the tile's keys of smaller digits.
            per_wave = np.zeros((THREADS // WAVE, RADIX), np.int64)
            np.add.at(per_wave, (wave, digit), 1)
            wave_before = np.cumsum(per_wave, axis=0) - per_wave
            tile_count = per_wave.sum(axis=0)
            s_start = np.cumsum(tile_count) - tile_count
            at = s_start[digit] + wave_before[wave, digit] + rank
            # The clamp min(at, kSortTile - 1) never binds: a bijection onto [0, count).
            assert at.max(initial=-1) < count <= TILE
            assert np.array_equal(np.sort(at), pos)
            s_keys = np.empty(count, np.int64)
            s_vals = np.empty(count, np.int64)
            s_keys[at] = k
            s_vals[at] = v
            # Digit offsets from the scan: the segment's tiles before this one
            # and the segment's digit totals (the exclusive scan at the
            # segment's end, a surplus tile's entry for the last segment).
            before_tiles = scan[:, t] - scan[:, first]
            seg_count = scan[:, first + tiles[s]] - scan[:, first]
            digit_start = np.cumsum(seg_count) - seg_count
            s_base = digit_start + before_tiles
            d_staged = (s_keys >> shift) & (RADIX - 1)
            rel = s_base[d_staged] + (np.arange(count) - s_start[d_staged])
            # The guard `rel >= n` never fires.
            assert rel.min(initial=0) >= 0 and rel.max(initial=-1) < n
            rows = starts[s] + rel
            assert np.all(out_k[rows] == -1), "an output row written twice"
            out_k[rows] = s_keys
            out_v[rows] = s_vals
    assert np.all(out_k >= 0), "an output row never written"
    return out_k, out_v


def model_sort(keys, sizes, bits):
    """All passes; pass 0 synthesises the values (the local row)."""
    starts, _, _, _ = plan(sizes)
    vals = np.concatenate([np.arange(n, dtype=np.int64) for n in sizes])
    k = keys.astype(np.int64)
    for shift in range(0, bits, 8):
        k, vals = one_pass(k, vals, sizes, shift)
    return vals


@pytest.mark.parametrize("sizes", [[1], [5], [4095], [4096], [4097], [1, 4096, 4097, 9000, 3],
                                   [8193] * 3, [30000]])
@pytest.mark.parametrize("kind", ["uniform", "duplicates", "equal"])
def test_scatter_arithmetic_is_a_stable_sort_and_guards_never_bind(sizes, kind):
    rng = np.random.default_rng(sum(sizes) + len(kind))
    total = sum(sizes)
    if kind == "uniform":
        keys = rng.integers(0, 1 << 30, total, dtype=np.int64)
    elif kind == "duplicates":
        keys = rng.integers(0, 40, total, dtype=np.int64) * 0x01010101
    else:
        keys = np.full(total, 0x2ABCDEF, np.int64)
    got = model_sort(keys, sizes, 30)
    starts = np.concatenate([[0], np.cumsum(sizes)[:-1]])
    for s, n in enumerate(sizes):
        seg = keys[starts[s]:starts[s] + n]
        assert np.array_equal(got[starts[s]:starts[s] + n], np.argsort(seg, kind="stable"))


def test_the_check_catches_a_wrong_offset():
    """The model's assertions are live: one digit offset moved by one row
    (a plausible slip in the scan arithmetic) trips them."""
    rng = np.random.default_rng(3)
    keys = rng.integers(0, 1 << 16, 9000, dtype=np.int64)
    vals = np.arange(9000, dtype=np.int64)
    real_cumsum = np.cumsum

    def shifted(a, axis=None):
        out = real_cumsum(a, axis=axis)
        if axis == 1:
            out = out.copy()
            out[7, 1:] += 1
        return out

    np.cumsum = shifted
    try:
        with pytest.raises(AssertionError):
            one_pass(keys, vals, [9000], 0)
    finally:
        np.cumsum = real_cumsum
