"""Pin the C oracle (CPU only).

Every oracle function is checked against something that does not restate it:
brute-force constructions, exhaustive enumeration, exact rational arithmetic,
numpy library routines, known answers, the invariants of the reference's own
tests (torchbvh tests/test_bvh_build.py:65-130, tests/test_knn.py) and, for
k-NN, two different algorithms (branch-and-bound vs brute force) that must
agree exactly.
"""

from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

import oracle
from parity import (
    assert_same_f32,
    assert_same_int,
    boundary_cloud,
    knn_pathological_clouds,
    pathological_clouds,
    single_child_cloud,
    unit_direction_points,
)


# ---------------------------------------------------------------------------
# Implicit tree closed forms vs a brute-force heap
# ---------------------------------------------------------------------------
def brute_tree(n: int):
    """Build the heap explicitly: 2^L leaf slots, the first n real; an
    internal node is real iff a child is; storage rows are ranks of real
    nodes in heap order."""
    L = 0
    while (1 << L) < n:
        L += 1
    size = (1 << (L + 1)) - 1
    real = np.zeros(size, bool)
    first_leaf = (1 << L) - 1
    real[first_leaf:first_leaf + n] = True
    for i in range(first_leaf - 1, -1, -1):
        real[i] = real[2 * i + 1] or real[2 * i + 2]
    rank = np.cumsum(real) - 1
    return L, real, rank


@pytest.mark.parametrize("n", list(range(1, 700)) + [1000, 1023, 1024, 1025, 4097, 10000, 65535])
def test_tree_closed_forms_match_brute_force_heap(n):
    L, real, rank = brute_tree(n)
    assert oracle.leaf_level(n) == L
    assert oracle.virtual_leaves(n) == (1 << L) - n
    assert oracle.real_node_count(n) == int(real.sum())
    for i in range(real.size):
        assert oracle.is_virtual(n, i) == (not real[i])
        if real[i]:
            assert oracle.memory_index(n, i) == rank[i]


@pytest.mark.parametrize(
    "n,nr,vl,L",
    [(10_000, 20_005, 6_384, 14), (1 << 20, 2_097_151, 0, 20), (65_536, 131_071, 0, 16),
     (1 << 22, 8_388_607, 0, 22), (200_000, None, 62_144, 18)],
)
def test_tree_facts_at_baseline_sizes(n, nr, vl, L):
    if nr is None:
        nr = int(brute_tree(n)[1].sum())
    assert oracle.real_node_count(n) == nr
    assert oracle.virtual_leaves(n) == vl
    assert oracle.leaf_level(n) == L


# ---------------------------------------------------------------------------
# Morton codes
# ---------------------------------------------------------------------------
def interleave(values: list[int], bits: int) -> int:
    out = 0
    D = len(values)
    for b in range(bits):
        for d, v in enumerate(values):
            out |= ((v >> b) & 1) << (D * b + d)
    return out


def test_spread_functions_exhaustive():
    assert oracle.split3(1023) == 0x09249249
    assert oracle.split2(0xFFFF) == 0x55555555
    for v in range(1024):
        assert oracle.split3(v) == sum(((v >> b) & 1) << (3 * b) for b in range(10))
    vs = np.arange(65536)
    expect = np.zeros_like(vs)
    for b in range(16):
        expect |= ((vs >> b) & 1) << (2 * b)
    got = np.array([oracle.split2(int(v)) for v in vs])
    assert np.array_equal(got, expect)


def test_morton_known_answers_3d():
    lo = np.zeros(3, np.float32)
    hi = np.ones(3, np.float32)
    pts = np.array([
        [0, 0, 0], [1, 1, 1], [1, 0, 0], [0, 1, 0], [0, 0, 1],
        [0.5, 0, 0], [0.25, 0.5, 0.75], [-5, 7, 0.5],
    ], np.float32)
    codes = oracle.morton_codes(pts, lo, hi)
    s = 0x09249249
    assert codes[0] == 0
    assert codes[1] == (1 << 30) - 1
    assert codes[2] == s and codes[3] == s << 1 and codes[4] == s << 2
    assert codes[5] == 1 << 27  # x cell 512: bit 9 of x -> bit 27
    assert codes[6] == interleave([256, 512, 768], 10)
    assert codes[7] == interleave([0, 1023, 512], 10)  # clamped outside the box


def test_morton_known_answers_2d_and_degenerate_axes():
    lo = np.array([-1, 2], np.float32)
    hi = np.array([3, 2], np.float32)  # axis 1 has zero extent -> cell 0
    pts = np.array([[-1, 2], [3, 2], [1, 100], [2, -100]], np.float32)
    codes = oracle.morton_codes(pts, lo, hi)
    assert codes[0] == 0
    assert codes[1] == 0x55555555  # x cell 65535, y cell 0
    assert codes[2] == interleave([32768, 0], 16)
    assert codes[3] == interleave([49152, 0], 16)
    full = oracle.morton_codes(np.array([[3, 5]], np.float32), np.array([-1, 1], np.float32),
                               np.array([3, 5], np.float32))
    assert full[0] == 0xFFFFFFFF


def test_morton_matches_numpy_ieee_quantisation():
    rng = np.random.default_rng(5)
    for D, bins, nbits in ((3, 1024, 10), (2, 65536, 16)):
        pts = (rng.standard_normal((5000, D)) * 3).astype(np.float32)
        lo, hi = oracle.bounds(pts)
        u = np.clip((pts - lo) / (hi - lo), np.float32(0), np.float32(1)).astype(np.float32)
        cells = np.minimum((u * np.float32(bins)).astype(np.uint32), bins - 1)
        expect = [interleave([int(c) for c in row], nbits) for row in cells]
        got = oracle.morton_codes(pts, lo, hi)
        assert np.array_equal(got.astype(np.int64), np.array(expect, np.int64))


def test_stable_argsort_matches_numpy_stable():
    rng = np.random.default_rng(7)
    for n, hi in ((1, 4), (2, 2), (1000, 8), (4097, 1 << 30), (70_000, 50)):
        keys = rng.integers(0, hi, n, dtype=np.uint32)
        assert_same_int(oracle.stable_argsort(keys), np.argsort(keys, kind="stable"), "argsort")


@pytest.mark.parametrize("dim", [2, 3])
def test_schedule_order_is_stable_sort_on_top_16_hilbert_bits(dim):
    """The schedule is pinned by its definition through a plain Python sort
    on (hilbert >> (bits - 16), query index) over the Hilbert indices of the
    queries' Morton cells (cells recomputed here with numpy's IEEE fp32
    quantisation): a wrong shift, an unstable sort, a full-code sort or the
    Morton curve all fail it."""
    rng = np.random.default_rng(61 + dim)
    q = rng.random((3000, dim), dtype=np.float32)
    lo = np.zeros(dim, np.float32)
    hi = np.ones(dim, np.float32)
    b = 10 if dim == 3 else 16
    cells = np.minimum((q * np.float32(1 << b)).astype(np.uint32), (1 << b) - 1)
    hil = oracle.hilbert_of_cells(cells, b).astype(np.int64)
    assert_same_int(oracle.hilbert_codes(q, lo, hi).astype(np.int64), hil, "hilbert codes")
    shift = (30 if dim == 3 else 32) - 16
    want = sorted(range(len(hil)), key=lambda i: (hil[i] >> shift, i))
    got = oracle.schedule_order(q, lo, hi)
    assert_same_int(got, np.array(want, np.int64), "schedule")
    codes = oracle.morton_codes(q, lo, hi).astype(np.int64)
    morton_sched = sorted(range(len(codes)), key=lambda i: (codes[i] >> shift, i))
    assert not np.array_equal(got, np.array(morton_sched))


def all_cells(dim: int, b: int) -> np.ndarray:
    axes = np.meshgrid(*[np.arange(1 << b)] * dim, indexing="ij")
    return np.stack([a.ravel() for a in axes], axis=1).astype(np.uint32)


@pytest.mark.parametrize("dim", [2, 3])
def test_hilbert_top_levels_depend_only_on_top_cell_levels(dim):
    """The schedule sorts on the top 16 index bits, and the GPU key computes
    only those: the index of the top 6 (3-D) / 8 (2-D) levels of the cell.
    That equals the full index's top bits (self-similarity)."""
    b, top = (10, 6) if dim == 3 else (16, 8)
    rng = np.random.default_rng(77 + dim)
    cells = rng.integers(0, 1 << b, (100_000, dim)).astype(np.uint32)
    full = oracle.hilbert_of_cells(cells, b).astype(np.uint64)
    coarse = oracle.hilbert_of_cells((cells >> (b - top)).astype(np.uint32), top).astype(np.uint64)
    assert np.array_equal(full >> np.uint64(dim * (b - top)), coarse)


@pytest.mark.parametrize("dim", [2, 3])
def test_hilbert_index_at_full_resolution_on_aligned_subcubes(dim):
    """At the schedule's resolution (10 bits per axis in 3-D, 16 in 2-D) the
    grid is too large to enumerate; by the prefix property every aligned
    sub-cube is a contiguous index range and a jump-free path through it,
    checked on random aligned 8^3 / 32^2 sub-cubes."""
    b = 10 if dim == 3 else 16
    side = 8 if dim == 3 else 32
    rng = np.random.default_rng(900 + dim)
    local = all_cells(dim, side.bit_length() - 1)
    for _ in range(20):
        corner = rng.integers(0, (1 << b) // side, dim) * side
        cells = (local + corner).astype(np.uint32)
        h = oracle.hilbert_of_cells(cells, b).astype(np.int64)
        hs = np.sort(h)
        assert hs[-1] - hs[0] == len(h) - 1, "not a contiguous range"
        path = cells[np.argsort(h)].astype(np.int64)
        assert np.all(np.abs(np.diff(path, axis=0)).sum(1) == 1)


@pytest.mark.parametrize("dim,b", [(2, 1), (2, 2), (2, 3), (2, 5), (3, 1), (3, 2), (3, 3), (3, 4)])
def test_hilbert_index_is_a_hilbert_curve(dim, b):
    """What makes an order a Hilbert curve, checked on every cell of small
    grids: a bijection onto [0, 2^(D*b)) starting at the origin, consecutive
    indices at unit L1 distance (no jumps), and every prefix of D*k bits
    covering exactly one aligned cube of side 2^(b-k)."""
    cells = all_cells(dim, b)
    h = oracle.hilbert_of_cells(cells, b).astype(np.int64)
    assert_same_int(np.sort(h), np.arange(len(h)), "bijection")
    path = cells[np.argsort(h)].astype(np.int64)
    assert np.all(path[0] == 0)
    assert np.all(np.abs(np.diff(path, axis=0)).sum(1) == 1), "consecutive cells must be adjacent"
    for k in range(1, b + 1):
        side = 1 << (b - k)
        for prefix in np.unique(h >> (dim * (b - k))):
            members = cells[(h >> (dim * (b - k))) == prefix].astype(np.int64)
            corner = members.min(0)
            assert np.all(corner % side == 0) and np.all(members.max(0) - corner == side - 1)
            assert len(members) == side ** dim


@pytest.mark.parametrize("dim", [2, 3])
def test_routed_order_is_stable_sort_on_route_then_code(dim):
    """Pinned by its definition through a plain Python sort on (route, code of
    the route's bounds, query index); 2-D needs the 33rd key bit."""
    rng = np.random.default_rng(81 + dim)
    q = rng.random((2500, dim), dtype=np.float32)
    routes = rng.random(2500) < 0.4
    tlo, thi = np.zeros(dim, np.float32), np.ones(dim, np.float32)
    flo, fhi = np.full(dim, -1.0, np.float32), np.full(dim, 2.0, np.float32)
    ct = oracle.morton_codes(q, tlo, thi).astype(np.int64)
    cf = oracle.morton_codes(q, flo, fhi).astype(np.int64)
    want = sorted(range(len(q)), key=lambda i: (int(routes[i]), ct[i] if routes[i] else cf[i], i))
    got = oracle.routed_order(q, routes, tlo, thi, flo, fhi)
    assert_same_int(got, np.array(want, np.int64), "routed order")


def test_routed_knn_offsets_false_route_indices():
    rng = np.random.default_rng(91)
    tp = rng.random((300, 3), dtype=np.float32)
    fp = rng.random((200, 3), dtype=np.float32) + 5.0
    q = np.concatenate((tp[:5], fp[:5])).astype(np.float32)
    routes = np.array([True] * 5 + [False] * 5)
    idx, dist = oracle.knn_routed(tp, fp, q, routes, 4)
    assert_same_int(idx[:5, 0], np.arange(5), "true self")
    assert_same_int(idx[5:, 0], 300 + np.arange(5), "false self, offset")
    assert (dist[:, 0] == 0).all()


def test_bounds_match_numpy_and_seed_semantics():
    rng = np.random.default_rng(9)
    p = rng.standard_normal((1000, 3)).astype(np.float32)
    lo, hi = oracle.bounds(p)
    assert_same_f32(lo, p.min(0), "lo")
    assert_same_f32(hi, p.max(0), "hi")
    # Seeds are +-1e30 (bvh_build.cu:466-467): coordinates beyond them clamp.
    big = np.full((4, 2), 3e30, np.float32)
    lo, hi = oracle.bounds(big)
    assert np.all(lo == np.float32(1e30)) and np.all(hi == np.float32(3e30))


@pytest.mark.parametrize("dim", [2, 3])
def test_point_order_equals_build_order_inside_the_seeds(dim):
    """Within +-1e30 the plain min/max of the point ordering equals the
    build's seeded bounds, so the two orders coincide."""
    rng = np.random.default_rng(30 + dim)
    for n in (1, 7, 5000):
        p = (rng.standard_normal((n, dim)) * 10).astype(np.float32)
        assert_same_int(oracle.morton_point_order(p), oracle.build(p)["sorted_indices"], f"n={n}")


@pytest.mark.parametrize("dim", [2, 3])
def test_point_order_spreads_clouds_beyond_the_seeds(dim):
    """A cloud along axis 0 lying entirely above 1e30, other axes constant:
    only axis 0 varies, so the codes order the points by their axis-0 cell
    over the points' own extent [min, max]: the minimum lands in cell 0, the
    maximum in the last cell, every cell step is at most one cell width of x,
    and ties keep input order.  The build's bounds stop at the 1e30 seed,
    which coarsens the cells and changes the order."""
    rng = np.random.default_rng(40 + dim)
    n = 4000
    p = np.zeros((n, dim), np.float32)
    p[:, 0] = (2e30 + rng.random(n) * 1e30).astype(np.float32)
    order = oracle.morton_point_order(p)
    x = p[order, 0].astype(np.float64)
    width = (p[:, 0].max() - p[:, 0].min()) / (1024 if dim == 3 else 65536)
    lo, hi = float(p[:, 0].min()), float(p[:, 0].max())
    assert x[0] - lo <= width * 1.0001 and hi - x[-1] <= width * 1.0001  # first and last cells
    assert np.all(np.diff(x) >= -width * 1.0001)
    # Ties within a cell keep input order (cells well inside their bounds,
    # so float64 rounding here cannot put a point in a neighbouring cell).
    cells = (x - lo) / width
    inner = np.abs(cells - np.round(cells)) > 1e-3
    for c in np.unique(np.floor(cells[inner]))[:50]:
        run = order[inner & (np.floor(cells) == c)]
        assert np.all(np.diff(run) > 0)
    assert not np.array_equal(order, oracle.build(p)["sorted_indices"])


# ---------------------------------------------------------------------------
# Build: reference invariants + brute-force subtree boxes
# ---------------------------------------------------------------------------
def check_build(points: np.ndarray) -> dict:
    n, D = points.shape
    b = oracle.build(points)
    L, real, _ = brute_tree(n)
    nr = int(real.sum())
    nodes = b["node_aabbs"]
    assert nodes.shape == (nr, 2 * D)
    assert b["num_real_nodes"] == nr and b["leaf_level"] == L
    assert b["virtual_leaves"] == (1 << L) - n
    # sorted_indices: the stable Morton order of the points.
    lo, hi = points.min(0), points.max(0)
    assert_same_f32(b["scene_min"], lo, "scene_min")
    assert_same_f32(b["scene_max"], hi, "scene_max")
    codes = oracle.morton_codes(points, lo, hi)
    assert_same_int(b["sorted_indices"], np.argsort(codes, kind="stable"), "sorted_indices")
    sp = points[b["sorted_indices"]]
    check_tree(b, sp, sp)
    return b


def check_tree(b: dict, leaf_lo: np.ndarray, leaf_hi: np.ndarray) -> None:
    """Every real node's box is the union of its leaf range's boxes (leaf
    boxes in sorted order); traversal arrays follow the heap."""
    n, D = leaf_lo.shape
    L, real, rank = brute_tree(n)
    nodes = b["node_aabbs"]
    first_leaf = (1 << L) - 1
    for i in np.nonzero(real)[0]:
        level = int(i + 1).bit_length() - 1
        span = 1 << (L - level)
        a = (i - ((1 << level) - 1)) * span
        box = nodes[rank[i]]
        assert_same_f32(box[:D], leaf_lo[a:min(a + span, n)].min(0), f"node {i} lo")
        assert_same_f32(box[D:], leaf_hi[a:min(a + span, n)].max(0), f"node {i} hi")
        row = rank[i]
        if i >= first_leaf:
            assert b["left_child_mem"][row] == -1 and b["right_child_mem"][row] == -1
            assert b["mem_to_leaf"][row] == i - first_leaf
        else:
            assert b["left_child_mem"][row] == rank[2 * i + 1]
            assert b["right_child_mem"][row] == (rank[2 * i + 2] if real[2 * i + 2] else -1)
            assert b["mem_to_leaf"][row] == -1


@pytest.mark.parametrize("case", range(len(pathological_clouds())))
def test_build_pathological_clouds(case):
    check_build(pathological_clouds()[case])


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("n", [1, 2, 3, 4, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65])
def test_build_boundary_sizes(n, dim):
    check_build(boundary_cloud(n, dim))


@pytest.mark.parametrize("n", [3, 5, 6, 9, 10, 17, 18])
def test_build_single_child_nodes(n):
    check_build(single_child_cloud(n))


@pytest.mark.parametrize("n,dim", [(1000, 3), (777, 2), (5000, 3)])
def test_build_random(n, dim):
    rng = np.random.default_rng(n + dim)
    check_build(rng.random((n, dim), dtype=np.float32))


def test_build_degenerate_extent_is_constant():
    b = check_build(np.array([[7.0, -3.0]] * 3, np.float32))
    assert np.all(b["node_aabbs"] == np.array([7.0, -3.0, 7.0, -3.0], np.float32))


# ---------------------------------------------------------------------------
# Primitive build: numpy boxes / centres / bounds, brute-force node boxes,
# and the reduction to the point build for degenerate primitives
# ---------------------------------------------------------------------------
def check_build_primitives(prims: np.ndarray) -> dict:
    n, V, D = prims.shape
    b = oracle.build_primitives(prims)
    L, real, _ = brute_tree(n)
    assert b["node_aabbs"].shape == (int(real.sum()), 2 * D) and b["leaf_level"] == L
    box_lo, box_hi = prims.min(1), prims.max(1)
    centers = prims[:, 0, :].copy()
    for v in range(1, V):
        centers = centers + prims[:, v, :]  # float32, vertex order
    centers = centers / np.float32(V)
    assert_same_f32(b["centers"], centers, "centers")
    lo, hi = box_lo.min(0), box_hi.max(0)
    assert_same_f32(b["scene_min"], lo, "scene_min")
    assert_same_f32(b["scene_max"], hi, "scene_max")
    codes = oracle.morton_codes(centers, lo, hi)
    assert_same_int(b["sorted_indices"], np.argsort(codes, kind="stable"), "sorted_indices")
    order = b["sorted_indices"]
    check_tree(b, box_lo[order], box_hi[order])
    return b


def random_primitives(rng, n: int, V: int, D: int, spread: float = 0.05) -> np.ndarray:
    """Primitives around random anchors in [-2, 2]^D, edges up to `spread`."""
    anchor = rng.random((n, 1, D), dtype=np.float32) * 4 - 2
    return (anchor + (rng.random((n, V, D), dtype=np.float32) - 0.5) * spread).astype(np.float32)


@pytest.mark.parametrize("V,D", [(2, 2), (3, 3)])
@pytest.mark.parametrize("n", [1, 2, 3, 5, 16, 17, 37, 1000])
def test_build_primitives_random(n, V, D):
    check_build_primitives(random_primitives(np.random.default_rng(100 * n + D), n, V, D))


@pytest.mark.parametrize("V,D", [(2, 2), (3, 3)])
def test_build_primitives_long_overlapping_edges(V, D):
    # Boxes spanning most of the scene: node boxes are far from the centres'.
    rng = np.random.default_rng(7 + D)
    check_build_primitives((rng.random((300, V, D), dtype=np.float32) * 4 - 2).astype(np.float32))


@pytest.mark.parametrize("V,D", [(2, 2), (3, 3)])
def test_build_primitives_degenerate_reduce_to_point_build(V, D):
    # Every vertex equal, on a 1/64 grid: the vertex sum is exact, so the
    # centre is the point and each leaf box is the point's; the primitive
    # build must then equal the (separately pinned) point build field by field.
    rng = np.random.default_rng(21 + D)
    pts = (rng.integers(-128, 128, (513, D)) / 64.0).astype(np.float32)
    prims = np.repeat(pts[:, None, :], V, axis=1)
    pb, b = check_build_primitives(prims), oracle.build(pts)
    for key in ("node_aabbs", "scene_min", "scene_max"):
        assert_same_f32(pb[key], b[key], key)
    for key in ("sorted_indices", "left_child_mem", "right_child_mem", "mem_to_leaf"):
        assert_same_int(pb[key], b[key], key)


def test_build_primitives_bounds_take_box_corners_not_centres():
    # Two segments whose centres coincide: scene bounds still cover the
    # vertices, and both leaves carry their own boxes.
    prims = np.array([[[0.0, 0.0], [2.0, 2.0]], [[0.0, 2.0], [2.0, 0.0]]], np.float32)
    b = check_build_primitives(prims)
    assert_same_f32(b["scene_min"], np.zeros(2, np.float32), "scene_min")
    assert_same_f32(b["scene_max"], np.full(2, 2.0, np.float32), "scene_max")
    assert_same_f32(b["centers"], np.ones((2, 2), np.float32), "centers")
    assert_same_int(b["sorted_indices"], np.array([0, 1]), "equal codes keep input order")


# ---------------------------------------------------------------------------
# Distances: the fused chain, checked with exact rational arithmetic
# ---------------------------------------------------------------------------
def round_f32(x: Fraction) -> np.float32:
    """Correctly round a rational to fp32 (nearest, ties to even)."""
    if x == 0:
        return np.float32(0)
    c = np.float32(float(x))
    cands = {c, np.nextafter(c, np.float32(np.inf)), np.nextafter(c, np.float32(-np.inf))}
    best = min(cands, key=lambda v: (abs(Fraction(float(v)) - x),
                                     int(np.array([v], np.float32).view(np.uint32)[0]) & 1))
    return np.float32(best)


def fused_chain(q, p) -> np.float32:
    s = None
    for d in range(len(q)):
        delta = abs(Fraction(float(np.float32(q[d]) - np.float32(p[d]))))
        s = round_f32(delta * delta) if s is None else round_f32(delta * delta + Fraction(float(s)))
    return s


def test_point_distance_is_correctly_rounded_fma_chain():
    rng = np.random.default_rng(11)
    for D in (2, 3):
        for _ in range(1500):
            scale = 10.0 ** rng.integers(-4, 5)
            q = (rng.standard_normal(D) * scale).astype(np.float32)
            p = (q + rng.standard_normal(D).astype(np.float32) * np.float32(scale * 1e-3)).astype(np.float32)
            got = np.float32(oracle.point_distance(q, p))
            assert_same_f32(got, fused_chain(q, p), f"dist {q} {p}")


# ---------------------------------------------------------------------------
# k-NN: branch-and-bound == brute force; brute force vs float64 truth
# ---------------------------------------------------------------------------
def check_knn(points, queries, k):
    bi, bd = oracle.knn_brute(points, queries, k)
    ti, td = oracle.knn(points, queries, k)
    assert_same_int(ti, bi, "bvh vs brute indices")
    assert_same_f32(td, bd, "bvh vs brute distances")
    # Rows ascending lexicographically.
    assert np.all((bd[:, :-1] < bd[:, 1:]) | ((bd[:, :-1] == bd[:, 1:]) & (bi[:, :-1] < bi[:, 1:])))
    # Against float64 truth: the chosen set is optimal up to rounding.
    p64 = points.astype(np.float64)
    for r in range(queries.shape[0]):
        d64 = ((queries[r].astype(np.float64) - p64) ** 2).sum(1)
        kth = np.sort(d64)[k - 1]
        chosen = d64[bi[r]]
        assert np.all(chosen <= kth * (1 + 1e-6) + 1e-30)
        np.testing.assert_allclose(bd[r], chosen, rtol=1e-6, atol=1e-30)
    return bi, bd


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 8, 16, 32])
def test_knn_uniform(dim, k):
    rng = np.random.default_rng(1000 + dim * 10 + k)
    check_knn(rng.random((300, dim), dtype=np.float32), rng.random((60, dim), dtype=np.float32), k)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 8, 16])
def test_knn_self_query(dim, k):
    rng = np.random.default_rng(2000 + dim * 10 + k)
    p = rng.random((48, dim), dtype=np.float32)
    bi, bd = check_knn(p, p, k)
    assert np.all(bd[:, 0] == 0) and np.array_equal(bi[:, 0], np.arange(48))


@pytest.mark.parametrize("case", range(len(knn_pathological_clouds())))
def test_knn_pathological(case):
    p, k = knn_pathological_clouds()[case]
    check_knn(p, p[: min(7, p.shape[0])] + np.float32(0.125), k)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 8, 16])
def test_knn_ties_resolve_to_lowest_index(dim, k):
    p = unit_direction_points(dim)
    q = np.zeros((2, dim), np.float32)
    bi, bd = check_knn(p, q, k)
    assert np.all(bd == 1.0)
    assert np.array_equal(bi, np.tile(np.arange(k), (2, 1)))
    dup = np.full((20, dim), 3.5, np.float32)
    bi, bd = check_knn(dup, np.full((3, dim), 3.5, np.float32), k)
    assert np.all(bd == 0) and np.array_equal(bi, np.tile(np.arange(k), (3, 1)))


def test_knn_clustered_and_duplicates_large():
    rng = np.random.default_rng(3)
    centres = rng.random((8, 3)).astype(np.float32)
    p = (centres[rng.integers(0, 8, 20_000)] + 0.02 * rng.standard_normal((20_000, 3))).astype(np.float32)
    p[100:200] = p[5]  # a block of exact duplicates
    q = (p[:400] + 0.005 * rng.standard_normal((400, 3))).astype(np.float32)
    bi, bd = oracle.knn_brute(p, q, 32)
    ti, td = oracle.knn(p, q, 32)
    assert_same_int(ti, bi, "indices")
    assert_same_f32(td, bd, "distances")


def test_torch_bruteforce_agrees_with_oracle_away_from_near_ties():
    import torch

    from oracle.torch_bruteforce import knn_bruteforce

    rng = np.random.default_rng(21)
    p = rng.random((4000, 3), dtype=np.float32)
    q = rng.random((300, 3), dtype=np.float32)
    ti, td = knn_bruteforce(torch.from_numpy(p), torch.from_numpy(q), 16)
    oi, od = oracle.knn_brute(p, q, 16)
    np.testing.assert_allclose(td.numpy(), od, rtol=1e-6, atol=0)
    gaps = np.diff(od, axis=1)
    safe = np.all(gaps > 1e-5 * od[:, 1:], axis=1)
    assert np.array_equal(ti.numpy()[safe], oi[safe])
