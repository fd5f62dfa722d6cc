"""GPU build parity against the oracle: Morton codes, sort permutation,
scene bounds, node AABBs and traversal arrays must be bit-exact.

Point sets restate the reference's build tests (torchbvh
tests/test_bvh_build.py:133-340) plus sizes around this library's tile and
subtree boundaries (4096-key sort tiles, 256-leaf tree groups)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import torchbvh_amd as tb
from parity import (
    assert_same_f32,
    assert_same_int,
    boundary_cloud,
    pathological_clouds,
    single_child_cloud,
)
from torchbvh_amd import _native
from torchbvh_amd._native import _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def check_single_build(points: np.ndarray) -> None:
    h = tb.build_bvh(dev(points))
    ref = oracle.build(points)
    for key in ("num_leaves", "num_real_nodes", "leaf_level", "virtual_leaves", "dim"):
        assert h[key] == ref[key], key
    assert "batch_size" not in h
    for key in ("scene_min", "scene_max", "node_aabbs"):
        assert tuple(h[key].shape) == ref[key].shape, key
        assert_same_f32(h[key].cpu().numpy(), ref[key], key)
    for key in ("sorted_indices", "left_child_mem", "right_child_mem", "mem_to_leaf"):
        t = h[key]
        assert t.dtype == (torch.int64 if key == "sorted_indices" else torch.int32), key
        assert_same_int(t.cpu().numpy(), ref[key], key)


@pytest.mark.parametrize("case", range(len(pathological_clouds())))
def test_build_pathological_clouds(case):
    check_single_build(pathological_clouds()[case])


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("n", [1, 2, 3, 4, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65])
def test_build_boundary_sizes(n, dim):
    check_single_build(boundary_cloud(n, dim))


@pytest.mark.parametrize("n", [3, 5, 6, 9, 10, 17, 18])
def test_build_single_child_nodes(n):
    check_single_build(single_child_cloud(n))


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("n", [255, 256, 257, 4095, 4096, 4097, 8193, 65536, 65537, 100_003])
def test_build_random_sizes_around_tiles(n, dim):
    rng = np.random.default_rng(n * 10 + dim)
    check_single_build(rng.random((n, dim), dtype=np.float32))


@pytest.mark.parametrize("dim", [2, 3])
def test_build_heavy_duplicates_keep_stable_order(dim):
    rng = np.random.default_rng(77 + dim)
    pts = rng.integers(0, 4, (20_000, dim)).astype(np.float32)  # few distinct codes
    check_single_build(pts)


@pytest.mark.parametrize("dim", [2, 3])
def test_batched_build_matches_per_cloud_oracle(dim):
    rng = np.random.default_rng(500 + dim)
    pts = rng.random((5, 3000, dim), dtype=np.float32)
    pts[2] *= 1e4
    pts[3] = 0.5  # fully degenerate cloud
    h = tb.build_bvh(dev(pts))
    assert isinstance(h, tb.BatchedBVHHandle) and h["batch_size"] == 5
    ref = oracle.build_batched(pts)
    for key in ("scene_min", "scene_max", "node_aabbs"):
        assert_same_f32(h[key].cpu().numpy(), ref[key], key)
    for key in ("sorted_indices", "left_child_mem", "right_child_mem", "mem_to_leaf"):
        assert_same_int(h[key].cpu().numpy(), ref[key], key)


def test_ragged_build_matches_per_cloud_oracle():
    rng = np.random.default_rng(900)
    counts = [1, 2, 4096, 4097, 300, 70_000, 17, 9000]
    pts = np.concatenate([rng.random((c, 3), dtype=np.float32) * (b + 1) for b, c in enumerate(counts)])
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    h = tb.build_bvh(dev(pts), batch_offsets=dev(offsets))
    assert isinstance(h, tb.RaggedBVHHandle)
    assert h["batch_size"] == len(counts)
    inner = h._handles
    for b, c in enumerate(counts):
        ref = oracle.build(pts[offsets[b]:offsets[b + 1]])
        for key in ("scene_min", "scene_max", "node_aabbs"):
            assert_same_f32(inner[b][key].cpu().numpy(), ref[key], f"cloud {b} {key}")
        for key in ("sorted_indices", "left_child_mem", "right_child_mem", "mem_to_leaf"):
            assert_same_int(inner[b][key].cpu().numpy(), ref[key], f"cloud {b} {key}")
        for key in ("num_leaves", "num_real_nodes", "leaf_level", "virtual_leaves"):
            assert inner[b][key] == ref[key]


@pytest.mark.parametrize("dim", [2, 3])
def test_morton_codes_bit_exact(dim):
    rng = np.random.default_rng(31 + dim)
    pts = (rng.standard_normal((3, 9000, dim)) * np.array([1.0, 1e3, 1e-3][:dim])).astype(np.float32)
    lo = np.stack([oracle.bounds(p)[0] for p in pts])
    hi = np.stack([oracle.bounds(p)[1] for p in pts])
    hi[1, 0] = lo[1, 0]  # a zero-extent axis
    codes = _C.morton_codes(dev(pts), dev(lo), dev(hi)).cpu().numpy()
    for b in range(3):
        assert_same_int(codes[b], oracle.morton_codes(pts[b], lo[b], hi[b]).astype(np.int64), f"codes {b}")


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("m", [1, 100, 4096, 4097, 50_000])
def test_query_order_bit_exact(dim, m):
    rng = np.random.default_rng(m + dim)
    q = rng.random((2, m, dim), dtype=np.float32) * 1.2 - 0.1  # some outside the scene box
    lo = np.zeros((2, dim), np.float32)
    hi = np.ones((2, dim), np.float32)
    order = _C.morton_sort_queries_narrow(dev(q), dev(lo), dev(hi)).cpu().numpy()
    for b in range(2):
        assert_same_int(order[b], oracle.query_order(q[b], lo[b], hi[b]), f"order {b}")


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("m", [1, 100, 4097, 50_000])
def test_schedule_order_bit_exact(dim, m):
    rng = np.random.default_rng(7 * m + dim)
    q = rng.random((2, m, dim), dtype=np.float32) * 1.2 - 0.1
    lo = np.zeros((2, dim), np.float32)
    hi = np.ones((2, dim), np.float32)
    order = _C.morton_sort_queries_narrow(dev(q), dev(lo), dev(hi), schedule=True).cpu().numpy()
    for b in range(2):
        assert_same_int(order[b], oracle.schedule_order(q[b], lo[b], hi[b]), f"schedule {b}")


def test_schedule_order_ragged_bit_exact():
    rng = np.random.default_rng(77)
    counts = [5, 0, 4097, 300]
    q = rng.random((sum(counts), 3), dtype=np.float32)
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    lo = np.zeros((4, 3), np.float32)
    hi = np.full((4, 3), 0.5, np.float32)
    order = _C.morton_sort_queries_ragged(dev(q), dev(offsets), dev(lo), dev(hi), 4,
                                          schedule=True).cpu().numpy()
    for b, c in enumerate(counts):
        seg = slice(offsets[b], offsets[b + 1])
        assert_same_int(order[seg], oracle.schedule_order(q[seg], lo[b], hi[b]), f"cloud {b}")


def test_build_is_deterministic_across_calls():
    rng = np.random.default_rng(5)
    p = dev(rng.random((50_000, 3), dtype=np.float32))
    a = tb.build_bvh(p)
    b = tb.build_bvh(p)
    assert torch.equal(a["node_aabbs"], b["node_aabbs"])
    assert torch.equal(a["sorted_indices"], b["sorted_indices"])


def assert_same_accel(a: torch.Tensor, b: torch.Tensor, counts: list[int], dim: int) -> None:
    """Accel buffers agree on every byte traversal can read: the `total`
    16-byte points, the records reachable from each cloud's root (boxes,
    child refs, parent link) and the bucket parent links (the last word of
    the row where each bucket starts).  Nothing else is ever written: the
    records of ranges that fit one bucket, the other last words, the
    padding after the points."""
    assert a.shape == b.shape
    total = sum(counts)
    pts = total * 16
    assert torch.equal(a[:pts], b[:pts]), "accel points differ"
    off = (pts + 255) // 256 * 256
    width = 4 * dim + 4
    ra = a[off:].cpu().numpy().view(np.int32).reshape(-1, width)
    rb = b[off:].cpu().numpy().view(np.int32).reshape(-1, width)
    assert ra.shape[0] == total
    start = 0
    for c, n in enumerate(counts):
        base = start  # cloud c's record rows follow its point rows
        start += n
        if n < 2:
            continue
        frontier = np.array([0])
        while frontier.size:
            rows = base + frontier
            assert np.array_equal(ra[rows, :width - 1], rb[rows, :width - 1]), f"cloud {c}: records differ"
            refs = rb[rows, 4 * dim:4 * dim + 2].ravel()
            buckets = base + (refs[refs < 0] & 0x0FFFFFFF)
            assert np.array_equal(ra[buckets, width - 1], rb[buckets, width - 1]), f"cloud {c}: bucket links differ"
            frontier = refs[refs >= 0]


def _standalone_accel(points: torch.Tensor, h) -> torch.Tensor:
    data = {k: h[k][None] for k in ("sorted_indices", "node_aabbs", "scene_min", "scene_max")}
    return _C.build_accel(points[None], data)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("n", [1, 5, 4097, 200_001])
def test_fused_accel_matches_standalone_build(n, dim):
    """The build that also emits the accel (one launch sequence) and the
    accel built afterwards from the finished BVH hold the same bytes."""
    rng = np.random.default_rng(n + 7 * dim)
    p = dev(rng.random((n, dim), dtype=np.float32))
    h = tb.build_bvh(p)
    fused = h._aux["accel"]
    assert fused is not None
    assert_same_accel(fused, _standalone_accel(p, h), [n], dim)


@pytest.mark.parametrize("dim", [2, 3])
def test_fused_accel_matches_standalone_above_the_cooperative_span_limit(dim):
    """Calls of more than 1.5M points finish the spanning radix-tree nodes
    in two phases (one lane per node of short extent, a sub-group of eight
    per longer one); calls up to it, a sub-group per node.  Both hold the
    standalone build's bytes (one lane and binary searches per node)."""
    rng = np.random.default_rng(90 + dim)
    p = dev(rng.random((1_700_000, dim), dtype=np.float32))
    h = tb.build_bvh(p)
    assert_same_accel(h._aux["accel"], _standalone_accel(p, h), [p.shape[0]], dim)


def test_fused_accel_matches_standalone_ragged():
    rng = np.random.default_rng(41)
    counts = [1, 3, 4096, 9000, 70_001, 2]
    pts = np.concatenate([rng.random((c, 3), dtype=np.float32) * (b + 1) for b, c in enumerate(counts)])
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    p, o = dev(pts), dev(offsets)
    h = tb.build_bvh(p, batch_offsets=o)
    fused = h._aux["accel"]
    packed = {k: h._aux["packed"][k] for k in ("sorted_indices", "node_aabbs", "scene_min", "scene_max")}
    assert_same_accel(fused, _C.build_accel_ragged(p, o, packed, counts), counts, 3)


def test_build_million_points_many_tiles():
    """245 sort tiles per pass: offsets scanned over many tiles and the
    reduction of many tile boxes, bit-exact against the oracle."""
    rng = np.random.default_rng(2024)
    check_single_build(rng.random((1_000_000, 3), dtype=np.float32))


def _check_accel_boxes(points: np.ndarray, accel: torch.Tensor, sorted_idx: np.ndarray, dim: int) -> int:
    """Walks the accel from the root: each record's child refs determine the
    children's point ranges (a bucket ref names its range; an internal child
    of a node covering [lo, hi] with index g covers [lo, g] on the left,
    [g + 1, hi] on the right); every stored child box must equal the exact
    min/max of its points.  Also checks the parent links the traversal
    resumes through: every reached record's parent word names the record
    that referenced it (-1 at the root), and the last word of the row where
    each bucket starts names the record that references the bucket.
    Returns the number of records checked."""
    n = points.shape[0]
    width = 4 * dim + 4
    off = (n * 16 + 255) // 256 * 256
    recs = accel.cpu().numpy()[off:off + n * width * 4].view(np.float32).reshape(-1, width)
    refs = recs[:, 4 * dim:4 * dim + 2].copy().view(np.int32)
    links = recs[:, 4 * dim + 2:].copy().view(np.int32)
    sp = points[sorted_idx]  # Morton order
    stack = [(0, 0, n - 1, -1)]
    checked = 0
    while stack:
        node, lo, hi, parent = stack.pop()
        assert int(links[node, 0]) == parent, f"record {node}: parent link"
        lref, rref = int(refs[node, 0]), int(refs[node, 1])
        if lref < 0:
            split = (lref & 0x0FFFFFFF) + ((lref >> 28) & 7)
        else:
            split = lref
        ranges = ((lo, split), (split + 1, hi))
        for c, (a, b) in enumerate(ranges):
            box = recs[node, c * 2 * dim:(c + 1) * 2 * dim]
            want = np.concatenate((sp[a:b + 1].min(0), sp[a:b + 1].max(0)))
            assert np.array_equal(box.view(np.uint32), want.astype(np.float32).view(np.uint32)), \
                f"record {node} child {c} range [{a}, {b}]"
            ref = (lref, rref)[c]
            if ref >= 0:
                stack.append((ref, a, b, node))
            else:
                assert (ref & 0x0FFFFFFF) == a and ((ref >> 28) & 7) + 1 == b - a + 1
                assert int(links[a, 1]) == node, f"bucket at {a}: parent link"
        checked += 1
    return checked


@pytest.mark.parametrize("case", ["uniform3", "clustered3", "uniform2", "duplicates3"])
def test_accel_records_hold_exact_child_boxes(case):
    rng = np.random.default_rng({"uniform3": 71, "clustered3": 72, "uniform2": 73, "duplicates3": 74}[case])
    if case == "uniform3":
        p = rng.random((150_000, 3), dtype=np.float32)
    elif case == "uniform2":
        p = rng.random((60_000, 2), dtype=np.float32)
    elif case == "clustered3":
        c = rng.random((8, 3), dtype=np.float32)
        p = (c[rng.integers(0, 8, 80_000)] + 0.02 * rng.standard_normal((80_000, 3))).astype(np.float32)
    else:
        p = rng.integers(0, 6, (20_000, 3)).astype(np.float32)
    h = tb.build_bvh(dev(p))
    checked = _check_accel_boxes(p, h._aux["accel"], h["sorted_indices"].cpu().numpy(), p.shape[1])
    assert checked > p.shape[0] // 8


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("B,n", [(1, 1), (1, 6), (1, 4097), (3, 70_001), (1, 200_001)])
def test_accel_from_tree_matches_fused_build(B, n, dim):
    """An accel rebuilt from node_aabbs and sorted_indices alone (leaf rows
    as the points, bounds from the root box) holds the fused build's bytes."""
    rng = np.random.default_rng(B * n + dim)
    pts = rng.random((B, n, dim), dtype=np.float32)
    data = _C.build_bvh_batched_cooperative(dev(pts), with_accel=True)
    L = _native.load()
    nodes, sidx = data["node_aabbs"].clone(), data["sorted_indices"].clone()
    accel = _native._accel_from_tree(nodes, sidx, dim)
    torch.cuda.synchronize()
    assert accel is not None and accel.numel() == data["accel"].numel()
    assert _native._registered_accel(nodes, sidx) is accel
    assert_same_accel(data["accel"], accel, [n] * B, dim)
    del L


def test_accel_from_tree_recovers_bounds_beyond_the_seeds():
    """A cloud lying entirely above 1e30 on one axis: the build's bounds are
    the seed (1e30) there, not the root box's minimum; the rebuilt accel
    must use the same bounds, hence the same codes and tree."""
    rng = np.random.default_rng(17)
    pts = rng.random((1, 5000, 3), dtype=np.float32)
    pts[..., 1] = 2e30 + pts[..., 1] * 1e30
    data = _C.build_bvh_batched_cooperative(dev(pts), with_accel=True)
    accel = _native._accel_from_tree(data["node_aabbs"].clone(), data["sorted_indices"].clone(), 3)
    torch.cuda.synchronize()
    assert_same_accel(data["accel"], accel, [5000], 3)
