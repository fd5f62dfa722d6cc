"""Non-finite coordinates.  The reference's distance takes, per axis,
max(lo - q, max(0, q - hi)) (torchbvh/csrc/geometry.cuh:3-18); max returns
its non-NaN operand, so a NaN difference counts 0 on that axis: a NaN query
coordinate, or a query and a point both at the same infinity.  The accel's
leaf distance must agree with that bit for bit, and both traversals must
return the oracle's results (brute force and the reference's DFS over the
implicit tree) for queries with NaN or infinite coordinates and for clouds
with infinite coordinates.

A NaN point coordinate is different: the node boxes' min/max skip NaN, so
no box bounds that point's (zero) distance on the NaN axis, and which
NaN-coordinate points a traversal reports depends on the order it visits
the tree.  The implicit-tree traversal follows the reference's order and
must match the oracle's DFS; the accel must return rows that are sorted,
hold distinct indices and carry each index's true distance."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import torchbvh_amd as tb
from parity import assert_same_f32, assert_same_int
from torchbvh_amd._native import _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
INF, NAN = np.float32(np.inf), np.float32(np.nan)


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def both_paths(points: np.ndarray, queries: np.ndarray, k: int):
    """(accel result, implicit-tree result) for one cloud."""
    h = tb.build_bvh(dev(points))
    q = dev(queries)
    accel = tb.query_knn(h, q, k)
    nodes, sidx = h["node_aabbs"][None], h["sorted_indices"][None]
    imp = _C.query_knn_batched_cached_bounds(nodes, sidx, q[None], h["num_leaves"], h["num_real_nodes"],
                                              h["dim"], k, accel=False)
    torch.cuda.synchronize()
    out = [(accel[0].cpu().numpy(), accel[1].cpu().numpy()), (imp[0][0].cpu().numpy(), imp[1][0].cpu().numpy())]
    tb.destroy_bvh(h)
    return out


def queries_with_nonfinite(rng, m: int, dim: int) -> np.ndarray:
    q = rng.random((m, dim), dtype=np.float32)
    kinds = rng.integers(0, 5, (m, dim))
    q[kinds == 1] = NAN
    q[kinds == 2] = INF
    q[kinds == 3] = -INF
    return q


@pytest.mark.parametrize("k", [4, 16, 32])
@pytest.mark.parametrize("dim", [2, 3])
def test_nonfinite_queries_match_oracle(k, dim):
    rng = np.random.default_rng(600 + k + dim)
    pts = rng.random((20_000, dim), dtype=np.float32)
    q = queries_with_nonfinite(rng, 3000, dim)
    ei, ed = oracle.knn_brute(pts, q, k)
    di, dd = oracle.knn(pts, q, k)
    assert_same_int(di, ei, "oracle DFS vs brute force")
    for name, (idx, dist) in zip(("accel", "implicit"), both_paths(pts, q, k)):
        assert_same_int(idx, ei, f"{name} indices")
        assert_same_f32(dist, ed, f"{name} distances")


@pytest.mark.parametrize("dim", [2, 3])
def test_infinite_point_coordinates_match_oracle(dim):
    """Points at +-inf on some axes (boxes then reach infinity and still
    bound every distance), queried from finite, infinite and NaN positions."""
    rng = np.random.default_rng(700 + dim)
    pts = rng.random((20_000, dim), dtype=np.float32)
    rows = rng.choice(20_000, 300, replace=False)
    pts[rows[:150], 0] = INF
    pts[rows[150:], dim - 1] = -INF
    q = queries_with_nonfinite(rng, 2000, dim)
    ei, ed = oracle.knn_brute(pts, q, 8)
    bvh = oracle.build(pts)
    di, dd = oracle.knn_bvh(bvh, q, 8)
    assert_same_int(di, ei, "oracle DFS vs brute force")
    h = tb.build_bvh(dev(pts))
    assert_same_f32(h["node_aabbs"].cpu().numpy(), bvh["node_aabbs"], "node_aabbs")
    assert_same_int(h["sorted_indices"].cpu().numpy(), bvh["sorted_indices"], "sorted_indices")
    tb.destroy_bvh(h)
    for name, (idx, dist) in zip(("accel", "implicit"), both_paths(pts, q, 8)):
        assert_same_int(idx, ei, f"{name} indices")
        assert_same_f32(dist, ed, f"{name} distances")


def test_nan_point_coordinates():
    rng = np.random.default_rng(800)
    pts = rng.random((20_000, 3), dtype=np.float32)
    pts[rng.choice(20_000, 200, replace=False), 1] = NAN
    q = rng.random((2000, 3), dtype=np.float32)
    bvh = oracle.build(pts)
    di, dd = oracle.knn_bvh(bvh, q, 16)
    (ai, ad), (ii, idd) = both_paths(pts, q, 16)
    assert_same_int(ii, di, "implicit indices vs the oracle's DFS")
    assert_same_f32(idd, dd, "implicit distances vs the oracle's DFS")
    # Accel: sorted rows of distinct indices, each with its true distance.
    assert np.all(ai >= 0)
    assert all(len(set(r)) == len(r) for r in ai.tolist())
    assert np.all(np.diff(ad, axis=1) >= 0)
    assert_same_f32(ad, oracle.pair_distances(pts, q, ai), "accel distances of its own indices")
