"""Radix-sort paths that the other GPU tests do not reach.

* More than 4096 tiles per pass (over 16.8M keys): the per-digit tile scan
  runs in several chunks.  Checked at full size through properties that do
  not depend on the size: the order is a permutation, the Morton codes are
  non-decreasing along it, and equal codes keep ascending input index (the
  stability the reference's CUB sort has, bvh_build.cu:580-594).
* Thousands of tiny ragged clouds (and clouds without queries): every
  segment-relative offset comes from scan[d][t] - scan[d][first tile],
  checked bit-exact against the oracle cloud by cloud; and the whole k-NN
  path over thousands of clouds, whose tree-pass groups, span work-groups
  and traversal waves mix clouds.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from parity import assert_same_f32, assert_same_int
from torchbvh_amd._native import _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("dim", [2, 3])
def test_point_order_over_4096_tiles_is_a_stable_code_sort(dim):
    n = 17_000_000  # 4151 tiles of 4096 keys
    g = torch.Generator(device=DEV).manual_seed(4151 + dim)
    p = torch.rand((1, n, dim), generator=g, device=DEV)
    p[0, : n // 4] = torch.floor(p[0, : n // 4] * 64) / 64  # many equal codes
    order = _C.morton_sort_points_batched(p)[0]
    assert order.shape == (n,) and order.dtype == torch.int64
    assert torch.equal(torch.bincount(order, minlength=n), torch.ones(n, dtype=torch.int64, device=DEV))
    codes = _C.morton_codes(p, p.amin(1).contiguous(), p.amax(1).contiguous())[0]
    sc = codes[order]
    assert bool((sc[1:] >= sc[:-1]).all()), "codes not sorted"
    ties = sc[1:] == sc[:-1]
    assert int(ties.sum()) > 1000
    assert bool((order[1:][ties] > order[:-1][ties]).all()), "equal codes out of input order"
    del p, order, codes, sc, ties
    torch.cuda.empty_cache()


def test_ragged_build_thousands_of_tiny_clouds():
    rng = np.random.default_rng(3000)
    counts = rng.integers(1, 41, 3000).tolist()
    counts[17] = 4097  # one cloud over a tile boundary among them
    pts = rng.random((sum(counts), 3), dtype=np.float32)
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    h = _C.build_bvh_ragged(dev(pts), dev(offsets), counts)
    node_offsets = h["node_offsets"].cpu().numpy()
    sorted_idx = h["sorted_indices"].cpu().numpy()
    nodes = h["node_aabbs"].cpu().numpy()
    smin, smax = h["scene_min"].cpu().numpy(), h["scene_max"].cpu().numpy()
    for b, c in enumerate(counts):
        ref = oracle.build(pts[offsets[b]:offsets[b + 1]])
        assert_same_int(sorted_idx[offsets[b]:offsets[b + 1]], ref["sorted_indices"], f"cloud {b} order")
        assert_same_f32(nodes[node_offsets[b]:node_offsets[b + 1]], ref["node_aabbs"], f"cloud {b} nodes")
        assert_same_f32(smin[b], ref["scene_min"], f"cloud {b} min")
        assert_same_f32(smax[b], ref["scene_max"], f"cloud {b} max")


def test_ragged_query_order_many_segments_some_empty():
    rng = np.random.default_rng(3001)
    counts = rng.integers(0, 30, 2500)
    counts[::7] = 0  # clouds without queries
    counts[5] = 9000
    q = rng.random((int(counts.sum()), 3), dtype=np.float32)
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    lo = rng.random((len(counts), 3), dtype=np.float32) * 0.5
    hi = lo + 0.5
    order = _C.morton_sort_queries_ragged(dev(q), dev(offsets), dev(lo), dev(hi), len(counts)).cpu().numpy()
    for b in range(len(counts)):
        a, e = offsets[b], offsets[b + 1]
        if a == e:
            continue
        assert_same_int(order[a:e], oracle.query_order(q[a:e], lo[b], hi[b]), f"cloud {b}")


@pytest.mark.parametrize("k,dim", [(16, 3), (8, 2)])
def test_ragged_knn_thousands_of_small_clouds(k, dim):
    """Ragged k-NN through the public API (fused accel build, span kernel,
    Hilbert schedule, accel traversal) over 2,000 clouds: mostly small ones
    (k to 600 points, so one tree-pass group or one span work-group holds
    many clouds), a few above one sort tile and one above a tree-pass group
    of 256 leaves per level.  (The public API, like the reference's, wants
    strictly increasing offsets, so every cloud has a query.)  Every cloud's
    rows must be the oracle's, bit for bit."""
    import torchbvh_amd as tb

    print(f"ragged knn: 2000 clouds k={k} dim={dim}", flush=True)
    rng = np.random.default_rng(7000 + k + dim)
    counts = rng.integers(k, 601, 2000)
    counts[[5, 700, 1500]] = [4097, 20_000, 70_000]
    qcounts = rng.integers(1, 40, 2000)
    qcounts[1500] = 3000
    pts = rng.random((int(counts.sum()), dim), dtype=np.float32)
    po = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    qo = np.concatenate(([0], np.cumsum(qcounts))).astype(np.int64)
    # Queries near each cloud's own points (each cloud sits in [0, 1)^D).
    q = np.concatenate([rng.random((int(m), dim), dtype=np.float32) for m in qcounts])
    h = tb.build_bvh(dev(pts), batch_offsets=dev(po))
    idx, dist = tb.query_knn(h, dev(q), k, query_offsets=dev(qo))
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    for b in range(len(counts)):
        ei, ed = oracle.knn(pts[po[b]:po[b + 1]], q[qo[b]:qo[b + 1]], k)
        assert_same_int(idx[qo[b]:qo[b + 1]], ei, f"cloud {b} indices (n={counts[b]})")
        assert_same_f32(dist[qo[b]:qo[b + 1]], ed, f"cloud {b} distances")


@pytest.mark.parametrize("use_accel", [True, False])
def test_batched_knn_many_equal_clouds(use_accel):
    """Batched input of 700 equal clouds: the segment table is computed in
    closed form by the first launch of the build and of the query ordering
    (no planning launch), for more clouds than work-groups of some passes;
    both traversals, every cloud against the oracle."""
    B, n, m, k = 700, 150, 24, 8
    print(f"batched knn: B={B} n={n} m={m} k={k} accel={use_accel}", flush=True)
    rng = np.random.default_rng(7100 + use_accel)
    p = rng.random((B, n, 3), dtype=np.float32)
    q = rng.random((B, m, 3), dtype=np.float32)
    d = _C.build_bvh_batched_cooperative(dev(p))
    order = _C.morton_sort_queries_narrow(dev(q), d["scene_min"], d["scene_max"])
    idx, dist = _C.query_knn_batched_cached_bounds_ordered(
        d["node_aabbs"], d["sorted_indices"], dev(q), order, d["num_leaves"], d["num_real_nodes"], 3, k,
        accel=None if use_accel else False)
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    for b in range(B):
        ei, ed = oracle.knn(p[b], q[b], k)
        assert_same_int(idx[b], ei, f"cloud {b} indices")
        assert_same_f32(dist[b], ed, f"cloud {b} distances")
