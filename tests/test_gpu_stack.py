"""The traversals' bounded stack: inputs whose trees are deep enough, or
whose boxes tie closely enough, that a lane's ring of LDS entries overflows,
drops entries and must resume through the parent links (the accel's stored
links, the implicit tree's closed forms).  Results must still be the
oracle's k nearest (distance, index) pairs, bit for bit.

Measured on a CPU model of the traversal (16-entry ring, as in the 3-D
k = 16 kernel): every query of the shell cloud drops entries and walks up
46 times; ~98% of the exponential-scale queries drop entries."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import torchbvh_amd as tb
from parity import assert_same_f32, assert_same_int

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def shell(rng, n: int, dim: int) -> np.ndarray:
    """Points on a sphere (circle) of radius 0.25 around (0.5, ...): from the
    centre, every box is within the k-th distance, so nothing is pruned and
    the stack grows to the tree's depth."""
    v = rng.standard_normal((n, dim)).astype(np.float32)
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    return (0.5 + 0.25 * v).astype(np.float32)


def exponential(rng, n: int, dim: int) -> np.ndarray:
    """Coordinates spread over 40 binary orders of magnitude: long chains of
    radix-tree nodes that split one Morton bit at a time."""
    e = rng.integers(0, 40, (n, dim))
    return (2.0 ** (-e) * rng.random((n, dim))).astype(np.float32)


def check(points: np.ndarray, queries: np.ndarray, k: int) -> None:
    with tb.BVH(dev(points)) as bvh:
        idx, dist = bvh.knn(dev(queries), k)
    torch.cuda.synchronize()
    ei, ed = oracle.knn_brute(points, queries, k)
    assert_same_int(idx.cpu().numpy(), ei, "indices")
    assert_same_f32(dist.cpu().numpy(), ed, "distances")


@pytest.mark.parametrize("k", [4, 8, 16, 32])
@pytest.mark.parametrize("dim", [2, 3])
def test_shell_queries_at_the_centre(k, dim):
    print(f"stack: shell dim={dim} k={k}", flush=True)
    rng = np.random.default_rng(300 + 10 * k + dim)
    pts = shell(rng, 100_000, dim)
    q = np.concatenate([np.full((64, dim), 0.5, np.float32),
                        (0.5 + 0.01 * rng.standard_normal((192, dim))).astype(np.float32)])
    check(pts, q, k)


@pytest.mark.parametrize("k", [4, 16, 32])
@pytest.mark.parametrize("dim", [2, 3])
def test_exponential_scales(k, dim):
    print(f"stack: exponential dim={dim} k={k}", flush=True)
    rng = np.random.default_rng(400 + 10 * k + dim)
    check(exponential(rng, 100_000, dim), exponential(rng, 4096, dim), k)


def test_ragged_clouds_with_deep_trees():
    """Ragged launch: clouds of every kind side by side, so lanes of one wave
    resume in different clouds (record rows follow each cloud's point rows)."""
    print("stack: ragged deep clouds", flush=True)
    rng = np.random.default_rng(500)
    clouds = [shell(rng, 30_000, 3), exponential(rng, 50_000, 3), rng.random((7, 3), dtype=np.float32),
              shell(rng, 5_000, 3)]
    queries = [np.full((100, 3), 0.5, np.float32), exponential(rng, 300, 3),
               rng.random((50, 3), dtype=np.float32), (0.5 + 0.05 * rng.standard_normal((200, 3))).astype(np.float32)]
    pts = np.concatenate(clouds)
    q = np.concatenate(queries)
    po = np.concatenate(([0], np.cumsum([len(c) for c in clouds]))).astype(np.int64)
    qo = np.concatenate(([0], np.cumsum([len(c) for c in queries]))).astype(np.int64)
    with tb.BVH(dev(pts), batch_offsets=dev(po)) as bvh:
        idx, dist = bvh.knn(dev(q), 4, query_offsets=dev(qo))
    torch.cuda.synchronize()
    ei, ed = oracle.knn_ragged(pts, po, q, qo, 4)
    assert_same_int(idx.cpu().numpy(), ei, "indices")
    assert_same_f32(dist.cpu().numpy(), ed, "distances")


@pytest.mark.parametrize("k,dim,n", [(4, 3, 600_000), (16, 2, 600_000), (16, 3, 2_200_000)])
def test_implicit_tree_ring_overflow(k, dim, n):
    """The implicit-tree traversal (the reference's layout, no accel) uses
    the same ring with the resume walk through closed-form parents.  A shell
    cloud of n points has L - 1 levels of internal nodes above the leaves'
    parents (19 for 600,000 points, 21 for 2,200,000), each of which defers
    its far child for a query at the centre: more than the ring holds (16
    entries for 3-D k = 4 and 2-D k = 16, 20 for 3-D k = 16).  Results must be
    the brute force's bit for bit."""
    from torchbvh_amd._native import _C

    print(f"stack: implicit shell dim={dim} k={k} n={n}", flush=True)
    rng = np.random.default_rng(900 + 10 * k + dim)
    pts = shell(rng, n, dim)
    q = np.concatenate([np.full((64, dim), 0.5, np.float32),
                        (0.5 + 0.02 * rng.standard_normal((128, dim))).astype(np.float32),
                        rng.random((64, dim), dtype=np.float32)])
    h = tb.build_bvh(dev(pts))
    nodes, sidx = h["node_aabbs"][None], h["sorted_indices"][None]
    idx, dist = _C.query_knn_batched_cached_bounds(nodes, sidx, dev(q)[None], h["num_leaves"],
                                                    h["num_real_nodes"], h["dim"], k, accel=False)
    torch.cuda.synchronize()
    tb.destroy_bvh(h)
    ei, ed = oracle.knn_brute(pts, q, k)
    assert_same_int(idx[0].cpu().numpy(), ei, "indices")
    assert_same_f32(dist[0].cpu().numpy(), ed, "distances")


# The 3-D k = 16 accel traversal has two ring layouts: compact 5-byte entries
# (24-bit refs) when every cloud has at most 2^20 points, full 6-byte entries
# above that.  The tests above run the compact one; these cross the limit.
COMPACT_CLOUD = 1 << 20


def test_shell_above_compact_limit_full_ring():
    """Shell cloud of 2^20 + 4096 points (full layout) queried from the
    centre: every lane's ring overflows and resumes through parent links."""
    print("stack: shell above the compact-ring limit, 3-D k=16", flush=True)
    rng = np.random.default_rng(1101)
    pts = shell(rng, COMPACT_CLOUD + 4096, 3)
    q = np.concatenate([np.full((64, 3), 0.5, np.float32),
                        (0.5 + 0.01 * rng.standard_normal((64, 3))).astype(np.float32)])
    check(pts, q, 16)


@pytest.mark.parametrize("n", [COMPACT_CLOUD, COMPACT_CLOUD + 1])
def test_uniform_at_the_compact_limit(n):
    """Exactly 2^20 points (compact ring, the widest 20-bit bucket starts and
    node indices) and one more (full ring), 4096 queries, 3-D k = 16."""
    print(f"stack: uniform n={n} 3-D k=16", flush=True)
    rng = np.random.default_rng(1200 + n % 7)
    pts = rng.random((n, 3), dtype=np.float32)
    q = np.concatenate([rng.random((4032, 3), dtype=np.float32),
                        pts[-64:] + np.float32(1e-4)]).astype(np.float32)
    with tb.BVH(dev(pts)) as bvh:
        idx, dist = bvh.knn(dev(q), 16)
    torch.cuda.synchronize()
    ei, ed = oracle.knn(pts, q, 16)
    assert_same_int(idx.cpu().numpy(), ei, "indices")
    assert_same_f32(dist.cpu().numpy(), ed, "distances")


def test_ragged_total_above_compact_limit():
    """Ragged 3-D k = 16 call whose clouds are each below 2^20 points but
    whose total is above: the launch takes the full ring (the limit applies
    to the call's total, which bounds every cloud)."""
    print("stack: ragged total above the compact-ring limit", flush=True)
    rng = np.random.default_rng(1301)
    clouds = [rng.random((600_000, 3), dtype=np.float32), shell(rng, 500_000, 3)]
    queries = [rng.random((1000, 3), dtype=np.float32),
               np.concatenate([np.full((64, 3), 0.5, np.float32), rng.random((500, 3), dtype=np.float32)])]
    pts = np.concatenate(clouds)
    q = np.concatenate(queries)
    po = np.concatenate(([0], np.cumsum([len(c) for c in clouds]))).astype(np.int64)
    qo = np.concatenate(([0], np.cumsum([len(c) for c in queries]))).astype(np.int64)
    with tb.BVH(dev(pts), batch_offsets=dev(po)) as bvh:
        idx, dist = bvh.knn(dev(q), 16, query_offsets=dev(qo))
    torch.cuda.synchronize()
    ei, ed = oracle.knn_ragged(pts, po, q, qo, 16)
    assert_same_int(idx.cpu().numpy(), ei, "indices")
    assert_same_f32(dist.cpu().numpy(), ed, "distances")
