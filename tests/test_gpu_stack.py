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
