"""Which structure the reference-style k-NN bindings traverse for tensors
the library did not just build, and which explicit accels they accept.

With accel=None, tensors the registry does not know are checked on the
device once: only the point BVH the build writes (degenerate leaf boxes,
internal boxes the merges of their children, leaves in Morton order,
indices in range) gets an accel built from it; anything else (a primitive
BVH, edited boxes, another leaf order) is answered by the implicit tree, as
the reference answers it (knn_query.cu:47-154 over whatever boxes it is
given).  An explicit accel must be one this library built for exactly those
node_aabbs (knn_query.cu:363-399 checks every tensor it is handed)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from parity import assert_same_f32, assert_same_int
from torchbvh_amd import _native
from torchbvh_amd._native import _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def knn_none(d: dict, nodes, sidx, q, k: int):
    return _C.query_knn_batched_cached_bounds(nodes, sidx, q, d["num_leaves"], d["num_real_nodes"], d["dim"], k)


def implicit_boxes(leaves: np.ndarray) -> np.ndarray:
    """Node rows of the implicit tree over `leaves` ((n, 2D) boxes in leaf
    order): each real internal node the min/max of its real children, a copy
    of the left one where the right one is virtual, rows in level order."""
    n, d2 = leaves.shape
    D = d2 // 2
    L = oracle.leaf_level(n)
    out = np.empty((oracle.real_node_count(n), d2), np.float32)
    first = (1 << L) - 1
    for j in range(n):
        out[oracle.memory_index(n, first + j)] = leaves[j]
    for lvl in range(L - 1, -1, -1):
        for i in range((1 << lvl) - 1, (1 << (lvl + 1)) - 1):
            if oracle.is_virtual(n, i):
                continue
            a = out[oracle.memory_index(n, 2 * i + 1)]
            if oracle.is_virtual(n, 2 * i + 2):
                out[oracle.memory_index(n, i)] = a
            else:
                b = out[oracle.memory_index(n, 2 * i + 2)]
                out[oracle.memory_index(n, i)] = np.concatenate([np.fmin(a[:D], b[:D]), np.fmax(a[D:], b[D:])])
    return out


@pytest.mark.parametrize("V,D", [(2, 2), (3, 3)])
def test_primitive_bvh_takes_the_implicit_tree(V, D):
    """A primitive BVH has the point build's shapes, but its leaves are
    boxes: the bindings answer with box distances, as the reference does."""
    rng = np.random.default_rng(900 + D)
    prims = (rng.random((1, 2000, 1, D), dtype=np.float32) + 0.03 * rng.random((1, 2000, V, D), dtype=np.float32))
    q = rng.random((1, 700, D), dtype=np.float32)
    d = _C.build_primitive_bvh_batched(dev(prims))
    print(f"primitive BVH V={V} D={D}", flush=True)
    idx, dist = knn_none(d, d["node_aabbs"], d["sorted_indices"], dev(q), 8)
    entry = _native._registry_entry(d["node_aabbs"], d["sorted_indices"])
    assert entry is not None and entry[2] is None  # registered for the implicit tree
    ei, ed = oracle.knn_bvh(oracle.build_primitives(prims[0]), q[0], 8)
    assert_same_int(idx[0].cpu().numpy(), ei, "indices")
    assert_same_f32(dist[0].cpu().numpy(), ed, "distances")
    # The second call takes the registered decision without a new check.
    idx2, dist2 = knn_none(d, d["node_aabbs"], d["sorted_indices"], dev(q), 8)
    assert torch.equal(idx, idx2) and torch.equal(dist, dist2)


def test_degenerate_primitives_are_a_point_bvh():
    """Segments whose two vertices coincide form the point build's BVH: the
    check passes and the accel answers, equal to the oracle's points k-NN."""
    rng = np.random.default_rng(910)
    pts = rng.random((2, 3000, 2), dtype=np.float32)
    prims = np.repeat(pts[:, :, None, :], 2, axis=2)
    q = rng.random((2, 600, 2), dtype=np.float32)
    d = _C.build_primitive_bvh_batched(dev(prims))
    idx, dist = knn_none(d, d["node_aabbs"], d["sorted_indices"], dev(q), 8)
    assert _native._registered_accel(d["node_aabbs"], d["sorted_indices"]) is not None
    for b in range(2):
        ei, ed = oracle.knn(pts[b], q[b], 8)
        assert_same_int(idx[b].cpu().numpy(), ei, f"cloud {b} indices")
        assert_same_f32(dist[b].cpu().numpy(), ed, f"cloud {b} distances")


def test_edited_boxes_take_the_implicit_tree():
    """A point BVH whose internal box was widened after the build is no
    longer the build's: the implicit tree answers (still the exact k-NN,
    since a wider box only costs visits)."""
    rng = np.random.default_rng(920)
    p = rng.random((1, 3000, 3), dtype=np.float32)
    q = rng.random((1, 500, 3), dtype=np.float32)
    d = _C.build_bvh_batched_cooperative(dev(p))
    nodes = d["node_aabbs"].clone()
    nodes[0, 5, :3] -= 0.25
    sidx = d["sorted_indices"].clone()
    idx, dist = knn_none(d, nodes, sidx, dev(q), 16)
    entry = _native._registry_entry(nodes, sidx)
    assert entry is not None and entry[2] is None
    ei, ed = oracle.knn_brute(p[0], q[0], 16)
    assert_same_int(idx[0].cpu().numpy(), ei, "indices")
    assert_same_f32(dist[0].cpu().numpy(), ed, "distances")


def test_consistent_bvh_in_another_leaf_order_takes_the_implicit_tree():
    """Leaves in reversed Morton order with every internal box recomputed:
    a valid BVH, but not in the order the accel's radix tree needs."""
    rng = np.random.default_rng(930)
    p = rng.random((3000, 3), dtype=np.float32)
    q = rng.random((400, 3), dtype=np.float32)
    order = oracle.build(p)["sorted_indices"][::-1].copy()
    leaves = np.concatenate([p[order], p[order]], axis=1)
    nodes = dev(implicit_boxes(leaves)[None])
    sidx = dev(order[None])
    d = {"num_leaves": 3000, "num_real_nodes": oracle.real_node_count(3000), "dim": 3}
    idx, dist = knn_none(d, nodes, sidx, dev(q[None]), 8)
    entry = _native._registry_entry(nodes, sidx)
    assert entry is not None and entry[2] is None
    ei, ed = oracle.knn_brute(p, q, 8)
    assert_same_int(idx[0].cpu().numpy(), ei, "indices")
    assert_same_f32(dist[0].cpu().numpy(), ed, "distances")
    # The same boxes in Morton order pass the check and take an accel.
    ref = oracle.build(p)
    mnodes, msidx = dev(ref["node_aabbs"][None]), dev(ref["sorted_indices"][None])
    midx, mdist = knn_none(d, mnodes, msidx, dev(q[None]), 8)
    assert _native._registered_accel(mnodes, msidx) is not None
    assert torch.equal(midx, idx) and torch.equal(mdist, dist)


def test_a_node_count_that_does_not_match_the_leaves_is_rejected():
    """A smaller, self-consistent num_real_nodes and node_aabbs for unknown
    tensors is refused before anything is built or launched."""
    rng = np.random.default_rng(940)
    p = rng.random((1, 1000, 3), dtype=np.float32)
    d = _C.build_bvh_batched_cooperative(dev(p))
    nr = d["num_real_nodes"] - 1
    nodes = d["node_aabbs"][:, :nr].clone()
    with pytest.raises(RuntimeError, match="num_real_nodes does not match num_leaves"):
        _C.query_knn_batched_cached_bounds(nodes, d["sorted_indices"].clone(), dev(p[:, :50]),
                                           d["num_leaves"], nr, 3, 4)
    assert _native._registry_entry(nodes, d["sorted_indices"]) is None


def test_an_explicit_accel_must_belong_to_the_tensors():
    """Two clouds of the same size: the accel of one is refused with the
    other's tensors (it would silently answer for the wrong cloud), a
    misaligned view is refused, and each accel is accepted with its own."""
    rng = np.random.default_rng(950)
    pa, pb = (dev(rng.random((1, 2000, 3), dtype=np.float32)) for _ in range(2))
    q = dev(rng.random((1, 300, 3), dtype=np.float32))
    da = _C.build_bvh_batched_cooperative(pa, with_accel=True)
    db = _C.build_bvh_batched_cooperative(pb, with_accel=True)
    args = (q, 2000, da["num_real_nodes"], 3, 8)
    with pytest.raises(RuntimeError, match="not built by this library for these node_aabbs"):
        _C.query_knn_batched_cached_bounds(db["node_aabbs"], db["sorted_indices"], *args, accel=da["accel"])
    with pytest.raises(RuntimeError, match="256-byte aligned"):
        _C.query_knn_batched_cached_bounds(da["node_aabbs"], da["sorted_indices"], *args,
                                           accel=da["accel"][16:])
    ia, dA = _C.query_knn_batched_cached_bounds(da["node_aabbs"], da["sorted_indices"], *args, accel=da["accel"])
    ib, dB = _C.query_knn_batched_cached_bounds(db["node_aabbs"], db["sorted_indices"], *args, accel=db["accel"])
    ea, _ = oracle.knn(pa[0].cpu().numpy(), q[0].cpu().numpy(), 8)
    eb, _ = oracle.knn(pb[0].cpu().numpy(), q[0].cpu().numpy(), 8)
    assert_same_int(ia[0].cpu().numpy(), ea, "cloud a")
    assert_same_int(ib[0].cpu().numpy(), eb, "cloud b")
    # Modified after the build: the accel no longer belongs to them.
    db["node_aabbs"].add_(0)
    with pytest.raises(RuntimeError, match="not built by this library"):
        _C.query_knn_batched_cached_bounds(db["node_aabbs"], db["sorted_indices"], *args, accel=db["accel"])
