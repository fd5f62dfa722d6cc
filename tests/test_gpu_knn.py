"""GPU k-NN parity against the oracle: indices identical and distances
bit-exact (the contract's tolerance is 1e-6 relative; the kernel and the
oracle evaluate the same fused chain, so equality is expected and tested).

Cases restate the reference's k-NN tests (torchbvh tests/test_knn.py,
tests/test_batched_knn.py, tests/test_ragged_knn.py) with index checks
everywhere, since ties now resolve to the lower index."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import torchbvh_amd as tb
from parity import (
    assert_same_f32,
    assert_same_int,
    knn_pathological_clouds,
    unit_direction_points,
)
from torchbvh_amd import _native
from torchbvh_amd._native import _C

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["scheduled", "input-order"])
def schedule_mode(request, monkeypatch):
    """Every case twice: query_knn with the traversal schedule forced on
    (threshold 0) and with its default, under which these small query sets
    traverse in input order."""
    from torchbvh_amd import _query

    if request.param == "scheduled":
        monkeypatch.setattr(_query, "SCHEDULE_MIN_QUERIES", 0)
    return request.param
DEV = torch.device("cuda")
DIST_RTOL = 1e-6  # contractual tolerance; checked in addition to bit equality


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def implicit_knn(h, queries: torch.Tensor, k: int, sort: bool):
    """The traversal over the reference's implicit tree (no accel)."""
    nodes, sidx, q = h["node_aabbs"][None], h["sorted_indices"][None], queries[None]
    if sort:
        order = _C.morton_sort_queries_narrow(q, h["scene_min"][None], h["scene_max"][None])
        out = _C.query_knn_batched_cached_bounds_ordered(
            nodes, sidx, q, order, h["num_leaves"], h["num_real_nodes"], h["dim"], k, accel=False)
    else:
        out = _C.query_knn_batched_cached_bounds(
            nodes, sidx, q, h["num_leaves"], h["num_real_nodes"], h["dim"], k, accel=False)
    return out[0][0], out[1][0]


def check_single(points: np.ndarray, queries: np.ndarray, k: int) -> None:
    h = tb.build_bvh(dev(points))
    assert h._aux["accel"] is not None
    ei, ed = oracle.knn(points, queries, k)
    qd = dev(queries)
    for sort in (True, False):
        for path, (idx, dist) in (("accel", tb.query_knn(h, qd, k, sort_queries=sort)),
                                  ("implicit", implicit_knn(h, qd, k, sort))):
            assert idx.dtype == torch.int64 and dist.dtype == torch.float32
            assert tuple(idx.shape) == (queries.shape[0], k)
            idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
            np.testing.assert_allclose(dist, ed, rtol=DIST_RTOL, atol=0)
            assert_same_int(idx, ei, f"{path} indices sort={sort}")
            assert_same_f32(dist, ed, f"{path} distances sort={sort}")


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 8, 16, 32])
def test_knn_uniform_random(dim, k):
    rng = np.random.default_rng(1000 + dim * 10 + k)
    check_single(rng.random((3000, dim), dtype=np.float32), rng.random((1500, dim), dtype=np.float32), k)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 8, 16, 32])
def test_knn_self_query(dim, k):
    rng = np.random.default_rng(2000 + dim * 10 + k)
    p = rng.random((777, dim), dtype=np.float32)
    check_single(p, p, k)
    idx, dist = tb.query_knn(tb.build_bvh(dev(p)), dev(p), k)
    assert torch.all(dist[:, 0] == 0)
    assert torch.equal(idx[:, 0].cpu(), torch.arange(777))


@pytest.mark.parametrize("k", [4, 8, 16, 32])
def test_knn_minimum_cloud_sizes(k):
    rng = np.random.default_rng(k)
    for n in (k, k + 1, 2 * k - 1):
        check_single(rng.random((n, 3), dtype=np.float32), rng.random((37, 3), dtype=np.float32), k)


@pytest.mark.parametrize("k", [4, 8])
def test_knn_displaced_curve(k):
    base = np.linspace(-2.0, 2.0, 32, dtype=np.float32)
    p = np.stack((base, np.sin(base), np.cos(base)), 1).astype(np.float32)
    check_single(p, p + np.array([0.07, -0.11, 0.05], np.float32), k)


@pytest.mark.parametrize("case", range(len(knn_pathological_clouds())))
def test_knn_pathological_clouds(case):
    p, k = knn_pathological_clouds()[case]
    check_single(p, p[: min(7, p.shape[0])] + np.float32(0.125), k)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 8, 16])
def test_knn_ties_take_lowest_indices(dim, k):
    p = unit_direction_points(dim)
    q = np.zeros((2, dim), np.float32)
    check_single(p, q, k)
    idx, dist = tb.query_knn(tb.build_bvh(dev(p)), dev(q), k)
    assert torch.all(dist == 1.0)
    assert torch.equal(idx.cpu(), torch.arange(k).repeat(2, 1))
    dup = np.full((20, dim), 3.5, np.float32)
    check_single(dup, np.full((3, dim), 3.5, np.float32), k)


@pytest.mark.parametrize("dim", [2, 3])
def test_knn_ties_take_lowest_indices_k32(dim):
    """K = 32 (the buffered-merge traversal): 16 copies of each unit
    direction, all at distance 1 from the origin, plus farther points."""
    eye = np.eye(dim, dtype=np.float32)
    dirs = np.concatenate([np.stack((eye[d], -eye[d])) for d in range(dim)])
    p = np.concatenate((np.repeat(dirs, 16, axis=0), 3.0 * dirs, 5.0 * dirs)).astype(np.float32)
    q = np.zeros((3, dim), np.float32)
    check_single(p, q, 32)
    idx, dist = tb.query_knn(tb.build_bvh(dev(p)), dev(q), 32)
    assert torch.all(dist == 1.0)
    assert torch.equal(idx.cpu(), torch.arange(32).repeat(3, 1))


@pytest.mark.parametrize("dim", [2, 3])
def test_batched_knn_k32_matches_oracle(dim):
    rng = np.random.default_rng(13150 + dim)
    p = rng.random((4, 3000, dim), dtype=np.float32)
    p[1, :1000] = p[1, 1000:2000]  # exact duplicates: ties by index
    q = rng.random((4, 700, dim), dtype=np.float32)
    idx, dist = tb.query_knn(tb.build_bvh(dev(p)), dev(q), 32)
    for b in range(4):
        ei, ed = oracle.knn(p[b], q[b], 32)
        assert_same_int(idx[b].cpu().numpy(), ei, f"batch {b} indices")
        assert_same_f32(dist[b].cpu().numpy(), ed, f"batch {b} distances")


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 8, 16, 32])
def test_knn_robust_matrix(dim, k):
    """tests/test_knn.py:327-356: random points, a tie block, duplicates and
    outliers, with exact, displaced, origin and outlier queries."""
    rng = np.random.default_rng(2400 + dim * 100 + k)
    rand = (rng.random((96, dim), dtype=np.float32) * 2 - 1).astype(np.float32)
    ties = np.zeros((k + 2, dim), np.float32)
    dup = np.full((2, dim), 0.25, np.float32)
    out = np.zeros((2, dim), np.float32)
    out[0, 0], out[1, 0] = 50.0, -50.0
    out[:, 1] = [30.0, -30.0]
    p = np.concatenate((rand, ties, dup, out)).astype(np.float32)
    disp = np.linspace(0.015, 0.045, dim, dtype=np.float32)
    q = np.concatenate((p[:19], p[19:38] + disp, np.zeros((5, dim), np.float32), out + 0.1 * disp,
                        rng.random((17, dim), dtype=np.float32) * 2 - 1)).astype(np.float32)
    check_single(p, q, k)


@pytest.mark.parametrize("dim", [2, 3])
def test_knn_clustered_duplicates_large(dim):
    rng = np.random.default_rng(40 + dim)
    centres = rng.random((8, dim)).astype(np.float32)
    p = (centres[rng.integers(0, 8, 60_000)] + 0.02 * rng.standard_normal((60_000, dim))).astype(np.float32)
    p[1000:1300] = p[3]
    q = (p[:5000] + 0.005 * rng.standard_normal((5000, dim))).astype(np.float32)
    check_single(p, q, 32)


def test_knn_queries_outside_scene_box():
    rng = np.random.default_rng(8)
    p = rng.random((5000, 3), dtype=np.float32)
    q = (rng.standard_normal((2000, 3)) * 5).astype(np.float32)
    check_single(p, q, 16)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("n", [16, 17, 31, 300])
@pytest.mark.parametrize("k", [4, 8, 16])
def test_batched_knn_matches_oracle_and_single_loop(dim, n, k):
    rng = np.random.default_rng(13100 + dim * 100 + n * 10 + k)
    p = rng.random((3, n, dim), dtype=np.float32)
    q = rng.random((3, 9, dim), dtype=np.float32)
    h = tb.build_bvh(dev(p))
    idx, dist, pos = tb.query_knn(h, dev(q), k, source_points=dev(p))
    assert tuple(idx.shape) == (3, 9, k) and tuple(pos.shape) == (3, 9, k, dim)
    for b in range(3):
        ei, ed = oracle.knn(p[b], q[b], k)
        assert_same_int(idx[b].cpu().numpy(), ei, f"batch {b} indices")
        assert_same_f32(dist[b].cpu().numpy(), ed, f"batch {b} distances")
        assert_same_f32(pos[b].cpu().numpy(), p[b][ei], f"batch {b} positions")
        si, sd = tb.query_knn(tb.build_bvh(dev(p[b])), dev(q[b]), k)
        assert torch.equal(si, idx[b]) and torch.equal(sd, dist[b])


def test_batched_no_cross_sample_leakage():
    rng = np.random.default_rng(13300)
    p = np.stack([rng.random((200, 3), dtype=np.float32) + 100.0 * b for b in range(4)])
    q = np.stack([p[b, :20] + 0.01 for b in range(4)]).astype(np.float32)
    h = tb.build_bvh(dev(p))
    idx, dist = tb.query_knn(h, dev(q), 8)
    assert int(idx.min()) >= 0 and int(idx.max()) < 200
    for b in range(4):
        ei, ed = oracle.knn(p[b], q[b], 8)
        assert_same_int(idx[b].cpu().numpy(), ei, "indices")


def _offsets(counts):
    return np.concatenate(([0], np.cumsum(counts))).astype(np.int64)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 8, 16, 32])
def test_ragged_knn_matches_oracle(dim, k):
    rng = np.random.default_rng(14100 + dim * 10 + k)
    counts = [k, k + 3, k + 9, 5000, 4097]
    qcounts = [3, 6, 4, 1000, 777]
    p = np.concatenate([rng.random((c, dim), dtype=np.float32) + 20.0 * b for b, c in enumerate(counts)])
    q = np.concatenate([rng.random((c, dim), dtype=np.float32) + 20.0 * b for b, c in enumerate(qcounts)])
    po, qo = _offsets(counts), _offsets(qcounts)
    h = tb.build_bvh(dev(p), batch_offsets=dev(po))
    idx, dist, pos = tb.query_knn(h, dev(q), k, query_offsets=dev(qo), source_points=dev(p))
    ei, ed = oracle.knn_ragged(p, po, q, qo, k)
    assert_same_int(idx.cpu().numpy(), ei, "indices")
    assert_same_f32(dist.cpu().numpy(), ed, "distances")
    packed = h._aux["packed"]
    ii, idd = _C.query_knn_ragged(packed["node_aabbs"], packed["sorted_indices"], dev(po),
                                  packed["node_offsets"], dev(q), dev(qo), None, len(counts), dim, k)
    assert_same_int(ii.cpu().numpy(), ei, "implicit ragged indices")
    assert_same_f32(idd.cpu().numpy(), ed, "implicit ragged distances")
    rows = np.repeat(po[:-1], qcounts)
    assert_same_f32(pos.cpu().numpy(), p[ei + rows[:, None]], "positions")


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 8, 16, 32])
def test_ragged_ties_take_lowest_local_indices(dim, k):
    eye = np.eye(dim, dtype=np.float32)
    dirs = np.concatenate([np.stack((eye[d], -eye[d])) for d in range(dim)])
    counts = [k + 3, k + 7, k + 11]
    qcounts = [2, 3, 1]
    shifts = [np.full(dim, -40.0, np.float32), np.full(dim, 40.0, np.float32),
              np.linspace(-25.0, 25.0, dim, dtype=np.float32)]
    d0 = np.zeros(dim, np.float32)
    d0[0] = 1.0
    d2 = np.zeros(dim, np.float32)
    d2[-1] = -1.0
    reps = (counts[1] + dirs.shape[0] - 1) // dirs.shape[0]
    samples = [np.tile(d0, (counts[0], 1)) + shifts[0],
               np.tile(dirs, (reps, 1))[: counts[1]] + shifts[1],
               np.tile(d2, (counts[2], 1)) + shifts[2]]
    p = np.concatenate(samples).astype(np.float32)
    q = np.concatenate([np.tile(s, (c, 1)) for s, c in zip(shifts, qcounts)]).astype(np.float32)
    po, qo = _offsets(counts), _offsets(qcounts)
    h = tb.build_bvh(dev(p), batch_offsets=dev(po))
    idx, dist = tb.query_knn(h, dev(q), k, query_offsets=dev(qo))
    ei, ed = oracle.knn_ragged(p, po, q, qo, k)
    assert_same_int(idx.cpu().numpy(), ei, "indices")
    assert_same_f32(dist.cpu().numpy(), ed, "distances")
    assert torch.all(dist == 1.0)
    assert torch.equal(idx.cpu(), torch.arange(k).repeat(6, 1))


def test_ragged_indices_are_local():
    rng = np.random.default_rng(14200)
    counts = [8, 11, 14]
    p = np.concatenate([rng.random((c, 3), dtype=np.float32) + 100.0 * b for b, c in enumerate(counts)])
    po = _offsets(counts)
    q = np.concatenate([p[po[b]:po[b] + 3] for b in range(3)])
    h = tb.build_bvh(dev(p), batch_offsets=dev(po))
    idx, dist = tb.query_knn(h, dev(q), 4, query_offsets=dev(_offsets([3, 3, 3])))
    for b, c in enumerate(counts):
        s = idx[3 * b:3 * b + 3]
        assert int(s.min()) >= 0 and int(s.max()) < c
    assert torch.all(dist[:, 0] == 0)


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 16, 32])
@pytest.mark.parametrize("use_accel", [True, False])
def test_spatial_output_is_ordered_output_in_launch_order(dim, k, use_accel):
    """`query_knn_batched_cached_bounds_spatial` (knn_query.cu:147-148,
    448-461): row [b, m] holds the result of query order[b, m]."""
    rng = np.random.default_rng(300 + dim * 10 + k)
    p = rng.random((3, 2000, dim), dtype=np.float32)
    q = rng.random((3, 777, dim), dtype=np.float32)
    h = tb.build_bvh(dev(p))
    qd = dev(q)
    order = _C.morton_sort_queries_narrow(qd, h["scene_min"], h["scene_max"])
    args = (h["node_aabbs"], h["sorted_indices"], qd, order, h["num_leaves"], h["num_real_nodes"], dim, k)
    accel = h._aux["accel"] if use_accel else False
    si, sd = _C.query_knn_batched_cached_bounds_spatial(*args, accel=accel)
    oi, od = _C.query_knn_batched_cached_bounds_ordered(*args, accel=accel)
    perm = order.unsqueeze(-1).expand(-1, -1, k)
    assert torch.equal(si, torch.gather(oi, 1, perm))
    assert torch.equal(sd, torch.gather(od, 1, perm))
    o = order.cpu().numpy()
    for b in range(3):
        ei, ed = oracle.knn(p[b], q[b][o[b]], k)
        assert_same_int(si[b].cpu().numpy(), ei, f"batch {b} indices")
        assert_same_f32(sd[b].cpu().numpy(), ed, f"batch {b} distances")


def _routed_case(dim, B, nt, nf, m, seed, frac=0.5):
    rng = np.random.default_rng(seed)
    tp = rng.random((B, nt, dim), dtype=np.float32)
    fp = (rng.random((B, nf, dim), dtype=np.float32) * 2.0 - 0.5).astype(np.float32)
    q = (rng.random((B, m, dim), dtype=np.float32) * 1.4 - 0.2).astype(np.float32)
    routes = rng.random((B, m)) < frac
    routes[0, :] = True    # a cloud whose queries all take the true route
    if B > 1:
        routes[1, :] = False  # ... and one whose queries all take the false route
    return tp, fp, q, routes


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("m", [1, 300, 5000])
def test_routed_order_bit_exact(dim, m):
    tp, fp, q, routes = _routed_case(dim, 3, 500, 400, m, 410 + m + dim)
    ht, hf = tb.build_bvh(dev(tp)), tb.build_bvh(dev(fp))
    order = _C.morton_sort_routed_queries_batched(dev(q), dev(routes), ht["scene_min"], ht["scene_max"],
                                                  hf["scene_min"], hf["scene_max"]).cpu().numpy()
    tmin, tmax = ht["scene_min"].cpu().numpy(), ht["scene_max"].cpu().numpy()
    fmin, fmax = hf["scene_min"].cpu().numpy(), hf["scene_max"].cpu().numpy()
    for b in range(3):
        want = oracle.routed_order(q[b], routes[b], tmin[b], tmax[b], fmin[b], fmax[b])
        assert_same_int(order[b], want, f"cloud {b} routed order")


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("k", [4, 16, 32])
@pytest.mark.parametrize("use_accel", [True, False])
def test_routed_knn_spatial_matches_oracle(dim, k, use_accel):
    tp, fp, q, routes = _routed_case(dim, 3, 900, 700, 640, 520 + dim * 10 + k)
    ht, hf = tb.build_bvh(dev(tp)), tb.build_bvh(dev(fp))
    qd, rd = dev(q), dev(routes)
    order = _C.morton_sort_routed_queries_batched(qd, rd, ht["scene_min"], ht["scene_max"],
                                                  hf["scene_min"], hf["scene_max"])
    kw = ({"true_accel": ht._aux["accel"], "false_accel": hf._aux["accel"]} if use_accel
          else {"true_accel": False, "false_accel": False})
    idx, dist = _C.query_knn_routed_batched_cached_bounds_spatial(
        ht["node_aabbs"], ht["sorted_indices"], hf["node_aabbs"], hf["sorted_indices"], qd, rd, order,
        ht["num_leaves"], ht["num_real_nodes"], hf["num_leaves"], hf["num_real_nodes"], dim, k, **kw)
    o = order.cpu().numpy()
    for b in range(3):
        ei, ed = oracle.knn_routed(tp[b], fp[b], q[b][o[b]], routes[b][o[b]], k)
        assert_same_int(idx[b].cpu().numpy(), ei, f"cloud {b} indices")
        assert_same_f32(dist[b].cpu().numpy(), ed, f"cloud {b} distances")


def test_reference_style_bindings_use_the_registered_accel():
    """A caller of the reference's `_C` surface builds with
    build_bvh_batched_cooperative(points) and passes the dict's tensors to
    the k-NN bindings: the result keeps exactly the reference's keys, and
    the query takes the accel registered with those tensors (identical to
    the implicit tree's result and the oracle's) until they are modified."""
    rng = np.random.default_rng(77)
    p = rng.random((2, 5000, 3), dtype=np.float32)
    q = rng.random((2, 900, 3), dtype=np.float32)
    pd, qd = dev(p), dev(q)
    d = _C.build_bvh_batched_cooperative(pd)
    assert set(d) == {"node_aabbs", "sorted_indices", "scene_min", "scene_max", "batch_size", "num_leaves",
                      "num_real_nodes", "leaf_level", "virtual_leaves", "dim", "left_child_mem",
                      "right_child_mem", "mem_to_leaf"}
    assert _native._registered_accel(d["node_aabbs"], d["sorted_indices"]) is not None
    order = _C.morton_sort_queries_narrow(qd, d["scene_min"], d["scene_max"])
    args = (d["node_aabbs"], d["sorted_indices"], qd, order, d["num_leaves"], d["num_real_nodes"], 3, 16)
    ai, ad = _C.query_knn_batched_cached_bounds_ordered(*args)
    ii, idd = _C.query_knn_batched_cached_bounds_ordered(*args, accel=False)
    assert torch.equal(ai, ii) and torch.equal(ad, idd)
    for b in range(2):
        ei, ed = oracle.knn(p[b], q[b], 16)
        assert_same_int(ai[b].cpu().numpy(), ei, f"cloud {b} indices")
        assert_same_f32(ad[b].cpu().numpy(), ed, f"cloud {b} distances")
    d["node_aabbs"].mul_(1.0)
    assert _native._registered_accel(d["node_aabbs"], d["sorted_indices"]) is None


def test_reference_style_bindings_on_cloned_tensors_build_an_accel():
    """The tensors a reference-style caller passes need not be the ones the
    build returned: a clone (or copy, or reload) gets an accel built from
    node_aabbs and sorted_indices alone on first use, registered for the
    next calls.  cfg2's size: results equal the registered path's on every
    row and the oracle's on a sample; the call takes the accel, not the
    implicit tree (printed timings: first call with the accel build,
    second from the registry)."""
    import time

    g = torch.Generator("cpu").manual_seed(2001)
    p = torch.rand((1, 1 << 20, 3), generator=g)
    q = torch.rand((1, 1 << 20, 3), generator=torch.Generator("cpu").manual_seed(2002))
    pd, qd = p.to(DEV), q.to(DEV)
    d = _C.build_bvh_batched_cooperative(pd)
    order = _C.morton_sort_queries_narrow(qd, d["scene_min"], d["scene_max"])
    args = (d["num_leaves"], d["num_real_nodes"], 3, 16)
    ri, rd = _C.query_knn_batched_cached_bounds_ordered(d["node_aabbs"], d["sorted_indices"], qd, order, *args)
    nodes, sidx = d["node_aabbs"].clone(), d["sorted_indices"].clone()
    assert _native._registered_accel(nodes, sidx) is None
    times = []
    for _ in range(2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ci, cd = _C.query_knn_batched_cached_bounds_ordered(nodes, sidx, qd, order, *args)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) * 1e3)
    print(f"cloned tensors: first call {times[0]:.3f} ms (accel built), second {times[1]:.3f} ms", flush=True)
    assert _native._registered_accel(nodes, sidx) is not None
    assert torch.equal(ci, ri) and torch.equal(cd, rd)
    rows = np.random.default_rng(5).choice(1 << 20, 4096, replace=False)
    ei, ed = oracle.knn_brute(p[0].numpy(), q[0].numpy()[rows], 16)
    assert_same_int(ci[0].cpu().numpy()[rows], ei, "indices")
    assert_same_f32(cd[0].cpu().numpy()[rows], ed, "distances")


def test_explicit_accel_smaller_than_the_layout_is_rejected():
    rng = np.random.default_rng(78)
    p = dev(rng.random((2, 3000, 3), dtype=np.float32))
    q = dev(rng.random((2, 100, 3), dtype=np.float32))
    d = _C.build_bvh_batched_cooperative(p)
    small = _C.build_bvh_batched_cooperative(p[:, :2000].contiguous(), with_accel=True)["accel"]
    with pytest.raises(RuntimeError, match="need"):
        _C.query_knn_batched_cached_bounds(d["node_aabbs"], d["sorted_indices"], q, d["num_leaves"],
                                           d["num_real_nodes"], 3, 4, accel=small)
