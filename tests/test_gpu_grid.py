"""Parity of the cell-block search (tbvh_knn_accel_grid, which batched accel
k-NN calls above GRID_MIN_QUERIES queries take) against the oracle's DFS
(the reference's traversal, knn_query.cu:47-154) and against the plain
accel traversal.

Covered: uniform clouds (most queries answered from their block, the rest
by the seeded fallback traversal), every k, 2-D and 3-D, ordered and
input-order launches, batched calls mixing a uniform cloud with a
clustered one (its long empty runs disable the search for that cloud), a
cloud on a plane (empty extent), clouds with NaN points (disabled: the
plain traversal's rows), queries outside the cloud's box and non-finite
queries, heavy exact ties (points on a coarse lattice), and the C ABI
directly: results bit-equal to tbvh_knn_accel, a short workspace refused,
no workspace meaning tbvh_knn_accel."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
import torchbvh_amd as tb
from parity import assert_same_f32, assert_same_int
from torchbvh_amd import _native
from torchbvh_amd._native import GRID_MIN_QUERIES, _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
Q = GRID_MIN_QUERIES + 4099  # above the threshold, not a multiple of the wave


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def check_single(p: np.ndarray, q: np.ndarray, k: int, what: str) -> None:
    print(f"grid {what}: n={p.shape[0]} q={q.shape[0]} D={p.shape[1]} k={k}", flush=True)
    h = tb.build_bvh(dev(p))
    idx, dist = tb.query_knn(h, dev(q), k)
    ei, ed = oracle.knn_bvh(oracle.build(p), q, k)
    assert_same_int(idx.cpu().numpy(), ei, f"{what} indices")
    assert_same_f32(dist.cpu().numpy(), ed, f"{what} distances")


@pytest.mark.parametrize("k", [4, 8, 16, 32])
def test_uniform_3d(k):
    rng = np.random.default_rng(100 + k)
    p = rng.random((150_000, 3), dtype=np.float32)
    q = rng.random((Q, 3), dtype=np.float32)
    check_single(p, q, k, f"uniform 3-D k={k}")


@pytest.mark.parametrize("k", [4, 8, 16, 32])
def test_uniform_2d(k):
    rng = np.random.default_rng(200 + k)
    p = rng.random((300_000, 2), dtype=np.float32)
    q = (p[rng.integers(0, p.shape[0], Q)] + rng.normal(0, 0.002, (Q, 2))).astype(np.float32)
    check_single(p, q, k, f"uniform 2-D k={k}")


def test_queries_outside_the_box_and_on_its_faces():
    rng = np.random.default_rng(7)
    p = (rng.random((120_000, 3), dtype=np.float32) * np.float32(2) - np.float32(1)).astype(np.float32)
    q = (rng.random((Q, 3), dtype=np.float32) * np.float32(3) - np.float32(1.5)).astype(np.float32)
    q[::5, 0] = p[:, 0].min()
    q[1::5, 1] = p[:, 1].max()
    check_single(p, q, 16, "outside and on faces")


def test_cloud_far_from_the_origin():
    """A unit cloud at 1e5: the coordinates' rounding (ulp 0.008) dwarfs a
    margin slack taken from the extent alone; the slack scales with the
    magnitudes, so blocks that cannot prove exactness fall back."""
    rng = np.random.default_rng(14)
    p = (rng.random((120_000, 3)) + 1e5).astype(np.float32)
    q = (rng.random((Q, 3)) + 1e5).astype(np.float32)
    check_single(p, q, 8, "far from the origin")


def test_lattice_ties():
    """Points on a coarse lattice, many of them equal: exact ties everywhere,
    resolved to the lower index by both paths."""
    rng = np.random.default_rng(8)
    p = (np.floor(rng.random((200_000, 3)) * 40) / 40).astype(np.float32)
    q = (np.floor(rng.random((Q, 3)) * 80) / 80).astype(np.float32)
    check_single(p, q, 8, "lattice ties")


def test_nonfinite_queries():
    rng = np.random.default_rng(9)
    p = rng.random((100_000, 3), dtype=np.float32)
    q = rng.random((Q, 3), dtype=np.float32)
    q[::97, 1] = np.nan
    q[5::101, 2] = np.inf
    q[7::103, 0] = -np.inf
    check_single(p, q, 16, "non-finite queries")


@pytest.mark.parametrize("k", [8, 16])
def test_void_sends_queries_through_every_stage(k):
    """A uniform cloud with a spherical hole of about two cells' radius:
    queries near its rim miss the first 3^3 block's margin and are decided by
    the second (5^3, cells beyond the first k-th distance dropped); queries
    deep inside keep too many cells or miss that margin too and take the
    traversal.  Every row against the oracle."""
    rng = np.random.default_rng(15 + k)
    p = rng.random((300_000, 3), dtype=np.float32)
    centre = np.float32(0.5)
    p = p[np.linalg.norm(p - centre, axis=1) > 0.07]
    q = rng.random((Q, 3), dtype=np.float32)
    inside = q.shape[0] // 4
    d = rng.normal(size=(inside, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    q[:inside] = (centre + d * rng.random((inside, 1)) * 0.09).astype(np.float32)
    check_single(p, q, k, f"void k={k}")


def test_clustered_cloud_falls_back():
    rng = np.random.default_rng(10)
    centres = rng.random((8, 3), dtype=np.float32)
    p = (centres[rng.integers(0, 8, 160_000)] + rng.normal(0, 0.01, (160_000, 3))).astype(np.float32)
    q = (p[rng.integers(0, p.shape[0], Q)] + rng.normal(0, 0.003, (Q, 3))).astype(np.float32)
    check_single(p, q, 16, "clustered")


def test_planar_cloud_falls_back():
    rng = np.random.default_rng(11)
    p = rng.random((100_000, 3), dtype=np.float32)
    p[:, 2] = 0.5
    q = rng.random((Q, 3), dtype=np.float32)
    check_single(p, q, 8, "planar")


def test_batched_mixed_clouds():
    """One uniform, one clustered and one scaled uniform cloud in one call:
    the search runs per cloud, disabled for the clustered one."""
    rng = np.random.default_rng(12)
    B, n, m = 3, 60_000, 50_000
    p = rng.random((B, n, 3), dtype=np.float32)
    centres = rng.random((4, 3), dtype=np.float32)
    p[1] = (centres[rng.integers(0, 4, n)] + rng.normal(0, 0.005, (n, 3))).astype(np.float32)
    p[2] = (p[2] * np.float32(1e3) + np.float32(7)).astype(np.float32)
    q = rng.random((B, m, 3), dtype=np.float32)
    q[2] = (q[2] * np.float32(1e3) + np.float32(7)).astype(np.float32)
    assert B * m > GRID_MIN_QUERIES
    h = tb.build_bvh(dev(p))
    idx, dist = tb.query_knn(h, dev(q), 16)
    for b in range(B):
        ei, ed = oracle.knn_bvh(oracle.build(p[b]), q[b], 16)
        assert_same_int(idx[b].cpu().numpy(), ei, f"cloud {b} indices")
        assert_same_f32(dist[b].cpu().numpy(), ed, f"cloud {b} distances")


def _call(L, fn, acc, node_aabbs, nr, qb, order, B, M, N, D, k, ws=None, ws_bytes=0):
    idx = torch.full((B, M, k), -7, dtype=torch.int64, device=DEV)
    dist = torch.full((B, M, k), -7.0, device=DEV)
    st = _native._stream(DEV)
    P = _native._ptr
    if fn == "grid":
        rc = L.tbvh_knn_accel_grid(P(acc), P(node_aabbs), nr, P(qb), P(order), B, M, N, D, k, P(idx), P(dist),
                                   P(ws) if ws is not None else None, ws_bytes, st)
    else:
        rc = L.tbvh_knn_accel(P(acc), P(qb), P(order), B, M, N, D, k, P(idx), P(dist), st)
    torch.cuda.synchronize()
    return rc, idx, dist


@pytest.mark.parametrize("ordered", [False, True])
def test_c_abi_grid_equals_accel_traversal(ordered):
    rng = np.random.default_rng(13)
    B, N, M, D, k = 2, 70_000, 40_000, 3, 16
    p = rng.random((B, N, D), dtype=np.float32)
    p[1, ::1000] = np.nan  # NaN points: cloud 1 is disabled, its rows are the traversal's
    q = rng.random((B, M, D), dtype=np.float32)
    h = tb.build_bvh(dev(p))
    acc = h._aux["accel"]
    qb = dev(q)
    order = _C.morton_sort_queries_narrow(qb, h["scene_min"], h["scene_max"], schedule=True) if ordered else None
    L = _native.load()
    need = ctypes.c_size_t(0)
    assert L.tbvh_knn_accel_grid_workspace_size(B, M, N, D, k, ctypes.byref(need)) == 0 and need.value > 0
    ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
    nr = int(h["num_real_nodes"])
    rc, gi, gd = _call(L, "grid", acc, h["node_aabbs"], nr, qb, order, B, M, N, D, k, ws, need.value)
    assert rc == 0, _native.load().tbvh_last_error()
    rc, ti, td = _call(L, "plain", acc, None, 0, qb, order, B, M, N, D, k)
    assert rc == 0
    assert torch.equal(gi, ti) and torch.equal(gd, td)
    # cloud 0 against the oracle as well
    ei, ed = oracle.knn_bvh(oracle.build(p[0]), q[0], k)
    assert_same_int(gi[0].cpu().numpy(), ei, "cloud 0 indices")
    assert_same_f32(gd[0].cpu().numpy(), ed, "cloud 0 distances")
    # a short workspace is refused before any launch; none runs the traversal
    rc, _, _ = _call(L, "grid", acc, h["node_aabbs"], nr, qb, order, B, M, N, D, k, ws, need.value - 256)
    assert rc != 0 and b"workspace" in L.tbvh_last_error()
    rc, ni, nd = _call(L, "grid", acc, h["node_aabbs"], nr, qb, order, B, M, N, D, k, None, 0)
    assert rc == 0 and torch.equal(ni, ti) and torch.equal(nd, td)
    rc, _, _ = _call(L, "grid", acc, h["node_aabbs"], nr + 1, qb, order, B, M, N, D, k, ws, need.value)
    assert rc != 0 and b"num_real_nodes" in L.tbvh_last_error()


@pytest.mark.parametrize("schedule", [False, True])
@pytest.mark.parametrize("D,k", [(3, 16), (2, 8)])
def test_c_abi_grid_spatial_equals_accel_spatial(schedule, D, k):
    """Spatial output (results in launch position, the MLS binding): the
    cell-block search through tbvh_knn_accel_grid_spatial against
    tbvh_knn_accel_spatial, bit for bit, with the full Morton order the
    reference binding produces and with the traversal schedule; and the
    _C binding (which takes it above GRID_MIN_QUERIES) against both."""
    rng = np.random.default_rng(17 + k)
    B, N, M = 2, 200_000, GRID_MIN_QUERIES // 2 + 901
    p = rng.random((B, N, D), dtype=np.float32)
    q = rng.random((B, M, D), dtype=np.float32)
    h = tb.build_bvh(dev(p))
    acc = h._aux["accel"]
    qb = dev(q)
    order = _C.morton_sort_queries_narrow(qb, h["scene_min"], h["scene_max"], schedule=schedule)
    L = _native.load()
    need = ctypes.c_size_t(0)
    assert L.tbvh_knn_accel_grid_workspace_size(B, M, N, D, k, ctypes.byref(need)) == 0 and need.value > 0
    ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
    nr = int(h["num_real_nodes"])
    P, st = _native._ptr, _native._stream(DEV)
    outs = []
    for grid in (True, False):
        idx = torch.full((B, M, k), -7, dtype=torch.int64, device=DEV)
        dist = torch.full((B, M, k), -7.0, device=DEV)
        if grid:
            rc = L.tbvh_knn_accel_grid_spatial(P(acc), P(h["node_aabbs"]), nr, P(qb), P(order), B, M, N, D, k,
                                               P(idx), P(dist), P(ws), need.value, st)
        else:
            rc = L.tbvh_knn_accel_spatial(P(acc), P(qb), P(order), B, M, N, D, k, P(idx), P(dist), st)
        assert rc == 0, L.tbvh_last_error()
        outs.append((idx, dist))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    bi, bd = _C.query_knn_batched_cached_bounds_spatial(h["node_aabbs"], h["sorted_indices"], qb, order,
                                                        h["num_leaves"], h["num_real_nodes"], D, k)
    assert torch.equal(bi, outs[1][0]) and torch.equal(bd, outs[1][1])
    # cloud 0 against the oracle, rows mapped back from launch position to input row
    o = order[0].cpu().numpy()
    ei, ed = oracle.knn_bvh(oracle.build(p[0]), q[0][o], k)
    assert_same_int(bi[0].cpu().numpy(), ei, "cloud 0 indices (launch order)")
    assert_same_f32(bd[0].cpu().numpy(), ed, "cloud 0 distances (launch order)")


def test_grid_spatial_and_rows_with_disabled_cloud_and_nonfinite_queries():
    """A batched call mixing a near-uniform cloud with a disabled one (NaN
    points), with NaN and infinite queries in both: the spatial-output and
    neighbour-row forms of the cell-block search equal the plain traversal's
    spatial and neighbour-row forms bit for bit (the disabled cloud and the
    non-finite queries go to the traversal)."""
    rng = np.random.default_rng(29)
    B, N, M, D, k, C = 2, 150_000, GRID_MIN_QUERIES // 2 + 333, 3, 16, 3
    p = rng.random((B, N, D), dtype=np.float32)
    p[1, ::997] = np.nan
    q = rng.random((B, M, D), dtype=np.float32)
    q[0, 5] = np.nan
    q[0, 77, 1] = np.inf
    q[1, 11, 2] = -np.inf
    src = rng.random((B, N, C), dtype=np.float32)
    h = tb.build_bvh(dev(p))
    acc = h._aux["accel"]
    qb, sb = dev(q), dev(src)
    order = _C.morton_sort_queries_narrow(qb, h["scene_min"], h["scene_max"])
    L = _native.load()
    need = ctypes.c_size_t(0)
    assert L.tbvh_knn_accel_grid_workspace_size(B, M, N, D, k, ctypes.byref(need)) == 0 and need.value > 0
    ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
    nr = int(h["num_real_nodes"])
    P, st = _native._ptr, _native._stream(DEV)

    def outs():
        return (torch.full((B, M, k), -7, dtype=torch.int64, device=DEV), torch.full((B, M, k), -7.0, device=DEV),
                torch.full((B, M, k, C), -7.0, device=DEV))

    gi, gd, _ = outs()
    ti, td, _ = outs()
    assert L.tbvh_knn_accel_grid_spatial(P(acc), P(h["node_aabbs"]), nr, P(qb), P(order), B, M, N, D, k, P(gi),
                                         P(gd), P(ws), need.value, st) == 0
    assert L.tbvh_knn_accel_spatial(P(acc), P(qb), P(order), B, M, N, D, k, P(ti), P(td), st) == 0
    torch.cuda.synchronize()
    assert torch.equal(gi, ti) and torch.equal(gd, td)
    gi, gd, gp = outs()
    ti, td, tp = outs()
    assert L.tbvh_knn_accel_grid_positions(P(acc), P(h["node_aabbs"]), nr, P(qb), P(order), B, M, N, D, k, P(sb), C,
                                           P(gi), P(gd), P(gp), P(ws), need.value, st) == 0
    assert L.tbvh_knn_accel_positions(P(acc), P(qb), P(order), B, M, N, D, k, P(sb), C, P(ti), P(td), P(tp), st) == 0
    torch.cuda.synchronize()
    assert torch.equal(gi, ti) and torch.equal(gd, td) and torch.equal(gp, tp)
