"""Parity of the routed cell-block search (tbvh_knn_accel_routed_grid_spatial,
which the routed binding `query_knn_routed_batched_cached_bounds_spatial`
takes above GRID_MIN_QUERIES queries) against the oracle's routed k-NN (the
reference's routed traversal, knn_query.cu:183-327) and, through the C ABI,
bit for bit against the routed accel traversal
(tbvh_knn_accel_routed_spatial).

Covered: 2-D and 3-D, every k the search runs for; true and false clouds
of different sizes and boxes (each searched at its own grid level); a
cloud whose queries all take the true route, one whose queries all take
the false route, one mixing both in every wave; queries outside the
boxes; clouds the table kernel disables (NaN points, a clustered cloud's
long empty runs) beside enabled ones, on either route; NaN and infinite
queries; a short workspace refused; no workspace meaning the traversal."""

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


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def routed_workspace(B, M, nt, nf, D, k) -> int:
    need = ctypes.c_size_t(0)
    assert _native.load().tbvh_knn_accel_routed_grid_workspace_size(B, M, nt, nf, D, k, ctypes.byref(need)) == 0
    return need.value


def routed_traversal(ht, hf, qd, rd, order, B, M, D, k):
    """The routed accel traversal alone, through the C ABI."""
    L = _native.load()
    P = _native._ptr
    idx = torch.full((B, M, k), -7, dtype=torch.int64, device=DEV)
    dist = torch.full((B, M, k), -7.0, device=DEV)
    rc = L.tbvh_knn_accel_routed_spatial(P(ht._aux["accel"]), P(hf._aux["accel"]), P(qd), P(rd), P(order), B, M,
                                         int(ht["num_leaves"]), int(hf["num_leaves"]), D, k, P(idx), P(dist),
                                         _native._stream(DEV))
    assert rc == 0, L.tbvh_last_error()
    return idx, dist


def routed_grid(ht, hf, qd, rd, order, B, M, D, k, ws, ws_bytes):
    """The routed cell-block search, through the C ABI: (status, indices, distances)."""
    L = _native.load()
    P = _native._ptr
    idx = torch.full((B, M, k), -7, dtype=torch.int64, device=DEV)
    dist = torch.full((B, M, k), -7.0, device=DEV)
    rc = L.tbvh_knn_accel_routed_grid_spatial(
        P(ht._aux["accel"]), P(ht["node_aabbs"]), int(ht["num_real_nodes"]), P(hf._aux["accel"]),
        P(hf["node_aabbs"]), int(hf["num_real_nodes"]), P(qd), P(rd), P(order), B, M, int(ht["num_leaves"]),
        int(hf["num_leaves"]), D, k, P(idx), P(dist), P(ws) if ws is not None else None, ws_bytes,
        _native._stream(DEV))
    return rc, idx, dist


# (D, k, true cloud, false cloud): sizes with a grid at both (the false
# cloud's level one below the true's where the levels allow it).
CASES = [(3, 4, 150_000, 135_000), (3, 8, 150_000, 35_000), (3, 16, 150_000, 40_000), (3, 32, 150_000, 40_000),
         (2, 8, 150_000, 40_000), (2, 16, 150_000, 40_000), (2, 32, 150_000, 40_000)]


@pytest.mark.parametrize("D,k,nt,nf", CASES)
def test_routed_grid_matches_oracle_and_traversal(D, k, nt, nf):
    B, M = 3, GRID_MIN_QUERIES // 3 + 777
    print(f"routed grid D={D} k={k} nt={nt} nf={nf} B={B} M={M}", flush=True)
    rng = np.random.default_rng(900 + 10 * D + k)
    tp = rng.random((B, nt, D), dtype=np.float32)
    fp = (rng.random((B, nf, D), dtype=np.float32) * 2.0 - 0.5).astype(np.float32)
    q = (rng.random((B, M, D), dtype=np.float32) * 1.4 - 0.2).astype(np.float32)
    routes = rng.random((B, M)) < 0.5
    routes[0, :] = True
    routes[1, :] = False
    assert routed_workspace(B, M, nt, nf, D, k) > 0
    ht, hf = tb.build_bvh(dev(tp)), tb.build_bvh(dev(fp))
    qd, rd = dev(q), dev(routes)
    order = _C.morton_sort_routed_queries_batched(qd, rd, ht["scene_min"], ht["scene_max"], hf["scene_min"],
                                                  hf["scene_max"])
    # The binding takes the cell-block search at this size.
    idx, dist = _C.query_knn_routed_batched_cached_bounds_spatial(
        ht["node_aabbs"], ht["sorted_indices"], hf["node_aabbs"], hf["sorted_indices"], qd, rd, order,
        ht["num_leaves"], ht["num_real_nodes"], hf["num_leaves"], hf["num_real_nodes"], D, k)
    ti, td = routed_traversal(ht, hf, qd, rd, order, B, M, D, k)
    torch.cuda.synchronize()
    assert torch.equal(idx, ti) and torch.equal(dist, td)
    o = order.cpu().numpy()
    for b in range(B):
        ei, ed = oracle.knn_routed(tp[b], fp[b], q[b][o[b]], routes[b][o[b]], k)
        assert_same_int(idx[b].cpu().numpy(), ei, f"cloud {b} indices")
        assert_same_f32(dist[b].cpu().numpy(), ed, f"cloud {b} distances")


@pytest.mark.parametrize("D,k", [(3, 16), (3, 32), (2, 8)])
def test_c_abi_routed_grid_disabled_clouds_and_nonfinite_queries(D, k):
    """Clouds the table kernel disables on either route (NaN points in the
    false cloud of batch 0, a clustered true cloud in batch 1: long empty
    runs of cells) beside enabled ones, NaN and infinite queries on both
    routes: every row equals the routed traversal's, bit for bit.  A short
    workspace is refused before any launch; none runs the traversal."""
    B, N, M = 2, 150_000, GRID_MIN_QUERIES // 2 + 501
    print(f"routed grid disabled clouds D={D} k={k}", flush=True)
    rng = np.random.default_rng(31 + D * 7 + k)
    tp = rng.random((B, N, D), dtype=np.float32)
    # batch 1's true cloud: two tight clusters
    c = rng.integers(0, 2, N)
    tp[1] = (0.1 + 0.8 * c[:, None] + rng.normal(0, 0.01, (N, D))).astype(np.float32)
    fp = (rng.random((B, N, D), dtype=np.float32) * 2.0 - 0.5).astype(np.float32)
    fp[0, ::991] = np.nan
    q = rng.random((B, M, D), dtype=np.float32)
    q[0, 3] = np.nan
    q[0, 100, 0] = np.inf
    q[1, 7, D - 1] = -np.inf
    q[1, 2000] = np.nan
    routes = rng.random((B, M)) < 0.5
    ht, hf = tb.build_bvh(dev(tp)), tb.build_bvh(dev(fp))
    qd, rd = dev(q), dev(routes)
    order = _C.morton_sort_routed_queries_batched(qd, rd, ht["scene_min"], ht["scene_max"], hf["scene_min"],
                                                  hf["scene_max"])
    need = routed_workspace(B, M, N, N, D, k)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    rc, gi, gd = routed_grid(ht, hf, qd, rd, order, B, M, D, k, ws, need)
    assert rc == 0, _native.load().tbvh_last_error()
    ti, td = routed_traversal(ht, hf, qd, rd, order, B, M, D, k)
    torch.cuda.synchronize()
    assert torch.equal(gi, ti) and torch.equal(gd, td)
    # Enabled cloud (batch 1's false cloud) rows against the oracle as well.
    o = order[1].cpu().numpy()
    sel = ~routes[1][o] & np.isfinite(q[1][o]).all(axis=1)
    ei, ed = oracle.knn(fp[1], q[1][o][sel], k)
    assert_same_int(gi[1].cpu().numpy()[sel], ei + N, "batch 1 false-route indices")
    assert_same_f32(gd[1].cpu().numpy()[sel], ed, "batch 1 false-route distances")
    rc, _, _ = routed_grid(ht, hf, qd, rd, order, B, M, D, k, ws, need - 256)
    assert rc == 2 and b"workspace" in _native.load().tbvh_last_error()
    rc, ni, nd = routed_grid(ht, hf, qd, rd, order, B, M, D, k, None, 0)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(ni, ti) and torch.equal(nd, td)


def test_routed_grid_repeated_calls_share_nothing():
    """Two routed cell-block calls in a row on one workspace, the second
    with fewer queries and the routes flipped: each equals the traversal
    (the workspace's counts and flags are cleared by every call)."""
    D, k, nt, nf = 3, 16, 150_000, 60_000
    rng = np.random.default_rng(4242)
    tp = rng.random((1, nt, D), dtype=np.float32)
    fp = rng.random((1, nf, D), dtype=np.float32)
    ht, hf = tb.build_bvh(dev(tp)), tb.build_bvh(dev(fp))
    M0 = GRID_MIN_QUERIES + 3000
    need = routed_workspace(1, M0, nt, nf, D, k)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    for M, flip in ((M0, False), (GRID_MIN_QUERIES + 65, True)):
        print(f"routed grid repeat M={M} flip={flip}", flush=True)
        q = rng.random((1, M, D), dtype=np.float32)
        routes = rng.random((1, M)) < 0.3
        if flip:
            routes = ~routes
        qd, rd = dev(q), dev(routes)
        order = _C.morton_sort_routed_queries_batched(qd, rd, ht["scene_min"], ht["scene_max"], hf["scene_min"],
                                                      hf["scene_max"])
        assert routed_workspace(1, M, nt, nf, D, k) <= need
        rc, gi, gd = routed_grid(ht, hf, qd, rd, order, 1, M, D, k, ws, need)
        assert rc == 0, _native.load().tbvh_last_error()
        ti, td = routed_traversal(ht, hf, qd, rd, order, 1, M, D, k)
        torch.cuda.synchronize()
        assert torch.equal(gi, ti) and torch.equal(gd, td)
