"""CPU oracle for torchbvh_amd's parity tests.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker (or, for the CPU baseline, as the thing timed on the host).  The
product path never imports it.

The arithmetic lives in ``oracle.c`` (a restatement of the reference's build
and k-NN path, see its header); this module wraps it with numpy arrays and
adds the batched / ragged loops the reference's Python layer performs
(torchbvh/_query.py:39-85, :120-366).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from .build_oracle import LIB_PATH, build as _build_lib

_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")


def lib():
    """Load (building on first use if absent) the compiled oracle."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            _build_lib()
        L = ctypes.CDLL(str(LIB_PATH))
        c_int, c_i64 = ctypes.c_int, ctypes.c_int64
        L.orc_leaf_level.argtypes = [c_int]
        L.orc_virtual_leaves.argtypes = [c_int]
        L.orc_real_node_count.argtypes = [c_int]
        L.orc_memory_index.argtypes = [c_int, c_int]
        L.orc_is_virtual.argtypes = [c_int, c_int]
        L.orc_split3.argtypes = [ctypes.c_uint32]
        L.orc_split3.restype = ctypes.c_uint32
        L.orc_split2.argtypes = [ctypes.c_uint32]
        L.orc_split2.restype = ctypes.c_uint32
        L.orc_morton.argtypes = [_f32p, c_int, _f32p, _f32p]
        L.orc_morton.restype = ctypes.c_uint32
        L.orc_morton_codes.argtypes = [_f32p, c_i64, c_int, _f32p, _f32p, _u32p]
        L.orc_hilbert_codes.argtypes = [_f32p, c_i64, c_int, _f32p, _f32p, _u32p]
        L.orc_hilbert_cells.argtypes = [_u32p, c_i64, c_int, c_int, _u32p]
        L.orc_bounds.argtypes = [_f32p, c_i64, c_int, _f32p, _f32p]
        L.orc_stable_argsort.argtypes = [_u32p, c_i64, _i64p]
        L.orc_build.argtypes = [_f32p, c_int, c_int, _f32p, _i64p, _f32p, _f32p, _i32p, _i32p, _i32p]
        L.orc_build_primitives.argtypes = [_f32p, c_int, c_int, c_int, _f32p, _i64p, _f32p, _f32p, _i32p,
                                           _i32p, _i32p, _f32p]
        L.orc_knn_brute.argtypes = [_f32p, c_i64, _f32p, c_i64, c_int, c_int, _i64p, _f32p]
        L.orc_knn_bvh.argtypes = [_f32p, _i64p, c_int, _f32p, c_i64, c_int, c_int, _i64p, _f32p]
        L.orc_point_dist.argtypes = [_f32p, _f32p, c_int]
        L.orc_point_dist.restype = ctypes.c_float
        L.orc_pair_distances.argtypes = [_f32p, _f32p, _i64p, c_i64, c_int, c_int, _f32p]
        L.orc_num_threads.restype = c_int
        L.orc_set_num_threads.argtypes = [c_int]
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


# ---------------------------------------------------------------------------
# Closed forms and primitives
# ---------------------------------------------------------------------------
def leaf_level(n: int) -> int:
    return lib().orc_leaf_level(n)


def virtual_leaves(n: int) -> int:
    return lib().orc_virtual_leaves(n)


def real_node_count(n: int) -> int:
    return lib().orc_real_node_count(n)


def memory_index(n: int, i: int) -> int:
    return lib().orc_memory_index(n, i)


def is_virtual(n: int, i: int) -> bool:
    return bool(lib().orc_is_virtual(n, i))


def split3(x: int) -> int:
    return int(lib().orc_split3(x))


def split2(x: int) -> int:
    return int(lib().orc_split2(x))


def bounds(points) -> tuple[np.ndarray, np.ndarray]:
    p = _f32(points)
    n, D = p.shape
    lo = np.empty(D, np.float32)
    hi = np.empty(D, np.float32)
    lib().orc_bounds(p, n, D, lo, hi)
    return lo, hi


def morton_codes(points, lo, hi) -> np.ndarray:
    p = _f32(points)
    n, D = p.shape
    out = np.empty(n, np.uint32)
    lib().orc_morton_codes(p, n, D, _f32(lo), _f32(hi), out)
    return out


def hilbert_codes(points, lo, hi) -> np.ndarray:
    """Hilbert index of each point's Morton cell (30 bits in 3-D, 32 in 2-D)."""
    p = _f32(points)
    n, D = p.shape
    out = np.empty(n, np.uint32)
    lib().orc_hilbert_codes(p, n, D, _f32(lo), _f32(hi), out)
    return out


def hilbert_of_cells(cells, bits: int) -> np.ndarray:
    """Hilbert index of integer cells (n, D) with `bits` bits per axis."""
    c = np.ascontiguousarray(cells, dtype=np.uint32)
    n, D = c.shape
    out = np.empty(n, np.uint32)
    lib().orc_hilbert_cells(c, n, D, bits, out)
    return out


def stable_argsort(keys) -> np.ndarray:
    k = np.ascontiguousarray(np.asarray(keys, dtype=np.uint32))
    perm = np.empty(k.shape[0], np.int64)
    lib().orc_stable_argsort(k, k.shape[0], perm)
    return perm


def point_distance(q, p) -> float:
    q = _f32(q)
    return float(lib().orc_point_dist(q, _f32(p), q.shape[0]))


# ---------------------------------------------------------------------------
# Build
# ---------------------------------------------------------------------------
def build(points) -> dict:
    """Single-cloud build; returns the reference's single-handle payload
    (torchbvh/_query.py:39-54, bindings.cpp:137-153) as numpy arrays."""
    p = _f32(points)
    n, D = p.shape
    nr = real_node_count(n)
    node_aabbs = np.empty((nr, 2 * D), np.float32)
    sorted_idx = np.empty(n, np.int64)
    lo = np.empty(D, np.float32)
    hi = np.empty(D, np.float32)
    left = np.empty(nr, np.int32)
    right = np.empty(nr, np.int32)
    leaf = np.empty(nr, np.int32)
    lib().orc_build(p, n, D, node_aabbs, sorted_idx, lo, hi, left, right, leaf)
    return {
        "node_aabbs": node_aabbs,
        "sorted_indices": sorted_idx,
        "scene_min": lo,
        "scene_max": hi,
        "num_leaves": n,
        "num_real_nodes": nr,
        "leaf_level": leaf_level(n),
        "virtual_leaves": virtual_leaves(n),
        "dim": D,
        "left_child_mem": left,
        "right_child_mem": right,
        "mem_to_leaf": leaf,
    }


def morton_point_order(points) -> np.ndarray:
    """Point ordering of one cloud (torchbvh/csrc/bvh_build.cu:723-740, used
    by FPS): Morton codes against the points' plain min / max
    (points.min(1) / max(1), :731-732; no +-1e30 seeds, unlike the build),
    then a stable order (the reference's torch.sort is not stable; the two
    agree wherever codes are distinct)."""
    p = _f32(points)
    return stable_argsort(morton_codes(p, p.min(0), p.max(0)))


def build_batched(points) -> dict:
    """[B, N, D] build: the single build per cloud, stacked."""
    p = _f32(points)
    parts = [build(p[b]) for b in range(p.shape[0])]
    out = dict(parts[0])
    for key in ("node_aabbs", "sorted_indices", "scene_min", "scene_max"):
        out[key] = np.stack([q[key] for q in parts])
    out["batch_size"] = p.shape[0]
    return out


# ---------------------------------------------------------------------------
# Query ordering and k-NN
# ---------------------------------------------------------------------------
def query_order(queries, scene_min, scene_max) -> np.ndarray:
    """Morton order of queries against a BVH's bounds
    (torchbvh/csrc/morton_sort.cu:212-262)."""
    return stable_argsort(morton_codes(queries, scene_min, scene_max))


def schedule_order(queries, scene_min, scene_max) -> np.ndarray:
    """Traversal schedule of this library's query_knn (no reference
    counterpart; the reference uses query_order above): stable order by the
    top 16 bits of the Hilbert index of the query's Morton cell, ties by
    ascending query index."""
    q = _f32(queries)
    bits = 30 if q.shape[1] == 3 else 32
    codes = hilbert_codes(q, scene_min, scene_max).astype(np.uint64)
    return stable_argsort((codes >> np.uint64(bits - 16)).astype(np.uint32))


def build_primitives(primitives) -> dict:
    """Primitive build of one sample ((n, V, D): 2-D segments or 3-D
    triangles; torchbvh/csrc/bvh_build.cu:60-93, 757-821), with the centres."""
    p = _f32(primitives)
    n, V, D = p.shape
    nr = real_node_count(n)
    out = {
        "node_aabbs": np.empty((nr, 2 * D), np.float32),
        "sorted_indices": np.empty(n, np.int64),
        "scene_min": np.empty(D, np.float32),
        "scene_max": np.empty(D, np.float32),
        "left_child_mem": np.empty(nr, np.int32),
        "right_child_mem": np.empty(nr, np.int32),
        "mem_to_leaf": np.empty(nr, np.int32),
        "centers": np.empty((n, D), np.float32),
    }
    lib().orc_build_primitives(p, n, V, D, out["node_aabbs"], out["sorted_indices"], out["scene_min"],
                               out["scene_max"], out["left_child_mem"], out["right_child_mem"],
                               out["mem_to_leaf"], out["centers"])
    out.update(num_leaves=n, num_real_nodes=nr, leaf_level=leaf_level(n), virtual_leaves=virtual_leaves(n),
               dim=D)
    return out


def routed_order(queries, routes, true_min, true_max, false_min, false_max) -> np.ndarray:
    """Routed query order of one cloud (torchbvh/csrc/morton_sort.cu:82-120,
    240-286): each query encoded against its route's bounds, composite key
    route << code_bits | code, stable order."""
    q = _f32(queries)
    r = np.asarray(routes, dtype=bool)
    bits = 30 if q.shape[1] == 3 else 32
    ct = morton_codes(q, true_min, true_max).astype(np.uint64)
    cf = morton_codes(q, false_min, false_max).astype(np.uint64)
    key = np.where(r, ct | (np.uint64(1) << np.uint64(bits)), cf)
    return np.argsort(key, kind="stable").astype(np.int64)


def knn_routed(true_points, false_points, queries, routes, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Routed k-NN of one cloud (torchbvh/csrc/knn_query.cu:183-327): a query
    with a true route searches the true points, else the false points, whose
    indices follow the true cloud's (+ len(true_points)); rows in query order."""
    q = _f32(queries)
    r = np.asarray(routes, dtype=bool)
    idx = np.empty((q.shape[0], k), np.int64)
    dist = np.empty((q.shape[0], k), np.float32)
    if r.any():
        idx[r], dist[r] = knn(true_points, q[r], k)
    if (~r).any():
        i, d = knn(false_points, q[~r], k)
        idx[~r], dist[~r] = i + len(true_points), d
    return idx, dist


def knn_brute(points, queries, k: int) -> tuple[np.ndarray, np.ndarray]:
    p = _f32(points)
    q = _f32(queries)
    D = p.shape[1]
    m = q.shape[0]
    idx = np.empty((m, k), np.int64)
    dist = np.empty((m, k), np.float32)
    lib().orc_knn_brute(p, p.shape[0], q, m, D, k, idx, dist)
    return idx, dist


def knn_bvh(bvh: dict, queries, k: int) -> tuple[np.ndarray, np.ndarray]:
    q = _f32(queries)
    m = q.shape[0]
    D = bvh["dim"]
    idx = np.empty((m, k), np.int64)
    dist = np.empty((m, k), np.float32)
    lib().orc_knn_bvh(
        _f32(bvh["node_aabbs"]),
        np.ascontiguousarray(bvh["sorted_indices"], dtype=np.int64),
        int(bvh["num_leaves"]),
        q,
        m,
        D,
        k,
        idx,
        dist,
    )
    return idx, dist


def knn(points, queries, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Exact k-NN of one cloud: build + branch-and-bound (identical to
    knn_brute by construction of the tie rule; tests pin the two against
    each other)."""
    return knn_bvh(build(points), queries, k)


def knn_ragged(points, point_offsets, queries, query_offsets, k: int):
    """Per-cloud loop over packed inputs (torchbvh/_query.py:347-366)."""
    p = _f32(points)
    q = _f32(queries)
    idx_parts, dist_parts = [], []
    for b in range(len(point_offsets) - 1):
        p0, p1 = int(point_offsets[b]), int(point_offsets[b + 1])
        q0, q1 = int(query_offsets[b]), int(query_offsets[b + 1])
        i, d = knn(p[p0:p1], q[q0:q1], k)
        idx_parts.append(i)
        dist_parts.append(d)
    return np.concatenate(idx_parts), np.concatenate(dist_parts)


def pair_distances(points, queries, indices) -> np.ndarray:
    """Fused-chain distance of each query row to each of its returned points."""
    p = _f32(points)
    q = _f32(queries)
    idx = np.ascontiguousarray(indices, dtype=np.int64)
    m, k = idx.shape
    out = np.empty((m, k), np.float32)
    lib().orc_pair_distances(p, q, idx, m, p.shape[1], k, out)
    return out


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(int(n))


def num_threads() -> int:
    return int(lib().orc_num_threads())


__all__ = [
    "LIB_PATH",
    "bounds",
    "build",
    "build_batched",
    "is_virtual",
    "knn",
    "knn_brute",
    "knn_bvh",
    "knn_ragged",
    "leaf_level",
    "memory_index",
    "morton_codes",
    "num_threads",
    "pair_distances",
    "point_distance",
    "query_order",
    "real_node_count",
    "set_num_threads",
    "split2",
    "split3",
    "stable_argsort",
    "virtual_leaves",
]
