"""Build and k-NN query entry points: validation, dispatch and handle payloads.

Public behaviour (signatures, dispatch, messages, payloads) follows
torchbvh/_query.py:29-405.  Ragged inputs differ in mechanism only: the
reference loops over clouds in Python with one native build/query per cloud
(:68-85, :299-366); here one segmented native build and one segmented
sort + k-NN launch sequence serve every cloud, and the per-cloud handles are
views into the packed result.
"""

from __future__ import annotations

import torch

from ._constants import SUPPORTED_DIMS
from ._handles import BVHHandle, BatchedBVHHandle, RaggedBVHHandle, live_payload
from ._native import _C
from ._validation import (
    check_build_extent,
    check_cuda_f32,
    check_k,
    check_offsets,
    check_ragged_points,
    check_source_points,
    dense,
    dense_offsets,
)


# ---------------------------------------------------------------------------
# Builders
# ---------------------------------------------------------------------------
def _build_bvh_single(points: torch.Tensor) -> BVHHandle:
    if points.dim() != 2:
        raise ValueError("build_bvh: points must have shape (N, D)")
    if points.size(1) not in SUPPORTED_DIMS:
        raise ValueError("build_bvh: D must be 2 or 3")
    check_cuda_f32("build_bvh", points, "points")
    # Sizes only, before any copy (an expanded view is rejected without
    # materialising it).
    check_build_extent("build_bvh", points)
    points = dense(points)
    batched = points.unsqueeze(0)
    data = _C.build_bvh_batched_cooperative(batched, with_accel=True)
    accel = data.pop("accel")
    # A single handle carries the payload without the batch dimension.
    del data["batch_size"]
    for key in ("node_aabbs", "sorted_indices", "scene_min", "scene_max"):
        data[key] = data[key].squeeze(0)
    return BVHHandle(data, aux={"accel": accel})


def _build_bvh_batched(points: torch.Tensor) -> BatchedBVHHandle:
    if points.dim() != 3:
        raise ValueError("build_bvh: batched points must have shape (B, N, D)")
    if points.size(2) not in SUPPORTED_DIMS:
        raise ValueError("build_bvh: D must be 2 or 3")
    check_cuda_f32("build_bvh", points, "points")
    # Sizes only, before any copy (an expanded view is rejected without
    # materialising it).
    check_build_extent("build_bvh", points)
    points = dense(points)
    data = _C.build_bvh_batched_cooperative(points, with_accel=True)
    accel = data.pop("accel")
    return BatchedBVHHandle(data, aux={"accel": accel})


def _build_bvh_ragged(points: torch.Tensor, batch_offsets: torch.Tensor) -> RaggedBVHHandle:
    points = dense(points)
    batch_offsets = dense_offsets(batch_offsets)
    offsets = check_ragged_points("build_bvh", points, batch_offsets)
    check_build_extent("build_bvh", points)
    counts = [b - a for a, b in zip(offsets, offsets[1:])]
    packed = _C.build_bvh_ragged(points, batch_offsets, counts, with_accel=True)
    accel = packed["accel"]
    dim = int(points.size(1))
    node_offsets = packed["host_node_offsets"]
    handles = []
    for b, n in enumerate(counts):
        n0, n1 = node_offsets[b], node_offsets[b + 1]
        p0, p1 = offsets[b], offsets[b + 1]
        handles.append(
            BVHHandle(
                {
                    "node_aabbs": packed["node_aabbs"][n0:n1],
                    "sorted_indices": packed["sorted_indices"][p0:p1],
                    "scene_min": packed["scene_min"][b],
                    "scene_max": packed["scene_max"][b],
                    "num_leaves": n,
                    "num_real_nodes": n1 - n0,
                    "leaf_level": (n - 1).bit_length(),
                    "virtual_leaves": (1 << (n - 1).bit_length()) - n,
                    "dim": dim,
                    "left_child_mem": packed["left_child_mem"][n0:n1],
                    "right_child_mem": packed["right_child_mem"][n0:n1],
                    "mem_to_leaf": packed["mem_to_leaf"][n0:n1],
                }
            )
        )
    return RaggedBVHHandle(
        {
            "batch_offsets": batch_offsets.clone(),
            "num_leaves_per_sample": torch.diff(batch_offsets).clone(),
            "batch_size": len(counts),
            "dim": dim,
        },
        handles,
        aux={
            "packed": packed,
            "host_offsets": offsets,
            "accel": accel,
        },
    )


def build_bvh(
    points: torch.Tensor,
    *,
    batch_offsets: torch.Tensor | None = None,
) -> BVHHandle | BatchedBVHHandle | RaggedBVHHandle:
    """Build a BVH; dispatches on the points' shape and ``batch_offsets``.

    - ``(N, D)`` → ``BVHHandle``
    - ``(B, N, D)`` → ``BatchedBVHHandle`` (independent trees per cloud)
    - ``(total_N, D)`` with ``batch_offsets`` ``(B + 1,)`` → ``RaggedBVHHandle``

    Ragged neighbour indices are local to each cloud.
    """
    if batch_offsets is not None:
        if points.dim() != 2:
            raise ValueError("build_bvh: ragged mode requires 2-D points (total_N, D)")
        return _build_bvh_ragged(points, batch_offsets)
    if points.dim() == 3:
        return _build_bvh_batched(points)
    if points.dim() == 2:
        return _build_bvh_single(points)
    raise ValueError("build_bvh: points must have shape (N, D) or (B, N, D)")


# ---------------------------------------------------------------------------
# Queries
# ---------------------------------------------------------------------------
# query_knn orders its traversal (the Hilbert schedule) only above this many
# queries.  Results do not depend on the order; below it the two-pass sort
# costs more than the coherence it buys (measured on MI355X with random-order
# queries: 10k-100k queries traverse 10-35% faster unsorted, sort included;
# from ~2^17-2^18 up the sorted order wins, 2x at 1M).
SCHEDULE_MIN_QUERIES = 1 << 17


def _schedule(sort_queries: bool, total_queries: int) -> bool:
    return sort_queries and total_queries > SCHEDULE_MIN_QUERIES


def _query_knn_single(
    bvh: BVHHandle,
    query_points: torch.Tensor,
    k: int,
    *,
    source_points: torch.Tensor | None = None,
    sort_queries: bool = True,
):
    check_k("query_knn", k)
    data = live_payload(bvh, BVHHandle, "query_knn")
    if query_points.dim() != 2:
        raise ValueError("query_knn: query_points must have shape (M, D)")
    if query_points.size(1) != data["dim"]:
        raise ValueError("query_knn: query_points second dimension must match BVH dim")
    check_cuda_f32("query_knn", query_points, "query_points")
    if query_points.device != data["sorted_indices"].device:
        raise ValueError("query_knn: query_points must be on the same device as the BVH")
    queries = dense(query_points).unsqueeze(0)
    node_aabbs = data["node_aabbs"].unsqueeze(0)
    sorted_indices = data["sorted_indices"].unsqueeze(0)
    accel = bvh._aux.get("accel")
    src = None
    if source_points is not None:
        check_source_points("query_knn", "single", source_points, data, data["sorted_indices"].device)
        src = dense(source_points).unsqueeze(0)
    if _schedule(sort_queries, int(queries.size(1))):
        order = _C.morton_sort_queries_narrow(
            queries, data["scene_min"].unsqueeze(0), data["scene_max"].unsqueeze(0), schedule=True
        )
        out = _C.query_knn_batched_cached_bounds_ordered(
            node_aabbs, sorted_indices, queries, order.contiguous(),
            data["num_leaves"], data["num_real_nodes"], data["dim"], k, accel=accel, source_points=src,
        )
    else:
        out = _C.query_knn_batched_cached_bounds(
            node_aabbs, sorted_indices, queries,
            data["num_leaves"], data["num_real_nodes"], data["dim"], k, accel=accel, source_points=src,
        )
    return tuple(t.squeeze(0) for t in out)


def _query_knn_batched(
    bvh: BatchedBVHHandle,
    query_points: torch.Tensor,
    k: int,
    *,
    source_points: torch.Tensor | None = None,
    sort_queries: bool = True,
):
    check_k("query_knn", k)
    data = live_payload(bvh, BatchedBVHHandle, "query_knn")
    if query_points.dim() != 3:
        raise ValueError("query_knn: batched query_points must have shape (B, M, D)")
    if query_points.size(0) != data["batch_size"]:
        raise ValueError("query_knn: query_points batch size must match BVH batch_size")
    if query_points.size(2) != data["dim"]:
        raise ValueError("query_knn: query_points last dimension must match BVH dim")
    check_cuda_f32("query_knn", query_points, "query_points")
    if query_points.device != data["sorted_indices"].device:
        raise ValueError("query_knn: query_points must be on the same device as the BVH")
    queries = dense(query_points)
    accel = bvh._aux.get("accel")
    src = None
    if source_points is not None:
        check_source_points("query_knn", "batched", source_points, data, data["sorted_indices"].device)
        src = dense(source_points)
    if _schedule(sort_queries, int(queries.size(0) * queries.size(1))):
        order = _C.morton_sort_queries_narrow(queries, data["scene_min"], data["scene_max"],
                                              schedule=True)
        return _C.query_knn_batched_cached_bounds_ordered(
            data["node_aabbs"], data["sorted_indices"], queries, order.contiguous(),
            data["num_leaves"], data["num_real_nodes"], data["dim"], k, accel=accel, source_points=src,
        )
    return _C.query_knn_batched_cached_bounds(
        data["node_aabbs"], data["sorted_indices"], queries,
        data["num_leaves"], data["num_real_nodes"], data["dim"], k, accel=accel, source_points=src,
    )


def _query_knn_ragged(
    bvh: RaggedBVHHandle,
    query_points: torch.Tensor,
    query_offsets: torch.Tensor,
    k: int,
    *,
    source_points: torch.Tensor | None = None,
):
    check_k("query_knn", k)
    data = live_payload(bvh, RaggedBVHHandle, "query_knn")
    if query_points.dim() != 2:
        raise ValueError("query_knn: ragged query_points must have shape (total_M, D)")
    if query_points.size(1) != data["dim"]:
        raise ValueError("query_knn: query_points second dimension must match BVH dim")
    check_cuda_f32("query_knn", query_points, "query_points")
    if query_points.device != data["batch_offsets"].device:
        raise ValueError("query_knn: query_points must be on the same device as the BVH")
    queries = dense(query_points)
    query_offsets = dense_offsets(query_offsets)
    q_offsets = check_offsets(
        "query_knn", query_offsets, total_rows=int(queries.size(0)), device=queries.device
    )
    if len(q_offsets) - 1 != data["batch_size"]:
        raise ValueError("query_knn: query_offsets batch size must match BVH batch_size")
    p_offsets = bvh._aux["host_offsets"]
    if any(b - a < k for a, b in zip(p_offsets, p_offsets[1:])):
        raise ValueError("query_knn: each source sample must contain at least k points")
    if source_points is not None:
        check_source_points("query_knn", "ragged", source_points, data, queries.device, p_offsets[-1])
        source_points = dense(source_points)

    packed = bvh._aux["packed"]
    order = None
    if _schedule(True, int(queries.size(0))):
        order = _C.morton_sort_queries_ragged(
            queries, query_offsets, packed["scene_min"], packed["scene_max"], data["batch_size"],
            schedule=True,
        )
    return _C.query_knn_ragged(
        packed["node_aabbs"], packed["sorted_indices"], data["batch_offsets"],
        packed["node_offsets"], queries, query_offsets, order, data["batch_size"],
        data["dim"], k, accel=bvh._aux.get("accel"), total_points=p_offsets[-1],
        source_points=source_points,
    )


def query_knn(
    bvh: BVHHandle | BatchedBVHHandle | RaggedBVHHandle,
    query_points: torch.Tensor,
    k: int,
    *,
    query_offsets: torch.Tensor | None = None,
    source_points: torch.Tensor | None = None,
    sort_queries: bool = True,
):
    """Exact k nearest neighbours; dispatches on the handle type.

    Returns ``(indices int64, squared_distances fp32)`` with rows ascending by
    (distance, index), or ``(indices, squared_distances, neighbor_positions)``
    when ``source_points`` is given.  Shapes: ``(M, k)`` single, ``(B, M, k)``
    batched, packed ``(total_M, k)`` ragged (``query_offsets`` required).
    """
    if isinstance(bvh, RaggedBVHHandle):
        if query_offsets is None:
            raise ValueError("query_knn: query_offsets is required when querying a ragged BVH")
        return _query_knn_ragged(bvh, query_points, query_offsets, k, source_points=source_points)
    if query_offsets is not None:
        raise TypeError("query_knn: query_offsets requires a RaggedBVHHandle")
    if isinstance(bvh, BatchedBVHHandle):
        return _query_knn_batched(
            bvh, query_points, k, source_points=source_points, sort_queries=sort_queries
        )
    return _query_knn_single(
        bvh, query_points, k, source_points=source_points, sort_queries=sort_queries
    )
