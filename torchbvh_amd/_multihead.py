"""Multi-head displaced queries on top of the batched build and k-NN.

Mirrors the reference's helpers (torchbvh/_multihead.py:38-190): every
sample's points ``pos: (B, N, D)`` get one BVH; the per-point, per-head
query positions ``q: (B, N, H, D)`` are flattened to ``(B, N*H, D)`` and
answered by the Morton-ordered batched k-NN; results are reshaped back.
Names, argument checks and their messages follow the reference; the k-NN
underneath is this library's (exact, ties to the lower index).
"""

from __future__ import annotations

import torch

from ._constants import EXACT_DISTANCE_EPSILON, SUPPORTED_DIMS
from ._handles import scoped_bvh
from ._native import _C
from ._query import _build_bvh_batched, _query_knn_batched
from ._validation import check_cuda_f32, dense, dense_offsets

__all__ = ["query_displaced_knn", "gather_neighbor_values", "interpolate_displaced"]


def _check_displaced(pos: torch.Tensor, q: torch.Tensor, op: str) -> None:
    """Shape, dtype and device checks of the displaced-query helpers
    (reference order and messages: _multihead.py:17-35)."""
    if pos.dim() != 3:
        raise ValueError(f"{op}: pos must have shape (B, N, D)")
    if q.dim() != 4:
        raise ValueError(f"{op}: q must have shape (B, N, H, D)")
    if pos.size(2) not in SUPPORTED_DIMS:
        raise ValueError(f"{op}: D must be 2 or 3")
    checks = (
        (q.size(0) == pos.size(0), "q batch size must match pos"),
        (q.size(1) == pos.size(1), "q point dimension must match pos"),
        (q.size(3) == pos.size(2), "q last dimension must match pos"),
        (q.size(2) >= 1, "q must contain at least one head"),
    )
    for ok, message in checks:
        if not ok:
            raise ValueError(f"{op}: {message}")
    check_cuda_f32(op, pos, "pos")
    check_cuda_f32(op, q, "q")
    if pos.device != q.device:
        raise ValueError(f"{op}: pos and q must be on the same device")


def query_displaced_knn(pos: torch.Tensor, q: torch.Tensor, k: int = 8, *,
                        return_positions: bool = True):
    """k nearest points of ``pos[b]`` to every displaced query ``q[b, n, h]``.

    Returns local indices and squared distances of shape ``(B, N, H, k)``
    and, with ``return_positions``, the neighbours' coordinates
    ``(B, N, H, k, D)``."""
    _check_displaced(pos, q, "query_displaced_knn")
    pos = dense(pos)
    q = dense(q)
    B, N, H, D = q.shape
    queries = q.reshape(B, N * H, D).contiguous()
    sources = pos.detach().contiguous()
    with scoped_bvh(_build_bvh_batched, sources) as bvh:
        out = _query_knn_batched(bvh, queries, k,
                                 source_points=sources if return_positions else None,
                                 sort_queries=True)
    shapes = ((B, N, H, k), (B, N, H, k), (B, N, H, k, D))
    return tuple(t.reshape(shape).contiguous() for t, shape in zip(out, shapes))


def gather_neighbor_values(values: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """``out[b, n, h, j] = values[b, indices[b, n, h, j], h]``: per-head
    values of each neighbour, from the matching head only."""
    op = "gather_neighbor_values"
    if values.dim() != 4:
        raise ValueError(f"{op}: values must have shape (B, N, H, Ch)")
    if indices.dim() != 4:
        raise ValueError(f"{op}: indices must have shape (B, N, H, k)")
    for axis, what in ((0, "batch size"), (1, "point dimension"), (2, "head dimension")):
        if values.size(axis) != indices.size(axis):
            raise ValueError(f"{op}: indices {what} must match values")
    if values.size(3) < 1:
        raise ValueError(f"{op}: values must have at least one channel")
    check_cuda_f32(op, values, "values")
    if indices.dtype != torch.int64:
        raise ValueError(f"{op}: indices must be int64")
    if values.device != indices.device:
        raise ValueError(f"{op}: values and indices must be on the same device")
    values = dense(values)
    indices = dense_offsets(indices)
    if indices.numel() > 0:
        lo, hi = torch.aminmax(indices)
        if int(lo) < 0 or int(hi) >= values.size(1):
            raise ValueError(f"{op}: indices must be local source indices")
    B, _, H, _ = values.shape
    batch = torch.arange(B, device=values.device).view(B, 1, 1, 1)
    head = torch.arange(H, device=values.device).view(1, 1, H, 1)
    return values[batch, indices, head]


def interpolate_displaced(pos: torch.Tensor, q: torch.Tensor, values: torch.Tensor, k: int = 8, *,
                          reduction: str = "weighted_mean") -> torch.Tensor:
    """Inverse-squared-distance weighted mean of the matching head's values
    over the k neighbours of each displaced query, ``w = 1 / (d2 + 1e-12)``
    normalised over the neighbours; a query with exact hits (d2 <= 1e-12)
    gets the plain mean of those neighbours' values instead."""
    op = "interpolate_displaced"
    if reduction != "weighted_mean":
        raise ValueError(f"{op}: reduction must be 'weighted_mean'")
    _check_displaced(pos, q, op)
    if values.dim() != 4:
        raise ValueError(f"{op}: values must have shape (B, N, H, Ch)")
    if values.size(0) != pos.size(0) or values.size(1) != pos.size(1):
        raise ValueError(f"{op}: values first two dimensions must match pos")
    if values.size(2) != q.size(2):
        raise ValueError(f"{op}: values head dimension must match q")
    if values.size(3) < 1:
        raise ValueError(f"{op}: values must have at least one channel")
    check_cuda_f32(op, values, "values")
    if values.device != pos.device:
        raise ValueError(f"{op}: values must be on the same device as pos")
    values = dense(values)
    indices, d2 = query_displaced_knn(dense(pos), dense(q), k, return_positions=False)
    eps = EXACT_DISTANCE_EPSILON
    exact = d2 <= eps
    weights = torch.reciprocal(d2 + eps)
    weights = weights / weights.sum(dim=-1, keepdim=True).clamp(min=eps)
    if not (values.requires_grad and torch.is_grad_enabled()):
        # One kernel: the same rank-by-rank sums and exact-hit select, with
        # no gathered copy and no host synchronisation.
        return _C.interpolate_neighbors(values, indices, weights, exact)
    neighbours = gather_neighbor_values(values, indices)  # (B, N, H, k, Ch)
    # Accumulated neighbour rank by neighbour rank, the reference's order of
    # fp32 additions (_multihead.py:123-144).
    weighted = torch.zeros_like(values)
    exact_sum = torch.zeros_like(values)
    for r in range(indices.size(-1)):
        v = neighbours[..., r, :]
        weighted = weighted + v * weights[..., r].unsqueeze(-1)
        exact_sum = exact_sum + v * exact[..., r].to(values.dtype).unsqueeze(-1)
    if exact.any():
        counts = exact.to(values.dtype).sum(dim=-1, keepdim=True).clamp(min=1.0)
        weighted = torch.where(exact.any(dim=-1, keepdim=True), exact_sum / counts, weighted)
    return weighted
