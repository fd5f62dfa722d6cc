"""``BVH``: owning wrapper with context-manager lifetime
(reference: torchbvh/_bvh_class.py:14-105)."""

from __future__ import annotations

import torch

from ._handles import BVHHandle, BatchedBVHHandle, RaggedBVHHandle, destroy_bvh
from ._query import _build_bvh_batched, _build_bvh_ragged, _build_bvh_single, query_knn
from ._validation import _as_contiguous, _as_contiguous_int64


class BVH:
    """BVH over ``(N, D)``, ``(B, N, D)`` or packed ``(total_N, D)`` points
    (with ``batch_offsets``).  Owns its handle; ``destroy`` is idempotent and
    runs on context-manager exit.  Handle fields are not exposed."""

    def __init__(self, points: torch.Tensor, *, batch_offsets: torch.Tensor | None = None) -> None:
        if batch_offsets is not None:
            if points.dim() != 2:
                raise ValueError("BVH: ragged mode requires 2-D points (total_N, D)")
            points = _as_contiguous(points)
            self._handle: BVHHandle | BatchedBVHHandle | RaggedBVHHandle = _build_bvh_ragged(
                points, _as_contiguous_int64(batch_offsets)
            )
        elif points.dim() == 3:
            points = _as_contiguous(points)
            self._handle = _build_bvh_batched(points)
        elif points.dim() == 2:
            points = _as_contiguous(points)
            self._handle = _build_bvh_single(points)
        else:
            raise ValueError("BVH: points must have shape (N, D) or (B, N, D)")
        self._points = points

    @property
    def destroyed(self) -> bool:
        return self._handle.destroyed

    def knn(
        self,
        query_points: torch.Tensor,
        k: int,
        *,
        query_offsets: torch.Tensor | None = None,
        source_points: torch.Tensor | None = None,
        sort_queries: bool = True,
    ):
        """Exact k-NN; ``query_offsets`` is required for ragged BVHs."""
        return query_knn(
            self._handle,
            query_points,
            k,
            query_offsets=query_offsets,
            source_points=source_points,
            sort_queries=sort_queries,
        )

    def interpolate(self, displaced_points, features, k: int = 8, *, return_grad: bool = False):
        """MLS interpolation belongs to the reference's MLS subsystem, which
        this library does not provide (only BVH build and k-NN)."""
        if isinstance(self._handle, RaggedBVHHandle):
            raise TypeError(
                "BVH.interpolate() is not supported for ragged inputs; "
                "use a single-sample or batched BVH"
            )
        raise NotImplementedError(
            "BVH.interpolate(): MLS interpolation is outside torchbvh_amd's scope "
            "(BVH build and exact k-NN only)"
        )

    def destroy(self) -> None:
        destroy_bvh(self._handle)

    def __enter__(self) -> "BVH":
        return self

    def __exit__(self, *args) -> None:
        self.destroy()
