"""``BVH``: an owning object around one handle, destroyed on context exit.

Contract (torchbvh/_bvh_class.py:14-105): the constructor's signature, shape
dispatch and messages, `knn`, `destroyed`, idempotent `destroy`, context
manager use, and no item access to the handle's fields.  MLS interpolation,
which the reference also hangs on this class, is outside this library's
scope (`interpolate` says so; ragged BVHs keep the reference's TypeError).
"""

from __future__ import annotations

import torch

from ._handles import AnyHandle, RaggedBVHHandle
from ._query import _build_bvh_batched, _build_bvh_ragged, _build_bvh_single, query_knn
from ._validation import dense, dense_offsets

# Builder for each accepted point rank, without offsets.
_BUILDERS = {2: _build_bvh_single, 3: _build_bvh_batched}


class BVH:
    """BVH over ``(N, D)``, ``(B, N, D)`` or packed ``(total_N, D)`` points
    (with ``batch_offsets``)."""

    def __init__(self, points: torch.Tensor, *, batch_offsets: torch.Tensor | None = None) -> None:
        if batch_offsets is not None:
            if points.dim() != 2:
                raise ValueError("BVH: ragged mode requires 2-D points (total_N, D)")
            handle = _build_bvh_ragged(dense(points), dense_offsets(batch_offsets))
        else:
            build = _BUILDERS.get(points.dim())
            if build is None:
                raise ValueError("BVH: points must have shape (N, D) or (B, N, D)")
            handle = build(dense(points))
        self._handle: AnyHandle = handle

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
        """Exact k-NN (see `query_knn`); ``query_offsets`` is required for
        ragged BVHs."""
        return query_knn(self._handle, query_points, k, query_offsets=query_offsets,
                         source_points=source_points, sort_queries=sort_queries)

    def interpolate(self, displaced_points, features, k: int = 8, *, return_grad: bool = False):
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
        self._handle.destroy()

    def __enter__(self) -> "BVH":
        return self

    def __exit__(self, *exc) -> None:
        self.destroy()
