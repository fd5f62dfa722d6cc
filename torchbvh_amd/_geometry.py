"""``PointGeometry``: an immutable point snapshot plus one batched BVH, reused
across queries within a forward (reference: torchbvh/_geometry.py:11-88)."""

from __future__ import annotations

from contextlib import contextmanager

import torch

from ._handles import _temporary_bvh
from ._query import _build_bvh_batched


class PointGeometry:
    """Own a detached copy of float32 CUDA points ``(N, D)`` or ``(B, N, D)``
    and a batched BVH over it.  Mutating the source tensor afterwards
    invalidates the object (checked through torch's version counter, data
    pointer, shape, strides, device and dtype)."""

    def __init__(self, points: torch.Tensor, *, experimental_fast: bool = False):
        if not isinstance(points, torch.Tensor) or points.ndim not in (2, 3):
            raise ValueError("PointGeometry: points must have shape (N, D) or (B, N, D)")
        if points.is_inference():
            raise ValueError("PointGeometry requires version-tracked source tensors")
        if not isinstance(experimental_fast, bool):
            raise TypeError("PointGeometry: experimental_fast must be bool")
        self.experimental_fast = experimental_fast
        self._source = points
        self._signature = self._source_signature(points)
        snapshot = points.detach().clone(memory_format=torch.contiguous_format)
        self._points = snapshot.unsqueeze(0) if points.ndim == 2 else snapshot
        self._bvh = _build_bvh_batched(self._points)

    @staticmethod
    def _source_signature(points: torch.Tensor):
        return (points._version, points.data_ptr(), tuple(points.shape),
                tuple(points.stride()), points.device, points.dtype)

    @property
    def destroyed(self) -> bool:
        return self._bvh.destroyed

    def validate(self, points: torch.Tensor) -> "PointGeometry":
        if self.destroyed:
            raise RuntimeError("PointGeometry has been destroyed")
        if points is not self._source:
            raise ValueError("PointGeometry belongs to a different source tensor")
        if self._source_signature(points) != self._signature:
            raise ValueError("PointGeometry source changed; rebuild geometry")
        return self

    @property
    def bvh(self):
        """The batched BVH handle (borrowed; do not destroy it)."""
        self.validate(self._source)
        return self._bvh

    @property
    def points(self) -> torch.Tensor:
        """The ``(B, N, D)`` snapshot the BVH was built over."""
        self.validate(self._source)
        return self._points

    def destroy(self) -> None:
        self._bvh.destroy()
        self._points = None
        self._source = None

    def __enter__(self) -> "PointGeometry":
        return self.validate(self._source)

    def __exit__(self, *args) -> None:
        self.destroy()


def _validate_geometry(points, geometry):
    if geometry is not None:
        if not isinstance(geometry, PointGeometry):
            raise TypeError("geometry must be a PointGeometry")
        geometry.validate(points)
    return geometry


@contextmanager
def _source_bvh(build_fn, points, geometry=None):
    if geometry is None:
        with _temporary_bvh(build_fn, points) as bvh:
            yield bvh
    else:
        yield geometry.bvh
