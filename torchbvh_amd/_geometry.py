"""``PointGeometry``: a frozen snapshot of a point tensor plus one batched BVH
over it, for reuse across the queries of one forward pass.

Contract (torchbvh/_geometry.py:11-88): the constructor's checks and
messages, `validate(points)` accepting only the very tensor it was made from
and only while that tensor is unchanged, the `bvh` property, `destroyed`,
and use as a context manager that destroys on exit.

"Unchanged" is decided by a stamp of the source tensor taken at
construction: its version counter (bumped by every in-place write), storage
address, shape, strides, device and dtype.  The BVH is built over a detached
contiguous copy, so later writes to the source can never reach it; they only
make `validate` refuse the stale geometry.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from ._query import _build_bvh_batched


class _Stamp(NamedTuple):
    version: int
    data_ptr: int
    shape: tuple
    stride: tuple
    device: torch.device
    dtype: torch.dtype

    @classmethod
    def of(cls, t: torch.Tensor) -> "_Stamp":
        return cls(t._version, t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.device, t.dtype)


class PointGeometry:
    """Own a detached copy of float32 CUDA points ``(N, D)`` or ``(B, N, D)``
    and a batched BVH over it (single clouds become a batch of one)."""

    def __init__(self, points: torch.Tensor, *, experimental_fast: bool = False):
        if not isinstance(points, torch.Tensor) or points.ndim not in (2, 3):
            raise ValueError("PointGeometry: points must have shape (N, D) or (B, N, D)")
        if points.is_inference():
            raise ValueError("PointGeometry requires version-tracked source tensors")
        if not isinstance(experimental_fast, bool):
            raise TypeError("PointGeometry: experimental_fast must be bool")
        self.experimental_fast = experimental_fast
        self._source = points
        self._stamp = _Stamp.of(points)
        snapshot = points.detach().clone(memory_format=torch.contiguous_format)
        self._snapshot = snapshot if points.ndim == 3 else snapshot.unsqueeze(0)
        self._bvh = _build_bvh_batched(self._snapshot)

    @property
    def destroyed(self) -> bool:
        return self._bvh.destroyed

    def validate(self, points: torch.Tensor) -> "PointGeometry":
        if self.destroyed:
            raise RuntimeError("PointGeometry has been destroyed")
        if points is not self._source:
            raise ValueError("PointGeometry belongs to a different source tensor")
        if _Stamp.of(points) != self._stamp:
            raise ValueError("PointGeometry source changed; rebuild geometry")
        return self

    @property
    def bvh(self):
        """The batched BVH handle (borrowed: destroy the geometry, not it)."""
        return self.validate(self._source)._bvh

    @property
    def points(self) -> torch.Tensor:
        """The ``(B, N, D)`` snapshot the BVH was built over."""
        return self.validate(self._source)._snapshot

    def destroy(self) -> None:
        self._bvh.destroy()
        self._snapshot = None
        self._source = None

    def __enter__(self) -> "PointGeometry":
        return self.validate(self._source)

    def __exit__(self, *exc) -> None:
        self.destroy()
