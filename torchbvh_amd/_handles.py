"""BVH handles: read-only mappings over the build payload with an explicit
lifetime (reference: torchbvh/_handles.py:7-120).

Single and batched handles expose exactly the reference's payload keys.
Library-private companions (packed ragged storage, offsets) live in
``handle._aux`` so the mapping's key set stays the reference's.
"""

from __future__ import annotations

from collections.abc import Iterator, Mapping
from contextlib import contextmanager

import torch


class _MappingBVHHandle(Mapping):
    """Liveness-checked mapping shared by all handle kinds."""

    _destroyed_message = "BVH handle has been destroyed"

    def __init__(self, data: Mapping, *, marker: str | None = None, aux: dict | None = None):
        self._data = dict(data)
        if marker is not None:
            self._data[marker] = True
        self._aux = dict(aux or {})
        self._destroyed = False

    @property
    def destroyed(self) -> bool:
        return self._destroyed

    def destroy(self) -> None:
        self._destroyed = True
        self._data.clear()
        self._aux.clear()

    def _require_live(self) -> dict:
        if self._destroyed:
            raise RuntimeError(self._destroyed_message)
        return self._data

    def __getitem__(self, key):
        return self._require_live()[key]

    def __iter__(self) -> Iterator:
        return iter(self._require_live())

    def __len__(self) -> int:
        return len(self._require_live())


class BVHHandle(_MappingBVHHandle):
    """Single-cloud BVH payload."""


class BatchedBVHHandle(_MappingBVHHandle):
    """Fixed-size batched BVH payload ([B, N, D] input)."""

    _destroyed_message = "Batched BVH handle has been destroyed"

    def __init__(self, data: Mapping, aux: dict | None = None):
        super().__init__(data, marker="_batched", aux=aux)


class RaggedBVHHandle(_MappingBVHHandle):
    """Packed ragged BVH: metadata keys plus one single-cloud view handle per
    cloud (``_handles``), all backed by one packed build."""

    _destroyed_message = "Ragged BVH handle has been destroyed"

    def __init__(self, data: Mapping, handles: list[BVHHandle], aux: dict | None = None):
        super().__init__(data, marker="_ragged", aux=aux)
        self._handles = list(handles)

    def destroy(self) -> None:
        if not self._destroyed:
            for handle in self._handles:
                handle.destroy()
        super().destroy()
        self._handles.clear()

    def _require_handles(self) -> list[BVHHandle]:
        self._require_live()
        return self._handles


def _bvh_data(bvh, prefix: str = "query_knn") -> Mapping:
    if isinstance(bvh, BVHHandle):
        return bvh._require_live()
    raise TypeError(f"{prefix}: bvh must be a BVHHandle returned by build_bvh")


def _batched_bvh_data(bvh, prefix: str = "query_knn") -> Mapping:
    if isinstance(bvh, BatchedBVHHandle):
        return bvh._require_live()
    raise TypeError(f"{prefix}: bvh must be a BatchedBVHHandle returned by build_bvh")


def _ragged_bvh_data(bvh, prefix: str = "query_knn"):
    if isinstance(bvh, RaggedBVHHandle):
        return bvh._require_live(), bvh._require_handles()
    raise TypeError(f"{prefix}: bvh must be a RaggedBVHHandle returned by build_bvh")


@contextmanager
def _temporary_bvh(build_fn, points: torch.Tensor):
    handle = build_fn(points)
    try:
        yield handle
    finally:
        destroy_bvh(handle)


def destroy_bvh(bvh: BVHHandle | BatchedBVHHandle | RaggedBVHHandle) -> None:
    """Destroy a handle and drop its tensor references (idempotent)."""
    if isinstance(bvh, _MappingBVHHandle):
        bvh.destroy()
        return
    raise TypeError("destroy_bvh: bvh must be a handle returned by build_bvh")
