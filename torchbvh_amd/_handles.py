"""BVH handles: read-only mappings over a build's payload with an explicit
lifetime.

The public face is the drop-in contract (torchbvh/_handles.py:7-120): three
handle types, the payload keys (batched and ragged handles add a `_batched` /
`_ragged` marker key), RuntimeError on use after destroy with a per-type
message, TypeError naming the expected handle type, and a ragged handle
that destroys its per-cloud handles with it.

Underneath, a handle owns one `_Storage`: the payload the mapping shows, the
library's private companions (`aux`: the k-NN accel, the packed ragged
build and its host offsets) and the child handles that are views into that
storage.  Destroying a handle drops the storage, so every tensor it held is
released at once; liveness is simply whether the storage is still there.
"""

from __future__ import annotations

from collections.abc import Iterator, Mapping
from contextlib import contextmanager
from typing import Callable, Union


class _Storage:
    __slots__ = ("payload", "aux", "children")

    def __init__(self, payload: dict, aux: dict, children: list):
        self.payload = payload
        self.aux = aux
        self.children = children


class _Handle(Mapping):
    """Mapping view of a live `_Storage`."""

    _label = "BVH handle"   # names the handle in the use-after-destroy message
    _marker: str | None = None

    def __init__(self, data: Mapping, aux: dict | None = None, children: list | None = None):
        payload = dict(data)
        if self._marker is not None:
            payload[self._marker] = True
        self._store: _Storage | None = _Storage(payload, dict(aux or {}), list(children or []))

    @property
    def destroyed(self) -> bool:
        return self._store is None

    def destroy(self) -> None:
        store, self._store = self._store, None
        if store is not None:
            for child in store.children:
                child.destroy()

    def _live(self) -> _Storage:
        if self._store is None:
            raise RuntimeError(f"{self._label} has been destroyed")
        return self._store

    @property
    def _aux(self) -> dict:
        """Private companions of the payload (empty once destroyed)."""
        return {} if self._store is None else self._store.aux

    def __getitem__(self, key):
        return self._live().payload[key]

    def __iter__(self) -> Iterator:
        return iter(self._live().payload)

    def __len__(self) -> int:
        return len(self._live().payload)


class BVHHandle(_Handle):
    """Single-cloud BVH payload."""


class BatchedBVHHandle(_Handle):
    """Fixed-size batched BVH payload ([B, N, D] input)."""

    _label = "Batched BVH handle"
    _marker = "_batched"

    def __init__(self, data: Mapping, aux: dict | None = None):
        super().__init__(data, aux)


class RaggedBVHHandle(_Handle):
    """Packed ragged BVH: metadata keys plus one single-cloud handle per cloud
    (views into the one packed build), destroyed together."""

    _label = "Ragged BVH handle"
    _marker = "_ragged"

    def __init__(self, data: Mapping, handles: list[BVHHandle], aux: dict | None = None):
        super().__init__(data, aux, handles)

    @property
    def _handles(self) -> list[BVHHandle]:
        """The per-cloud handles (empty once destroyed)."""
        return [] if self._store is None else self._store.children


AnyHandle = Union[BVHHandle, BatchedBVHHandle, RaggedBVHHandle]


def live_payload(bvh, kind: type, prefix: str = "query_knn") -> Mapping:
    """The payload of a live handle of exactly the expected kind; TypeError
    naming that kind for anything else, RuntimeError if destroyed."""
    if not isinstance(bvh, kind):
        raise TypeError(f"{prefix}: bvh must be a {kind.__name__} returned by build_bvh")
    return bvh._live().payload


def destroy_bvh(bvh: AnyHandle) -> None:
    """Destroy a handle and drop its tensor references (idempotent)."""
    if not isinstance(bvh, _Handle):
        raise TypeError("destroy_bvh: bvh must be a handle returned by build_bvh")
    bvh.destroy()


@contextmanager
def scoped_bvh(build: Callable[..., AnyHandle], *args):
    """A handle built for the duration of a `with` block."""
    handle = build(*args)
    try:
        yield handle
    finally:
        handle.destroy()
