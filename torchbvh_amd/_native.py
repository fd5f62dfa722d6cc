"""ctypes binding of the C-ABI library and torch-facing wrappers.

``_C`` mirrors the reference's native module surface for this path
(torchbvh/csrc/bindings.cpp:155-199): ``build_bvh_batched_cooperative``,
``morton_sort_queries_narrow``, ``query_knn_batched_cached_bounds`` and
``query_knn_batched_cached_bounds_ordered`` take and return torch tensors with
the reference's shapes and dtypes, plus the ragged entry points this library
adds (one launch sequence for all clouds).  Outputs and workspaces are
allocated with torch on the input's device; every launch goes on the current
stream of that device.  Native precondition failures raise ``RuntimeError``
like the reference's ``TORCH_CHECK``.

The library must be built (``python -m torchbvh_amd._build``); there is no
fallback: without it every call raises.
"""

from __future__ import annotations

import ctypes
import functools
import threading
import weakref
from pathlib import Path
from typing import NamedTuple

import torch

from ._build import LIB_PATH

_lock = threading.Lock()
_lib = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_szp = ctypes.POINTER(ctypes.c_size_t)

# TBVH_ABI_VERSION of include/torchbvh_amd.h that these declarations follow.
ABI_VERSION = 2


def _declare(L) -> None:
    L.tbvh_abi_version.restype = _int
    L.tbvh_last_error.restype = ctypes.c_char_p
    L.tbvh_leaf_level.argtypes = [_i64]
    L.tbvh_leaf_level.restype = _int
    L.tbvh_virtual_leaves.argtypes = [_i64]
    L.tbvh_virtual_leaves.restype = _i64
    L.tbvh_real_node_count.argtypes = [_i64]
    L.tbvh_real_node_count.restype = _i64
    L.tbvh_build_workspace_size.argtypes = [_i64, _i64, _int, _szp]
    L.tbvh_build.argtypes = [_vp, _i64, _i64, _int] + [_vp] * 7 + [_vp, ctypes.c_size_t, _vp]
    L.tbvh_build_ragged_workspace_size.argtypes = [_i64, _i64, _int, _szp]
    L.tbvh_build_ragged.argtypes = (
        [_vp, _vp, _i64, _i64, _int] + [_vp] * 8 + [_i64, _vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_build_with_accel.argtypes = (
        [_vp, _i64, _i64, _int] + [_vp] * 8 + [_vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_build_with_accel_noalloc.argtypes = [_vp, _i64, _i64, _int] + [_vp] * 9
    L.tbvh_build_ragged_with_accel.argtypes = (
        [_vp, _vp, _i64, _i64, _int] + [_vp] * 8 + [_i64, _vp, _vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_build_primitives_workspace_size.argtypes = [_i64, _i64, _int, _int, _szp]
    L.tbvh_build_primitives.argtypes = (
        [_vp, _i64, _i64, _int, _int] + [_vp] * 7 + [_vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_morton_sort_points_workspace_size.argtypes = [_i64, _i64, _int, _szp]
    L.tbvh_morton_sort_points.argtypes = [_vp, _i64, _i64, _int, _vp, _vp, ctypes.c_size_t, _vp]
    L.tbvh_sort_queries_workspace_size.argtypes = [_i64, _i64, _int, _szp]
    L.tbvh_sort_queries.argtypes = [_vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    L.tbvh_sort_queries_ragged_workspace_size.argtypes = [_i64, _i64, _int, _szp]
    L.tbvh_sort_queries_ragged.argtypes = (
        [_vp, _vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_schedule_queries.argtypes = L.tbvh_sort_queries.argtypes
    L.tbvh_schedule_queries_ragged.argtypes = L.tbvh_sort_queries_ragged.argtypes
    L.tbvh_sort_routed_queries_workspace_size.argtypes = [_i64, _i64, _int, _szp]
    L.tbvh_sort_routed_queries.argtypes = (
        [_vp, _vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_knn_routed_spatial.argtypes = (
        [_vp] * 7 + [_i64] * 6 + [_int, _int, _vp, _vp, _vp]
    )
    L.tbvh_knn_accel_routed_spatial.argtypes = (
        [_vp] * 5 + [_i64] * 4 + [_int, _int, _vp, _vp, _vp]
    )
    L.tbvh_knn_accel_routed_grid_workspace_size.argtypes = [_i64, _i64, _i64, _i64, _int, _int, _vp]
    L.tbvh_knn_accel_routed_grid_spatial.argtypes = (
        [_vp, _vp, _i64, _vp, _vp, _i64] + [_vp] * 3 + [_i64] * 4
        + [_int, _int, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_morton_codes.argtypes = [_vp, _i64, _i64, _int, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    L.tbvh_knn.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, _vp, _vp, _vp]
    L.tbvh_knn_spatial.argtypes = L.tbvh_knn.argtypes
    L.tbvh_knn_ragged.argtypes = (
        [_vp] * 7 + [_i64, _i64, _int, _int, _vp, _vp, _vp]
    )
    L.tbvh_accel_size.argtypes = [_i64, _i64, _int, _szp]
    L.tbvh_accel_workspace_size.argtypes = [_i64, _i64, _int, _szp]
    L.tbvh_accel_build.argtypes = [_vp] * 5 + [_i64, _i64, _int, _vp, _vp, ctypes.c_size_t, _vp]
    L.tbvh_accel_build_from_tree.argtypes = [_vp, _vp, _i64, _i64, _i64, _int, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    L.tbvh_accel_build_ragged.argtypes = (
        [_vp] * 6 + [_i64, _i64, _int, _vp, _vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_knn_accel.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _vp, _vp, _vp]
    L.tbvh_knn_accel_spatial.argtypes = L.tbvh_knn_accel.argtypes
    L.tbvh_knn_accel_grid_workspace_size.argtypes = [_i64, _i64, _i64, _int, _int, _vp]
    L.tbvh_knn_accel_grid.argtypes = (
        [_vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _int, _int, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_knn_accel_ragged.argtypes = (
        [_vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _int, _int, _vp, _vp, _vp]
    )
    L.tbvh_knn_accel_positions.argtypes = (
        [_vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _vp, _int, _vp, _vp, _vp, _vp]
    )
    L.tbvh_knn_accel_grid_spatial.argtypes = L.tbvh_knn_accel_grid.argtypes
    L.tbvh_knn_accel_grid_positions.argtypes = (
        [_vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _int, _int, _vp, _int, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp]
    )
    L.tbvh_knn_accel_ragged_positions.argtypes = (
        [_vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _int, _int, _vp, _int, _vp, _vp, _vp, _vp]
    )
    L.tbvh_interpolate_neighbors.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _vp]
    for name in (
        "tbvh_build_workspace_size", "tbvh_build", "tbvh_build_ragged_workspace_size",
        "tbvh_build_ragged", "tbvh_build_with_accel", "tbvh_build_ragged_with_accel",
        "tbvh_sort_queries_workspace_size", "tbvh_sort_queries",
        "tbvh_sort_queries_ragged_workspace_size", "tbvh_sort_queries_ragged",
        "tbvh_schedule_queries", "tbvh_schedule_queries_ragged",
        "tbvh_morton_codes", "tbvh_knn", "tbvh_knn_ragged", "tbvh_accel_size",
        "tbvh_accel_workspace_size", "tbvh_accel_build", "tbvh_accel_build_ragged",
        "tbvh_knn_accel", "tbvh_knn_accel_ragged", "tbvh_knn_spatial", "tbvh_knn_accel_spatial",
        "tbvh_knn_accel_grid_workspace_size", "tbvh_knn_accel_grid", "tbvh_knn_accel_grid_spatial",
        "tbvh_knn_accel_positions", "tbvh_knn_accel_grid_positions", "tbvh_knn_accel_ragged_positions",
        "tbvh_sort_routed_queries_workspace_size", "tbvh_sort_routed_queries",
        "tbvh_knn_routed_spatial", "tbvh_knn_accel_routed_spatial",
        "tbvh_knn_accel_routed_grid_workspace_size", "tbvh_knn_accel_routed_grid_spatial",
        "tbvh_build_primitives_workspace_size", "tbvh_build_primitives",
        "tbvh_morton_sort_points_workspace_size", "tbvh_morton_sort_points",
        "tbvh_interpolate_neighbors", "tbvh_build_with_accel_noalloc", "tbvh_accel_build_from_tree",
    ):
        getattr(L, name).restype = _int


def library_path() -> Path:
    return LIB_PATH


def load():
    """Load the native library (torch's HIP runtime is loaded first, so the
    library binds to the same runtime instance as torch)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"torchbvh_amd: native library {LIB_PATH} is not built; "
                    "run `python -m torchbvh_amd._build` (hipcc, gfx950)"
                )
            L = ctypes.CDLL(str(LIB_PATH))
            _declare(L)
            if L.tbvh_abi_version() != ABI_VERSION:
                raise RuntimeError(
                    f"torchbvh_amd: {LIB_PATH} has ABI version {L.tbvh_abi_version()}, these bindings "
                    f"need {ABI_VERSION}; rebuild it with `python -m torchbvh_amd._build`"
                )
            _lib = L
    return _lib


def _last_error() -> str:
    msg = load().tbvh_last_error()
    return msg.decode() if msg else "unknown error"


def _check(status: int) -> None:
    if status != 0:
        raise RuntimeError(_last_error())


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _size(fn, *args) -> int:
    out = ctypes.c_size_t(0)
    _check(fn(*args, ctypes.byref(out)))
    return out.value


def _require(cond: bool, op: str, message: str) -> None:
    if not cond:
        raise RuntimeError(f"{op}: {message}")


def _require_device_f32(op: str, t: torch.Tensor, name: str) -> None:
    _require(t.is_cuda and t.is_contiguous() and t.dtype == torch.float32, op,
             f"{name} must be contiguous CUDA float32")


def _require_device_i64(op: str, t: torch.Tensor, name: str) -> None:
    _require(t.is_cuda and t.is_contiguous() and t.dtype == torch.int64, op,
             f"{name} must be contiguous CUDA int64")


# ---------------------------------------------------------------------------
# Closed forms
# ---------------------------------------------------------------------------
def leaf_level(n: int) -> int:
    return int(load().tbvh_leaf_level(n))


def virtual_leaves(n: int) -> int:
    return int(load().tbvh_virtual_leaves(n))


def real_node_count(n: int) -> int:
    return int(load().tbvh_real_node_count(n))


# Largest cloud the acceleration structure supports (28-bit bucket starts).
MAX_ACCEL_CLOUD = 1 << 28

# Batched accel k-NN calls with more queries than this take the cell-block
# search (tbvh_knn_accel_grid); below it its three extra launches cost more
# than it saves.
GRID_MIN_QUERIES = 1 << 17


@functools.lru_cache(maxsize=256)
def _grid_workspace_size(B: int, M: int, n: int, D: int, k: int) -> int:
    """Workspace bytes of the cell-block search for this call shape, 0
    where it does not run (tbvh_knn_accel_grid_workspace_size)."""
    need = ctypes.c_size_t(0)
    _check(load().tbvh_knn_accel_grid_workspace_size(B, M, n, D, k, ctypes.byref(need)))
    return int(need.value)


@functools.lru_cache(maxsize=256)
def _routed_grid_workspace_size(B: int, M: int, n_true: int, n_false: int, D: int, k: int) -> int:
    """Workspace bytes of the routed cell-block search, 0 where it does not
    run (tbvh_knn_accel_routed_grid_workspace_size)."""
    need = ctypes.c_size_t(0)
    _check(load().tbvh_knn_accel_routed_grid_workspace_size(B, M, n_true, n_false, D, k, ctypes.byref(need)))
    return int(need.value)


# ---------------------------------------------------------------------------
# Accel registry: a reference-style caller builds with the batched binding
# and later passes only the BVH's tensors to the k-NN bindings.  The build
# registers its accel under its node_aabbs; a k-NN call with accel=None
# whose node_aabbs and sorted_indices are those tensors or views of all
# their elements (the reference's single-cloud path squeezes the batch
# dimension at build time and unsqueezes it per query, _query.py:51-53,139),
# unmodified since (torch's version counters, which views share), traverses
# the accel instead of the implicit tree - identical results, about 10x
# fewer node visits.  Tensors it does not know (a clone, a copy, a reload)
# are checked on the device once (tbvh_accel_build_from_tree: leaf rows
# degenerate boxes, internal rows the merges of their children, leaf codes
# in order, indices in range - the point BVH the build writes) and get an
# accel built from node_aabbs and sorted_indices alone (the same bytes the
# build would have written); tensors that fail the check (a primitive BVH,
# edited boxes, another Morton order) are registered for the implicit tree,
# which answers for any boxes as the reference does.  accel=False forces
# the implicit tree.  Entries go when the registered node_aabbs is freed.
# ---------------------------------------------------------------------------
class _Held(NamedTuple):
    """A tensor the registry refers to without keeping it alive: its root
    (the tensor that owns the memory of a view), data pointer, element count
    and version when it was recorded."""

    root: weakref.ref
    ptr: int
    numel: int
    version: int

    def matches(self, t: torch.Tensor) -> bool:
        return (_root(t) is self.root() and t.data_ptr() == self.ptr and t.numel() == self.numel
                and t.is_contiguous() and t._version == self.version)


def _root(t: torch.Tensor) -> torch.Tensor:
    return t._base if t._base is not None else t


def _held(t: torch.Tensor, callback=None) -> _Held:
    return _Held(weakref.ref(_root(t), callback), t.data_ptr(), t.numel(), t._version)


_accel_registry: dict[int, tuple] = {}  # node_aabbs data pointer -> (_Held nodes, _Held order, accel | None)


def _register_accel(node_aabbs: torch.Tensor, sorted_indices: torch.Tensor, accel: torch.Tensor | None) -> None:
    """Record which accel answers for these tensors (None: the implicit
    tree).  A built accel is also recorded as belonging to them."""
    key = node_aabbs.data_ptr()

    def _drop(ref, key=key):
        entry = _accel_registry.get(key)
        if entry is not None and entry[0].root is ref:
            del _accel_registry[key]

    _accel_registry[key] = (_held(node_aabbs, _drop), _held(sorted_indices), accel)
    if accel is not None:
        _record_accel(accel, node_aabbs, int(sorted_indices.numel()))


def _registry_entry(node_aabbs: torch.Tensor, sorted_indices: torch.Tensor):
    entry = _accel_registry.get(node_aabbs.data_ptr())
    if entry is None or not (entry[0].matches(node_aabbs) and entry[1].matches(sorted_indices)):
        return None
    return entry


def _registered_accel(node_aabbs: torch.Tensor, sorted_indices: torch.Tensor):
    """The accel registered for these tensors, unmodified, or None (also
    when they are registered for the implicit tree)."""
    entry = _registry_entry(node_aabbs, sorted_indices)
    return None if entry is None else entry[2]


# Provenance of every accel this library builds: the node_aabbs it was
# built with and the point count it covers, so that an accel handed in
# explicitly is used only with the BVH it belongs to (an accel of another
# cloud of the same size would silently answer for that cloud).
_accel_owners: dict[int, tuple] = {}  # accel data pointer -> (accel ref, _Held nodes, total points)


def _record_accel(accel: torch.Tensor, node_aabbs: torch.Tensor, total_points: int) -> None:
    key = accel.data_ptr()

    def _drop(ref, key=key):
        entry = _accel_owners.get(key)
        if entry is not None and entry[0] is ref:
            del _accel_owners[key]

    _accel_owners[key] = (weakref.ref(accel, _drop), _held(node_aabbs), int(total_points))


def _fusable_source(source_points, device, lead: tuple) -> bool:
    """True when the traversal's epilogue can gather `source_points` rows:
    contiguous float32 on the queries' device with the points' leading
    shape (`lead`) and at most 4096 columns, and no gradient to carry (the
    reference's indexing is differentiable; a source that needs one takes
    the torch gather)."""
    if source_points is not None and torch.is_grad_enabled() and source_points.requires_grad:
        return False
    return (source_points is not None and isinstance(source_points, torch.Tensor)
            and source_points.is_cuda and source_points.device == device
            and source_points.dtype == torch.float32 and source_points.is_contiguous()
            and source_points.dim() == len(lead) + 1 and tuple(source_points.shape[:-1]) == lead
            and 1 <= source_points.size(-1) <= 4096)


def _with_positions(indices, distances, positions, source_points):
    """(indices, distances) or, when neighbour rows were asked for, also
    the rows: the fused result, or source_points[.., indices] gathered here."""
    if source_points is None:
        return indices, distances
    if positions is None:
        if indices.dim() == 3:  # batched: [B, M, k] indices into [B, N, C] rows
            B, M, k = indices.shape
            rows = source_points.gather(1, indices.reshape(B, M * k, 1).expand(B, M * k, source_points.size(-1)))
            positions = rows.reshape(B, M, k, source_points.size(-1))
        else:
            positions = source_points[indices]
    return indices, distances, positions


def _accel_belongs(accel: torch.Tensor, node_aabbs: torch.Tensor, total_points: int) -> bool:
    """True when this library built `accel` (the tensor itself or a view of
    all of it) for `node_aabbs` over `total_points` points, and node_aabbs
    has not been modified since."""
    owner = _accel_owners.get(accel.data_ptr())
    return (owner is not None and owner[0]() is _root(accel) and owner[2] == total_points
            and owner[1].matches(node_aabbs))


def _check_accel(op: str, accel, clouds: int, total_points: int, dim: int, device: torch.device,
                 node_aabbs: torch.Tensor) -> None:
    """An accel tensor handed in by the caller must be a contiguous 1-D
    uint8 tensor on the queries' device, 256-byte aligned (the kernels read
    it in 16-byte rows), at least as large as the layout for these clouds
    (the traversal then never reads outside it; it also bounds-checks every
    child ref and parent link against its cloud), and one this library built
    for exactly these node_aabbs, unmodified since: an accel of another
    cloud would silently answer for that cloud, and links corrupted into a
    cycle would keep the traversal running."""
    _require(isinstance(accel, torch.Tensor) and accel.dtype == torch.uint8 and accel.dim() == 1
             and accel.is_contiguous(), op, "accel must be a contiguous 1-D uint8 tensor")
    _require(accel.is_cuda and accel.device == device, op, "accel must be on the queries' device")
    _require(accel.data_ptr() % 256 == 0, op, "accel must be 256-byte aligned")
    need = _size(load().tbvh_accel_size, clouds, total_points, dim)
    _require(accel.numel() >= need, op,
             f"accel holds {accel.numel()} bytes; {clouds} cloud(s) of {total_points} points in total "
             f"need {need}")
    _require(_accel_belongs(accel, node_aabbs, total_points), op,
             "accel was not built by this library for these node_aabbs (or they were modified since)")


def _accel_from_tree(node_aabbs: torch.Tensor, sorted_indices: torch.Tensor, dim: int):
    """The accel of a batched BVH known only by its node_aabbs [B, nr, 2D]
    and sorted_indices [B, N], built and registered on first use; None (and
    registered as such) when a cloud is too large for one or the tensors are
    not the point BVH the build writes (checked on the device; the one host
    synchronisation of this path)."""
    B, N = int(sorted_indices.size(0)), int(sorted_indices.size(1))
    if N > MAX_ACCEL_CLOUD:
        _register_accel(node_aabbs, sorted_indices, None)
        return None
    L = load()
    dev = node_aabbs.device
    with torch.cuda.device(dev):
        accel = torch.empty(_size(L.tbvh_accel_size, B, B * N, dim), dtype=torch.uint8, device=dev)
        defects = torch.empty(1, dtype=torch.int32, device=dev)
        ws = _workspace(_size(L.tbvh_accel_workspace_size, B, B * N, dim), dev)
        _check(L.tbvh_accel_build_from_tree(_ptr(node_aabbs), _ptr(sorted_indices), B, N,
                                            int(node_aabbs.size(1)), int(dim), _ptr(accel), _ptr(defects),
                                            _ptr(ws), ws.numel(), _stream(dev)))
        if int(defects.item()) != 0:
            accel = None
    _register_accel(node_aabbs, sorted_indices, accel)
    return accel


def _pick_accel(op: str, accel, node_aabbs: torch.Tensor, sorted_indices: torch.Tensor, dim: int):
    """accel argument of the batched k-NN bindings (inputs already checked):
    False forces the implicit tree; a tensor is checked and used; None takes
    what the registry holds for these tensors (an accel, or the implicit
    tree), or checks them and builds one from them."""
    if accel is False:
        return None
    B, N = int(sorted_indices.size(0)), int(sorted_indices.size(1))
    if accel is None:
        entry = _registry_entry(node_aabbs, sorted_indices)
        return entry[2] if entry is not None else _accel_from_tree(node_aabbs, sorted_indices, dim)
    _check_accel(op, accel, B, B * N, dim, sorted_indices.device, node_aabbs)
    return accel


# ---------------------------------------------------------------------------
# Native operations (reference `_C` surface)
# ---------------------------------------------------------------------------
class _NativeOps:
    """Torch-level wrappers over the C ABI, named as the reference's `_C`."""

    @staticmethod
    def build_bvh_batched_cooperative(points: torch.Tensor, *, with_accel: bool | None = None) -> dict:
        """Batched build (bvh_build.cu:679-721).  Unless `with_accel` is
        False (and N <= MAX_ACCEL_CLOUD) the same launch sequence also builds
        the k-NN acceleration structure: returned under "accel" (None when
        too large) if `with_accel` is True; otherwise only registered for
        the k-NN bindings, so the result holds exactly the reference's keys."""
        op = "build_bvh_batched_cooperative"
        _require_device_f32(op, points, "points")
        _require(points.dim() == 3 and points.size(0) >= 1 and points.size(1) >= 1
                 and points.size(2) in (2, 3), op, "points must have shape (B, N, 2|3)")
        L = load()
        B, N, D = (int(s) for s in points.shape)
        dev = points.device
        with torch.cuda.device(dev):
            ws_bytes = _size(L.tbvh_build_workspace_size, B, N, D)
            nr = real_node_count(N)
            node_aabbs = torch.empty((B, nr, 2 * D), dtype=torch.float32, device=dev)
            sorted_indices = torch.empty((B, N), dtype=torch.int64, device=dev)
            scene_min = torch.empty((B, D), dtype=torch.float32, device=dev)
            scene_max = torch.empty((B, D), dtype=torch.float32, device=dev)
            left = torch.empty(nr, dtype=torch.int32, device=dev)
            right = torch.empty(nr, dtype=torch.int32, device=dev)
            leaf = torch.empty(nr, dtype=torch.int32, device=dev)
            ws = _workspace(ws_bytes, dev)
            accel = None
            if with_accel is not False and N <= MAX_ACCEL_CLOUD:
                accel = torch.empty(_size(L.tbvh_accel_size, B, B * N, D), dtype=torch.uint8,
                                    device=dev)
                _check(L.tbvh_build_with_accel(
                    _ptr(points), B, N, D, _ptr(node_aabbs), _ptr(sorted_indices),
                    _ptr(scene_min), _ptr(scene_max), _ptr(left), _ptr(right), _ptr(leaf),
                    _ptr(accel), _ptr(ws), ws.numel(), _stream(dev)))
            else:
                _check(L.tbvh_build(
                    _ptr(points), B, N, D, _ptr(node_aabbs), _ptr(sorted_indices),
                    _ptr(scene_min), _ptr(scene_max), _ptr(left), _ptr(right), _ptr(leaf),
                    _ptr(ws), ws.numel(), _stream(dev)))
        out = {
            "node_aabbs": node_aabbs,
            "sorted_indices": sorted_indices,
            "scene_min": scene_min,
            "scene_max": scene_max,
            "batch_size": B,
            "num_leaves": N,
            "num_real_nodes": nr,
            "leaf_level": leaf_level(N),
            "virtual_leaves": virtual_leaves(N),
            "dim": D,
            "left_child_mem": left,
            "right_child_mem": right,
            "mem_to_leaf": leaf,
        }
        if accel is not None:
            _register_accel(node_aabbs, sorted_indices, accel)
        if with_accel:
            out["accel"] = accel
        return out

    @staticmethod
    def build_primitive_bvh_batched(primitives: torch.Tensor) -> dict:
        """Batched BVH over segments (B, F, 2, 2) or triangles (B, F, 3, 3):
        leaves are the primitives' vertex boxes, ordered by the Morton codes
        of their centres (bvh_build.cu:757-821).  Same payload as the point
        build, with F leaves per cloud."""
        op = "build_primitive_bvh_batched"
        _require_device_f32(op, primitives, "primitives")
        _require(primitives.dim() == 4, op, "primitives must have shape (B, F, V, D)")
        _require(primitives.size(0) >= 1, op, "batch size must be at least 1")
        _require(primitives.size(1) >= 1, op, "each sample must contain at least one primitive")
        B, F, V, D = (int(s) for s in primitives.shape)
        _require((V, D) in ((2, 2), (3, 3)), op, "expected 2-D segments or 3-D triangles")
        L = load()
        dev = primitives.device
        with torch.cuda.device(dev):
            ws_bytes = _size(L.tbvh_build_primitives_workspace_size, B, F, V, D)
            nr = real_node_count(F)
            node_aabbs = torch.empty((B, nr, 2 * D), dtype=torch.float32, device=dev)
            sorted_indices = torch.empty((B, F), dtype=torch.int64, device=dev)
            scene_min = torch.empty((B, D), dtype=torch.float32, device=dev)
            scene_max = torch.empty((B, D), dtype=torch.float32, device=dev)
            left = torch.empty(nr, dtype=torch.int32, device=dev)
            right = torch.empty(nr, dtype=torch.int32, device=dev)
            leaf = torch.empty(nr, dtype=torch.int32, device=dev)
            ws = _workspace(ws_bytes, dev)
            _check(L.tbvh_build_primitives(
                _ptr(primitives), B, F, V, D, _ptr(node_aabbs), _ptr(sorted_indices),
                _ptr(scene_min), _ptr(scene_max), _ptr(left), _ptr(right), _ptr(leaf),
                _ptr(ws), ws.numel(), _stream(dev)))
        return {
            "node_aabbs": node_aabbs,
            "sorted_indices": sorted_indices,
            "scene_min": scene_min,
            "scene_max": scene_max,
            "batch_size": B,
            "num_leaves": F,
            "num_real_nodes": nr,
            "leaf_level": leaf_level(F),
            "virtual_leaves": virtual_leaves(F),
            "dim": D,
            "left_child_mem": left,
            "right_child_mem": right,
            "mem_to_leaf": leaf,
        }

    @staticmethod
    def morton_sort_points_batched(points: torch.Tensor) -> torch.Tensor:
        """Cloud-local Morton order of every cloud's points against its own
        bounds (bvh_build.cu:723-740), as `sorted_indices` of the build."""
        op = "morton_sort_points_batched"
        _require(isinstance(points, torch.Tensor) and points.is_cuda and points.is_contiguous()
                 and points.dtype == torch.float32, op, "points must be contiguous CUDA float32")
        _require(points.dim() == 3 and points.size(0) >= 1 and points.size(1) >= 1
                 and points.size(2) in (2, 3), op, "points must have shape (B, N, 2|3)")
        L = load()
        B, N, D = (int(s) for s in points.shape)
        dev = points.device
        with torch.cuda.device(dev):
            ws_bytes = _size(L.tbvh_morton_sort_points_workspace_size, B, N, D)
            order = torch.empty((B, N), dtype=torch.int64, device=dev)
            ws = _workspace(ws_bytes, dev)
            _check(L.tbvh_morton_sort_points(_ptr(points), B, N, D, _ptr(order), _ptr(ws), ws.numel(),
                                             _stream(dev)))
        return order

    @staticmethod
    def build_bvh_ragged(points: torch.Tensor, batch_offsets: torch.Tensor,
                         counts: list[int], *, with_accel: bool = False) -> dict:
        """Segmented build of packed clouds; `counts` are the host-side cloud
        sizes (already validated).  Returns packed tensors and per-cloud node
        offsets; with `with_accel` (and every cloud <= MAX_ACCEL_CLOUD) also
        the acceleration structure under "accel" (None otherwise)."""
        op = "build_bvh_ragged"
        _require_device_f32(op, points, "points")
        _require_device_i64(op, batch_offsets, "batch_offsets")
        L = load()
        T, D = (int(s) for s in points.shape)
        B = len(counts)
        dev = points.device
        node_counts = [real_node_count(c) for c in counts]
        total_nodes = sum(node_counts)
        with torch.cuda.device(dev):
            ws_bytes = _size(L.tbvh_build_ragged_workspace_size, B, T, D)
            node_aabbs = torch.empty((total_nodes, 2 * D), dtype=torch.float32, device=dev)
            sorted_indices = torch.empty(T, dtype=torch.int64, device=dev)
            scene_min = torch.empty((B, D), dtype=torch.float32, device=dev)
            scene_max = torch.empty((B, D), dtype=torch.float32, device=dev)
            left = torch.empty(total_nodes, dtype=torch.int32, device=dev)
            right = torch.empty(total_nodes, dtype=torch.int32, device=dev)
            leaf = torch.empty(total_nodes, dtype=torch.int32, device=dev)
            node_offsets = torch.empty(B + 1, dtype=torch.int64, device=dev)
            ws = _workspace(ws_bytes, dev)
            accel = None
            if with_accel and max(counts) <= MAX_ACCEL_CLOUD:
                accel = torch.empty(_size(L.tbvh_accel_size, B, T, D), dtype=torch.uint8,
                                    device=dev)
                _check(L.tbvh_build_ragged_with_accel(
                    _ptr(points), _ptr(batch_offsets), B, T, D, _ptr(node_aabbs),
                    _ptr(sorted_indices), _ptr(scene_min), _ptr(scene_max), _ptr(left),
                    _ptr(right), _ptr(leaf), _ptr(node_offsets), total_nodes, _ptr(accel),
                    _ptr(ws), ws.numel(), _stream(dev)))
            else:
                _check(L.tbvh_build_ragged(
                    _ptr(points), _ptr(batch_offsets), B, T, D, _ptr(node_aabbs),
                    _ptr(sorted_indices), _ptr(scene_min), _ptr(scene_max), _ptr(left),
                    _ptr(right), _ptr(leaf), _ptr(node_offsets), total_nodes,
                    _ptr(ws), ws.numel(), _stream(dev)))
        if accel is not None:
            _record_accel(accel, node_aabbs, T)
        host_node_offsets = [0]
        for c in node_counts:
            host_node_offsets.append(host_node_offsets[-1] + c)
        return {
            "node_aabbs": node_aabbs,
            "sorted_indices": sorted_indices,
            "scene_min": scene_min,
            "scene_max": scene_max,
            "left_child_mem": left,
            "right_child_mem": right,
            "mem_to_leaf": leaf,
            "node_offsets": node_offsets,
            "host_node_offsets": host_node_offsets,
            "accel": accel,
        }

    @staticmethod
    def build_accel(points: torch.Tensor, data: dict) -> torch.Tensor | None:
        """Acceleration structure for a batched build payload ([B, N, D]
        points and the tensors `build_bvh_batched_cooperative` returned);
        None when a cloud exceeds MAX_ACCEL_CLOUD points."""
        op = "build_accel"
        _require_device_f32(op, points, "points")
        B, N, D = (int(s) for s in points.shape)
        if N > MAX_ACCEL_CLOUD:
            return None
        L = load()
        dev = points.device
        with torch.cuda.device(dev):
            nbytes = _size(L.tbvh_accel_size, B, B * N, D)
            ws_bytes = _size(L.tbvh_accel_workspace_size, B, B * N, D)
            accel = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            ws = _workspace(ws_bytes, dev)
            _check(L.tbvh_accel_build(
                _ptr(points), _ptr(data["sorted_indices"]), _ptr(data["node_aabbs"]),
                _ptr(data["scene_min"]), _ptr(data["scene_max"]), B, N, D, _ptr(accel),
                _ptr(ws), ws.numel(), _stream(dev)))
        _record_accel(accel, data["node_aabbs"], B * N)
        return accel

    @staticmethod
    def build_accel_ragged(points: torch.Tensor, batch_offsets: torch.Tensor, packed: dict,
                           counts: list[int]) -> torch.Tensor | None:
        op = "build_accel_ragged"
        _require_device_f32(op, points, "points")
        if max(counts) > MAX_ACCEL_CLOUD:
            return None
        L = load()
        T, D = (int(s) for s in points.shape)
        B = len(counts)
        dev = points.device
        with torch.cuda.device(dev):
            nbytes = _size(L.tbvh_accel_size, B, T, D)
            ws_bytes = _size(L.tbvh_accel_workspace_size, B, T, D)
            accel = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            ws = _workspace(ws_bytes, dev)
            _check(L.tbvh_accel_build_ragged(
                _ptr(points), _ptr(batch_offsets), _ptr(packed["sorted_indices"]),
                _ptr(packed["node_aabbs"]), _ptr(packed["scene_min"]), _ptr(packed["scene_max"]),
                B, T, D, _ptr(accel), _ptr(ws), ws.numel(), _stream(dev)))
        _record_accel(accel, packed["node_aabbs"], T)
        return accel

    @staticmethod
    def morton_sort_queries_narrow(queries: torch.Tensor, scene_min: torch.Tensor,
                                   scene_max: torch.Tensor, *, schedule: bool = False) -> torch.Tensor:
        """Stable Morton order of [B, M, D] queries against per-cloud bounds.
        With ``schedule`` only the top 16 code bits are sorted (the
        traversal schedule ``query_knn`` uses; results do not depend on it)."""
        op = "morton_sort_queries_narrow"
        _require_device_f32(op, queries, "queries")
        _require(scene_min.is_cuda and scene_max.is_cuda and scene_min.is_contiguous()
                 and scene_max.is_contiguous(), op, "bounds must be contiguous CUDA tensors")
        _require(queries.dim() == 3 and queries.size(2) in (2, 3), op,
                 "queries must have shape (B, M, 2|3)")
        _require(scene_min.shape == scene_max.shape and scene_min.dim() == 2
                 and scene_min.size(0) == queries.size(0)
                 and scene_min.size(1) == queries.size(2), op, "bounds shape mismatch")
        _require(scene_min.dtype == torch.float32 and scene_max.dtype == torch.float32, op,
                 "bounds must be float32")
        L = load()
        B, M, D = (int(s) for s in queries.shape)
        dev = queries.device
        order = torch.empty((B, M), dtype=torch.int64, device=dev)
        if M == 0:
            return order
        fn = L.tbvh_schedule_queries if schedule else L.tbvh_sort_queries
        with torch.cuda.device(dev):
            ws_bytes = _size(L.tbvh_sort_queries_workspace_size, B, M, D)
            ws = _workspace(ws_bytes, dev)
            _check(fn(_ptr(queries), B, M, D, _ptr(scene_min), _ptr(scene_max), _ptr(order),
                      _ptr(ws), ws.numel(), _stream(dev)))
        return order

    @staticmethod
    def morton_sort_queries_ragged(queries: torch.Tensor, query_offsets: torch.Tensor,
                                   scene_min: torch.Tensor, scene_max: torch.Tensor,
                                   batch_size: int, *, schedule: bool = False) -> torch.Tensor:
        op = "morton_sort_queries_ragged"
        _require_device_f32(op, queries, "queries")
        _require_device_i64(op, query_offsets, "query_offsets")
        L = load()
        T, D = (int(s) for s in queries.shape)
        dev = queries.device
        order = torch.empty(T, dtype=torch.int64, device=dev)
        if T == 0:
            return order
        fn = L.tbvh_schedule_queries_ragged if schedule else L.tbvh_sort_queries_ragged
        with torch.cuda.device(dev):
            ws_bytes = _size(L.tbvh_sort_queries_ragged_workspace_size, batch_size, T, D)
            ws = _workspace(ws_bytes, dev)
            _check(fn(_ptr(queries), _ptr(query_offsets), batch_size, T, D, _ptr(scene_min),
                      _ptr(scene_max), _ptr(order), _ptr(ws), ws.numel(), _stream(dev)))
        return order

    @staticmethod
    def morton_codes(rows: torch.Tensor, scene_min: torch.Tensor,
                     scene_max: torch.Tensor) -> torch.Tensor:
        """Diagnostic: the Morton kernel's u32 codes (as int64) of [B, M, D]
        rows against per-cloud bounds [B, D]."""
        op = "morton_codes"
        _require_device_f32(op, rows, "rows")
        _require(rows.dim() == 3 and rows.size(2) in (2, 3), op, "rows must have shape (B, M, 2|3)")
        _require_device_f32(op, scene_min, "scene_min")
        _require_device_f32(op, scene_max, "scene_max")
        L = load()
        B, M, D = (int(s) for s in rows.shape)
        dev = rows.device
        codes = torch.empty((B, M), dtype=torch.int32, device=dev)
        if M == 0:
            return codes.to(torch.int64)
        with torch.cuda.device(dev):
            ws_bytes = _size(L.tbvh_sort_queries_workspace_size, B, M, D)
            ws = _workspace(ws_bytes, dev)
            _check(L.tbvh_morton_codes(
                _ptr(rows), B, M, D, _ptr(scene_min), _ptr(scene_max), _ptr(codes),
                _ptr(ws), ws.numel(), _stream(dev)))
        return codes.to(torch.int64) & 0xFFFFFFFF

    @staticmethod
    def _knn(op, node_aabbs, sorted_indices, query_points, query_order, num_leaves,
             num_real_nodes, dim, k, accel=None, spatial=False, source_points=None):
        _require(dim in (2, 3), op, "D must be 2 or 3")
        _require_device_f32(op, query_points, "query_points")
        _require(query_points.dim() == 3 and query_points.size(2) == dim, op,
                 "query_points must have shape (B, M, D)")
        _require_device_f32(op, node_aabbs, "node_aabbs")
        _require(node_aabbs.dim() == 3 and node_aabbs.size(0) == query_points.size(0)
                 and node_aabbs.size(1) == num_real_nodes and node_aabbs.size(2) == 2 * dim,
                 op, "node_aabbs has incompatible shape")
        _require_device_i64(op, sorted_indices, "sorted_indices")
        _require(sorted_indices.dim() == 2 and sorted_indices.size(0) == query_points.size(0)
                 and sorted_indices.size(1) == num_leaves, op,
                 "sorted_indices has incompatible shape")
        if query_order is not None:
            _require_device_i64(op, query_order, "query_order")
            _require(query_order.dim() == 2 and query_order.shape == query_points.shape[:2],
                     op, "query_order must have shape (B, M)")
        _require(num_leaves >= k, op, "num_leaves must be >= k")
        _require(1 <= num_leaves <= 1 << 30 and num_real_nodes == real_node_count(num_leaves), op,
                 "num_real_nodes does not match num_leaves")
        dev = query_points.device
        for t in (node_aabbs, sorted_indices) + ((query_order,) if query_order is not None else ()):
            _require(t.device == dev, op, "all inputs must share a device")
        accel = _pick_accel(op, accel, node_aabbs, sorted_indices, int(dim))
        B, M = int(query_points.size(0)), int(query_points.size(1))
        indices = torch.empty((B, M, k), dtype=torch.int64, device=dev)
        distances = torch.empty((B, M, k), dtype=torch.float32, device=dev)
        fused = _fusable_source(source_points, dev, (B, int(num_leaves))) and accel is not None
        positions = None
        if fused:
            C = int(source_points.size(-1))
            positions = torch.empty((B, M, k, C), dtype=torch.float32, device=dev)
        if M == 0:
            return _with_positions(indices, distances, positions, source_points)
        L = load()
        with torch.cuda.device(dev):
            grid = (accel is not None and B * M > GRID_MIN_QUERIES
                    and _grid_workspace_size(B, M, int(num_leaves), int(dim), int(k)) > 0)
            if fused and grid and not spatial:
                # The cell-block search with the neighbour rows (the same
                # rows as tbvh_knn_accel_positions).
                need = _grid_workspace_size(B, M, int(num_leaves), int(dim), int(k))
                ws = torch.empty(need, dtype=torch.uint8, device=dev)
                _check(L.tbvh_knn_accel_grid_positions(
                    _ptr(accel), _ptr(node_aabbs), int(num_real_nodes), _ptr(query_points), _ptr(query_order),
                    B, M, int(num_leaves), int(dim), int(k), _ptr(source_points), C, _ptr(indices),
                    _ptr(distances), _ptr(positions), _ptr(ws), need, _stream(dev)))
            elif fused:
                _check(L.tbvh_knn_accel_positions(
                    _ptr(accel), _ptr(query_points), _ptr(query_order), B, M, int(num_leaves),
                    int(dim), int(k), _ptr(source_points), C, _ptr(indices), _ptr(distances),
                    _ptr(positions), _stream(dev)))
            elif grid:
                need = _grid_workspace_size(B, M, int(num_leaves), int(dim), int(k))
                # The cell-block search first (same results; see
                # tbvh_knn_accel_grid), where the clouds allow a grid and
                # it measured faster (a nonzero workspace).
                ws = torch.empty(need, dtype=torch.uint8, device=dev)
                fn = L.tbvh_knn_accel_grid_spatial if spatial else L.tbvh_knn_accel_grid
                _check(fn(
                    _ptr(accel), _ptr(node_aabbs), int(num_real_nodes), _ptr(query_points), _ptr(query_order),
                    B, M, int(num_leaves), int(dim), int(k), _ptr(indices), _ptr(distances),
                    _ptr(ws), need, _stream(dev)))
            elif accel is not None:
                fn = L.tbvh_knn_accel_spatial if spatial else L.tbvh_knn_accel
                _check(fn(
                    _ptr(accel), _ptr(query_points), _ptr(query_order), B, M, int(num_leaves),
                    int(dim), int(k), _ptr(indices), _ptr(distances), _stream(dev)))
            else:
                fn = L.tbvh_knn_spatial if spatial else L.tbvh_knn
                _check(fn(
                    _ptr(node_aabbs), _ptr(sorted_indices), _ptr(query_points), _ptr(query_order),
                    B, M, int(num_leaves), int(num_real_nodes), int(dim), int(k),
                    _ptr(indices), _ptr(distances), _stream(dev)))
        return _with_positions(indices, distances, positions, source_points)

    @classmethod
    def query_knn_batched_cached_bounds(cls, node_aabbs, sorted_indices, query_points,
                                        num_leaves, num_real_nodes, dim, k, *, accel=None,
                                        source_points=None):
        """Unordered traversal.  `accel`: an accel tensor (identical results,
        fewer node visits), None for the one the batched build registered
        with these tensors (if any), False for the implicit tree.  With
        `source_points` ([B, num_leaves, C]) also returns the neighbours'
        rows [B, M, k, C] (source_points[b, indices[b, m, j]]), gathered in
        the traversal's epilogue when it runs on an accel and the source is
        contiguous float32, else with a torch gather afterwards."""
        return cls._knn("query_knn_batched_cached_bounds", node_aabbs, sorted_indices,
                        query_points, None, num_leaves, num_real_nodes, dim, k, accel,
                        source_points=source_points)

    @classmethod
    def query_knn_batched_cached_bounds_ordered(cls, node_aabbs, sorted_indices, query_points,
                                                query_order, num_leaves, num_real_nodes, dim, k,
                                                *, accel=None, source_points=None):
        """Morton-ordered traversal; `accel` and `source_points` as for the
        unordered one."""
        return cls._knn("query_knn_batched_cached_bounds_ordered", node_aabbs, sorted_indices,
                        query_points, query_order, num_leaves, num_real_nodes, dim, k, accel,
                        source_points=source_points)

    @classmethod
    def query_knn_batched_cached_bounds_spatial(cls, node_aabbs, sorted_indices, query_points,
                                                query_order, num_leaves, num_real_nodes, dim, k,
                                                *, accel=None):
        """Reference binding `query_knn_batched_cached_bounds_spatial`
        (bindings.cpp:199): as the ordered traversal, but row [b, m] of the
        output holds query query_order[b, m] (launch order).  `accel` as for
        the unordered traversal."""
        op = "query_knn_batched_cached_bounds_spatial"
        _require(query_order is not None, op, "query_order is required")
        return cls._knn(op, node_aabbs, sorted_indices, query_points, query_order, num_leaves,
                        num_real_nodes, dim, k, accel, spatial=True)

    @staticmethod
    def morton_sort_routed_queries_batched(queries: torch.Tensor, routes: torch.Tensor,
                                           true_scene_min: torch.Tensor, true_scene_max: torch.Tensor,
                                           false_scene_min: torch.Tensor,
                                           false_scene_max: torch.Tensor) -> torch.Tensor:
        """Reference binding `morton_sort_routed_queries_batched`
        (morton_sort.cu:288-329): stable order of (route, Morton code against
        the route's bounds) per cloud."""
        op = "morton_sort_routed_queries_batched"
        _require_device_f32(op, queries, "queries")
        _require(queries.dim() == 3 and queries.size(2) in (2, 3), op, "queries must have shape (B, M, D)")
        _require(routes.is_cuda and routes.is_contiguous() and routes.dtype == torch.bool, op,
                 "routes must be contiguous CUDA bool")
        _require(routes.dim() == 2 and tuple(routes.shape) == tuple(queries.shape[:2]), op,
                 "routes must have shape (B, M)")
        B, M, D = (int(s) for s in queries.shape)
        for t in (true_scene_min, true_scene_max, false_scene_min, false_scene_max):
            _require_device_f32(op, t, "scene bounds")
            _require(tuple(t.shape) == (B, D), op, "each scene bound must have shape (B, D)")
        dev = queries.device
        for t in (routes, true_scene_min, true_scene_max, false_scene_min, false_scene_max):
            _require(t.device == dev, op, "all inputs must share a device")
        L = load()
        order = torch.empty((B, M), dtype=torch.int64, device=dev)
        if M == 0:
            return order
        with torch.cuda.device(dev):
            ws = _workspace(_size(L.tbvh_sort_routed_queries_workspace_size, B, M, D), dev)
            _check(L.tbvh_sort_routed_queries(
                _ptr(queries), _ptr(routes), B, M, D, _ptr(true_scene_min), _ptr(true_scene_max),
                _ptr(false_scene_min), _ptr(false_scene_max), _ptr(order), _ptr(ws), ws.numel(),
                _stream(dev)))
        return order

    @staticmethod
    def query_knn_routed_batched_cached_bounds_spatial(
            true_node_aabbs, true_sorted_indices, false_node_aabbs, false_sorted_indices, query_points,
            routes, query_order, true_num_leaves, true_num_real_nodes, false_num_leaves,
            false_num_real_nodes, dim, k, *, true_accel=None, false_accel=None):
        """Reference binding `query_knn_routed_batched_cached_bounds_spatial`
        (knn_query.cu:463-539): routed search, output rows in launch order,
        false-route indices offset by true_num_leaves.  With both accels
        (passed, or registered by the batched builds; False forces the
        implicit trees) the accelerated traversal (identical results)."""
        op = "query_knn_routed_batched_cached_bounds_spatial"
        _require(dim in (2, 3), op, "D must be 2 or 3")
        _require_device_f32(op, query_points, "query_points")
        _require(query_points.dim() == 3 and query_points.size(2) == dim, op,
                 "query_points must have shape (B, M, D)")
        B, M = int(query_points.size(0)), int(query_points.size(1))
        _require(routes.is_cuda and routes.is_contiguous() and routes.dtype == torch.bool
                 and tuple(routes.shape) == (B, M), op, "routes must be contiguous CUDA bool (B, M)")
        _require_device_i64(op, query_order, "query_order")
        _require(tuple(query_order.shape) == (B, M), op, "query_order must have shape (B, M)")
        for nodes, nr, name in ((true_node_aabbs, true_num_real_nodes, "true_node_aabbs"),
                                (false_node_aabbs, false_num_real_nodes, "false_node_aabbs")):
            _require_device_f32(op, nodes, name)
            _require(tuple(nodes.shape) == (B, nr, 2 * dim), op, f"{name} has incompatible shape")
        for srt, n, name in ((true_sorted_indices, true_num_leaves, "true_sorted_indices"),
                             (false_sorted_indices, false_num_leaves, "false_sorted_indices")):
            _require_device_i64(op, srt, name)
            _require(tuple(srt.shape) == (B, n), op, f"{name} has incompatible shape")
        _require(true_num_leaves >= k and false_num_leaves >= k, op, "both source counts must be >= k")
        for n, nr in ((true_num_leaves, true_num_real_nodes), (false_num_leaves, false_num_real_nodes)):
            _require(n <= 1 << 30 and nr == real_node_count(n), op, "num_real_nodes does not match num_leaves")
        dev = query_points.device
        indices = torch.empty((B, M, k), dtype=torch.int64, device=dev)
        distances = torch.empty((B, M, k), dtype=torch.float32, device=dev)
        if M == 0:
            return indices, distances
        true_accel = _pick_accel(op, true_accel, true_node_aabbs, true_sorted_indices, int(dim))
        false_accel = _pick_accel(op, false_accel, false_node_aabbs, false_sorted_indices, int(dim))
        L = load()
        with torch.cuda.device(dev):
            need = 0
            if true_accel is not None and false_accel is not None and B * M > GRID_MIN_QUERIES:
                need = _routed_grid_workspace_size(B, M, int(true_num_leaves), int(false_num_leaves),
                                                   int(dim), int(k))
            if need > 0:
                # The cell-block search in each query's route's structure
                # first (the same results; see tbvh_knn_accel_grid).
                ws = torch.empty(need, dtype=torch.uint8, device=dev)
                _check(L.tbvh_knn_accel_routed_grid_spatial(
                    _ptr(true_accel), _ptr(true_node_aabbs), int(true_num_real_nodes), _ptr(false_accel),
                    _ptr(false_node_aabbs), int(false_num_real_nodes), _ptr(query_points), _ptr(routes),
                    _ptr(query_order), B, M, int(true_num_leaves), int(false_num_leaves), int(dim), int(k),
                    _ptr(indices), _ptr(distances), _ptr(ws), need, _stream(dev)))
            elif true_accel is not None and false_accel is not None:
                _check(L.tbvh_knn_accel_routed_spatial(
                    _ptr(true_accel), _ptr(false_accel), _ptr(query_points), _ptr(routes),
                    _ptr(query_order), B, M, int(true_num_leaves), int(false_num_leaves), int(dim),
                    int(k), _ptr(indices), _ptr(distances), _stream(dev)))
            else:
                _check(L.tbvh_knn_routed_spatial(
                    _ptr(true_node_aabbs), _ptr(true_sorted_indices), _ptr(false_node_aabbs),
                    _ptr(false_sorted_indices), _ptr(query_points), _ptr(routes), _ptr(query_order),
                    B, M, int(true_num_leaves), int(true_num_real_nodes), int(false_num_leaves),
                    int(false_num_real_nodes), int(dim), int(k), _ptr(indices), _ptr(distances),
                    _stream(dev)))
        return indices, distances

    @staticmethod
    def query_knn_ragged(node_aabbs, sorted_indices, point_offsets, node_offsets, query_points,
                         query_offsets, query_order, batch_size, dim, k, *, accel=None,
                         total_points=None, source_points=None):
        op = "query_knn_ragged"
        if accel is False:  # the implicit trees, as for the batched bindings
            accel = None
        _require_device_f32(op, query_points, "query_points")
        _require_device_f32(op, node_aabbs, "node_aabbs")
        _require_device_i64(op, sorted_indices, "sorted_indices")
        for name, t in (("point_offsets", point_offsets), ("node_offsets", node_offsets),
                        ("query_offsets", query_offsets)):
            _require_device_i64(op, t, name)
        T = int(query_points.size(0))
        dev = query_points.device
        if accel is not None:
            _require(total_points is not None, op, "total_points is required with an accel")
            _check_accel(op, accel, int(batch_size), int(total_points), int(dim), dev, node_aabbs)
        indices = torch.empty((T, k), dtype=torch.int64, device=dev)
        distances = torch.empty((T, k), dtype=torch.float32, device=dev)
        # Neighbour rows (packed like the points; indices are cloud-local):
        # fused in the traversal with an accel, else gathered by the caller.
        fused = (accel is not None and total_points is not None
                 and _fusable_source(source_points, dev, (int(total_points),)))
        positions = None
        if fused:
            C = int(source_points.size(-1))
            positions = torch.empty((T, k, C), dtype=torch.float32, device=dev)
        if T == 0:
            if source_points is None:
                return indices, distances
            return indices, distances, source_points.new_empty((0, k) + tuple(source_points.shape[1:]))
        L = load()
        with torch.cuda.device(dev):
            if fused:
                _check(L.tbvh_knn_accel_ragged_positions(
                    _ptr(accel), _ptr(point_offsets), int(total_points), _ptr(query_points),
                    _ptr(query_offsets), _ptr(query_order), int(batch_size), T, int(dim), int(k),
                    _ptr(source_points), C, _ptr(indices), _ptr(distances), _ptr(positions), _stream(dev)))
            elif accel is not None:
                _check(L.tbvh_knn_accel_ragged(
                    _ptr(accel), _ptr(point_offsets), int(total_points), _ptr(query_points),
                    _ptr(query_offsets), _ptr(query_order), int(batch_size), T, int(dim), int(k),
                    _ptr(indices), _ptr(distances), _stream(dev)))
            else:
                _check(L.tbvh_knn_ragged(
                    _ptr(node_aabbs), _ptr(sorted_indices), _ptr(point_offsets), _ptr(node_offsets),
                    _ptr(query_points), _ptr(query_offsets), _ptr(query_order), int(batch_size), T,
                    int(dim), int(k), _ptr(indices), _ptr(distances), _stream(dev)))
        if source_points is None:
            return indices, distances
        if positions is None:  # not fused: rows of each query's cloud, indices cloud-local
            counts = query_offsets[1:] - query_offsets[:-1]
            starts = point_offsets[:-1].repeat_interleave(counts, output_size=T)
            positions = source_points[indices + starts[:, None]]
        return indices, distances, positions

    @staticmethod
    def interpolate_neighbors(values, indices, weights, exact):
        """Rank loop and exact-hit select of `interpolate_displaced`
        (_multihead.py:123-144) in one kernel: values (B, N, H, C);
        indices, weights, exact (B, N, H, k).  Returns (B, N, H, C)."""
        op = "interpolate_neighbors"
        _require_device_f32(op, values, "values")
        _require_device_i64(op, indices, "indices")
        _require_device_f32(op, weights, "weights")
        _require(exact.dtype == torch.bool and exact.is_contiguous(), op, "exact must be a contiguous bool tensor")
        B, N, H, C = (int(x) for x in values.shape)
        k = int(indices.size(-1))
        for name, t in (("indices", indices), ("weights", weights), ("exact", exact)):
            _require(tuple(t.shape) == (B, N, H, k) and t.device == values.device, op,
                     f"{name} must have shape (B, N, H, k) on the values' device")
        out = torch.empty_like(values)
        if out.numel() == 0:
            return out
        dev = values.device
        with torch.cuda.device(dev):
            _check(load().tbvh_interpolate_neighbors(
                _ptr(values), _ptr(indices), _ptr(weights), _ptr(exact), B, N, H, C, k, _ptr(out),
                _stream(dev)))
        return out


_C = _NativeOps()
