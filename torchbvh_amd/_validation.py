"""Argument checks of the public API.

What a caller can observe is the drop-in contract: the exception type
(ValueError), each message and the order in which the checks run (the
reference's tests match the messages by regex; they are defined in
torchbvh/_validation.py:1-75).  Here the checks are data: ordered tables of
(predicate, message) rules, walked by one function, so each table reads as
the specification of one argument.
"""

from __future__ import annotations

from collections.abc import Callable, Sequence

import torch

from ._constants import SUPPORTED_DIMS, SUPPORTED_K

# The reference's wording ("k must be 4, 8, or 16", which its tests match)
# stays a prefix of the message, and the one extension is named after it.
K_MESSAGE = "k must be 4, 8, or 16 (32 is also supported)"

Rule = tuple[Callable[..., bool], str]


def _walk(prefix: str, rules: Sequence[Rule], *subject, **names) -> None:
    """Raise ValueError for the first rule whose predicate fails."""
    for holds, message in rules:
        if not holds(*subject):
            raise ValueError(f"{prefix}: {message.format(**names)}")


# A float32 point/query tensor on the GPU; contiguity is a separate rule
# because most entry points copy non-contiguous input instead of rejecting it.
_CUDA_F32: Sequence[Rule] = (
    (lambda t: t.is_cuda, "{name} must be a CUDA tensor"),
    (lambda t: t.dtype == torch.float32, "{name} must be float32"),
)
_CONTIGUOUS: Sequence[Rule] = ((lambda t: t.is_contiguous(), "{name} must be contiguous"),)

# Ragged offsets: first the tensor (shape, dtype, placement), then, read back
# to the host once, the values.
_OFFSETS_TENSOR: Sequence[Rule] = (
    (lambda t, dev: t.dim() == 1, "offsets must have shape (B + 1,)"),
    (lambda t, dev: t.numel() >= 2, "offsets must contain at least two entries"),
    (lambda t, dev: t.dtype == torch.int64, "offsets must be int64"),
    (lambda t, dev: t.is_cuda, "offsets must be a CUDA tensor"),
    (lambda t, dev: t.is_contiguous(), "offsets must be contiguous"),
    (lambda t, dev: t.device == dev, "offsets must be on the same device as the packed tensor"),
)
_OFFSETS_VALUES: Sequence[Rule] = (
    (lambda v, total: v[0] == 0, "offsets must start at 0"),
    (lambda v, total: v[-1] == total, "final offset must match the packed tensor length"),
    (lambda v, total: all(b > a for a, b in zip(v, v[1:])), "offsets must be strictly increasing"),
)

# Packed ragged points (before their offsets).
_RAGGED_POINTS: Sequence[Rule] = (
    (lambda t: t.dim() == 2, "points must have shape (total_N, D)"),
    (lambda t: t.size(1) in SUPPORTED_DIMS, "D must be 2 or 3"),
    *_CUDA_F32,
    *_CONTIGUOUS,
)


# Build extent (sizes only, checked before any copy so that an expanded view
# is rejected without materialising it): every row of the call must have a
# signed 32-bit index.
_INT32_MAX = 2**31 - 1
_BUILD_EXTENT: Sequence[Rule] = (
    (lambda t: (t.size(0) if t.dim() == 2 else t.size(0) * t.size(1)) <= _INT32_MAX,
     "total point count must fit in signed int32"),
)


def _first_only(rules: Sequence[Rule]) -> Sequence[Rule]:
    """Rules on one tensor, restated for a subject of (tensor, *context)."""
    return tuple((lambda t, *_, holds=holds: holds(t), message) for holds, message in rules)


# source_points of a k-NN call, per handle layout; the subject is (tensor,
# payload, BVH device, packed point count): shape against the payload
# first, then dtype and placement.
_SOURCE_TAIL: Sequence[Rule] = (
    *_first_only(_CUDA_F32),
    (lambda t, data, dev, total: t.device == dev, "{name} must be on the same device as the BVH"),
)
_SOURCE_POINTS: dict[str, Sequence[Rule]] = {
    "single": (
        (lambda t, data, dev, total: t.dim() == 2, "{name} must have shape (N, D)"),
        (lambda t, data, dev, total: t.size(0) == data["num_leaves"],
         "{name} first dimension must match BVH num_leaves"),
        (lambda t, data, dev, total: t.size(1) == data["dim"], "{name} second dimension must match BVH dim"),
        *_SOURCE_TAIL,
    ),
    "batched": (
        (lambda t, data, dev, total: t.dim() == 3, "{name} must have shape (B, N, D)"),
        (lambda t, data, dev, total: t.size(0) == data["batch_size"],
         "{name} batch size must match BVH batch_size"),
        (lambda t, data, dev, total: t.size(1) == data["num_leaves"],
         "{name} second dimension must match BVH num_leaves"),
        (lambda t, data, dev, total: t.size(2) == data["dim"], "{name} last dimension must match BVH dim"),
        *_SOURCE_TAIL,
    ),
    "ragged": (
        (lambda t, data, dev, total: t.dim() == 2, "ragged {name} must have shape (total_N, D)"),
        (lambda t, data, dev, total: t.size(0) == total, "{name} first dimension must match BVH total_N"),
        (lambda t, data, dev, total: t.size(1) == data["dim"], "{name} second dimension must match BVH dim"),
        *_SOURCE_TAIL,
    ),
}


def check_build_extent(prefix: str, points: torch.Tensor) -> None:
    _walk(prefix, _BUILD_EXTENT, points)


def check_source_points(prefix: str, layout: str, source_points: torch.Tensor, data, device: torch.device,
                        total_rows: int | None = None) -> None:
    """`source_points` of a k-NN call on a handle of `layout` ("single",
    "batched" or "ragged") with payload `data` on `device`; `total_rows` is
    the packed point count of a ragged BVH."""
    _walk(prefix, _SOURCE_POINTS[layout], source_points, data, device, total_rows, name="source_points")


def check_k(prefix: str, k: int) -> None:
    if k not in SUPPORTED_K:
        raise ValueError(f"{prefix}: {K_MESSAGE}")


def check_cuda_f32(prefix: str, tensor: torch.Tensor, name: str) -> None:
    _walk(prefix, _CUDA_F32, tensor, name=name)


def check_offsets(prefix: str, offsets: torch.Tensor, *, total_rows: int, device: torch.device) -> list[int]:
    """Validate a (B + 1,) int64 offsets tensor and return its values as host
    ints (one device-to-host read)."""
    _walk(prefix, _OFFSETS_TENSOR, offsets, device)
    values = [int(v) for v in offsets.detach().cpu().tolist()]
    _walk(prefix, _OFFSETS_VALUES, values, total_rows)
    return values


def check_ragged_points(prefix: str, points: torch.Tensor, offsets: torch.Tensor) -> list[int]:
    _walk(prefix, _RAGGED_POINTS, points, name="points")
    return check_offsets(prefix, offsets, total_rows=int(points.size(0)), device=points.device)


def dense(tensor: torch.Tensor) -> torch.Tensor:
    """The tensor itself when contiguous, else a contiguous copy."""
    return tensor.contiguous()


def dense_offsets(offsets: torch.Tensor) -> torch.Tensor:
    """Like `dense` for int64 offsets; other dtypes pass through unchanged so
    that check_offsets reports the dtype rather than a copy's."""
    return offsets.contiguous() if offsets.dtype == torch.int64 else offsets
