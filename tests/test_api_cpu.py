"""Public-API behaviour that is decided before any GPU work (CPU only):
package surface, constants and argument validation with the reference's
error types and messages (torchbvh tests/test_python_api.py,
tests/test_batched_python_api.py, tests/test_ragged_python_api.py)."""

from __future__ import annotations

import subprocess
import sys

import pytest
import torch

import torchbvh_amd as tb


def test_import_never_builds_or_loads_the_native_library():
    code = (
        "import torchbvh_amd, torchbvh_amd._native as n, sys; "
        "sys.exit(0 if n._lib is None else 1)"
    )
    assert subprocess.run([sys.executable, "-c", code]).returncode == 0


def test_public_surface():
    for name in ("BVH", "PointGeometry", "BVHHandle", "BatchedBVHHandle", "RaggedBVHHandle",
                 "build_bvh", "query_knn", "destroy_bvh", "SUPPORTED_K", "SUPPORTED_DIMS"):
        assert name in tb.__all__ and hasattr(tb, name)
    assert tb.SUPPORTED_K == (4, 8, 16, 32)
    assert tb.SUPPORTED_DIMS == (2, 3)
    assert not hasattr(tb.BVH, "__getitem__")


def test_query_rejects_non_handles():
    with pytest.raises(TypeError, match="BVHHandle"):
        tb.query_knn(object(), torch.empty((4, 2)), 4)
    with pytest.raises(TypeError, match="BVHHandle"):
        tb.query_knn({"dim": 2}, torch.empty((4, 2)), 4)


def test_destroy_rejects_plain_mapping():
    with pytest.raises(TypeError, match="handle returned by build_bvh"):
        tb.destroy_bvh({})


def test_build_validation_messages():
    with pytest.raises(ValueError, match="D must be 2 or 3"):
        tb.build_bvh(torch.zeros((4, 4)))
    with pytest.raises(ValueError, match="CUDA"):
        tb.build_bvh(torch.zeros((4, 2)))
    with pytest.raises(ValueError, match="shape"):
        tb.build_bvh(torch.zeros((1, 2, 4, 2)))
    with pytest.raises(ValueError, match="ragged mode requires 2-D points"):
        tb.build_bvh(torch.zeros((1, 4, 2)), batch_offsets=torch.tensor([0, 4]))
    with pytest.raises(ValueError, match="CUDA"):
        tb.build_bvh(torch.zeros((4, 2)), batch_offsets=torch.tensor([0, 4]))
    with pytest.raises(ValueError, match="D must be 2 or 3"):
        tb.build_bvh(torch.zeros((4, 5)), batch_offsets=torch.tensor([0, 4]))


def test_bvh_class_validation():
    with pytest.raises(ValueError, match=r"\(N, D\) or \(B, N, D\)"):
        tb.BVH(torch.zeros(4))
    with pytest.raises(ValueError, match="ragged mode requires 2-D points"):
        tb.BVH(torch.zeros((1, 4, 2)), batch_offsets=torch.tensor([0, 4]))


def test_point_geometry_validation():
    with pytest.raises(ValueError, match="shape"):
        tb.PointGeometry(torch.zeros(4))
    with torch.inference_mode():
        frozen = torch.zeros((4, 2))
    with pytest.raises(ValueError, match="version-tracked"):
        tb.PointGeometry(frozen)
    with pytest.raises(TypeError, match="experimental_fast"):
        tb.PointGeometry(torch.zeros((4, 2)), experimental_fast=1)


def test_k_message_lists_supported_values():
    """The reference's tests match "k must be 4, 8, or 16"; the message keeps
    that wording and names the k = 32 extension after it."""
    from torchbvh_amd._validation import check_k

    for k in (4, 8, 16, 32):
        check_k("query_knn", k)
    for k in (0, 1, 5, 12, 64):
        with pytest.raises(ValueError, match="k must be 4, 8, or 16") as err:
            check_k("query_knn", k)
        assert "32 is also supported" in str(err.value)


def test_handle_lifecycle_without_gpu():
    h = tb.BVHHandle({"dim": 3})
    assert not h.destroyed and h["dim"] == 3 and list(h) == ["dim"]
    tb.destroy_bvh(h)
    assert h.destroyed
    tb.destroy_bvh(h)
    with pytest.raises(RuntimeError, match="destroyed"):
        _ = h["dim"]
    inner = [tb.BVHHandle({"dim": 2}), tb.BVHHandle({"dim": 2})]
    r = tb.RaggedBVHHandle({"dim": 2}, inner)
    assert r["_ragged"] is True
    tb.destroy_bvh(r)
    assert r.destroyed and all(h.destroyed for h in inner)
    b = tb.BatchedBVHHandle({"dim": 2})
    assert b["_batched"] is True
    with pytest.raises(RuntimeError, match="Batched BVH handle has been destroyed"):
        b.destroy() or b["dim"]


@pytest.mark.parametrize("layout,good,cases", [
    ("single", (6, 3), [((6,), "source_points must have shape \\(N, D\\)"),
                        ((5, 3), "source_points first dimension must match BVH num_leaves"),
                        ((6, 2), "source_points second dimension must match BVH dim")]),
    ("batched", (2, 6, 3), [((6, 3), "source_points must have shape \\(B, N, D\\)"),
                            ((3, 6, 3), "source_points batch size must match BVH batch_size"),
                            ((2, 5, 3), "source_points second dimension must match BVH num_leaves"),
                            ((2, 6, 2), "source_points last dimension must match BVH dim")]),
    ("ragged", (9, 3), [((9,), "ragged source_points must have shape \\(total_N, D\\)"),
                        ((8, 3), "source_points first dimension must match BVH total_N"),
                        ((9, 2), "source_points second dimension must match BVH dim")]),
])
def test_source_points_rules_in_the_reference_order(layout, good, cases):
    """The source_points checks of query_knn (_query.py:197-215, 261-271 in
    the reference): shape against the handle first, then a CUDA float32
    tensor, then the BVH's device; each failure is a ValueError with the
    reference's message."""
    from torchbvh_amd._validation import check_source_points

    data = {"num_leaves": 6, "dim": 3, "batch_size": 2}
    cpu = torch.device("cpu")
    for shape, message in cases:
        with pytest.raises(ValueError, match=f"^query_knn: {message}$"):
            check_source_points("query_knn", layout, torch.zeros(shape), data, cpu, 9)
    # Right shape: the next rule is the device (CUDA), then the dtype.
    with pytest.raises(ValueError, match="source_points must be a CUDA tensor"):
        check_source_points("query_knn", layout, torch.zeros(good), data, cpu, 9)


def test_build_extent_rule_counts_every_row_without_materialising():
    from torchbvh_amd._validation import check_build_extent

    big = torch.zeros(1, 3).expand(1 << 16, 1 << 15, 3)  # 2^31 rows as a view
    with pytest.raises(ValueError, match="build_bvh: total point count must fit in signed int32"):
        check_build_extent("build_bvh", big)
    check_build_extent("build_bvh", torch.zeros(1, 3).expand((1 << 31) - 1, 3))
