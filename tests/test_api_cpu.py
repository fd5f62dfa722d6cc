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
