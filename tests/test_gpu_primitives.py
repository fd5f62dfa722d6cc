"""GPU parity of the primitive build and the point ordering against the
oracle: scene bounds, sort permutation, node boxes and traversal arrays
bit-exact.

Primitive sets follow the reference's ray tests (torchbvh
tests/test_raytrace.py:94-116: segments (3, 37, 2, 2) and triangles
(3, 29, 3, 3) in [-2, 2]) plus sizes around this library's 4096-primitive
tiles, each of which contributes one partial box to its sample's bounds."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from parity import assert_same_f32, assert_same_int
from torchbvh_amd._native import _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

SHAPES = [(2, 2), (3, 3)]


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def random_primitives(rng, B: int, F: int, V: int, D: int, spread: float = 0.05) -> np.ndarray:
    anchor = rng.random((B, F, 1, D), dtype=np.float32) * 4 - 2
    return (anchor + (rng.random((B, F, V, D), dtype=np.float32) - 0.5) * spread).astype(np.float32)


def check_primitive_build(prims: np.ndarray) -> dict:
    B, F, V, D = prims.shape
    h = _C.build_primitive_bvh_batched(dev(prims))
    for b in range(B):
        ref = oracle.build_primitives(prims[b])
        for key in ("num_leaves", "num_real_nodes", "leaf_level", "virtual_leaves", "dim"):
            assert h[key] == ref[key], key
        for key in ("scene_min", "scene_max", "node_aabbs"):
            assert_same_f32(h[key][b].cpu().numpy(), ref[key], f"sample {b} {key}")
        assert_same_int(h["sorted_indices"][b].cpu().numpy(), ref["sorted_indices"], f"sample {b} order")
        if b == 0:
            for key in ("left_child_mem", "right_child_mem", "mem_to_leaf"):
                assert h[key].dtype == torch.int32
                assert_same_int(h[key].cpu().numpy(), ref[key], key)
    assert h["batch_size"] == B and h["sorted_indices"].dtype == torch.int64
    return h


@pytest.mark.parametrize("V,D", SHAPES)
def test_primitive_build_reference_test_shapes(V, D):
    rng = np.random.default_rng(8102 + D)
    F = 37 if D == 2 else 29
    check_primitive_build((rng.random((3, F, V, D), dtype=np.float32) * 4 - 2).astype(np.float32))


@pytest.mark.parametrize("V,D", SHAPES)
@pytest.mark.parametrize("F", [1, 2, 3, 17, 256, 257, 4095, 4096, 4097, 50_001])
def test_primitive_build_sizes_around_tiles(F, V, D):
    check_primitive_build(random_primitives(np.random.default_rng(F + 10 * D), 2, F, V, D))


@pytest.mark.parametrize("V,D", SHAPES)
def test_primitive_build_degenerate_equals_point_build(V, D):
    rng = np.random.default_rng(33 + D)
    pts = (rng.integers(-128, 128, (2, 5000, D)) / 64.0).astype(np.float32)
    prims = np.repeat(pts[:, :, None, :], V, axis=2)
    h = check_primitive_build(prims)
    p = _C.build_bvh_batched_cooperative(dev(pts))
    for key in ("node_aabbs", "sorted_indices", "scene_min", "scene_max", "left_child_mem"):
        assert torch.equal(h[key], p[key]), key


def test_primitive_build_many_tiles():
    """62 tiles per sample: the per-cloud reduction of many tile boxes and
    sort offsets accumulated over many tiles."""
    check_primitive_build(random_primitives(np.random.default_rng(77), 2, 250_000, 3, 3))


def test_primitive_build_rejects_bad_shapes():
    bad = torch.zeros((1, 4, 3, 2), device=DEV)
    with pytest.raises(RuntimeError, match="expected 2-D segments or 3-D triangles"):
        _C.build_primitive_bvh_batched(bad)
    with pytest.raises(RuntimeError, match="at least one primitive"):
        _C.build_primitive_bvh_batched(torch.zeros((1, 0, 3, 3), device=DEV))


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("n", [1, 7, 4097, 100_003])
def test_morton_sort_points_matches_oracle(n, dim):
    rng = np.random.default_rng(n + dim)
    pts = rng.random((3, n, dim), dtype=np.float32)
    pts[1] *= 1e3
    pts[2, : n // 2] = 0.25  # heavy duplicates: stable order
    order = _C.morton_sort_points_batched(dev(pts))
    assert order.shape == (3, n) and order.dtype == torch.int64
    got = order.cpu().numpy()
    for b in range(3):
        assert_same_int(got[b], oracle.morton_point_order(pts[b]), f"cloud {b}")
    assert torch.equal(order, _C.build_bvh_batched_cooperative(dev(pts))["sorted_indices"])


@pytest.mark.parametrize("dim", [2, 3])
def test_morton_sort_points_bounds_are_unseeded(dim):
    """Clouds lying entirely beyond +-1e30 on one axis: the ordering's bounds
    are the points' own min/max (so that axis still spreads over the Morton
    grid), where the build's bounds stop at the 1e30 seed."""
    rng = np.random.default_rng(900 + dim)
    pts = rng.random((3, 5000, dim), dtype=np.float32)
    pts[0, :, 0] = 2e30 + pts[0, :, 0] * 1e30
    pts[1, :, dim - 1] = -(2e30 + pts[1, :, dim - 1] * 1e30)
    got = _C.morton_sort_points_batched(dev(pts)).cpu().numpy()
    built = _C.build_bvh_batched_cooperative(dev(pts))["sorted_indices"].cpu().numpy()
    for b in range(3):
        assert_same_int(got[b], oracle.morton_point_order(pts[b]), f"cloud {b}")
        assert_same_int(built[b], oracle.build(pts[b])["sorted_indices"], f"cloud {b} (seeded build)")
    assert not np.array_equal(got[0], built[0]) and not np.array_equal(got[1], built[1])
    assert np.array_equal(got[2], built[2])
