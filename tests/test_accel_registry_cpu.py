"""The accel registry behind the reference-style k-NN bindings (CPU
tensors stand in for device ones: the registry only compares tensors)."""

from __future__ import annotations

import gc

import torch

from torchbvh_amd import _native


def test_registered_accel_follows_the_build_tensors_and_their_views():
    nodes = torch.rand(2, 7, 6)
    order = torch.arange(8).repeat(2, 1)
    accel = torch.zeros(16, dtype=torch.uint8)
    _native._register_accel(nodes, order, accel)
    assert _native._registered_accel(nodes, order) is accel
    assert _native._registered_accel(nodes[None], order[None]) is accel  # views of every element
    assert _native._registered_accel(nodes.clone(), order) is None
    assert _native._registered_accel(nodes, order.clone()) is None
    assert _native._registered_accel(nodes[:1], order) is None  # a part is not the BVH
    assert _native._pick_accel("op", False, nodes, order, 3) is None
    assert _native._pick_accel("op", None, nodes, order, 3) is accel


def test_explicit_accel_tensors_are_checked_before_launch():
    """An accel handed in explicitly must be contiguous 1-D uint8 on the
    queries' device and as large as the layout for the BVH's clouds; these
    checks run before any native call."""
    import pytest

    nodes = torch.rand(2, 7, 6)
    order = torch.arange(8).repeat(2, 1)
    for bad in (torch.ones(1), torch.zeros((2, 8), dtype=torch.uint8),
                torch.zeros(32, dtype=torch.uint8)[::2]):
        with pytest.raises(RuntimeError, match="contiguous 1-D uint8"):
            _native._pick_accel("op", bad, nodes, order, 3)
    with pytest.raises(RuntimeError, match="queries' device"):
        _native._pick_accel("op", torch.zeros(1 << 12, dtype=torch.uint8), nodes, order, 3)


def test_modified_tensors_lose_the_accel():
    nodes = torch.rand(1, 3, 4)
    order = torch.arange(2)[None]
    accel = torch.zeros(4, dtype=torch.uint8)
    _native._register_accel(nodes, order, accel)
    nodes[None].mul_(1.0)  # in place through a view: the shared version counter moves
    assert _native._registered_accel(nodes, order) is None
    nodes2 = torch.rand(1, 3, 4)
    order2 = torch.arange(2)[None]
    _native._register_accel(nodes2, order2, accel)
    order2.add_(0)
    assert _native._registered_accel(nodes2, order2) is None


def test_entry_goes_with_the_build_tensor():
    nodes = torch.rand(1, 3, 4)
    key = nodes.data_ptr()
    _native._register_accel(nodes, torch.arange(2)[None], torch.zeros(4, dtype=torch.uint8))
    assert key in _native._accel_registry
    del nodes
    gc.collect()
    assert key not in _native._accel_registry


def test_explicit_accels_belong_to_the_tensors_they_were_built_for():
    """Every accel the library builds is recorded with the node_aabbs it
    was built for and its point count; an explicit accel is accepted only
    with those tensors (or views of all of them), unmodified."""
    nodes = torch.rand(2, 7, 6)
    order = torch.arange(8).repeat(2, 1)
    accel = torch.zeros(64, dtype=torch.uint8)
    _native._register_accel(nodes, order, accel)
    assert _native._accel_belongs(accel, nodes, 16)
    assert _native._accel_belongs(accel[:], nodes[None], 16)  # views of every element
    assert not _native._accel_belongs(accel, nodes, 8)  # another point count
    assert not _native._accel_belongs(accel, nodes.clone(), 16)  # a copy of the tensors
    assert not _native._accel_belongs(accel.clone(), nodes, 16)  # a copy of the accel
    other = torch.rand(2, 7, 6)  # another cloud of the same size
    assert not _native._accel_belongs(accel, other, 16)
    nodes.add_(0)  # modified since the build
    assert not _native._accel_belongs(accel, nodes, 16)
    unrecorded = torch.zeros(64, dtype=torch.uint8)
    assert not _native._accel_belongs(unrecorded, other, 16)


def test_the_registry_follows_views_of_the_build_tensors():
    """The reference's single-cloud path squeezes the batch dimension at
    build time and unsqueezes it for every query (_query.py:51-53,139): the
    registered accel is found through such views while the handle holds them,
    and the entry goes with the last of them."""
    nodes = torch.rand(1, 7, 6)
    order = torch.arange(8)[None]
    accel = torch.zeros(16, dtype=torch.uint8)
    _native._register_accel(nodes, order, accel)
    held_nodes, held_order = nodes.squeeze(0), order.squeeze(0)
    key = nodes.data_ptr()
    del nodes, order
    gc.collect()
    assert _native._registered_accel(held_nodes.unsqueeze(0), held_order.unsqueeze(0)) is accel
    del held_nodes, held_order
    gc.collect()
    assert key not in _native._accel_registry


def test_tensors_registered_for_the_implicit_tree():
    """Tensors the device check found not to be a point BVH are registered
    with no accel: the bindings then take the implicit tree without
    checking again."""
    nodes = torch.rand(1, 7, 6)
    order = torch.arange(4)[None]
    _native._register_accel(nodes, order, None)
    assert _native._registry_entry(nodes, order) is not None
    assert _native._registered_accel(nodes, order) is None
    assert _native._pick_accel("op", None, nodes, order, 3) is None
