"""The no-allocation build entry point (tbvh_build_with_accel_noalloc), called
through the C ABI, against tbvh_build_with_accel on the same inputs: every
output (node AABBs, sorted indices, bounds, traversal arrays and the accel
bytes) must be bit-identical, on two calls in a row (the second with a
smaller cloud, so stale scratch contents from the first would show), and a
k-NN over its accel must match the oracle."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from torchbvh_amd import _native

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def _outputs(B: int, N: int, D: int) -> dict:
    L = _native.load()
    nr = _native.real_node_count(N)
    accel_bytes = _native._size(L.tbvh_accel_size, B, B * N, D)
    return {
        "node_aabbs": torch.full((B, nr, 2 * D), float("nan"), dtype=torch.float32, device=DEV),
        "sorted_indices": torch.full((B, N), -7, dtype=torch.int64, device=DEV),
        "scene_min": torch.full((B, D), float("nan"), dtype=torch.float32, device=DEV),
        "scene_max": torch.full((B, D), float("nan"), dtype=torch.float32, device=DEV),
        "left": torch.full((nr,), -7, dtype=torch.int32, device=DEV),
        "right": torch.full((nr,), -7, dtype=torch.int32, device=DEV),
        "leaf": torch.full((nr,), -7, dtype=torch.int32, device=DEV),
        "accel": torch.full((accel_bytes,), 0xA5, dtype=torch.uint8, device=DEV),
    }


def _out_ptrs(o: dict) -> list:
    p = _native._ptr
    return [p(o["node_aabbs"]), p(o["sorted_indices"]), p(o["scene_min"]), p(o["scene_max"]),
            p(o["left"]), p(o["right"]), p(o["leaf"]), p(o["accel"])]


def _build_workspace(points: torch.Tensor) -> dict:
    L = _native.load()
    B, N, D = points.shape
    o = _outputs(B, N, D)
    ws = _native._workspace(_native._size(L.tbvh_build_workspace_size, B, N, D), DEV)
    _native._check(L.tbvh_build_with_accel(_native._ptr(points), B, N, D, *_out_ptrs(o), _native._ptr(ws),
                                           ws.numel(), _native._stream(DEV)))
    return o


def _build_noalloc(points: torch.Tensor) -> dict:
    L = _native.load()
    B, N, D = points.shape
    o = _outputs(B, N, D)
    _native._check(L.tbvh_build_with_accel_noalloc(_native._ptr(points), B, N, D, *_out_ptrs(o),
                                                   _native._stream(DEV)))
    return o


def _assert_identical(a: dict, b: dict) -> None:
    for key in a:
        x, y = a[key].cpu(), b[key].cpu()
        if x.dtype == torch.float32:
            x, y = x.view(torch.int32), y.view(torch.int32)
        assert torch.equal(x, y), key


@pytest.mark.parametrize("dim", [2, 3])
def test_noalloc_build_matches_workspace_build_twice(dim):
    print(f"no-alloc build, dim={dim}: 2 x 300000 points, then 3 x 5000", flush=True)
    g = torch.Generator("cpu").manual_seed(9100 + dim)
    big = torch.rand((2, 300_000, dim), generator=g).to(DEV)
    small = torch.rand((3, 5_000, dim), generator=g).to(DEV)
    for points in (big, small):
        ref = _build_workspace(points)
        got = _build_noalloc(points)
        torch.cuda.synchronize()
        _assert_identical(ref, got)


def test_noalloc_accel_answers_knn_like_oracle():
    print("no-alloc build + accel k-NN vs oracle: 20000 points, 4096 queries, k=16", flush=True)
    g = torch.Generator("cpu").manual_seed(9200)
    pts = torch.rand((1, 20_000, 3), generator=g)
    qs = torch.rand((1, 4096, 3), generator=g)
    o = _build_noalloc(pts.to(DEV))
    L = _native.load()
    q = qs.to(DEV)
    idx = torch.empty((1, 4096, 16), dtype=torch.int64, device=DEV)
    dist = torch.empty((1, 4096, 16), dtype=torch.float32, device=DEV)
    _native._check(L.tbvh_knn_accel(_native._ptr(o["accel"]), _native._ptr(q), None, 1, 4096, 20_000, 3, 16,
                                    _native._ptr(idx), _native._ptr(dist), _native._stream(DEV)))
    torch.cuda.synchronize()
    ei, ed = oracle.knn(pts[0].numpy(), qs[0].numpy(), 16)
    assert np.array_equal(idx[0].cpu().numpy(), ei)
    assert np.array_equal(dist[0].cpu().numpy().view(np.uint32), ed.view(np.uint32))


def test_noalloc_rejects_clouds_beyond_its_scratch():
    L = _native.load()
    pts = torch.zeros((1, 1 << 23, 3), dtype=torch.float32, device=DEV)
    # Null outputs and a small real accel: should the size check ever pass,
    # the build's own null-pointer check still stops the call before any
    # launch, so nothing is written.
    accel = torch.empty(256, dtype=torch.uint8, device=DEV)
    o = [None] * 7 + [_native._ptr(accel)]
    assert L.tbvh_build_with_accel_noalloc(_native._ptr(pts), 1, 1 << 23, 3, *o, _native._stream(DEV)) == 2
    assert "scratch array" in L.tbvh_last_error().decode()
