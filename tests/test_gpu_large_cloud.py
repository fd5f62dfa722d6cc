"""A cloud above 2^28 points: the accel is not built (its bucket refs hold
28-bit starts), so the build runs without it and k-NN takes the implicit-tree
traversal.  Both run at their real maximum-size indices (~5.4e8 heap nodes).

Points form a 646^3 integer grid (269,586,136 > 2^28 points), generated on
the device in row-major order, so point (i, j, l) has index
(i * 646 + j) * 646 + l.  The k nearest grid points of any query lie within
+-3 cells of it (or of its nearest grid cell, for a query just outside; the
test's queries were checked against a +-10 neighbourhood), so the oracle
brute force over that 7^3 neighbourhood, with candidates in ascending global
index order, gives the exact expected indices (exact ties: lower index) and
bit-exact distances.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import torchbvh_amd as tb
from parity import assert_same_f32, assert_same_int
from torchbvh_amd._native import MAX_ACCEL_CLOUD

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
G = 646


def grid_points() -> torch.Tensor:
    ax = torch.arange(G, device=DEV, dtype=torch.float32)
    return torch.stack(torch.meshgrid(ax, ax, ax, indexing="ij"), dim=-1).reshape(-1, 3).contiguous()


def expected(q: np.ndarray, k: int, reach: int = 3) -> tuple[np.ndarray, np.ndarray]:
    base = np.clip(np.floor(q).astype(np.int64), 0, G - 1)
    r = np.arange(-reach, reach + 1)
    cells = np.stack(np.meshgrid(r, r, r, indexing="ij"), -1).reshape(-1, 3) + base
    cells = cells[np.all((cells >= 0) & (cells < G), axis=1)]
    gidx = (cells[:, 0] * G + cells[:, 1]) * G + cells[:, 2]
    order = np.argsort(gidx)
    cand, gidx = cells[order].astype(np.float32), gidx[order]
    li, ld = oracle.knn(cand, q[None, :].astype(np.float32), k)
    return gidx[li[0]], ld[0]


@pytest.mark.parametrize("k", [16])
def test_cloud_above_accel_limit_uses_implicit_traversal(k):
    n = G ** 3
    assert n > MAX_ACCEL_CLOUD
    p = grid_points()
    assert p.shape == (n, 3)
    h = tb.build_bvh(p)
    assert h._aux["accel"] is None
    assert h["num_leaves"] == n and h["sorted_indices"].shape == (n,)
    rng = np.random.default_rng(646)
    q = (rng.integers(0, G, (300, 3)) + np.array([0.137, 0.291, 0.413]) +
         rng.random((300, 3)) * 0.05).astype(np.float32)
    # Corner, faces and just outside the grid (within 0.6 of a face).
    q[:4] = [[0.137, 0.291, 0.413], [G - 1.2, G - 1.3, G - 1.1], [0.5, G - 0.7, 300.2], [-0.4, G - 0.4, 12.3]]
    idx, dist = tb.query_knn(h, torch.from_numpy(q).to(DEV), k)
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    for r in range(q.shape[0]):
        ei, ed = expected(q[r], k)
        assert_same_int(idx[r], ei, f"query {r} indices")
        assert_same_f32(dist[r], ed, f"query {r} distances")
    del h, p
    torch.cuda.empty_cache()
