"""Seeded sweep over shapes, k and point distributions: every case's k-NN
indices and distances (and the build's permutation and node boxes) must
equal the oracle's bit for bit.  Covers combinations the targeted tests do
not pin one by one: batched and ragged inputs of awkward sizes, degenerate
axes (points on a line or a plane), heavy duplicates, clustered data,
queries far outside the clouds, and both traversal orders."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import torchbvh_amd as tb
from parity import assert_same_f32, assert_same_int
from torchbvh_amd import _query

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def make_points(rng, n: int, dim: int, kind: str) -> np.ndarray:
    if kind == "uniform":
        p = rng.random((n, dim))
    elif kind == "clusters":
        c = rng.random((5, dim))
        p = c[rng.integers(0, 5, n)] + 0.01 * rng.standard_normal((n, dim))
    elif kind == "line":
        t = rng.random(n)
        p = np.stack([t * (d + 1) for d in range(dim)], 1)
    elif kind == "plane":
        p = rng.random((n, dim))
        p[:, -1] = 0.5
    elif kind == "duplicates":
        base = rng.random((max(1, n // 10), dim))
        p = base[rng.integers(0, len(base), n)]
    else:  # "wide": mixed scales
        p = rng.standard_normal((n, dim)) * np.array([1e4, 1e-2, 1.0][:dim])
    return p.astype(np.float32)


def make_queries(rng, p: np.ndarray, m: int) -> np.ndarray:
    lo, hi = p.min(0), p.max(0)
    span = np.maximum(hi - lo, 1e-3)
    q = lo + (rng.random((m, p.shape[1])) * 1.4 - 0.2) * span
    q[: m // 8] = p[rng.integers(0, len(p), m // 8)]  # exact hits
    return q.astype(np.float32)


KINDS = ("uniform", "clusters", "line", "plane", "duplicates", "wide")
CASES = [(seed, KINDS[seed % len(KINDS)]) for seed in range(96)]


@pytest.mark.parametrize("scheduled", [False, True])
@pytest.mark.parametrize("seed,kind", CASES)
def test_sweep_single_and_batched(seed, kind, scheduled, monkeypatch):
    if scheduled:
        monkeypatch.setattr(_query, "SCHEDULE_MIN_QUERIES", 0)
    rng = np.random.default_rng(7000 + seed)
    dim = 2 + seed % 2
    k = (4, 8, 16, 32)[(seed // 2) % 4]
    B = 1 + seed % 3
    n = int(np.exp(rng.uniform(np.log(k), np.log(40_000))))
    m = int(rng.integers(1, 3000))
    pts = np.stack([make_points(rng, n, dim, kind) for _ in range(B)])
    qs = np.stack([make_queries(rng, pts[b], m) for b in range(B)])
    if B == 1:
        h = tb.build_bvh(dev(pts[0]))
        idx, dist = tb.query_knn(h, dev(qs[0]), k)
        idx, dist = idx[None], dist[None]
        perm = h["sorted_indices"][None]
        nodes = h["node_aabbs"][None]
    else:
        h = tb.build_bvh(dev(pts))
        idx, dist = tb.query_knn(h, dev(qs), k)
        perm, nodes = h["sorted_indices"], h["node_aabbs"]
    for b in range(B):
        ref = oracle.build(pts[b])
        assert_same_int(perm[b].cpu().numpy(), ref["sorted_indices"], f"cloud {b} permutation")
        assert_same_f32(nodes[b].cpu().numpy(), ref["node_aabbs"], f"cloud {b} node boxes")
        ei, ed = oracle.knn(pts[b], qs[b], k)
        assert_same_int(idx[b].cpu().numpy(), ei, f"cloud {b} indices (n={n}, m={m}, k={k}, {kind})")
        assert_same_f32(dist[b].cpu().numpy(), ed, f"cloud {b} distances")


@pytest.mark.parametrize("seed", range(24))
def test_sweep_ragged(seed):
    rng = np.random.default_rng(9000 + seed)
    dim = 2 + seed % 2
    k = (4, 8, 16, 32)[seed % 4]
    counts = [int(c) for c in rng.integers(k, 9000, 1 + seed % 5)]
    qcounts = [int(c) for c in rng.integers(0, 1500, len(counts))]
    kind = KINDS[seed % len(KINDS)]
    pts = [make_points(rng, c, dim, kind) for c in counts]
    qs = [make_queries(rng, p, max(m, 1))[:m] for p, m in zip(pts, qcounts)]
    po = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    qo = np.concatenate(([0], np.cumsum(qcounts))).astype(np.int64)
    h = tb.build_bvh(dev(np.concatenate(pts)), batch_offsets=dev(po))
    idx, dist = tb.query_knn(h, dev(np.concatenate(qs).reshape(-1, dim)), k, query_offsets=dev(qo))
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    for b in range(len(counts)):
        if qcounts[b] == 0:
            continue
        ei, ed = oracle.knn(pts[b], qs[b], k)
        assert_same_int(idx[qo[b]:qo[b + 1]], ei, f"cloud {b} indices")
        assert_same_f32(dist[qo[b]:qo[b + 1]], ed, f"cloud {b} distances")
