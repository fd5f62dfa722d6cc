"""Parity of the small-cloud path (one work-group per cloud: bounds, keys
and the whole stable sort in LDS, csrc/small.hip) against the oracle, at
its limits: 4,096 rows (4 keys per thread) and 12,288 rows (12 keys per
thread), the general path just past them, heavy duplicates (stability),
many tiny clouds, ragged calls, the query orders and the point ordering."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import torchbvh_amd as tb
from parity import assert_same_f32, assert_same_int
from torchbvh_amd._native import _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
LIMIT = 12_288


def dev(a) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def check_payload(got: dict, ref: dict, what: str) -> None:
    for key in ("scene_min", "scene_max", "node_aabbs"):
        assert_same_f32(got[key].cpu().numpy(), ref[key], f"{what} {key}")
    for key in ("sorted_indices", "left_child_mem", "right_child_mem", "mem_to_leaf"):
        assert_same_int(got[key].cpu().numpy(), ref[key], f"{what} {key}")


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("n", [1, 5, 1000, 4095, 4096, 4097, 10_000, LIMIT - 1, LIMIT, LIMIT + 1])
def test_single_build_and_knn_across_the_limits(n, dim):
    print(f"small path build n={n} dim={dim}", flush=True)
    rng = np.random.default_rng(n + 10 * dim)
    p = rng.random((n, dim), dtype=np.float32)
    q = rng.random((min(n, 3000), dim), dtype=np.float32)
    h = tb.build_bvh(dev(p))
    ref = oracle.build(p)
    check_payload(h, ref, f"n={n}")
    if n >= 4:
        idx, dist = tb.query_knn(h, dev(q), 4)
        ei, ed = oracle.knn_bvh(ref, q, 4)
        assert_same_int(idx.cpu().numpy(), ei, "indices")
        assert_same_f32(dist.cpu().numpy(), ed, "distances")


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("n", [4096, LIMIT])
def test_heavy_duplicates_keep_ascending_index(n, dim):
    """Few distinct codes: every pass must keep equal keys in row order."""
    rng = np.random.default_rng(40 + dim)
    p = rng.integers(0, 3, (n, dim)).astype(np.float32)
    check_payload(tb.build_bvh(dev(p)), oracle.build(p), "duplicates")


@pytest.mark.parametrize("B,n", [(16, 10_000), (300, 37), (3, LIMIT)])
def test_batched_small_clouds(B, n):
    rng = np.random.default_rng(B * 7 + n)
    p = rng.random((B, n, 3), dtype=np.float32)
    p[0] *= 1e3
    if B > 2:
        p[2] = 0.25  # a fully degenerate cloud
    h = tb.build_bvh(dev(p))
    ref = oracle.build_batched(p)
    check_payload(h, ref, f"B={B} n={n}")
    q = rng.random((B, 200, 3), dtype=np.float32)
    idx, dist = tb.query_knn(h, dev(q), 4)
    for b in (0, B - 1):
        ei, ed = oracle.knn(p[b], q[b], 4)
        assert_same_int(idx[b].cpu().numpy(), ei, f"cloud {b} indices")
        assert_same_f32(dist[b].cpu().numpy(), ed, f"cloud {b} distances")


@pytest.mark.parametrize("counts", [[1, 5000, 3, 7_000], [LIMIT], [7] * 40, [LIMIT - 10, 11]])
def test_ragged_small_calls(counts):
    rng = np.random.default_rng(sum(counts))
    p = np.concatenate([rng.random((c, 3), dtype=np.float32) * (b + 1) for b, c in enumerate(counts)])
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    h = tb.build_bvh(dev(p), batch_offsets=dev(offsets))
    for b, c in enumerate(counts):
        check_payload(h._handles[b], oracle.build(p[offsets[b]:offsets[b + 1]]), f"cloud {b}")
    if min(counts) >= 4:
        q = rng.random((len(p), 3), dtype=np.float32)
        idx, dist = tb.query_knn(h, dev(q), 4, query_offsets=dev(offsets))
        ei, ed = oracle.knn_ragged(p, offsets, q, offsets, 4)
        assert_same_int(idx.cpu().numpy(), ei, "indices")
        assert_same_f32(dist.cpu().numpy(), ed, "distances")


@pytest.mark.parametrize("dim", [2, 3])
@pytest.mark.parametrize("m", [4096, LIMIT, LIMIT + 1])
def test_query_orders_across_the_limit(m, dim):
    rng = np.random.default_rng(m * 3 + dim)
    q = rng.random((2, m, dim), dtype=np.float32) * 1.2 - 0.1
    q[1, ::3] = q[1, 0]  # repeated queries: ties keep ascending index
    lo = np.zeros((2, dim), np.float32)
    hi = np.ones((2, dim), np.float32)
    full = _C.morton_sort_queries_narrow(dev(q), dev(lo), dev(hi)).cpu().numpy()
    sched = _C.morton_sort_queries_narrow(dev(q), dev(lo), dev(hi), schedule=True).cpu().numpy()
    for b in range(2):
        assert_same_int(full[b], oracle.query_order(q[b], lo[b], hi[b]), f"order {b}")
        assert_same_int(sched[b], oracle.schedule_order(q[b], lo[b], hi[b]), f"schedule {b}")


def test_ragged_query_order_with_an_empty_cloud():
    rng = np.random.default_rng(78)
    counts = [9, 0, 12_000, 1]
    q = rng.random((sum(counts), 3), dtype=np.float32)
    offsets = np.concatenate(([0], np.cumsum(counts))).astype(np.int64)
    lo = np.zeros((4, 3), np.float32)
    hi = np.full((4, 3), 0.7, np.float32)
    for schedule, ref in ((False, oracle.query_order), (True, oracle.schedule_order)):
        order = _C.morton_sort_queries_ragged(dev(q), dev(offsets), dev(lo), dev(hi), 4,
                                              schedule=schedule).cpu().numpy()
        for b in range(4):
            seg = slice(offsets[b], offsets[b + 1])
            assert_same_int(order[seg], ref(q[seg], lo[b], hi[b]), f"cloud {b} schedule={schedule}")


@pytest.mark.parametrize("dim", [2, 3])
def test_point_ordering_small(dim):
    """morton_sort_points_batched (unseeded bounds) through the small path."""
    rng = np.random.default_rng(91 + dim)
    p = (rng.random((4, 9000, dim), dtype=np.float32) * 3 - 1).astype(np.float32)
    got = _C.morton_sort_points_batched(dev(p)).cpu().numpy()
    for b in range(4):
        assert_same_int(got[b], oracle.morton_point_order(p[b]), f"cloud {b}")
