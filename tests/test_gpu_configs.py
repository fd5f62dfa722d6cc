"""Parity at the BASELINE configs' full sizes.

Build outputs are compared bit-exactly in full, and every k-NN row of every
config exactly against the oracle's DFS (the reference's traversal,
knn_query.cu:47-154, restated; OpenMP over the queries), as the reference's
tests check indices on every row (tests/test_knn.py:124-157).  Every row is
also checked for size-independent properties: indices in range, rows
strictly ascending by (distance, index), and each distance bit-equal to the
fused-chain distance of the returned point."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
import oracle
import torchbvh_amd as tb
from parity import assert_same_f32, assert_same_int

pytestmark = [pytest.mark.gpu, pytest.mark.slow]
DEV = torch.device("cuda")


def build_parity(h, ref) -> None:
    for key in ("scene_min", "scene_max", "node_aabbs"):
        assert_same_f32(h[key].cpu().numpy(), ref[key], key)
    for key in ("sorted_indices", "left_child_mem", "right_child_mem", "mem_to_leaf"):
        assert_same_int(h[key].cpu().numpy(), ref[key], key)


def row_properties(points, queries, idx, dist, k) -> None:
    n = points.shape[0]
    assert idx.shape == (queries.shape[0], k)
    assert idx.min() >= 0 and idx.max() < n
    d, i = dist, idx
    ok = (d[:, :-1] < d[:, 1:]) | ((d[:, :-1] == d[:, 1:]) & (i[:, :-1] < i[:, 1:]))
    assert ok.all(), "rows not strictly ascending by (distance, index)"
    assert_same_f32(dist, oracle.pair_distances(points, queries, idx), "returned distances")


def run_single(cfg: str) -> None:
    w = bench.make_workload(cfg)
    p, q, k = w["points"].numpy(), w["queries"].numpy(), w["k"]
    print(f"[{cfg}] n={p.shape[0]} q={q.shape[0]} k={k}", flush=True)
    h = tb.build_bvh(w["points"].to(DEV))
    ref = oracle.build(p)
    build_parity(h, ref)
    idx, dist = tb.query_knn(h, w["queries"].to(DEV), k)
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    row_properties(p, q, idx, dist, k)
    ei, ed = oracle.knn_bvh(ref, q, k)
    assert_same_int(idx, ei, f"{cfg} indices")
    assert_same_f32(dist, ed, f"{cfg} distances")
    print(f"[{cfg}] all {q.shape[0]} rows equal the oracle's", flush=True)


def test_config2_uniform_1m_k16_all_rows():
    run_single("cfg2")


def test_config4_2d_4m_k8_all_rows():
    run_single("cfg4")


def test_config3_batched_32x65536_k16_all_rows():
    w = bench.make_workload("cfg3")
    p, q, k = w["points"].numpy(), w["queries"].numpy(), w["k"]
    h = tb.build_bvh(w["points"].to(DEV))
    idx, dist = tb.query_knn(h, w["queries"].to(DEV), k)
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    for b in range(p.shape[0]):
        ref = oracle.build(p[b])
        assert_same_f32(h["node_aabbs"][b].cpu().numpy(), ref["node_aabbs"], f"cloud {b} nodes")
        assert_same_int(h["sorted_indices"][b].cpu().numpy(), ref["sorted_indices"], f"cloud {b} order")
        row_properties(p[b], q[b], idx[b], dist[b], k)
        ei, ed = oracle.knn_bvh(ref, q[b], k)
        assert_same_int(idx[b], ei, f"cloud {b} indices")
        assert_same_f32(dist[b], ed, f"cloud {b} distances")
        if b % 8 == 7:
            print(f"[cfg3] clouds 0-{b} equal", flush=True)
    print(f"[cfg3] all {p.shape[0]} x {q.shape[1]} rows equal the oracle's", flush=True)


def test_config5_ragged_torus_k32_all_rows():
    w = bench.make_workload("cfg5")
    p, q, k = w["points"].numpy(), w["queries"].numpy(), w["k"]
    off = w["offsets"].numpy()
    h = tb.build_bvh(w["points"].to(DEV), batch_offsets=w["offsets"].to(DEV))
    idx, dist = tb.query_knn(h, w["queries"].to(DEV), k, query_offsets=w["query_offsets"].to(DEV))
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    for b in range(len(off) - 1):
        s0, s1 = off[b], off[b + 1]
        ref = oracle.build(p[s0:s1])
        inner = h._handles[b]
        assert_same_f32(inner["node_aabbs"].cpu().numpy(), ref["node_aabbs"], f"cloud {b} nodes")
        assert_same_int(inner["sorted_indices"].cpu().numpy(), ref["sorted_indices"], f"cloud {b} order")
        row_properties(p[s0:s1], q[s0:s1], idx[s0:s1], dist[s0:s1], k)
        ei, ed = oracle.knn_bvh(ref, q[s0:s1], k)
        assert_same_int(idx[s0:s1], ei, f"cloud {b} indices")
        assert_same_f32(dist[s0:s1], ed, f"cloud {b} distances")
        if b % 8 == 7:
            print(f"[cfg5] clouds 0-{b} equal", flush=True)
    print(f"[cfg5] all {q.shape[0]} rows of {len(off) - 1} clouds equal the oracle's", flush=True)
