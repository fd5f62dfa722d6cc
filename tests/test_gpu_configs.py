"""Parity at the BASELINE configs' full sizes.

Build outputs are compared bit-exactly in full.  k-NN rows are compared
exactly against the oracle for every query of config 2 and for a seeded
sample of queries elsewhere; every row of every config is also checked for
size-independent properties: indices in range, rows strictly ascending by
(distance, index), and each distance bit-equal to the fused-chain distance of
the returned point."""

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
SAMPLE = 20_000


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


def sample_rows(m: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(m, size=min(SAMPLE, m), replace=False))


def run_single(cfg: str, all_rows: bool) -> None:
    w = bench.make_workload(cfg)
    p, q, k = w["points"].numpy(), w["queries"].numpy(), w["k"]
    print(f"[{cfg}] n={p.shape[0]} q={q.shape[0]} k={k}", flush=True)
    h = tb.build_bvh(w["points"].to(DEV))
    ref = oracle.build(p)
    build_parity(h, ref)
    idx, dist = tb.query_knn(h, w["queries"].to(DEV), k)
    idx, dist = idx.cpu().numpy(), dist.cpu().numpy()
    row_properties(p, q, idx, dist, k)
    rows = np.arange(q.shape[0]) if all_rows else sample_rows(q.shape[0], 7)
    ei, ed = oracle.knn_bvh(ref, q[rows], k)
    assert_same_int(idx[rows], ei, f"{cfg} indices")
    assert_same_f32(dist[rows], ed, f"{cfg} distances")


def test_config2_uniform_1m_k16_all_rows():
    run_single("cfg2", all_rows=True)


def test_config4_2d_4m_k8():
    run_single("cfg4", all_rows=False)


def test_config3_batched_32x65536_k16():
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
        rows = sample_rows(q.shape[1], 100 + b)[: SAMPLE // 32]
        ei, ed = oracle.knn_bvh(ref, q[b][rows], k)
        assert_same_int(idx[b][rows], ei, f"cloud {b} indices")
        assert_same_f32(dist[b][rows], ed, f"cloud {b} distances")


def test_config5_ragged_torus_k32():
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
        rows = sample_rows(s1 - s0, 200 + b)[: SAMPLE // 64]
        ei, ed = oracle.knn_bvh(ref, q[s0:s1][rows], k)
        assert_same_int(idx[s0:s1][rows], ei, f"cloud {b} indices")
        assert_same_f32(dist[s0:s1][rows], ed, f"cloud {b} distances")
