"""Public API contract on the GPU: lifecycle, dispatch, validation messages,
payload keys/shapes/dtypes, source-point gathers and PointGeometry reuse
(restating torchbvh tests/test_python_api.py, tests/test_bvh_class.py,
tests/test_batched_python_api.py, tests/test_ragged_python_api.py,
tests/test_noncontiguous_public_api.py, tests/test_point_geometry.py:30-41)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import torchbvh_amd as tb
import torchbvh_amd._query as query_module
from parity import assert_same_f32, assert_same_int

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

SINGLE_KEYS = {"node_aabbs", "sorted_indices", "scene_min", "scene_max", "num_leaves",
               "num_real_nodes", "leaf_level", "virtual_leaves", "dim", "left_child_mem",
               "right_child_mem", "mem_to_leaf"}


def rand(*shape, seed=0):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.rand(shape, generator=g).to(DEV)


def offsets(values):
    return torch.tensor(values, device=DEV, dtype=torch.int64)


@pytest.mark.parametrize("dim", [2, 3])
def test_single_lifecycle_and_payload(dim):
    pts = rand(24, dim, seed=7000 + dim)
    q = pts[:6] + 0.01
    bvh = tb.build_bvh(pts)
    assert isinstance(bvh, tb.BVHHandle) and not bvh.destroyed
    assert set(bvh) == SINGLE_KEYS
    assert bvh["dim"] == dim and bvh["node_aabbs"].shape == (bvh["num_real_nodes"], 2 * dim)
    idx, dist = tb.query_knn(bvh, q, 4)
    assert idx.shape == (6, 4) and torch.all(dist[:, :-1] <= dist[:, 1:])
    tb.destroy_bvh(bvh)
    assert bvh.destroyed
    with pytest.raises(RuntimeError, match="destroyed"):
        tb.query_knn(bvh, q, 4)
    with pytest.raises(RuntimeError, match="destroyed"):
        _ = bvh["dim"]
    tb.destroy_bvh(bvh)


def test_single_query_validation():
    pts = rand(16, 3, seed=1)
    bvh = tb.build_bvh(pts)
    with pytest.raises(ValueError, match="k must be 4, 8, or 16"):
        tb.query_knn(bvh, pts, 5)
    with pytest.raises(TypeError, match="BVHHandle"):
        tb.query_knn(dict(bvh), pts[:3], 4)
    with pytest.raises(ValueError, match="shape"):
        tb.query_knn(bvh, pts.unsqueeze(0), 4)
    with pytest.raises(ValueError, match="second dimension"):
        tb.query_knn(bvh, rand(4, 2), 4)
    with pytest.raises(ValueError, match="float32"):
        tb.query_knn(bvh, pts.double(), 4)
    with pytest.raises(ValueError, match="CUDA"):
        tb.query_knn(bvh, pts.cpu(), 4)
    with pytest.raises(TypeError, match="RaggedBVHHandle"):
        tb.query_knn(bvh, pts, 4, query_offsets=offsets([0, 16]))
    # Fewer points than k: the native check (RuntimeError, as TORCH_CHECK).
    small = tb.build_bvh(rand(3, 3, seed=2))
    with pytest.raises(RuntimeError, match="num_leaves must be >= k"):
        tb.query_knn(small, rand(2, 3), 4)


def test_sort_queries_routes_through_ordered_traversal(monkeypatch):
    pts = rand(16, 3, seed=3)
    bvh = tb.build_bvh(pts)
    calls = []

    def fake_sort(qb, lo, hi, schedule=False):
        assert schedule  # query_knn orders its traversal with the schedule sort
        calls.append(("sort", tuple(qb.shape)))
        B, M, _ = qb.shape
        return torch.arange(M, device=qb.device).expand(B, M).contiguous()

    def fake_ordered(*args, accel=None, source_points=None):
        assert accel is not None and source_points is None
        calls.append(("ordered", tuple(args[3].shape), args[-1]))
        B, M, _ = args[2].shape
        k = int(args[-1])
        return (torch.zeros((B, M, k), device=DEV, dtype=torch.int64),
                torch.zeros((B, M, k), device=DEV))

    def fake_unordered(*args, **kwargs):
        raise AssertionError("unordered route must not be used when sort_queries=True")

    monkeypatch.setattr(query_module, "SCHEDULE_MIN_QUERIES", 0)
    monkeypatch.setattr(query_module._C, "morton_sort_queries_narrow", fake_sort)
    monkeypatch.setattr(query_module._C, "query_knn_batched_cached_bounds_ordered", fake_ordered)
    monkeypatch.setattr(query_module._C, "query_knn_batched_cached_bounds", fake_unordered)
    idx, dist = tb.query_knn(bvh, pts[:5].contiguous(), 4, sort_queries=True)
    assert idx.shape == (5, 4)
    assert calls == [("sort", (1, 5, 3)), ("ordered", (1, 5), 4)]


def test_small_query_sets_traverse_in_input_order(monkeypatch):
    """Up to SCHEDULE_MIN_QUERIES queries, query_knn skips the schedule sort
    even with sort_queries=True (the order never changes results); above it
    the schedule is used."""
    pts = rand(16, 3, seed=4)
    bvh = tb.build_bvh(pts)
    calls = []
    real_sort = query_module._C.morton_sort_queries_narrow

    def counting_sort(*args, **kwargs):
        calls.append("sort")
        return real_sort(*args, **kwargs)

    monkeypatch.setattr(query_module._C, "morton_sort_queries_narrow", counting_sort)
    q = pts[:6].contiguous()
    want = tb.query_knn(bvh, q, 4, sort_queries=False)
    got = tb.query_knn(bvh, q, 4, sort_queries=True)
    assert calls == []
    monkeypatch.setattr(query_module, "SCHEDULE_MIN_QUERIES", 5)
    got_sched = tb.query_knn(bvh, q, 4, sort_queries=True)
    assert calls == ["sort"]
    for a, b in ((got, want), (got_sched, want)):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_batched_lifecycle_and_validation():
    pts = rand(3, 17, 3, seed=13001)
    q = rand(3, 5, 3, seed=13002)
    bvh = tb.build_bvh(pts)
    assert isinstance(bvh, tb.BatchedBVHHandle)
    assert set(bvh) == SINGLE_KEYS | {"batch_size", "_batched"}
    assert bvh["batch_size"] == 3 and bvh["sorted_indices"].shape == (3, 17)
    for b in range(3):
        assert torch.equal(bvh["sorted_indices"][b].sort().values.cpu(), torch.arange(17))
    idx, dist, pos = tb.query_knn(bvh, q, 4, source_points=pts)
    assert pos.shape == (3, 5, 4, 3)
    with pytest.raises(ValueError, match="shape"):
        tb.query_knn(bvh, q[0], 4)
    with pytest.raises(ValueError, match="batch size"):
        tb.query_knn(bvh, q[:1], 4)
    with pytest.raises(ValueError, match="last dimension"):
        tb.query_knn(bvh, rand(3, 4, 2), 4)
    with pytest.raises(ValueError, match="float32"):
        tb.query_knn(bvh, q.double(), 4)
    with pytest.raises(ValueError, match="source_points"):
        tb.query_knn(bvh, q, 4, source_points=pts[:2])
    tb.destroy_bvh(bvh)
    with pytest.raises(RuntimeError, match="destroyed"):
        tb.query_knn(bvh, q, 4)
    with pytest.raises(ValueError, match="shape"):
        tb.build_bvh(pts.unsqueeze(0))


def test_ragged_lifecycle_payload_and_cascade_destroy():
    counts = [9, 17, 12]
    pts = torch.cat([rand(c, 3, seed=14001 + b) + 10.0 * b for b, c in enumerate(counts)])
    q = torch.cat([rand(c, 3, seed=14100 + b) + 10.0 * b for b, c in enumerate([4, 7, 5])])
    bo, qo = offsets([0, 9, 26, 38]), offsets([0, 4, 11, 16])
    bvh = tb.build_bvh(pts, batch_offsets=bo)
    assert isinstance(bvh, tb.RaggedBVHHandle)
    assert bvh["batch_size"] == 3 and bvh["dim"] == 3
    assert torch.equal(bvh["batch_offsets"], bo)
    assert torch.equal(bvh["num_leaves_per_sample"].cpu(), torch.tensor(counts))
    inner = list(bvh._handles)
    assert len(inner) == 3 and all(set(h) == SINGLE_KEYS for h in inner)
    idx, dist, pos = tb.query_knn(bvh, q, 4, query_offsets=qo, source_points=pts)
    assert idx.shape == (16, 4) and pos.shape == (16, 4, 3)
    for b, c in enumerate(counts):
        s = idx[int(qo[b]):int(qo[b + 1])]
        assert int(s.min()) >= 0 and int(s.max()) < c
    # Inner handles are usable single-cloud BVHs over their segment.
    si, sd = tb.query_knn(inner[1], q[4:11].contiguous(), 4)
    assert torch.equal(si, idx[4:11]) and torch.equal(sd, dist[4:11])
    tb.destroy_bvh(bvh)
    assert bvh.destroyed and all(h.destroyed for h in inner)
    with pytest.raises(RuntimeError, match="destroyed"):
        tb.query_knn(bvh, q, 4, query_offsets=qo)
    tb.destroy_bvh(bvh)


@pytest.mark.parametrize(
    "bad,match",
    [
        (lambda o: o.view(1, -1), "shape"),
        (lambda o: o.to(torch.int32), "int64"),
        (lambda o: o.cpu(), "CUDA"),
        (lambda o: offsets([1, 4, 8]), "start at 0"),
        (lambda o: offsets([0, 4, 7]), "final offset"),
        (lambda o: offsets([0, 8, 8]), "strictly increasing"),
    ],
)
def test_ragged_build_rejects_bad_offsets(bad, match):
    with pytest.raises(ValueError, match=match):
        tb.build_bvh(rand(8, 2), batch_offsets=bad(offsets([0, 4, 8])))


def test_ragged_query_validation():
    pts = rand(11, 2, seed=5)
    q = rand(8, 2, seed=6)
    bvh = tb.build_bvh(pts, batch_offsets=offsets([0, 3, 11]))
    with pytest.raises(ValueError, match="k must be 4, 8, or 16"):
        tb.query_knn(bvh, q, 5, query_offsets=offsets([0, 4, 8]))
    with pytest.raises(ValueError, match="batch size"):
        tb.query_knn(bvh, q, 4, query_offsets=offsets([0, 2, 5, 8]))
    with pytest.raises(ValueError, match="at least k"):
        tb.query_knn(bvh, q, 4, query_offsets=offsets([0, 4, 8]))
    with pytest.raises(ValueError, match="query_offsets is required"):
        tb.query_knn(bvh, q, 4)
    with pytest.raises(ValueError, match="second dimension"):
        tb.query_knn(bvh, rand(8, 3), 2 + 2, query_offsets=offsets([0, 4, 8]))
    single = tb.build_bvh(pts)
    batched = tb.build_bvh(pts.view(1, 11, 2).contiguous())
    for h in (single, batched):
        with pytest.raises(TypeError, match="RaggedBVHHandle"):
            tb.query_knn(h, q, 4, query_offsets=offsets([0, 8]))


def test_ragged_neighbor_positions_carry_gradients_to_source_only():
    counts = [8, 10, 12]
    g = torch.Generator("cpu").manual_seed(51030)
    pts = torch.cat([torch.randn((c, 3), generator=g) + 20.0 * b for b, c in enumerate(counts)])
    pts = pts.to(DEV).requires_grad_()
    q = torch.cat([pts.detach()[sum(counts[:b]):sum(counts[:b]) + m] + 0.025
                   for b, m in enumerate([3, 4, 5])]).requires_grad_()
    bvh = tb.build_bvh(pts, batch_offsets=offsets([0, 8, 18, 30]))
    idx, dist, pos = tb.query_knn(bvh, q, 4, query_offsets=offsets([0, 3, 7, 12]), source_points=pts)
    assert not idx.requires_grad and not dist.requires_grad and pos.requires_grad
    pos.square().sum().backward()
    assert pts.grad is not None and torch.count_nonzero(pts.grad) > 0
    assert q.grad is None


def test_bvh_class_delegation_and_lifecycle():
    base = torch.linspace(-1.0, 1.0, 20, device=DEV)
    pts = torch.stack((base, base.square() - 0.25, torch.sin(2.0 * base)), 1).contiguous()
    q = (pts[3:8] + 0.02).contiguous()
    with tb.BVH(pts) as bvh:
        assert not bvh.destroyed and not hasattr(bvh, "__getitem__")
        ic, dc = bvh.knn(q, 4)
        ic2, dc2, pc = bvh.knn(q, 4, source_points=pts)
        with pytest.raises(NotImplementedError):
            bvh.interpolate(q, torch.zeros((20, 2), device=DEV))
    assert bvh.destroyed
    bvh.destroy()
    with pytest.raises(RuntimeError):
        bvh.knn(q, 4)
    h = tb.build_bvh(pts)
    fi, fd = tb.query_knn(h, q, 4)
    assert torch.equal(ic, fi) and torch.equal(dc, fd) and torch.equal(ic2, fi)
    assert torch.equal(pc, pts[fi])
    ragged = tb.BVH(pts, batch_offsets=offsets([0, 10, 20]))
    with pytest.raises(TypeError, match="interpolate"):
        ragged.interpolate(q, torch.zeros((20, 2), device=DEV))
    ri, rd = ragged.knn(q, 4, query_offsets=offsets([0, 2, 5]))
    assert ri.shape == (5, 4)
    ragged.destroy()
    assert ragged.destroyed


def test_noncontiguous_inputs_match_contiguous():
    wide = rand(300, 4, seed=9)
    pts = wide[:, :3]
    assert not pts.is_contiguous()
    qw = rand(50, 5, seed=10)
    q = qw[:, 1:4]
    a_i, a_d = tb.query_knn(tb.build_bvh(pts), q, 8)
    b_i, b_d = tb.query_knn(tb.build_bvh(pts.contiguous()), q.contiguous(), 8)
    assert torch.equal(a_i, b_i) and torch.equal(a_d, b_d)
    with tb.BVH(pts) as bvh:
        c_i, _, c_p = bvh.knn(q, 8, source_points=pts)
    assert torch.equal(c_i, a_i)
    assert torch.equal(c_p, pts[a_i])


@pytest.mark.parametrize("batched", [False, True])
@pytest.mark.parametrize("dim", [2, 3])
def test_point_geometry_snapshot_and_validation(batched, dim):
    shape = (2, 31, dim + 1) if batched else (31, dim + 1)
    pts = rand(*shape, seed=719)[..., :dim]
    geo = tb.PointGeometry(pts)
    with geo as g:
        h = g.bvh
        assert isinstance(h, tb.BatchedBVHHandle)
        snap = g.points.cpu().numpy()
        for b in range(snap.shape[0]):
            ref = oracle.build(snap[b])
            assert_same_f32(h["node_aabbs"][b].cpu().numpy(), ref["node_aabbs"], "geometry nodes")
            assert_same_int(h["sorted_indices"][b].cpu().numpy(), ref["sorted_indices"], "geometry order")
        q = rand(2 if batched else 1, 13, dim, seed=3)
        idx, dist = tb.query_knn(h, q, 4)
        assert idx.shape == (q.shape[0], 13, 4)
    assert geo.destroyed
    with pytest.raises(RuntimeError, match="destroyed"):
        geo.validate(pts)


def test_point_geometry_rejects_other_or_mutated_sources():
    pts = rand(2, 32, 2)
    geo = tb.PointGeometry(pts)
    with pytest.raises(ValueError, match="different source"):
        geo.validate(pts.clone())
    pts.add_(1)
    with pytest.raises(ValueError, match="source changed"):
        geo.validate(pts)
    geo.destroy()
    geo.destroy()


def test_quickstart_config1_end_to_end():
    """README-sized quickstart (10k points, 10k queries, k=4)."""
    import bench

    w = bench.make_workload("cfg1")
    pts, q = w["points"].to(DEV), w["queries"].to(DEV)
    with tb.BVH(pts) as bvh:
        neighbors, distances_sq = bvh.knn(q, k=4)
    assert neighbors.shape == (10_000, 4) and torch.isfinite(distances_sq).all()
    ei, ed = oracle.knn(w["points"].numpy(), w["queries"].numpy(), 4)
    assert_same_int(neighbors.cpu().numpy(), ei, "cfg1 indices")
    assert_same_f32(distances_sq.cpu().numpy(), ed, "cfg1 distances")


def _displaced_inputs(B=2, N=24, H=3, D=3, C=4, seed=20500):
    g = torch.Generator().manual_seed(seed)
    pos = torch.rand((B, N, D), generator=g)
    pos = pos + 8.0 * torch.arange(B, dtype=torch.float32).view(B, 1, 1)
    q = pos[:, :, None, :] + 0.015 * torch.randn((B, N, H, D), generator=g)
    values = torch.randn((B, N, H, C), generator=g)
    return pos.to(DEV).contiguous(), q.to(DEV).contiguous(), values.to(DEV).contiguous()


@pytest.mark.parametrize("dim", [2, 3])
def test_query_displaced_knn_matches_flattened_batched_query(dim):
    """tests/test_displaced_query.py:88-150: local indices, ascending
    distances, positions of the returned points; identical to one batched
    query over the flattened heads."""
    pos, q, _ = _displaced_inputs(B=3, N=28, H=2, D=dim)
    idx, d2, npos = tb.query_displaced_knn(pos, q, 4)
    assert idx.shape == (3, 28, 2, 4) and d2.shape == (3, 28, 2, 4) and npos.shape == (3, 28, 2, 4, dim)
    assert int(idx.min()) >= 0 and int(idx.max()) < 28
    assert torch.all(d2[..., :-1] <= d2[..., 1:])
    b = torch.arange(3, device=DEV).view(3, 1, 1, 1)
    assert torch.equal(npos, pos[b, idx])
    fi, fd = tb.query_knn(tb.build_bvh(pos), q.reshape(3, 56, dim), 4)
    assert torch.equal(idx, fi.reshape(3, 28, 2, 4)) and torch.equal(d2, fd.reshape(3, 28, 2, 4))
    i2, dd2 = tb.query_displaced_knn(pos, q, 4, return_positions=False)
    assert torch.equal(i2, idx) and torch.equal(dd2, d2)
    with pytest.raises(ValueError, match="k must be"):
        tb.query_displaced_knn(pos, q, 5)


def test_gather_neighbor_values_uses_matching_head_only():
    values = torch.arange(2 * 5 * 3 * 2, dtype=torch.float32, device=DEV).reshape(2, 5, 3, 2)
    idx = torch.tensor([4, 0, 2, 1], device=DEV).expand(2, 5, 3, 4).contiguous()
    out = tb.gather_neighbor_values(values, idx)
    assert out.shape == (2, 5, 3, 4, 2)
    for b in range(2):
        for h in range(3):
            assert torch.equal(out[b, :, h], values[b, idx[b, :, h], h])
    with pytest.raises(ValueError, match="local source indices"):
        tb.gather_neighbor_values(values, idx + 5)


def test_interpolate_displaced_weighted_mean_and_exact_hits():
    """Weighted mean w = 1/(d2 + 1e-12) normalised; exact hits average."""
    pos, q, values = _displaced_inputs(B=2, N=20, H=3, D=3, C=5, seed=7)
    q[:, :, 0] = pos  # head 0 hits its own point exactly
    out = tb.interpolate_displaced(pos, q, values, 4)
    idx, d2 = tb.query_displaced_knn(pos, q, 4, return_positions=False)
    nv = tb.gather_neighbor_values(values, idx)
    w = torch.reciprocal(d2 + 1e-12)
    w = w / w.sum(-1, keepdim=True).clamp(min=1e-12)
    want = torch.zeros_like(values)
    for r in range(4):
        want = want + nv[..., r, :] * w[..., r].unsqueeze(-1)
    exact = d2 <= 1e-12
    ex = torch.zeros_like(values)
    for r in range(4):
        ex = ex + nv[..., r, :] * exact[..., r].float().unsqueeze(-1)
    ex = ex / exact.float().sum(-1, keepdim=True).clamp(min=1.0)
    want = torch.where(exact.any(-1, keepdim=True), ex, want)
    assert torch.equal(out, want)
    assert exact[:, :, 0, 0].all()  # head 0's nearest neighbour is its own point


def test_build_rejects_more_than_int32_points_without_copying():
    """_query.py:30-35: total point count must fit in signed int32; checked
    on the sizes, so an expanded (stride-0) view is never materialised."""
    one = torch.zeros((1, 1, 3), device=DEV)
    before = torch.cuda.memory_allocated(DEV)
    with pytest.raises(ValueError, match="build_bvh: total point count must fit in signed int32"):
        tb.build_bvh(one[0].expand(2**31, 3))
    with pytest.raises(ValueError, match="build_bvh: total point count must fit in signed int32"):
        tb.build_bvh(one.expand(2, 2**30, 3))
    assert torch.cuda.memory_allocated(DEV) == before


def test_readme_example_runs():
    """tests/test_readme_examples.py:19-35 for this package's README: its
    Python example runs as written and returns the documented shapes."""
    import re
    from pathlib import Path

    readme = (Path(__file__).resolve().parents[1] / "README.md").read_text(encoding="utf-8")
    examples = re.findall(r"```python\n(.*?)\n```", readme, re.DOTALL)
    assert len(examples) == 1
    ns: dict = {}
    exec(compile(examples[0], "README.md", "exec"), ns)
    assert ns["idx"].shape == (10_000, 16) and ns["idx"].dtype == torch.int64
    assert ns["d2"].dtype == torch.float32 and (ns["d2"].diff(dim=1) >= 0).all()
    assert ns["idx_b"].shape == (4, 2_000, 8)
