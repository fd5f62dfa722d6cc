"""Benchmark: BVH build + exact k-NN on one MI355X.

Default workload: 1,048,576 uniform 3-D points,
1,048,576 uniform queries, k = 16, fp32.  One step = build the BVH, Morton-
order the queries, run the traversal — the whole hot path, inputs resident in
HBM.  Prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg2]
                    [--cpu-seconds S] [--no-cpu-baseline]
    python bench.py --published   # the reference's published latency rows
    python bench.py --extras      # spatial/routed k-NN, gather, primitive build, point order
    python bench.py --copy-floor  # plain device copies at the build kernels' byte counts

The synthetic workloads of every BASELINE config are defined here
(``make_workload``) and shared with the parity tests.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

import torch

# ---------------------------------------------------------------------------
# Workloads (seeds and shapes as fixed for the BASELINE configs; generated on
# the CPU so GPU, oracle and CPU baseline see bit-identical inputs)
# ---------------------------------------------------------------------------
CONFIGS = {
    "cfg1": "3D k-NN, 10,000 uniform points / 10,000 uniform queries, k=4",
    "cfg2": "3D k-NN, 1,048,576 uniform points / 1,048,576 uniform queries, k=16",
    "cfg3": "batched 3D k-NN, 32 x 65,536 Gaussian-mixture clouds, displaced self-queries, k=16",
    "cfg4": "2D k-NN, 4,194,304 uniform points, jittered self-queries, k=8",
    "cfg5": "ragged 3D k-NN, 64 torus clouds of 1,000-200,000 points, AABB-uniform queries, k=32",
}


def _gen(seed: int) -> torch.Generator:
    return torch.Generator("cpu").manual_seed(seed)


def make_workload(name: str, scale: float = 1.0) -> dict:
    """Return CPU tensors for a BASELINE config.

    ``scale`` < 1 shrinks the point/query counts (same distributions and
    seeds) for quick parity runs; 1.0 is the configured size.
    """
    if name == "cfg1":
        n = max(int(10_000 * scale), 16)
        pts = torch.rand((n, 3), generator=_gen(1001))
        q = torch.rand((n, 3), generator=_gen(1002))
        return {"kind": "single", "points": pts, "queries": q, "k": 4}
    if name == "cfg2":
        n = max(int((1 << 20) * scale), 16)
        pts = torch.rand((n, 3), generator=_gen(2001))
        q = torch.rand((n, 3), generator=_gen(2002))
        return {"kind": "single", "points": pts, "queries": q, "k": 16}
    if name == "cfg3":
        B, n = 32, max(int(65_536 * scale), 16)
        centres = torch.rand((B, 8, 3), generator=_gen(3001))
        comp = torch.randint(0, 8, (B, n), generator=_gen(3002))
        base = torch.gather(centres, 1, comp.unsqueeze(-1).expand(-1, -1, 3))
        pts = base + 0.02 * torch.randn((B, n, 3), generator=_gen(3003))
        q = pts + 0.005 * torch.randn((B, n, 3), generator=_gen(3004))
        return {"kind": "batched", "points": pts.contiguous(), "queries": q.contiguous(), "k": 16}
    if name == "cfg4":
        n = max(int((1 << 22) * scale), 16)
        pts = torch.rand((n, 2), generator=_gen(4001))
        q = pts + 0.01 * torch.randn((n, 2), generator=_gen(4002))
        return {"kind": "single", "points": pts, "queries": q.contiguous(), "k": 8}
    if name == "cfg5":
        B = 64
        sizes = torch.randint(1_000, 200_001, (B,), generator=_gen(5001))
        sizes = [max(int(s * scale), 40) for s in sizes.tolist()]
        total = sum(sizes)
        # Angles uniform in [0, 2pi)^2 (not area-uniform on the torus).
        ang = torch.rand((total, 2), generator=_gen(5002)) * (2.0 * math.pi)
        theta, phi = ang[:, 0], ang[:, 1]
        R, r = 0.35, 0.1
        ring = R + r * torch.cos(phi)
        pts = torch.stack((ring * torch.cos(theta), ring * torch.sin(theta), r * torch.sin(phi)), 1)
        pts = pts + 0.5 + 0.002 * torch.randn((total, 3), generator=_gen(5003))
        offsets = [0]
        for s in sizes:
            offsets.append(offsets[-1] + s)
        u = torch.rand((total, 3), generator=_gen(5004))
        q = torch.empty_like(pts)
        for b in range(B):
            p0, p1 = offsets[b], offsets[b + 1]
            lo = pts[p0:p1].amin(0)
            hi = pts[p0:p1].amax(0)
            q[p0:p1] = lo + u[p0:p1] * (hi - lo)
        off = torch.tensor(offsets, dtype=torch.int64)
        return {"kind": "ragged", "points": pts.contiguous(), "queries": q.contiguous(),
                "k": 32, "offsets": off, "query_offsets": off.clone()}
    raise ValueError(f"unknown config {name!r}")


# ---------------------------------------------------------------------------
# Algorithmic bytes: fixed per-unit formulas, independent of this
# implementation's pass count
# ---------------------------------------------------------------------------
def real_node_count(n: int) -> int:
    L = (n - 1).bit_length()
    return 2 * n - 1 + bin((1 << L) - n).count("1")


def build_bytes(n: int, D: int) -> int:
    return n * (12 * D + 80) + 8 * D * real_node_count(n)


def qsort_bytes(q: int, D: int) -> int:
    """Full Morton sort of the queries (the reference binding): read the
    queries, write 4-byte keys, four 8-bit LSD passes of 16 bytes per
    (key, index) pair, write a 4-byte order."""
    return q * (4 * D + 72)


def qschedule_bytes(q: int, D: int) -> int:
    """The traversal schedule query_knn runs instead: the same terms with
    two passes (the top 16 key bits) in place of four."""
    return q * (4 * D + 40)


def knn_bytes(q: int, D: int, k: int) -> int:
    return q * (4 * D + 4 + 12 * k)


HBM_PEAK_GBS = 8000.0
PROFILES = Path(__file__).resolve().parent / "profiles"


def measured_traffic(config: str):
    """HBM bytes per k-NN call measured by rocprofv3 (FETCH_SIZE and
    WRITE_SIZE of the call's kernels, each scaled by the same counter's
    reading for a copy of known size), as recorded in
    profiles/knn_call_<config>_counters.md on the line
    ``traffic_bytes_per_call: <bytes>``; None when absent."""
    path = PROFILES / f"knn_call_{config}_counters.md"
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_call:"):
                return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        pass
    return None


# ---------------------------------------------------------------------------
# CPU baseline: the reference's brute-force test oracle (tests/test_knn.py:10-12)
# with the (distance, index) tie rule, timed on a bounded sample of queries.
# ---------------------------------------------------------------------------
def job_clouds(w: dict) -> list:
    """(points, queries) of every cloud of a workload, as CPU numpy arrays."""
    pts, q = w["points"].numpy(), w["queries"].numpy()
    if w["kind"] == "batched":
        return [(pts[b], q[b]) for b in range(pts.shape[0])]
    if w["kind"] == "ragged":
        po, qo = w["offsets"].tolist(), w["query_offsets"].tolist()
        return [(pts[po[b]:po[b + 1]], q[qo[b]:qo[b + 1]]) for b in range(len(po) - 1)]
    return [(pts, q)]


def _cpu_model() -> str:
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return model


def _query_sample(clouds: list, per_cloud: int, seed: int) -> list:
    """A seeded sample of at most `per_cloud` queries of every cloud (local
    indices, sorted)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    return [np.sort(rng.choice(len(q), min(per_cloud, len(q)), replace=False)) for _, q in clouds]


def cpu_baseline(clouds: list, k: int, per_cloud: int = 4096, seconds: float = 20.0) -> dict:
    """The reference's CPU path, which is its tests' brute force
    (tests/test_knn.py:10-12: (q[:, None] - p[None]).square().sum(-1) then
    top-k) with the (distance, index) tie rule (top-k of the int64 composite
    float_bits(d) << 32 | index), on every host core this process may run
    on.  Timed on a seeded sample of up to `per_cloud` queries per cloud
    against all of that cloud's points (fewer when a short probe shows the
    sample would take much more than `seconds`), in chunks of at most 2^26
    pairs, and extrapolated to the job by (query, point) pairs: brute force
    costs exactly that many distance evaluations."""
    from oracle.torch_bruteforce import knn_bruteforce

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)

    def run(samples) -> float:
        t = time.perf_counter()
        for (p, q), sel in zip(clouds, samples):
            if len(sel):
                chunk = max(1, min(256, (1 << 26) // max(len(p), 1)))
                knn_bruteforce(torch.from_numpy(p), torch.from_numpy(q[sel]), k, chunk=chunk)
        return time.perf_counter() - t

    def pairs(samples) -> int:
        return sum(len(sel) * len(p) for sel, (p, _) in zip(samples, clouds))

    # The probe runs on the largest cloud: on a small one the per-call cost
    # dominates and the rate (hence the sample) comes out far too low.
    big = max(range(len(clouds)), key=lambda b: len(clouds[b][0]))
    probe = [_query_sample(clouds[b:b + 1], 32, 97)[0] if b == big else [] for b in range(len(clouds))]
    run(probe)  # warm-up: thread pool, allocator
    rate = pairs(probe) / max(run(probe), 1e-9)  # pairs per second
    while per_cloud > 16 and pairs(_query_sample(clouds, per_cloud, 98)) > 1.5 * rate * seconds:
        per_cloud //= 2
    samples = _query_sample(clouds, per_cloud, 98)
    dt = run(samples)
    Q = sum(len(q) for _, q in clouds)
    n_sampled = sum(len(s) for s in samples)
    total = dt * sum(len(q) * len(p) for p, q in clouds) / pairs(samples)
    return {
        "value": Q / total,
        "unit": "queries/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"the reference tests' torch brute force (squared differences summed, top-k of the "
                   f"(distance, index) composite), torch {torch.__version__} on {cores} threads "
                   f"(os.sched_getaffinity; os.cpu_count() = {os.cpu_count()}); {n_sampled} of {Q} queries "
                   f"(up to {per_cloud} per cloud, seeded) against all points in {dt:.3g} s, extrapolated "
                   f"by (query, point) pairs to the job: {total:.3g} s; CPU: {_cpu_model()}"),
    }


def cpu_port_dfs(clouds: list, k: int, seconds: float) -> dict:
    """The whole job on the host with the C oracle, which restates the
    reference's GPU algorithm (implicit-tree build, DFS k-NN with the sorted
    candidate list).  Every cloud is built in full (one thread); the k-NN is
    timed on a uniform sample of the job's queries sized to about `seconds`
    (OpenMP over queries) and extrapolated to all of them."""
    import numpy as np

    import oracle

    threads = len(os.sched_getaffinity(0))
    oracle.lib().orc_set_num_threads(threads)
    t0 = time.perf_counter()
    bvhs = [oracle.build(p) for p, _ in clouds]
    t_build = time.perf_counter() - t0
    starts = np.cumsum([0] + [len(q) for _, q in clouds])
    Q = int(starts[-1])
    rng = np.random.default_rng(99)

    def timed(n: int) -> float:
        sel = np.sort(rng.choice(Q, n, replace=False))
        parts = np.searchsorted(sel, starts)
        t = time.perf_counter()
        for b, (bvh, (_, q)) in enumerate(zip(bvhs, clouds)):
            local = sel[parts[b]:parts[b + 1]] - starts[b]
            if len(local):
                oracle.knn_bvh(bvh, q[local], k)
        return time.perf_counter() - t

    probe = min(Q, 2048)
    timed(probe)  # warm-up: thread pool, caches
    per_query = timed(probe) / probe
    n, dt = probe, 0.0
    for _ in range(3):  # per-cloud call costs make small samples read slow: rescale
        n = int(min(Q, max(n, seconds / per_query)))
        dt = timed(n)
        per_query = dt / n
        if n == Q or dt >= 0.5 * seconds:
            break
    total = t_build + Q * per_query
    return {
        "value": Q / total,
        "unit": "queries/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"C oracle (restated reference build + DFS k-NN, gcc -O2): all {len(clouds)} "
                   f"cloud(s) built on 1 thread in {t_build:.3g} s; k-NN of {n} of {Q} queries "
                   f"(uniform sample) on {threads} threads in {dt:.3g} s; extrapolated job "
                   f"time {total:.3g} s; CPU: {_cpu_model()}"),
    }


# ---------------------------------------------------------------------------
# Bench
# ---------------------------------------------------------------------------
# The reference's only published numbers for this path: one-shot build +
# k = 4 k-NN latencies, `with BVH(points) as bvh: bvh.knn(queries, k=4)`, Q = N,
# uniform inputs from np.random.default_rng(20260923 + dim*10 + points + batch),
# one warm-up then the median of 3 synchronized wall-clock calls
# (torchbvh benchmarks/third_party.py:95-114, :138-140, :188-193), measured on
# an RTX 3500 Ada Generation Laptop GPU
# (benchmarks/results/third_party_0.3.2_2026-10-07.csv, rows knn,torchbvh).
PUBLISHED_MS = {  # (batch, dim, points) -> ms
    (1, 2, 10_000): 0.679, (1, 2, 20_000): 0.859, (1, 2, 30_000): 1.209, (1, 2, 40_000): 1.416,
    (1, 2, 50_000): 1.829, (1, 3, 10_000): 0.852, (1, 3, 20_000): 1.285, (1, 3, 30_000): 1.579,
    (1, 3, 40_000): 2.498, (1, 3, 50_000): 2.967, (16, 2, 10_000): 1.454, (16, 2, 20_000): 2.883,
    (16, 2, 30_000): 4.454, (16, 2, 40_000): 5.962, (16, 2, 50_000): 7.814, (16, 3, 10_000): 2.978,
    (16, 3, 20_000): 5.559, (16, 3, 30_000): 8.114, (16, 3, 40_000): 15.467, (16, 3, 50_000): 20.623,
}


def published_latencies() -> int:
    """Same protocol on this GPU for every published row; one JSON line each."""
    import time as _t

    import numpy as np

    import torchbvh_amd as tb

    for (batch, dim, n), ref_ms in PUBLISHED_MS.items():
        rng = np.random.default_rng(20260923 + dim * 10 + n + batch)
        p = torch.from_numpy(rng.random((batch, n, dim), dtype=np.float32)).to("cuda")
        q = torch.from_numpy(rng.random((batch, n, dim), dtype=np.float32)).to("cuda")
        p_in, q_in = (p[0], q[0]) if batch == 1 else (p, q)

        def call():
            with tb.BVH(p_in) as bvh:
                return bvh.knn(q_in, k=4)

        def timed(repeats: int) -> float:
            samples = []
            for _ in range(repeats):
                torch.cuda.synchronize()
                t0 = _t.perf_counter()
                call()
                torch.cuda.synchronize()
                samples.append(1e3 * (_t.perf_counter() - t0))
            return float(np.median(samples))

        call()
        torch.cuda.synchronize()
        ms = timed(3)
        print(json.dumps({"metric": "build+kNN latency (reference protocol)", "batch": batch, "dim": dim,
                          "points": n, "queries": n, "k": 4, "ms": round(ms, 4),
                          "ms_median_of_25": round(timed(25), 4), "reference_ms": ref_ms,
                          "reference_hardware": "RTX 3500 Ada Generation Laptop GPU",
                          "speedup": round(ref_ms / ms, 2)}), flush=True)
    return 0


def extras() -> int:
    """The rows either side of the hot path (spatial-output k-NN, routed
    ordering + k-NN, neighbour-position gather, primitive build, point
    ordering), each timed with device events at a stated size and reported
    against its algorithmic bytes; one JSON line each."""
    import numpy as np

    import torchbvh_amd as tb
    from torchbvh_amd._native import _C

    dev = torch.device("cuda:0")

    def timed(fn, reps: int = 20, warmup: int = 3) -> float:
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    def line(row: str, workload: str, ms: float, nbytes: int, formula: str) -> None:
        gbs = nbytes / (ms * 1e-3) / 1e9
        print(json.dumps({"row": row, "workload": workload, "ms": round(ms, 4),
                          "algorithmic_bytes": nbytes, "bytes_formula": formula, "gb_per_s": round(gbs, 1),
                          "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}), flush=True)

    D, K = 3, 16
    w = make_workload("cfg2")
    p, q = w["points"].to(dev)[None].contiguous(), w["queries"].to(dev)[None].contiguous()
    N = Q = p.shape[1]
    d = _C.build_bvh_batched_cooperative(p)
    nr = d["num_real_nodes"]

    def spatial():
        order = _C.morton_sort_queries_narrow(q, d["scene_min"], d["scene_max"])
        return _C.query_knn_batched_cached_bounds_spatial(d["node_aabbs"], d["sorted_indices"], q, order,
                                                          N, nr, D, K)
    line("(f)1 spatial-output k-NN (MLS call pattern: full Morton order, launch-order output)",
         "cfg2: 1M uniform 3-D points and queries, k=16", timed(spatial),
         qsort_bytes(Q, D) + knn_bytes(Q, D, K), "Q(4D+72) + Q(4D+4+12K)")

    g = torch.Generator("cpu").manual_seed(6001)
    nt = nf = N // 2
    tp = torch.rand((1, nt, D), generator=g).to(dev)
    fp = (torch.rand((1, nf, D), generator=g) * 2 - 0.5).to(dev)
    routes = (torch.rand((1, Q), generator=g) < 0.5).to(dev)
    dt, df = _C.build_bvh_batched_cooperative(tp), _C.build_bvh_batched_cooperative(fp)

    def routed():
        order = _C.morton_sort_routed_queries_batched(q, routes, dt["scene_min"], dt["scene_max"],
                                                      df["scene_min"], df["scene_max"])
        return _C.query_knn_routed_batched_cached_bounds_spatial(
            dt["node_aabbs"], dt["sorted_indices"], df["node_aabbs"], df["sorted_indices"], q, routes, order,
            nt, dt["num_real_nodes"], nf, df["num_real_nodes"], D, K)
    line("(f)2 routed ordering + routed spatial k-NN (two trees, per-query route)",
         "cfg2 queries, true/false clouds of 512k uniform points each, 50% routes, k=16", timed(routed),
         qsort_bytes(Q, D) + Q + knn_bytes(Q, D, K), "Q(4D+72) + Q (routes) + Q(4D+4+12K)")

    h = tb.build_bvh(p[0])
    src = p[0].contiguous()
    plain = timed(lambda: tb.query_knn(h, q[0], K))
    with_rows = timed(lambda: tb.query_knn(h, q[0], K, source_points=src))
    line("(f)3 neighbour-position gather fused in the k-NN epilogue (query_knn source_points): added time",
         "cfg2, k=16 (query_knn with source_points minus without)", with_rows - plain,
         Q * K * (2 * 4 * D), "QK(2*4D): neighbour row read, row written")

    Bm, Nm, Hm, Km = 4, 65_536, 4, 8
    pos = torch.rand((Bm, Nm, D), generator=g).to(dev)
    qd = (pos[:, :, None, :] + (torch.rand((Bm, Nm, Hm, D), generator=g).to(dev) - 0.5) * 0.02).contiguous()
    vals = torch.rand((Bm, Nm, Hm, 16), generator=g).to(dev)
    Qm = Bm * Nm * Hm
    line("(f)3 multi-head displaced-query k-NN (query_displaced_knn: build + k-NN + neighbour rows)",
         "4 clouds x 65,536 3-D points, 4 heads, k=8", timed(lambda: tb.query_displaced_knn(pos, qd, Km)),
         build_bytes(Nm, D) * Bm + qsort_bytes(Qm, D) + knn_bytes(Qm, D, Km) + Qm * Km * 2 * 4 * D,
         "B(build) + Q(4D+72) + Q(4D+4+12K) + QK(2*4D), Q = B*N*H")
    line("(f)3 multi-head interpolation (interpolate_displaced, 16 channels)",
         "4 clouds x 65,536 3-D points, 4 heads, k=8", timed(lambda: tb.interpolate_displaced(pos, qd, vals, Km)),
         build_bytes(Nm, D) * Bm + qsort_bytes(Qm, D) + knn_bytes(Qm, D, Km) + Qm * Km * 16 * 4 + Qm * 16 * 4,
         "as above without rows + QK*4C gathered values + Q*4C written, C = 16")

    F, V = 1 << 20, 3
    anchor = torch.rand((1, F, 1, D), generator=g)
    prims = (anchor + (torch.rand((1, F, V, D), generator=g) - 0.5) * 0.01).contiguous().to(dev)
    nrf = real_node_count(F)
    line("(f)4 primitive BVH build (triangles)", "1M triangles in [0,1)^3", timed(lambda: _C.build_primitive_bvh_batched(prims)),
         F * (4 * V * D + 24 * D + 80) + 8 * D * nrf,
         "F(4VD + 24D + 80) + 8D nr: vertices, centres and boxes, keys, sort, leaf boxes, nodes")
    line("(f)4 point Morton ordering (FPS)", "cfg2 points", timed(lambda: _C.morton_sort_points_batched(p)),
         N * (8 * D + 76), "N(8D + 76): two point reads, keys, sort, int64 order")
    return 0


COPY_FLOOR_MB = (0.004, 2, 4, 8, 16, 32, 64, 128, 256, 512)


def copy_floor() -> int:
    """What a plain device copy reaches at the byte counts of the build
    kernels: a copy moving `total` bytes (total / 2 read, total / 2
    written), 200 back to back between two events, as the build's launches
    run.  A kernel cannot beat the copy of its own bytes, so these are the
    per-launch ceilings against which the build kernels' fractions of peak
    are read.  One JSON line per size."""
    dev = torch.device("cuda:0")
    reps = 200
    for mb in COPY_FLOOR_MB:
        total = int(mb * 1e6) // 8 * 8
        src = torch.ones(total // 8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        us = 1e3 * e0.elapsed_time(e1) / reps
        gbs = total / (us * 1e-6) / 1e9
        print(json.dumps({"copy_floor_total_bytes": total, "us_per_copy": round(us, 3),
                          "gb_per_s": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}), flush=True)
        del src, dst
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg2", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-queries", type=int, default=4096,
                    help="queries per cloud of the CPU baseline's sample (brute force)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="host time budget of the C-oracle DFS's sampled k-NN")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--implicit-reps", type=int, default=1,
                    help="also time the traversal over the implicit tree (0 = skip)")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="end with a 256 MiB device copy (for rocprofv3 counter calibration)")
    ap.add_argument("--published", action="store_true",
                    help="instead: time the reference's published latency rows with its protocol")
    ap.add_argument("--extras", action="store_true",
                    help="instead: time the rows either side of the path (spatial, routed, gather, primitives)")
    ap.add_argument("--copy-floor", action="store_true",
                    help="instead: time plain device copies at the build kernels' byte counts")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "sharding across GPUs is not implemented", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    if args.published:
        return published_latencies()
    if args.extras:
        return extras()
    if args.copy_floor:
        return copy_floor()

    import torchbvh_amd as tb

    dev = torch.device("cuda:0")
    w = make_workload(args.config)
    k = w["k"]
    pts = w["points"].to(dev)
    qs = w["queries"].to(dev)
    D = pts.shape[-1]
    kind = w["kind"]
    if kind == "ragged":
        off = w["offsets"].to(dev)
        qoff = w["query_offsets"].to(dev)
        total_q = qs.shape[0]
        sizes = w["offsets"].diff().tolist()
        b_bytes = sum(build_bytes(n, D) for n in sizes)
    elif kind == "batched":
        total_q = qs.shape[0] * qs.shape[1]
        b_bytes = qs.shape[0] * build_bytes(pts.shape[1], D)
    else:
        total_q = qs.shape[0]
        b_bytes = build_bytes(pts.shape[0], D)
    s_bytes = qschedule_bytes(total_q, D)
    full_sort_bytes = qsort_bytes(total_q, D)
    n_bytes = knn_bytes(total_q, D, k)

    from torchbvh_amd._native import _C
    from torchbvh_amd._query import SCHEDULE_MIN_QUERIES

    # query_knn schedules the traversal only above SCHEDULE_MIN_QUERIES
    # queries (below it, input order is faster, schedule included).
    scheduled = total_q > SCHEDULE_MIN_QUERIES

    def step(events=None):
        """One pass of the hot path: build (BVH + accel), query ordering,
        traversal.  The build goes through the public API; the query calls
        the native ops in the order ``tb.query_knn`` does, with an event
        between each phase (all on torch's current stream, the stream the
        kernels are launched on)."""
        if events:
            events[0].record()
        if kind == "ragged":
            bvh = tb.build_bvh(pts, batch_offsets=off)
        else:
            bvh = tb.build_bvh(pts)
        if events:
            events[1].record()
        if kind == "ragged":
            packed = bvh._aux["packed"]
            order = (_C.morton_sort_queries_ragged(qs, qoff, packed["scene_min"], packed["scene_max"],
                                                   bvh["batch_size"], schedule=True)
                     if scheduled else None)
            if events:
                events[2].record()
            out = _C.query_knn_ragged(
                packed["node_aabbs"], packed["sorted_indices"], bvh["batch_offsets"], packed["node_offsets"],
                qs, qoff, order, bvh["batch_size"], D, k, accel=bvh._aux["accel"],
                total_points=bvh._aux["host_offsets"][-1])
        else:
            one = kind == "single"
            qb = qs.unsqueeze(0) if one else qs
            smin = bvh["scene_min"].unsqueeze(0) if one else bvh["scene_min"]
            smax = bvh["scene_max"].unsqueeze(0) if one else bvh["scene_max"]
            nodes = bvh["node_aabbs"].unsqueeze(0) if one else bvh["node_aabbs"]
            sidx = bvh["sorted_indices"].unsqueeze(0) if one else bvh["sorted_indices"]
            if scheduled:
                order = _C.morton_sort_queries_narrow(qb, smin, smax, schedule=True)
            if events:
                events[2].record()
            if scheduled:
                out = _C.query_knn_batched_cached_bounds_ordered(
                    nodes, sidx, qb, order, bvh["num_leaves"], bvh["num_real_nodes"], D, k,
                    accel=bvh._aux["accel"])
            else:
                out = _C.query_knn_batched_cached_bounds(
                    nodes, sidx, qb, bvh["num_leaves"], bvh["num_real_nodes"], D, k, accel=bvh._aux["accel"])
        if events:
            events[3].record()
        return bvh, out

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    build_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    query_ms = sum(e[1].elapsed_time(e[3]) for e in evs) / args.steps
    sort_ms = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    trav_ms = sum(e[2].elapsed_time(e[3]) for e in evs) / args.steps

    # The reference binding's full Morton sort of the queries (30 / 32 key
    # bits, four passes; for ragged input the segmented form of its
    # per-cloud calls), which query_knn replaces with the two-pass schedule;
    # timed on its own, outside the timed region.
    bvh, _ = step()
    if kind == "ragged":
        packed = bvh._aux["packed"]

        def full_sort():
            return _C.morton_sort_queries_ragged(qs, qoff, packed["scene_min"], packed["scene_max"],
                                                 bvh["batch_size"])
    else:
        one = kind == "single"
        qb = qs.unsqueeze(0) if one else qs
        smin = bvh["scene_min"].unsqueeze(0) if one else bvh["scene_min"]
        smax = bvh["scene_max"].unsqueeze(0) if one else bvh["scene_max"]

        def full_sort():
            return _C.morton_sort_queries_narrow(qb, smin, smax)
    for _ in range(2):
        full_sort()
    ef = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ef[0].record()
    for _ in range(10):
        full_sort()
    ef[1].record()
    torch.cuda.synchronize()
    full_sort_ms = ef[0].elapsed_time(ef[1]) / 10

    implicit_ms = None
    if kind != "ragged" and args.implicit_reps > 0:
        # The same query over the reference's implicit tree, for comparison
        # (outside the timed region).
        bvh, _ = step()
        one = kind == "single"
        qb = qs.unsqueeze(0) if one else qs
        smin = bvh["scene_min"].unsqueeze(0) if one else bvh["scene_min"]
        smax = bvh["scene_max"].unsqueeze(0) if one else bvh["scene_max"]
        nodes = bvh["node_aabbs"].unsqueeze(0) if one else bvh["node_aabbs"]
        sidx = bvh["sorted_indices"].unsqueeze(0) if one else bvh["sorted_indices"]
        order = _C.morton_sort_queries_narrow(qb, smin, smax, schedule=True)
        ei = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ei[0].record()
        for _ in range(args.implicit_reps):
            _C.query_knn_batched_cached_bounds_ordered(
                nodes, sidx, qb, order, bvh["num_leaves"], bvh["num_real_nodes"], D, k, accel=False)
        ei[1].record()
        torch.cuda.synchronize()
        implicit_ms = ei[0].elapsed_time(ei[1]) / args.implicit_reps

    if args.calibration_copy:
        # A plain device copy of known size, for scaling rocprofv3's
        # FETCH_SIZE / WRITE_SIZE counters (not part of the measurement).
        src = torch.ones(64 * 1024 * 1024, device=dev)
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()

    value = total_q / (ms_per_step * 1e-3)
    trav_gbs = n_bytes / (trav_ms * 1e-3) / 1e9 if trav_ms > 0 else None
    # Which kernels the timed k-NN call runs: batched calls above
    # GRID_MIN_QUERIES take the cell-block search where the clouds allow a
    # grid (a nonzero workspace), the rest the accel traversal alone.
    from torchbvh_amd import _native as native
    ws = ctypes.c_size_t(0)
    clouds, per_cloud = (1, pts.shape[0]) if kind == "single" else (pts.shape[0], pts.shape[1])
    grid = (kind != "ragged" and total_q > native.GRID_MIN_QUERIES
            and native.load().tbvh_knn_accel_grid_workspace_size(
                clouds, total_q // clouds, per_cloud, D, k, ctypes.byref(ws)) == 0
            and ws.value > 0)
    call_what = ("k-NN call: cell-block passes (grid_knn_kernel; grid_knn2_kernel for 3-D k = 8, 16) and the "
                 "traversal of what they leave (knn_accel_kernel)" if grid else "knn_accel_kernel (traversal)")
    traffic = measured_traffic(args.config)
    line = {
        "metric": "k-NN queries/sec + BVH build ms, 1M pts/1M queries k=16 3D fp32, 1 GPU",
        "value": value,
        "unit": "queries/s (end-to-end: build + query ordering + traversal per step)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch CPU generator, BASELINE config shapes)",
        "config": {
            "workload": CONFIGS[args.config],
            "config_id": args.config,
            "points": int(pts.numel() // D),
            "queries": int(total_q),
            "k": k,
            "dim": D,
        },
        "build_ms": build_ms,
        "query_ms": query_ms,
        "query_sort_ms": sort_ms,
        "query_sort_what": ("traversal schedule: stable 2-pass radix sort on the top 16 bits of Hilbert keys"
                            if scheduled else "none: at most SCHEDULE_MIN_QUERIES queries run in input order"),
        "traversal_ms": trav_ms,
        "traversal_implicit_tree_ms": implicit_ms,
        "queries_per_s_excl_build": total_q / (query_ms * 1e-3) if query_ms > 0 else None,
        "build_hbm_frac_algorithmic": (b_bytes / (build_ms * 1e-3) / 1e9) / HBM_PEAK_GBS,
        "query_sort_hbm_frac_algorithmic": ((s_bytes / (sort_ms * 1e-3) / 1e9) / HBM_PEAK_GBS
                                            if sort_ms and scheduled else None),
        "query_sort_bytes_formula": "Q(4D+40): queries read, 4-B keys, 2 passes x 16 B, 4-B order",
        "query_sort_full_ms": full_sort_ms,
        "query_sort_full_what": "reference binding morton_sort_queries_narrow: 30/32-bit Morton keys, 4 passes",
        "query_sort_full_hbm_frac_algorithmic": ((full_sort_bytes / (full_sort_ms * 1e-3) / 1e9) / HBM_PEAK_GBS
                                                 if full_sort_ms else None),
        "query_sort_full_bytes_formula": "Q(4D+72)",
        "roofline": {
            "bound": "hbm",
            "kernel": call_what,
            "achieved": trav_gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": (trav_gbs / HBM_PEAK_GBS) if trav_gbs else None,
            "traffic": traffic,
        },
    }
    if not args.no_cpu_baseline:
        clouds = job_clouds(w)
        line["cpu_baseline"] = cpu_baseline(clouds, k, args.cpu_queries, args.cpu_seconds * 2)
        line["cpu_port_bvh_dfs"] = cpu_port_dfs(clouds, k, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
