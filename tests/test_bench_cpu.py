"""bench.py's host-side pieces: the CPU baseline's contract fields and the
one-GPU guard (no GPU needed)."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def test_cpu_baseline_fields_on_the_small_config():
    import os

    w = bench.make_workload("cfg1")
    clouds = bench.job_clouds(w)
    assert len(clouds) == 1 and clouds[0][0].shape == (10_000, 3)
    r = bench.cpu_baseline(clouds, w["k"], 256)
    assert set(r) == {"value", "unit", "cores", "kind", "sample"}
    assert r["kind"] == "port" and r["unit"] == "queries/s"
    assert r["value"] > 0 and r["cores"] == len(os.sched_getaffinity(0))
    assert "brute force" in r["sample"] and "256 of 10000" in r["sample"]
    d = bench.cpu_port_dfs(clouds, w["k"], 0.05)
    assert set(d) == set(r) and d["value"] > 0 and "C oracle" in d["sample"]


def test_cpu_baseline_sample_extrapolates_by_pairs():
    """Ragged clouds are sampled at different fractions: the sample's time
    scales by (query, point) pairs."""
    import numpy as np

    rng = np.random.default_rng(1)
    clouds = [(rng.random((n, 3), dtype=np.float32), rng.random((m, 3), dtype=np.float32))
              for n, m in ((300, 50), (2000, 400))]
    r = bench.cpu_baseline(clouds, 4, 64)
    assert "114 of 450" in r["sample"]  # all 50 of the first cloud, 64 of the second


def test_query_sort_byte_formulas():
    assert bench.qsort_bytes(10, 3) == 10 * (12 + 4 + 4 * 16 + 4)
    assert bench.qschedule_bytes(10, 3) == 10 * (12 + 4 + 2 * 16 + 4)


def test_job_clouds_split_batched_and_ragged_workloads():
    w = bench.make_workload("cfg3")
    clouds = bench.job_clouds(w)
    assert len(clouds) == 32 and all(p.shape == (65_536, 3) for p, _ in clouds)
    w = bench.make_workload("cfg5")
    clouds = bench.job_clouds(w)
    off = w["offsets"].tolist()
    assert [len(p) for p, _ in clouds] == [b - a for a, b in zip(off, off[1:])]
    assert sum(len(q) for _, q in clouds) == w["queries"].shape[0]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
