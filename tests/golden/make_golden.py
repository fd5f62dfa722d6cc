"""Writes tests/golden/golden.npz: expected outputs for the reference's own
test inputs, computed by this repository's CPU oracle.

Run from the repository root: `python tests/golden/make_golden.py`.

Inputs restate the reference's test cases (torchbvh tests/test_bvh_build.py
:133-340, tests/test_knn.py:160-324, tests/test_raytrace.py:94-116); the
outputs are the oracle's, whose every function is pinned independently in
tests/test_oracle.py.  The fixtures freeze those expected values so that a
change to the oracle or to the library shows up as a diff against data,
not only against the other implementation.

Layout: one flat archive, keys `<case>__<field>`; cases `build<i>`,
`knn<i>`, `ties<dim>_<k>`, `sched<dim>` and `prims<dim>`.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import oracle  # noqa: E402
from parity import knn_pathological_clouds, pathological_clouds, unit_direction_points  # noqa: E402

BUILD_FIELDS = ("node_aabbs", "sorted_indices", "scene_min", "scene_max", "left_child_mem",
                "right_child_mem", "mem_to_leaf")


def cases() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    for i, p in enumerate(pathological_clouds()):
        b = oracle.build(p)
        out[f"build{i}__points"] = p
        out[f"build{i}__morton"] = oracle.morton_codes(p, b["scene_min"], b["scene_max"])
        for f in BUILD_FIELDS:
            out[f"build{i}__{f}"] = b[f]
    for i, (p, k) in enumerate(knn_pathological_clouds()):
        q = (p[: min(7, p.shape[0])] + np.float32(0.125)).astype(np.float32)
        idx, dist = oracle.knn(p, q, k)
        out[f"knn{i}__points"], out[f"knn{i}__queries"] = p, q
        out[f"knn{i}__k"] = np.array(k, np.int64)
        out[f"knn{i}__indices"], out[f"knn{i}__distances"] = idx, dist
    for dim in (2, 3):
        p = unit_direction_points(dim)
        q = np.zeros((2, dim), np.float32)
        for k in (4, 8, 16):
            idx, dist = oracle.knn(p, q, k)
            out[f"ties{dim}_{k}__points"], out[f"ties{dim}_{k}__queries"] = p, q
            out[f"ties{dim}_{k}__k"] = np.array(k, np.int64)
            out[f"ties{dim}_{k}__indices"], out[f"ties{dim}_{k}__distances"] = idx, dist
        rng = np.random.default_rng(500 + dim)
        q = (rng.random((300, dim), dtype=np.float32) * 1.2 - 0.1).astype(np.float32)
        lo, hi = np.zeros(dim, np.float32), np.ones(dim, np.float32)
        out[f"sched{dim}__queries"], out[f"sched{dim}__lo"], out[f"sched{dim}__hi"] = q, lo, hi
        out[f"sched{dim}__morton_order"] = oracle.query_order(q, lo, hi)
        out[f"sched{dim}__schedule_order"] = oracle.schedule_order(q, lo, hi)
        F = 37 if dim == 2 else 29
        prims = (np.random.default_rng(8102 + dim).random((F, dim, dim), dtype=np.float32) * 4 - 2)
        b = oracle.build_primitives(prims.astype(np.float32))
        out[f"prims{dim}__primitives"] = prims.astype(np.float32)
        for f in BUILD_FIELDS:
            out[f"prims{dim}__{f}"] = b[f]
    return out


if __name__ == "__main__":
    data = cases()
    path = Path(__file__).with_name("golden.npz")
    np.savez_compressed(path, **data)
    print(f"wrote {path} ({path.stat().st_size} bytes, {len(data)} arrays)")
