"""Committed golden fixtures (tests/golden/golden.npz, written by
tests/golden/make_golden.py from the reference's own test inputs).

CPU: the oracle still produces every fixture bit for bit.
GPU: the HIP library matches every fixture bit for bit — Morton codes,
permutations, node boxes and traversal arrays of the reference's build test
clouds, k-NN indices and distances (including exact ties), the Morton and
schedule query orders, and primitive builds."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

sys.path.insert(0, str(Path(__file__).parent / "golden"))

from make_golden import BUILD_FIELDS, cases  # noqa: E402
from parity import assert_same_f32, assert_same_int  # noqa: E402

GOLDEN = Path(__file__).parent / "golden" / "golden.npz"


def golden() -> dict[str, np.ndarray]:
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def case_names(g: dict, prefix: str) -> list[str]:
    return sorted({k.split("__")[0] for k in g if k.startswith(prefix)})


def assert_same(actual, expected, what: str) -> None:
    expected = np.asarray(expected)
    if expected.dtype.kind == "f":
        assert_same_f32(actual, expected, what)
    else:
        assert_same_int(actual, expected, what)


def test_oracle_reproduces_golden_fixtures():
    g = golden()
    fresh = cases()
    assert sorted(fresh) == sorted(g)
    for k in g:
        assert fresh[k].dtype == g[k].dtype and fresh[k].shape == g[k].shape, k
        assert_same(fresh[k], g[k], k)


@pytest.mark.gpu
def test_library_matches_golden_fixtures():
    import torchbvh_amd as tb
    from torchbvh_amd._native import _C

    dev = torch.device("cuda")
    g = golden()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    for c in case_names(g, "build"):
        p = g[f"{c}__points"]
        h = _C.build_bvh_batched_cooperative(t(p[None]))
        for f in BUILD_FIELDS:
            got = h[f] if f in ("left_child_mem", "right_child_mem", "mem_to_leaf") else h[f][0]
            assert_same(got.cpu().numpy(), g[f"{c}__{f}"], f"{c} {f}")
        codes = _C.morton_codes(t(p[None]), h["scene_min"], h["scene_max"])[0]
        assert_same(codes.cpu().numpy(), g[f"{c}__morton"], f"{c} morton")
    for c in case_names(g, "knn") + case_names(g, "ties"):
        p, q, k = g[f"{c}__points"], g[f"{c}__queries"], int(g[f"{c}__k"])
        idx, dist = tb.query_knn(tb.build_bvh(t(p)), t(q), k)
        assert_same(idx.cpu().numpy(), g[f"{c}__indices"], f"{c} indices")
        assert_same(dist.cpu().numpy(), g[f"{c}__distances"], f"{c} distances")
    for c in case_names(g, "sched"):
        q, lo, hi = (t(g[f"{c}__{f}"][None]) for f in ("queries", "lo", "hi"))
        assert_same(_C.morton_sort_queries_narrow(q, lo, hi)[0].cpu().numpy(), g[f"{c}__morton_order"],
                    f"{c} Morton order")
        assert_same(_C.morton_sort_queries_narrow(q, lo, hi, schedule=True)[0].cpu().numpy(),
                    g[f"{c}__schedule_order"], f"{c} schedule order")
    for c in case_names(g, "prims"):
        h = _C.build_primitive_bvh_batched(t(g[f"{c}__primitives"][None]))
        for f in BUILD_FIELDS:
            got = h[f] if f in ("left_child_mem", "right_child_mem", "mem_to_leaf") else h[f][0]
            assert_same(got.cpu().numpy(), g[f"{c}__{f}"], f"{c} {f}")
