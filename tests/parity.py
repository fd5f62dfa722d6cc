"""Helpers shared by the parity tests: point-set fixtures restated from the
reference's test-suite (torchbvh tests/test_bvh_build.py, tests/test_knn.py)
and exact comparisons against the C oracle."""

from __future__ import annotations

import numpy as np
import torch

import oracle


def bits(a) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    return a.view(np.uint32)


def assert_same_f32(actual, expected, what: str) -> None:
    a, e = bits(actual), bits(expected)
    if not np.array_equal(a, e):
        bad = np.argwhere(a != e)
        first = tuple(bad[0])
        raise AssertionError(
            f"{what}: {len(bad)} of {a.size} fp32 values differ bitwise; first at {first}: "
            f"{np.asarray(actual)[first]!r} vs {np.asarray(expected)[first]!r}"
        )


def assert_same_int(actual, expected, what: str) -> None:
    a, e = np.asarray(actual), np.asarray(expected)
    assert a.shape == e.shape, f"{what}: shape {a.shape} vs {e.shape}"
    if not np.array_equal(a, e):
        bad = np.argwhere(a != e)
        first = tuple(bad[0])
        raise AssertionError(
            f"{what}: {len(bad)} of {a.size} values differ; first at {first}: "
            f"{a[first]!r} vs {e[first]!r}"
        )


def np32(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu().numpy()
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


# ---------------------------------------------------------------------------
# Point sets from the reference's build tests (tests/test_bvh_build.py:133-340)
# ---------------------------------------------------------------------------
def boundary_cloud(n: int, dim: int) -> np.ndarray:
    """tests/test_bvh_build.py:166-179."""
    base = np.arange(n, dtype=np.float32)
    cols = [((base * (d + 3)) % 11) + base * np.float32(0.125 + 0.25 * d) for d in range(dim)]
    return np.stack(cols, axis=1).astype(np.float32)


def single_child_cloud(n: int) -> np.ndarray:
    """tests/test_bvh_build.py:307-321."""
    a = np.arange(n, dtype=np.float32)
    return np.stack((a, np.remainder(a, 3), -a), axis=1).astype(np.float32)


def linspace32(a, b, n) -> np.ndarray:
    return torch.linspace(a, b, n, dtype=torch.float32).numpy()


def pathological_clouds() -> list[np.ndarray]:
    """tests/test_bvh_build.py:133-164, :182-304, :324-340."""
    f = lambda rows: np.asarray(rows, dtype=np.float32)  # noqa: E731
    return [
        f([[0.0, 0.0], [1.0, 0.0], [0.25, 0.75], [0.25, 0.75], [2.0, -1.0]]),
        f([[1.0, 2.0, 0.0], [1.0, 2.0, 0.0], [3.0, 2.0, -1.0], [0.0, 2.0, 4.0],
           [5.0, 2.0, 4.0], [2.0, 2.0, 4.0]]),
        f([[4.0, -2.0]]),
        f([[-1.0, 3.0, 5.0]]),
        f([[0.0, 0.0], [10.0, -2.0]]),
        f([[0.0, 0.0, 0.0], [10.0, -2.0, 0.5]]),
        np.stack((linspace32(-3.0, 3.0, 9), linspace32(6.0, -6.0, 9)), 1),
        np.stack((linspace32(-2.0, 2.0, 11), linspace32(4.0, -4.0, 11), linspace32(1.0, 9.0, 11)), 1),
        f([[-2.0, -1.0, 7.0], [-1.0, 2.0, 7.0], [0.0, -3.0, 7.0], [1.0, 4.0, 7.0],
           [2.0, -5.0, 7.0], [3.0, 6.0, 7.0]]),
        np.full((9, 3), 2.5, np.float32),
        f([[0.0, 0.0], [1.0e6, 1.0e-3], [2.0e6, -1.0e-3], [3.0e6, 2.0e-3], [4.0e6, -2.0e-3]]),
        f([[0.0, 0.0, 0.0], [1.0e-3, 1.0e6, 2.0], [-1.0e-3, 2.0e6, -2.0], [2.0e-3, 3.0e6, 4.0],
           [-2.0e-3, 4.0e6, -4.0]]),
        f([[1.0e-7, -2.0e-7], [1.5e-7, -2.5e-7], [2.0e-7, -1.5e-7], [2.5e-7, -3.0e-7],
           [3.0e-7, -1.0e-7]]),
        f([[1.0, 1.0e-6, -1.0e3], [2.0, 1.5e-6, -5.0e2], [3.0, 2.0e-6, 0.0], [4.0, 2.5e-6, 5.0e2],
           [5.0, 3.0e-6, 1.0e3], [6.0, 3.5e-6, 1.5e3], [7.0, 4.0e-6, 2.0e3]]),
        f([[1.0e-4, -1.0e8], [2.0e-4, -5.0e7], [3.0e-4, 0.0], [4.0e-4, 5.0e7], [5.0e-4, 1.0e8]]),
        f([[-1.0e6, 1.0e-5, 2.0], [-5.0e5, 2.0e-5, 2.0], [0.0, 3.0e-5, 2.0], [5.0e5, 4.0e-5, 2.0],
           [1.0e6, 5.0e-5, 2.0], [1.5e6, 6.0e-5, 2.0]]),
        f([[7.0, -3.0], [7.0, -3.0], [7.0, -3.0]]),
    ]


def knn_pathological_clouds() -> list[tuple[np.ndarray, int]]:
    """tests/test_knn.py:160-258 (points, k)."""
    f = lambda rows: np.asarray(rows, dtype=np.float32)  # noqa: E731
    rng = np.random.default_rng(1601)
    return [
        (np.stack((linspace32(-3.0, 3.0, 17), linspace32(6.0, -6.0, 17)), 1), 4),
        (np.stack((linspace32(-2.0, 2.0, 19), linspace32(4.0, -4.0, 19), linspace32(1.0, 9.0, 19)), 1), 8),
        (f([[-2.0, -1.0, 7.0], [-1.0, 2.0, 7.0], [0.0, -3.0, 7.0], [1.0, 4.0, 7.0],
            [2.0, -5.0, 7.0], [3.0, 6.0, 7.0], [4.0, -7.0, 7.0], [5.0, 8.0, 7.0],
            [6.0, -9.0, 7.0], [7.0, 10.0, 7.0], [8.0, -11.0, 7.0], [9.0, 12.0, 7.0]]), 4),
        (np.full((18, 3), 2.5, np.float32), 16),
        (f([[0.0, 0.0], [1.0e6, 1.0e-3], [2.0e6, -1.0e-3], [3.0e6, 2.0e-3], [4.0e6, -2.0e-3],
            [5.0e6, 3.0e-3], [6.0e6, -3.0e-3], [7.0e6, 4.0e-3], [8.0e6, -4.0e-3]]), 8),
        (f([[0.0, 0.0, 0.0], [1.0e-3, 1.0e6, 2.0], [-1.0e-3, 2.0e6, -2.0], [2.0e-3, 3.0e6, 4.0],
            [-2.0e-3, 4.0e6, -4.0], [3.0e-3, 5.0e6, 6.0], [-3.0e-3, 6.0e6, -6.0],
            [4.0e-3, 7.0e6, 8.0], [-4.0e-3, 8.0e6, -8.0]]), 8),
        (np.concatenate((rng.random((20, 2), dtype=np.float32), f([[1000.0, -1000.0]]))), 4),
    ]


def unit_direction_points(dim: int) -> np.ndarray:
    """tests/test_knn.py:282-324: 4 copies of each unit direction + 3x each."""
    eye = np.eye(dim, dtype=np.float32)
    dirs = np.concatenate([np.stack((eye[d], -eye[d])) for d in range(dim)])
    return np.concatenate((np.repeat(dirs, 4, axis=0), 3.0 * dirs)).astype(np.float32)
