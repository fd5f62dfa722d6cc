"""C-ABI checks that need no GPU: the library loads, exports every symbol the
public header declares, its closed forms agree with the oracle, and argument
errors are reported (status + message) before anything is launched."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

import oracle
from torchbvh_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "torchbvh_amd.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tbvh_\w+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    names = declared_functions()
    for required in ("tbvh_build", "tbvh_build_workspace_size", "tbvh_build_ragged",
                     "tbvh_sort_queries", "tbvh_sort_queries_ragged", "tbvh_knn",
                     "tbvh_knn_ragged", "tbvh_last_error", "tbvh_abi_version"):
        assert required in names


@pytest.mark.parametrize("compiler,lang,std", [("gcc", "c", "c99"), ("g++", "c++", "c++17")])
def test_header_compiles_standalone(compiler, lang, std):
    """The public header is plain C (and C++-includable): no HIP or torch
    types, self-contained includes."""
    import shutil
    import subprocess

    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} not available")
    r = subprocess.run([compiler, "-fsyntax-only", "-x", lang, f"-std={std}", "-Wall", "-Wextra", "-Werror",
                        str(HEADER)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_library_exports_every_declared_symbol():
    L = _native.load()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, f"not exported: {missing}"
    assert L.tbvh_abi_version() == 2


@pytest.mark.parametrize("n", list(range(1, 300)) + [10_000, 65_536, 1 << 20, 4_194_304, 200_000, 1 << 30])
def test_closed_forms_match_oracle(n):
    assert _native.leaf_level(n) == oracle.leaf_level(n)
    assert _native.virtual_leaves(n) == oracle.virtual_leaves(n)
    assert _native.real_node_count(n) == oracle.real_node_count(n)


def test_closed_forms_reject_out_of_range():
    assert _native.real_node_count(0) == -1
    assert _native.real_node_count((1 << 30) + 1) == -1


def _err(L) -> str:
    return L.tbvh_last_error().decode()


FAKE = ctypes.c_void_p(0x100000)  # never dereferenced: every call below fails validation


def test_build_argument_errors():
    L = _native.load()
    size = ctypes.c_size_t()
    assert L.tbvh_build_workspace_size(1, 10, 4, ctypes.byref(size)) == 1
    assert "D must be 2 or 3" in _err(L)
    assert L.tbvh_build_workspace_size(0, 10, 3, ctypes.byref(size)) == 1
    assert L.tbvh_build_workspace_size(1 << 20, 1 << 12, 3, ctypes.byref(size)) == 1
    assert "int32" in _err(L)
    assert L.tbvh_build_workspace_size(2, 1000, 3, ctypes.byref(size)) == 0
    assert size.value > 0 and _err(L) == ""
    need = size.value
    # Workspace too small: rejected before any launch.
    args = [FAKE, 2, 1000, 3] + [FAKE] * 7
    assert L.tbvh_build(*args, FAKE, need - 1, None) == 2
    assert "workspace" in _err(L)
    # Null output.
    args = [FAKE, 2, 1000, 3, None] + [FAKE] * 6
    assert L.tbvh_build(*args, FAKE, need, None) == 1
    assert "null" in _err(L)
    # Misaligned workspace.
    args = [FAKE, 2, 1000, 3] + [FAKE] * 7
    assert L.tbvh_build(*args, ctypes.c_void_p(0x100004), need, None) == 1
    assert "aligned" in _err(L)


def test_knn_argument_errors():
    L = _native.load()
    nr = _native.real_node_count(100)
    base = [FAKE, FAKE, FAKE, None, 1, 10]
    assert L.tbvh_knn(*base, 100, nr, 3, 5, FAKE, FAKE, None) == 1
    assert "k must be 4, 8, or 16 (32 is also supported)" in _err(L)
    assert L.tbvh_knn(*base, 100, nr, 4, 8, FAKE, FAKE, None) == 1
    assert "D must be 2 or 3" in _err(L)
    assert L.tbvh_knn(*base, 3, _native.real_node_count(3), 3, 4, FAKE, FAKE, None) == 1
    assert "num_leaves must be >= k" in _err(L)
    assert L.tbvh_knn(*base, 100, nr + 1, 3, 4, FAKE, FAKE, None) == 1
    assert "num_real_nodes" in _err(L)
    assert L.tbvh_knn(FAKE, None, FAKE, None, 1, 10, 100, nr, 3, 4, FAKE, FAKE, None) == 1
    assert "null" in _err(L)
    # M == 0 is a no-op success (nothing launched).
    assert L.tbvh_knn(None, None, None, None, 1, 0, 100, nr, 3, 4, None, None, None) == 0


def test_sort_and_ragged_argument_errors():
    L = _native.load()
    size = ctypes.c_size_t()
    assert L.tbvh_sort_queries_workspace_size(1, -1, 3, ctypes.byref(size)) == 1
    assert L.tbvh_sort_queries(None, 1, 0, 3, None, None, None, None, 0, None) == 0
    assert L.tbvh_build_ragged_workspace_size(3, 2, 3, ctypes.byref(size)) == 1
    assert L.tbvh_knn_ragged(*([FAKE] * 7), 2, 10, 3, 7, FAKE, FAKE, None) == 1
    assert "k must be" in _err(L)
    # total_nodes below any valid tree size is rejected.
    assert L.tbvh_build_ragged(FAKE, FAKE, 2, 100, 3, *([FAKE] * 8), 10, FAKE, 1 << 20, None) == 1
    assert "total_nodes" in _err(L)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setattr(_native, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(RuntimeError, match="not built"):
        _native.load()


def test_accel_argument_errors():
    L = _native.load()
    size = ctypes.c_size_t()
    assert L.tbvh_accel_size(2, 1, 3, ctypes.byref(size)) == 1
    assert L.tbvh_accel_size(2, 1000, 3, ctypes.byref(size)) == 0
    assert size.value == ((1000 * 16 + 255) // 256) * 256 + 1000 * 16 * 4  # points, then one record row per point
    assert L.tbvh_accel_workspace_size(1, 1000, 2, ctypes.byref(size)) == 0
    need = size.value
    args = [FAKE] * 5 + [1, 1000, 2, FAKE]
    assert L.tbvh_accel_build(*args, FAKE, need - 1, None) == 2
    assert L.tbvh_accel_build(*([FAKE] * 5), 1, (1 << 28) + 1, 3, FAKE, FAKE, 1 << 40, None) == 1
    assert "2^28" in _err(L)
    assert L.tbvh_knn_accel(FAKE, FAKE, None, 1, 10, 3, 3, 4, FAKE, FAKE, None) == 1
    assert "num_leaves must be >= k" in _err(L)
    assert L.tbvh_knn_accel(None, None, None, 1, 0, 100, 3, 4, None, None, None) == 0


def test_grid_knn_workspace_and_argument_errors():
    L = _native.load()
    size = ctypes.c_size_t()
    # Too small for a grid of 4 cells per axis: no workspace (then the call is tbvh_knn_accel).
    assert L.tbvh_knn_accel_grid_workspace_size(1, 10, 20, 3, 4, ctypes.byref(size)) == 0 and size.value == 0
    # 2^20 points, k = 16 in 3-D: 4 points per cell, 2^18 cells; then flags, the two lists'
    # 8 x 64 counts each (32 words apart), the two lists (8 x 64 sub-lists, each for the
    # 64-query tiles of one eighth of the tiles with one residue mod 64), the bounds.
    M = 1000
    up = lambda x: (x + 255) // 256 * 256
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 1 << 20, 3, 16, ctypes.byref(size)) == 0
    table = (1 << 18) + 1
    tiles = (M + 63) // 64
    seg = ((tiles + 7) // 8 + 63) // 64 * 64
    expect = up(up(up(up(table * 4) + 4) + 2 * 512 * 32 * 4) + 512 * seg * 4)
    expect = up(expect + 512 * seg * 4)
    assert size.value == up(expect + M * 4)
    # k = 32 keeps at least 4 points per cell: 2^18 cells.
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 1 << 20, 3, 32, ctypes.byref(size)) == 0
    assert size.value == up(expect + M * 4)
    # Clouds of 2^24 points or more keep the traversal (run starts are packed into 24 bits).
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 1 << 24, 3, 16, ctypes.byref(size)) == 0 and size.value == 0
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 1 << 20, 4, 16, ctypes.byref(size)) == 1
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 1 << 20, 3, 5, ctypes.byref(size)) == 1
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 1 << 20, 3, 16, None) == 1
    # k = 4 keeps the traversal below 2^17 points per cloud, and 2-D clouds below 2^15 points.
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 1 << 16, 3, 4, ctypes.byref(size)) == 0 and size.value == 0
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 1 << 20, 2, 4, ctypes.byref(size)) == 0 and size.value == 0
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 10_000, 2, 8, ctypes.byref(size)) == 0 and size.value == 0
    # 10,000 points at k = 16 in 3-D: level 3 leaves 19.5 points per cell (4.9 x rho): no grid.
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, 10_000, 3, 16, ctypes.byref(size)) == 0 and size.value == 0
    N = 1 << 16
    assert L.tbvh_knn_accel_grid_workspace_size(1, M, N, 3, 8, ctypes.byref(size)) == 0 and size.value > 0
    need = size.value
    nr = _native.real_node_count(N)
    args = lambda nr_, ws, ws_bytes: (FAKE, FAKE, nr_, FAKE, None, 1, M, N, 3, 8, FAKE, FAKE, ws, ws_bytes, None)
    assert L.tbvh_knn_accel_grid(*args(nr + 1, FAKE, need)) == 1
    assert "num_real_nodes" in _err(L)
    assert L.tbvh_knn_accel_grid(*args(nr, FAKE, need - 1)) == 2
    assert "workspace" in _err(L)
    assert L.tbvh_knn_accel_grid(*args(nr, ctypes.c_void_p(0x100008), need)) == 1
    assert "aligned" in _err(L)
    assert L.tbvh_knn_accel_grid(FAKE, None, nr, FAKE, None, 1, M, N, 3, 8, FAKE, FAKE, FAKE, need, None) == 1
    assert "node_aabbs" in _err(L)
    assert L.tbvh_knn_accel_grid(None, None, 0, None, None, 1, 0, N, 3, 8, None, None, None, 0, None) == 0
    # The spatial form needs the launch order; the neighbour-row form its source and rows, then
    # the same checks as the plain form.
    sp = lambda order, nr_, ws_bytes: (FAKE, FAKE, nr_, FAKE, order, 1, M, N, 3, 8, FAKE, FAKE, FAKE, ws_bytes, None)
    assert L.tbvh_knn_accel_grid_spatial(*sp(None, nr, need)) == 1
    assert "null" in _err(L)
    assert L.tbvh_knn_accel_grid_spatial(*sp(FAKE, nr + 1, need)) == 1
    assert "num_real_nodes" in _err(L)
    assert L.tbvh_knn_accel_grid_spatial(*sp(FAKE, nr, need - 1)) == 2
    pos = lambda src, cols, nr_, ws_bytes: (FAKE, FAKE, nr_, FAKE, None, 1, M, N, 3, 8, src, cols, FAKE, FAKE, FAKE,
                                            FAKE, ws_bytes, None)
    assert L.tbvh_knn_accel_grid_positions(*pos(None, 3, nr, need)) == 1
    assert "source" in _err(L)
    assert L.tbvh_knn_accel_grid_positions(*pos(FAKE, 0, nr, need)) == 1
    assert "source_cols" in _err(L)
    assert L.tbvh_knn_accel_grid_positions(*pos(FAKE, 3, nr + 1, need)) == 1
    assert "num_real_nodes" in _err(L)
    assert L.tbvh_knn_accel_grid_positions(*pos(FAKE, 3, nr, need - 1)) == 2
    assert "workspace" in _err(L)


def test_routed_grid_workspace_and_argument_errors():
    """The routed cell-block search's workspace: the true route's tables,
    then the false route's (each at its own cloud's level), flags for both
    structures' clouds, then the counts, lists and bounds as in the plain
    search; none where either cloud takes no grid.  Argument errors before
    any launch."""
    L = _native.load()
    size = ctypes.c_size_t()
    up = lambda x: (x + 255) // 256 * 256
    B, M = 2, 1000
    # True clouds of 2^20 points (k = 16, 3-D: level 6, 2^18 cells), false clouds of 2^17 (level 5).
    assert L.tbvh_knn_accel_routed_grid_workspace_size(B, M, 1 << 20, 1 << 17, 3, 16, ctypes.byref(size)) == 0
    tiles = (B * M + 63) // 64
    seg = ((tiles + 7) // 8 + 63) // 64 * 64
    end = up(up(B * ((1 << 18) + 1) * 4) + B * ((1 << 15) + 1) * 4)
    end = up(end + 2 * B * 4)
    end = up(end + 2 * 512 * 32 * 4)
    end = up(up(end + 512 * seg * 4) + 512 * seg * 4)
    assert size.value == up(end + B * M * 4)
    # Swapped clouds: the true route's table is the smaller one, the total the same.
    assert L.tbvh_knn_accel_routed_grid_workspace_size(B, M, 1 << 17, 1 << 20, 3, 16, ctypes.byref(size)) == 0
    assert size.value == up(end + B * M * 4)
    # Either cloud without a grid: none (the call is then tbvh_knn_accel_routed_spatial).
    assert L.tbvh_knn_accel_routed_grid_workspace_size(B, M, 1 << 20, 1000, 3, 4, ctypes.byref(size)) == 0
    assert size.value == 0
    assert L.tbvh_knn_accel_routed_grid_workspace_size(B, M, 1 << 24, 1 << 20, 3, 16, ctypes.byref(size)) == 0
    assert size.value == 0
    assert L.tbvh_knn_accel_routed_grid_workspace_size(B, M, 1 << 20, 1 << 20, 3, 5, ctypes.byref(size)) == 1
    assert L.tbvh_knn_accel_routed_grid_workspace_size(B, M, 1 << 20, 1 << 20, 4, 16, ctypes.byref(size)) == 1
    assert L.tbvh_knn_accel_routed_grid_workspace_size(B, M, 1 << 20, 8, 3, 16, ctypes.byref(size)) == 1
    assert "source counts" in _err(L)
    assert L.tbvh_knn_accel_routed_grid_workspace_size(B, M, 1 << 20, 1 << 20, 3, 16, None) == 1
    N = 1 << 17
    assert L.tbvh_knn_accel_routed_grid_workspace_size(B, M, N, N, 3, 8, ctypes.byref(size)) == 0
    need = size.value
    assert need > 0
    nr = _native.real_node_count(N)

    def call(nr_t=nr, nr_f=nr, ws=FAKE, ws_bytes=need, nodes_f=FAKE, routes=FAKE, accel_f=FAKE, Mq=M):
        return L.tbvh_knn_accel_routed_grid_spatial(FAKE, FAKE, nr_t, accel_f, nodes_f, nr_f, FAKE, routes, FAKE,
                                                    B, Mq, N, N, 3, 8, FAKE, FAKE, ws, ws_bytes, None)
    assert call(nr_f=nr + 1) == 1
    assert "num_real_nodes" in _err(L)
    assert call(nr_t=nr - 1) == 1
    assert "num_real_nodes" in _err(L)
    assert call(ws_bytes=need - 1) == 2
    assert "workspace" in _err(L)
    assert call(ws=ctypes.c_void_p(0x100008)) == 1
    assert "aligned" in _err(L)
    assert call(nodes_f=None) == 1
    assert "node_aabbs" in _err(L)
    assert call(routes=None) == 1
    assert "null" in _err(L)
    assert call(accel_f=ctypes.c_void_p(0x100010)) == 1
    assert "aligned" in _err(L)
    assert L.tbvh_knn_accel_routed_grid_spatial(None, None, 0, None, None, 0, None, None, None, B, 0, N, N, 3, 8,
                                                None, None, None, 0, None) == 0


def test_accel_from_tree_and_accel_alignment_errors():
    """tbvh_accel_build_from_tree checks the node count against the tree
    over N points and needs its defects word; every k-NN accel entry point
    refuses an accel that is not 256-byte aligned.  All before any launch."""
    L = _native.load()
    size = ctypes.c_size_t()
    assert L.tbvh_accel_workspace_size(2, 2000, 3, ctypes.byref(size)) == 0
    need = size.value
    nr = _native.real_node_count(1000)
    assert L.tbvh_accel_build_from_tree(FAKE, FAKE, 2, 1000, nr - 1, 3, FAKE, FAKE, FAKE, need, None) == 1
    assert "num_real_nodes does not match num_leaves" in _err(L)
    assert L.tbvh_accel_build_from_tree(FAKE, FAKE, 2, 1000, nr, 3, FAKE, None, FAKE, need, None) == 1
    assert "null" in _err(L)
    mis = ctypes.c_void_p(0x100010)
    assert L.tbvh_knn_accel(mis, FAKE, None, 1, 10, 100, 3, 4, FAKE, FAKE, None) == 1
    assert "aligned" in _err(L)
    assert L.tbvh_knn_accel_spatial(mis, FAKE, FAKE, 1, 10, 100, 3, 4, FAKE, FAKE, None) == 1
    assert "aligned" in _err(L)
    assert L.tbvh_knn_accel_ragged(mis, FAKE, 100, FAKE, FAKE, None, 1, 10, 3, 4, FAKE, FAKE, None) == 1
    assert "aligned" in _err(L)
    assert L.tbvh_knn_accel_routed_spatial(FAKE, mis, FAKE, FAKE, FAKE, 1, 10, 100, 100, 3, 4, FAKE, FAKE,
                                           None) == 1
    assert "aligned" in _err(L)


def test_build_with_accel_argument_errors():
    L = _native.load()
    size = ctypes.c_size_t()
    assert L.tbvh_build_workspace_size(2, 1000, 3, ctypes.byref(size)) == 0
    need = size.value
    outs = [FAKE] * 7
    # Null accel.
    assert L.tbvh_build_with_accel(FAKE, 2, 1000, 3, *outs, None, FAKE, need, None) == 1
    assert "accel is null" in _err(L)
    # Misaligned accel.
    assert L.tbvh_build_with_accel(FAKE, 2, 1000, 3, *outs, ctypes.c_void_p(0x100010), FAKE,
                                   need, None) == 1
    assert "aligned" in _err(L)
    # Clouds above 2^28 points.
    assert L.tbvh_build_with_accel(FAKE, 1, (1 << 28) + 1, 3, *outs, FAKE, FAKE, 1 << 40,
                                   None) == 1
    assert "2^28" in _err(L)
    # Workspace too small.
    assert L.tbvh_build_with_accel(FAKE, 2, 1000, 3, *outs, FAKE, FAKE, need - 1, None) == 2
    # Ragged: null accel, then total_nodes too small.
    assert L.tbvh_build_ragged_with_accel(FAKE, FAKE, 2, 100, 3, *([FAKE] * 8), 1000, None,
                                          FAKE, 1 << 20, None) == 1
    assert "accel is null" in _err(L)
    assert L.tbvh_build_ragged_with_accel(FAKE, FAKE, 2, 100, 3, *([FAKE] * 8), 10, FAKE,
                                          FAKE, 1 << 20, None) == 1
    assert "total_nodes" in _err(L)


def test_spatial_knn_requires_an_order():
    L = _native.load()
    nr = _native.real_node_count(100)
    assert L.tbvh_knn_spatial(FAKE, FAKE, FAKE, None, 1, 10, 100, nr, 3, 4, FAKE, FAKE, None) == 1
    assert "null" in _err(L)
    assert L.tbvh_knn_accel_spatial(FAKE, FAKE, None, 1, 10, 100, 3, 4, FAKE, FAKE, None) == 1
    assert "null" in _err(L)
    assert L.tbvh_knn_accel_spatial(FAKE, FAKE, FAKE, 1, 10, 100, 3, 5, FAKE, FAKE, None) == 1
    assert "k must be" in _err(L)


def test_primitive_build_and_point_sort_argument_errors():
    L = _native.load()
    size = ctypes.c_size_t()
    # Only 2-D segments and 3-D triangles.
    for V, D in ((3, 2), (2, 3), (4, 3), (1, 1)):
        assert L.tbvh_build_primitives_workspace_size(1, 10, V, D, ctypes.byref(size)) == 1
        assert "expected 2-D segments or 3-D triangles" in _err(L)
    assert L.tbvh_build_primitives_workspace_size(0, 10, 3, 3, ctypes.byref(size)) == 1
    assert L.tbvh_build_primitives_workspace_size(2, 1000, 3, 3, ctypes.byref(size)) == 0
    need = size.value
    # The centres and leaf boxes are workspace: more than the point build's.
    point_size = ctypes.c_size_t()
    assert L.tbvh_build_workspace_size(2, 1000, 3, ctypes.byref(point_size)) == 0
    assert need >= point_size.value + 2 * 1000 * 9 * 4
    outs = [FAKE] * 7
    assert L.tbvh_build_primitives(None, 2, 1000, 3, 3, *outs, FAKE, need, None) == 1
    assert "null" in _err(L)
    assert L.tbvh_build_primitives(FAKE, 2, 1000, 3, 3, *outs, FAKE, need - 1, None) == 2
    assert L.tbvh_build_primitives(FAKE, 2, 1000, 3, 3, *outs, ctypes.c_void_p(0x100010), need,
                                   None) == 1
    assert "aligned" in _err(L)
    # Point ordering: bounds live in the workspace after the build layout.
    assert L.tbvh_morton_sort_points_workspace_size(2, 1000, 4, ctypes.byref(size)) == 1
    assert L.tbvh_morton_sort_points_workspace_size(2, 1000, 3, ctypes.byref(size)) == 0
    assert size.value > point_size.value
    assert L.tbvh_morton_sort_points(FAKE, 2, 1000, 3, None, FAKE, size.value, None) == 1
    assert L.tbvh_morton_sort_points(FAKE, 2, 1000, 3, FAKE, FAKE, size.value - 1, None) == 2


def test_knn_positions_argument_errors():
    """The fused-row entry points check their source and positions pointers
    and the row width before the traversal's own checks."""
    L = _native.load()
    NUL = None
    args = lambda src, cols, pos: (FAKE, FAKE, FAKE, 1, 10, 100, 3, 16, src, cols, FAKE, FAKE, pos, None)  # noqa: E731
    assert L.tbvh_knn_accel_positions(*args(NUL, 3, FAKE)) == 1
    assert "null source or positions" in _err(L)
    assert L.tbvh_knn_accel_positions(*args(FAKE, 3, NUL)) == 1
    assert "null source or positions" in _err(L)
    for cols in (0, -1, 4097):
        assert L.tbvh_knn_accel_positions(*args(FAKE, cols, FAKE)) == 1
        assert "source_cols must be in [1, 4096]" in _err(L)
    # Then the traversal's own checks apply (k here).
    bad_k = (FAKE, FAKE, FAKE, 1, 10, 100, 3, 5, FAKE, 3, FAKE, FAKE, FAKE, None)
    assert L.tbvh_knn_accel_positions(*bad_k) == 1
    assert "k must be 4, 8, or 16 (32 is also supported)" in _err(L)
    ragged = (FAKE, FAKE, 100, FAKE, FAKE, FAKE, 2, 10, 3, 16, NUL, 3, FAKE, FAKE, FAKE, None)
    assert L.tbvh_knn_accel_ragged_positions(*ragged) == 1
    assert "tbvh_knn_accel_ragged_positions" in _err(L) and "null source" in _err(L)


def test_interpolate_neighbors_argument_errors():
    """Shape and pointer checks of the interpolation entry point come before
    any launch; an empty cloud set is a no-op."""
    L = _native.load()
    args = lambda B, N, H, C, k, v=FAKE: (v, FAKE, FAKE, FAKE, B, N, H, C, k, FAKE, None)  # noqa: E731
    for bad in ((-1, 4, 2, 3, 8), (1, -1, 2, 3, 8), (1, 4, 0, 3, 8), (1, 4, 2, 0, 8), (1, 4, 2, 3, 0)):
        assert L.tbvh_interpolate_neighbors(*args(*bad)) == 1
        assert "need B >= 0, N >= 0, H >= 1, C >= 1 and k >= 1" in _err(L)
    assert L.tbvh_interpolate_neighbors(*args(1, 4, 2, 3, 8, None)) == 1
    assert "null input or output" in _err(L)
    for huge in ((1, 1 << 20, 1 << 10, 1 << 12, 8), (1 << 40, 1 << 40, 1 << 10, 1, 8),
                 (1 << 62, 4, 1, 1, 8), (1, 1, 1 << 32, 1 << 32, 8)):
        assert L.tbvh_interpolate_neighbors(*args(*huge)) == 1  # no int64 wrap past the check
        assert "exceeds 2^40" in _err(L)
    assert L.tbvh_interpolate_neighbors(*args(0, 4, 2, 3, 8, None)) == 0


def test_build_noalloc_argument_errors():
    """The no-allocation build rejects bad arguments and sizes beyond its
    scratch array before touching the GPU."""
    L = _native.load()
    outs = [FAKE] * 7
    assert L.tbvh_build_with_accel_noalloc(FAKE, 1, 1000, 3, *outs, None, None) == 1
    assert "accel is null" in _err(L)
    assert L.tbvh_build_with_accel_noalloc(FAKE, 1, 1000, 4, *outs, FAKE, None) == 1
    assert "D must be 2 or 3" in _err(L)
    assert L.tbvh_build_with_accel_noalloc(FAKE, 0, 1000, 3, *outs, FAKE, None) == 1
    # 8M points need more workspace than the 64 MiB array holds.
    size = ctypes.c_size_t()
    assert L.tbvh_build_workspace_size(1, 1 << 23, 3, ctypes.byref(size)) == 0
    assert size.value > 64 << 20
    assert L.tbvh_build_with_accel_noalloc(FAKE, 1, 1 << 23, 3, *outs, FAKE, None) == 2
    assert "scratch array holds 67108864" in _err(L)
