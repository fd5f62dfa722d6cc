"""The build and k-NN launch sequences under HIP graph capture.

No entry point synchronises, allocates device memory itself or clears
memory with a memset, so after a warm-up the whole build + query can be
captured in a graph (torch's CUDA-graph API on ROCm).  Each replay here
follows new points copied into the captured input, with eager work and
synchronisations between replays, and must equal the eager results bit
for bit (indices, distances, node boxes, permutation)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import torchbvh_amd as tb
from torchbvh_amd import _query

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def cloud(seed: int, n: int, dim: int) -> torch.Tensor:
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.rand((n, dim), generator=g).to(DEV)


@pytest.mark.parametrize("dim,k", [(3, 16), (2, 8)])
def test_build_and_knn_replay_under_graph_capture(dim, k, monkeypatch):
    monkeypatch.setattr(_query, "SCHEDULE_MIN_QUERIES", 0)  # capture the schedule sort too
    n, m = 60_000, 20_000
    p = cloud(1, n, dim)
    q = cloud(2, m, dim)

    def step():
        h = tb.build_bvh(p)
        idx, dist = tb.query_knn(h, q, k)
        return h["node_aabbs"], h["sorted_indices"], idx, dist

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()

    for r in range(4):
        p.copy_(cloud(10 + r, n, dim))
        q.copy_(cloud(20 + r, m, dim))
        graph.replay()
        torch.cuda.synchronize()
        want = step()  # eager, between replays
        torch.cuda.synchronize()
        for name, a, b in zip(("node_aabbs", "sorted_indices", "indices", "distances"), out, want):
            assert torch.equal(a, b), f"replay {r}: {name} differs from the eager result"
        assert int(out[2].min()) >= 0 and int(out[2].max()) < n
