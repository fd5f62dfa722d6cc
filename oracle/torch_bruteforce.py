"""Brute-force k-NN in torch on the CPU — the reference's test oracle
(tests/test_knn.py:10-12: ``(q[:, None] - p[None]).square().sum(-1)`` then
``topk(largest=False)``) with the (distance, index) tie rule.

TEST INFRASTRUCTURE ONLY (oracle package): tests use it as a second,
independent checker.

Ties: top-k runs on the int64 composite ``float_bits(d) << 32 | index``.
Squared distances are >= 0, so their IEEE bit patterns order like the values
and the composite orders lexicographically by (distance, index).  Distances
here are torch's unfused ``square().sum()`` (they can differ from the fused
chain of the GPU kernel in the last bit); parity tests use the C oracle.
"""

from __future__ import annotations

import torch


def knn_bruteforce(points: torch.Tensor, queries: torch.Tensor, k: int,
                   chunk: int = 16) -> tuple[torch.Tensor, torch.Tensor]:
    points = points.float().contiguous()
    queries = queries.float().contiguous()
    n = points.shape[0]
    idx_col = torch.arange(n, dtype=torch.int64)
    out_i, out_d = [], []
    for s in range(0, queries.shape[0], chunk):
        q = queries[s : s + chunk]
        d = (q[:, None, :] - points[None, :, :]).square().sum(dim=-1)
        key = (d.view(torch.int32).to(torch.int64) << 32) | idx_col
        top = key.topk(k, dim=1, largest=False, sorted=True).values
        out_i.append(top & 0xFFFFFFFF)
        out_d.append((top >> 32).to(torch.int32).view(torch.float32))
    return torch.cat(out_i), torch.cat(out_d)
