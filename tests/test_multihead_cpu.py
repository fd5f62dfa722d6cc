"""Argument checks of the displaced-query helpers that fire before any GPU
work (reference messages: torchbvh/_multihead.py:17-35, 92-110, 166-182;
tests/test_displaced_query.py:70-85)."""

import pytest
import torch

import torchbvh_amd as tb


def inputs(B=2, N=6, H=3, D=3, C=4):
    pos = torch.rand(B, N, D)
    q = pos[:, :, None, :].repeat(1, 1, H, 1)
    return pos, q, torch.rand(B, N, H, C)


@pytest.mark.parametrize(
    "bad_pos,bad_q,match",
    [
        (lambda p: p[0], lambda q: q, "pos.*shape"),
        (lambda p: p, lambda q: q.reshape(q.size(0), q.size(1) * q.size(2), q.size(3)), "q.*shape"),
        (lambda p: p[:1], lambda q: q, "batch size"),
        (lambda p: p, lambda q: q[:, :3], "point dimension"),
        (lambda p: p, lambda q: q[..., :2], "last dimension"),
        (lambda p: p, lambda q: q[:, :, :0], "at least one head"),
        (lambda p: p[..., :1], lambda q: q[..., :1], "D must be 2 or 3"),
    ],
)
def test_query_displaced_knn_shape_validation(bad_pos, bad_q, match):
    pos, q, _ = inputs()
    with pytest.raises(ValueError, match=match):
        tb.query_displaced_knn(bad_pos(pos), bad_q(q), 4)


def test_gather_neighbor_values_shape_validation():
    values = torch.rand(2, 5, 3, 4)
    idx = torch.zeros(2, 5, 3, 4, dtype=torch.int64)
    with pytest.raises(ValueError, match="values must have shape"):
        tb.gather_neighbor_values(values[0], idx)
    with pytest.raises(ValueError, match="indices must have shape"):
        tb.gather_neighbor_values(values, idx[0])
    with pytest.raises(ValueError, match="batch size"):
        tb.gather_neighbor_values(values, idx[:1])
    with pytest.raises(ValueError, match="point dimension"):
        tb.gather_neighbor_values(values, idx[:, :2])
    with pytest.raises(ValueError, match="head dimension"):
        tb.gather_neighbor_values(values, idx[:, :, :1])
    with pytest.raises(ValueError, match="at least one channel"):
        tb.gather_neighbor_values(values[..., :0], idx)


def test_interpolate_displaced_argument_validation():
    pos, q, values = inputs()
    with pytest.raises(ValueError, match="reduction must be 'weighted_mean'"):
        tb.interpolate_displaced(pos, q, values, reduction="max")
    with pytest.raises(ValueError, match="pos must have shape"):
        tb.interpolate_displaced(pos[0], q, values)
