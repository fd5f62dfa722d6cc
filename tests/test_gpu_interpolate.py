"""The fused interpolation kernel of interpolate_displaced: bit-identical to
the reference's tensor formula (torchbvh/_multihead.py:123-144, 186-190), evaluated
here with torch on the same k-NN result, for vector and scalar channel
layouts, exact hits of several multiplicities, and the autograd path."""

from __future__ import annotations

import pytest
import torch

import torchbvh_amd as tb
from torchbvh_amd._native import _C

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def inputs(B, N, H, D, C, seed, dup=0):
    g = torch.Generator().manual_seed(seed)
    pos = torch.rand((B, N, D), generator=g)
    if dup:  # points repeated dup times: exact hits of that multiplicity
        pos[:, : N // 2] = pos[:, : N // (2 * dup)].repeat_interleave(dup, dim=1)[:, : N // 2]
    q = pos[:, :, None, :] + 0.02 * torch.randn((B, N, H, D), generator=g)
    q[:, ::3, 0] = pos[:, ::3]  # every third point's head 0 sits on it
    values = torch.randn((B, N, H, C), generator=g)
    return pos.to(DEV), q.to(DEV).contiguous(), values.to(DEV)


def tensor_formula(values, idx, d2):
    """The reference's sequence of tensor operations, one rank at a time."""
    B, N, H, C = values.shape
    k = idx.size(-1)
    b = torch.arange(B, device=DEV).view(B, 1, 1, 1)
    h = torch.arange(H, device=DEV).view(1, 1, H, 1)
    nv = values[b, idx, h]
    exact = d2 <= 1e-12
    w = torch.reciprocal(d2 + 1e-12)
    w = w / w.sum(-1, keepdim=True).clamp(min=1e-12)
    want = torch.zeros_like(values)
    ex = torch.zeros_like(values)
    for r in range(k):
        want = want + nv[..., r, :] * w[..., r].unsqueeze(-1)
        ex = ex + nv[..., r, :] * exact[..., r].float().unsqueeze(-1)
    ex = ex / exact.float().sum(-1, keepdim=True).clamp(min=1.0)
    return torch.where(exact.any(-1, keepdim=True), ex, want), exact


@pytest.mark.parametrize("C", [1, 3, 4, 16, 33, 64])
@pytest.mark.parametrize("k,dim", [(4, 2), (8, 3), (16, 3), (32, 2)])
def test_fused_matches_tensor_formula(C, k, dim):
    pos, q, values = inputs(2, 257, 3, dim, C, seed=100 * C + k)
    out = tb.interpolate_displaced(pos, q, values, k)
    idx, d2 = tb.query_displaced_knn(pos, q, k, return_positions=False)
    want, exact = tensor_formula(values, idx, d2)
    assert exact.any()
    assert torch.equal(out, want)


@pytest.mark.parametrize("dup", [2, 3, 5])
def test_exact_hits_of_several_points_average(dup):
    pos, q, values = inputs(2, 300, 2, 3, 8, seed=31 + dup, dup=dup)
    out = tb.interpolate_displaced(pos, q, values, 8)
    idx, d2 = tb.query_displaced_knn(pos, q, 8, return_positions=False)
    want, exact = tensor_formula(values, idx, d2)
    assert (exact.sum(-1) >= dup).any()
    assert torch.equal(out, want)


def test_gradient_path_agrees_and_differentiates():
    pos, q, values = inputs(1, 200, 2, 3, 6, seed=5)
    fused = tb.interpolate_displaced(pos, q, values, 8)
    v = values.clone().requires_grad_(True)
    traced = tb.interpolate_displaced(pos, q, v, 8)
    assert traced.requires_grad
    assert torch.equal(traced.detach(), fused)
    traced.sum().backward()
    assert v.grad is not None and torch.isfinite(v.grad).all()
    with torch.no_grad():
        assert torch.equal(tb.interpolate_displaced(pos, q, v, 8), fused)


def test_misaligned_values_take_the_scalar_layout():
    """C % 4 == 0 but values start 4 bytes past a 16-byte boundary."""
    pos, q, values = inputs(1, 128, 2, 2, 8, seed=9)
    store = torch.empty(values.numel() + 1, device=DEV)
    shifted = store[1:].view(values.shape)
    shifted.copy_(values)
    assert shifted.data_ptr() % 16 != 0
    idx, d2 = tb.query_displaced_knn(pos, q, 4, return_positions=False)
    assert torch.equal(tb.interpolate_displaced(pos, q, shifted, 4), tensor_formula(values, idx, d2)[0])


def test_binding_out_of_range_indices_contribute_zero():
    g = torch.Generator().manual_seed(3)
    B, N, H, C, k = 2, 10, 2, 5, 4
    values = torch.randn((B, N, H, C), generator=g).to(DEV)
    idx = torch.randint(-3, N + 3, (B, N, H, k), generator=g).to(DEV)
    w = torch.rand((B, N, H, k), generator=g).to(DEV)
    exact = torch.zeros((B, N, H, k), dtype=torch.bool, device=DEV)
    out = _C.interpolate_neighbors(values, idx, w, exact)
    valid = (idx >= 0) & (idx < N)
    b = torch.arange(B, device=DEV).view(B, 1, 1, 1)
    h = torch.arange(H, device=DEV).view(1, 1, H, 1)
    nv = values[b, idx.clamp(0, N - 1), h] * valid.unsqueeze(-1)
    want = torch.zeros_like(values)
    for r in range(k):
        want = want + nv[..., r, :] * w[..., r].unsqueeze(-1)
    assert torch.equal(out, want)


def test_binding_empty_and_shape_errors():
    values = torch.zeros((0, 4, 2, 3), device=DEV)
    idx = torch.zeros((0, 4, 2, 8), dtype=torch.int64, device=DEV)
    w = torch.zeros((0, 4, 2, 8), device=DEV)
    ex = torch.zeros((0, 4, 2, 8), dtype=torch.bool, device=DEV)
    assert _C.interpolate_neighbors(values, idx, w, ex).shape == (0, 4, 2, 3)
    with pytest.raises(RuntimeError, match="weights must have shape"):
        _C.interpolate_neighbors(values, idx, w[..., :4], ex)
    with pytest.raises(RuntimeError, match="exact must be a contiguous bool"):
        _C.interpolate_neighbors(values, idx, w, ex.to(torch.uint8))


def test_binding_beyond_one_grid_of_work_items():
    """1 x 2^24 x 17 rows of one channel: more items than one capped grid
    (2^20 work-groups of 256) holds, so the grid-stride loop's second lap
    runs; rows each side of the lap boundary, and the last rows, are checked
    against the tensor formula (~17 GB of device memory)."""
    B, N, H, C, k = 1, 1 << 24, 17, 1, 4
    rows = B * N * H
    lap = (1 << 20) * 256
    assert rows > lap
    g = torch.Generator(device=DEV).manual_seed(11)
    values = torch.randn((B, N, H, C), generator=g, device=DEV)
    idx = torch.randint(0, N, (B, N, H, k), generator=g, device=DEV)
    w = torch.rand((B, N, H, k), generator=g, device=DEV)
    exact = torch.rand((B, N, H, k), generator=g, device=DEV) < 0.05
    out = _C.interpolate_neighbors(values, idx, w, exact).view(rows, C)
    flat_idx, flat_w, flat_e = idx.view(rows, k), w.view(rows, k), exact.view(rows, k)
    vflat = values.view(N * H, C)
    for lo in (0, lap - 4096, rows - 4096):
        r = torch.arange(lo, lo + 8192 if lo < rows - 8192 else rows, device=DEV)
        h = r % H
        nv = vflat[flat_idx[r] * H + h[:, None]]  # (rows, k, C)
        e = flat_e[r]
        want = torch.zeros((len(r), C), device=DEV)
        ex = torch.zeros((len(r), C), device=DEV)
        for j in range(k):
            want = want + nv[:, j] * flat_w[r, j].unsqueeze(-1)
            ex = ex + nv[:, j] * e[:, j].float().unsqueeze(-1)
        ex = ex / e.float().sum(-1, keepdim=True).clamp(min=1.0)
        want = torch.where(e.any(-1, keepdim=True), ex, want)
        assert torch.equal(out[r], want), f"rows from {lo}"
    del values, idx, w, exact, out, flat_idx, flat_w, flat_e, vflat
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dim,k,duplicates", [(2, 4, False), (3, 8, True)])
def test_values_only_gradient_boundary(dim, k, duplicates):
    """tests/test_gradient_boundaries.py:104-143: with pos, the displacement
    and values all requiring gradients, the output differentiates in values
    only; indices, distances and neighbour positions carry no gradient.
    Exact hits (head 0 sits on its point; duplicated points) are included."""
    g = torch.Generator().manual_seed(40 + dim)
    n = 16
    base = torch.rand((2, n, dim), generator=g)
    if duplicates:
        base[:, 8:] = base[:, :8]
    pos = base.to(DEV).requires_grad_(True)
    disp = torch.zeros((2, n, 3, dim), device=DEV)
    disp[:, :, 1, 0] = 0.02
    disp[:, :, 2, 0] = torch.linspace(-0.03, 0.03, n, device=DEV)
    rho = disp.requires_grad_(True)
    q = (pos[:, :, None, :] + rho).contiguous()
    q.retain_grad()
    feats = torch.stack([base[..., 0], base[..., 1], base[..., 0].square() + 0.25,
                         torch.sin(4 * base[..., 0]), torch.cos(3 * base[..., 1])], -1)
    values = feats[:, :, None, :].repeat(1, 1, 3, 1).contiguous().to(DEV).requires_grad_(True)

    out = tb.interpolate_displaced(pos, q, values, k)
    idx, d2, rows = tb.query_displaced_knn(pos, q, k)
    assert out.shape == values.shape and torch.isfinite(out).all()
    assert (d2[:, :, 0] <= 1e-12).any()
    assert not idx.requires_grad and not d2.requires_grad and not rows.requires_grad
    with torch.no_grad():  # the fused kernel gives the same values
        assert torch.equal(tb.interpolate_displaced(pos, q, values, k), out.detach())
    out.square().mean().backward()
    assert values.grad is not None and torch.isfinite(values.grad).all() and values.grad.abs().sum() > 0
    assert pos.grad is None and rho.grad is None and q.grad is None
