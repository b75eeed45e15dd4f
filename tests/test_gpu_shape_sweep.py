"""A seeded sweep of row counts and widths through the bandwidth kernels.

The shapes are drawn once, from a fixed seed: widths anywhere in 1..4096
(half of them from the widths where the kernels change layout: 64, 128, 256,
512, 1024, 2048, 4096 and their neighbours) and row counts log-uniform in
1..70000, so the sweep crosses every launch plan (16-lane groups, four-row
groups per block from 4 to 8, wide rows, the scalar path, the batched
dweight reduce) at sizes the fixed-shape tests do not pick.  Bars as in
test_gpu_kernels: the CPU oracle within 1e-5 of scale for fp32 RMSNorm, 2
fp16 ulps (on under 1% of elements) for SwiGLU, and bit equality for the
fused norms against their compositions.
"""
from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch

import oracle
from reversability_amd._hip import ops

pytestmark = pytest.mark.gpu
EPS = float(torch.finfo(torch.float32).eps)
EDGE_WIDTHS = [4, 8, 12, 64, 100, 128, 132, 252, 256, 260, 384, 512, 516, 1000, 1020, 1024,
               1028, 2048, 2052, 4092, 4096]


def _shapes(seed: int, count: int, max_elems: int, vec_only: bool):
    rng = random.Random(seed)
    out = []
    while len(out) < count:
        width = rng.choice(EDGE_WIDTHS) if rng.random() < 0.5 else rng.randrange(1, 4097)
        if vec_only and width % 4:
            continue
        rows = max(1, int(math.exp(rng.uniform(0, math.log(70000)))))
        if rows * width <= max_elems:
            out.append((rows, width))
    return out


def _rel_max(a: np.ndarray, b: np.ndarray) -> float:
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def _fp16_ulps(a: np.ndarray, b: np.ndarray):
    """Largest distance in fp16 ulps and the fraction of elements that differ."""
    ai = a.view(np.int16).astype(np.int32)
    bi = b.view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    d = np.abs(ai - bi)
    return int(d.max()), float((d > 0).mean())


@pytest.mark.parametrize("rows,width", _shapes(7, 24, 3_000_000, False))
def test_rmsnorm_sweep_matches_oracle(cuda_device, rows, width):
    g = torch.Generator().manual_seed(rows * 4099 + width)
    x = torch.randn(rows, width, generator=g)
    w = 1 + 0.02 * torch.randn(width, generator=g)
    dy = torch.randn(rows, width, generator=g)
    y, rstd = ops.rmsnorm_fwd(x.to(cuda_device), w.to(cuda_device), EPS)
    dx, dw = ops.rmsnorm_bwd(x.to(cuda_device), w.to(cuda_device), dy.to(cuda_device), rstd)
    oy, orstd = oracle.rmsnorm_fwd(x.numpy(), w.numpy(), EPS)
    odx, odw = oracle.rmsnorm_bwd(x.numpy(), w.numpy(), dy.numpy(), EPS)
    for got, want in ((y, oy), (rstd, orstd), (dx, odx), (dw, odw)):
        assert _rel_max(got.cpu().numpy(), want) <= 1e-5


@pytest.mark.parametrize("rows,width", _shapes(11, 16, 3_000_000, True))
def test_accumulating_backward_sweep(cuda_device, rows, width):
    """fp16 incoming gradient, dh and the fp16 copy: dx = the plain backward's
    dx + dh and dx16 its cast, bit for bit; dweight within fp32 summation
    error (the accumulating backward may sum its rows in another order)."""
    g = torch.Generator().manual_seed(rows * 4099 + width + 1)
    x = torch.randn(rows, width, generator=g).to(cuda_device)
    w = (1 + 0.02 * torch.randn(width, generator=g)).to(cuda_device)
    dy = torch.randn(rows, width, generator=g).half().to(cuda_device)
    dh = torch.randn(rows, width, generator=g).to(cuda_device)
    _, rstd = ops.rmsnorm_fwd(x, w, EPS)
    dx_plain, dw_plain = ops.rmsnorm_bwd(x, w, dy, rstd)
    dx, dx16, dw = ops.rmsnorm_bwd_acc(x, w, dy, rstd, dh, True)
    assert torch.equal(dx, dx_plain + dh)
    assert torch.equal(dx16, (dx_plain + dh).half())
    assert float((dw - dw_plain).abs().max()) <= 1e-5 * float(dw_plain.abs().max())


@pytest.mark.parametrize("rows,width", _shapes(23, 16, 3_000_000, True))
def test_fused_norms_sweep_match_compositions(cuda_device, rows, width):
    """sub + norm (with and without the re-add), add + norm and midpoint
    update + norm against the residual kernel followed by the fp16 norm."""
    g = torch.Generator().manual_seed(rows * 4099 + width + 2)
    x = torch.randn(rows, width, generator=g).to(cuda_device)
    f = torch.randn(rows, width, generator=g).half().to(cuda_device)
    m = torch.randn(rows, width, generator=g).half().to(cuda_device)
    w = (1 + 0.02 * torch.randn(width, generator=g)).to(cuda_device)
    d_ref = ops.residual_axpy(x, f, -1)
    y_ref, r_ref = ops.rmsnorm_fwd(d_ref, w, EPS, True)
    d, h, y, r = ops.sub_rmsnorm_fwd16(x, f, w, EPS, False)
    assert torch.equal(d, d_ref) and torch.equal(y, y_ref) and torch.equal(r, r_ref)
    h_ref = ops.residual_axpy(d_ref, f, 1)
    yh_ref, rh_ref = ops.rmsnorm_fwd(h_ref, w, EPS, True)
    h_add, y_add, r_add = ops.add_rmsnorm_fwd16(d_ref, f, w, EPS)
    assert torch.equal(h_add, h_ref) and torch.equal(y_add, yh_ref) and torch.equal(r_add, rh_ref)
    d2, h2, y2, r2 = ops.sub_rmsnorm_fwd16(x, f, w, EPS, True)
    assert torch.equal(d2, d_ref) and torch.equal(h2, h_ref)
    assert torch.equal(y2, yh_ref) and torch.equal(r2, rh_ref)
    scale, sign = (0.5, -1) if (rows + width) % 2 else (0.25, 1)
    o_ref = ops.midpoint_update(x, f, m, scale, sign)
    ym_ref, rm_ref = ops.rmsnorm_fwd(o_ref, w, EPS, True)
    o, ym, rm = ops.midpoint_rmsnorm_fwd16(x, f, m, w, EPS, scale, sign)
    assert torch.equal(o, o_ref) and torch.equal(ym, ym_ref) and torch.equal(rm, rm_ref)


@pytest.mark.parametrize("rows,width", _shapes(57, 24, 2_000_000, False))
def test_swiglu_sweep_matches_oracle(cuda_device, rows, width):
    half = max(1, width // 2)
    g = torch.Generator().manual_seed(rows * 4099 + width + 3)
    u = torch.randn(rows, 2 * half, generator=g).half()
    dy = torch.randn(rows, half, generator=g).half()
    o = ops.swiglu_fwd(u.to(cuda_device)).cpu().numpy()
    du = ops.swiglu_bwd(u.to(cuda_device), dy.to(cuda_device)).cpu().numpy()
    for got, want in ((o, oracle.swiglu_fwd(u.numpy())),
                      (du, oracle.swiglu_bwd(u.numpy(), dy.numpy()))):
        ulps, frac = _fp16_ulps(got, want)
        assert ulps <= 2 and frac < 0.01, (ulps, frac)
