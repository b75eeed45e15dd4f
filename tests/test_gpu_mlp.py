"""GPU parity of the MFMA MLP projections (reversability_amd.mlp).

Each GEMM output is compared with the same contraction accumulated in fp64 on
the fp16-rounded operands (the values autocast feeds the GEMM).  Any GEMM that
accumulates in fp32 -- MFMA here, cuBLAS in the reference -- may differ from
that truth by the fp32 accumulation bound K * 2^-24 * sum_k |a_k b_k| before
its final fp16 rounding, so the bar per element is

    |out - truth| <= ulp_fp16(truth) + K * 2^-24 * sum_k |a_k b_k|,

plus relative-L2 agreement (1e-3).  The SwiGLU parts are checked against the
CPU oracle applied to the kernel's own pre-activations.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from reversability_amd import mlp

pytestmark = pytest.mark.gpu


def ulps(actual: torch.Tensor, expected: torch.Tensor) -> torch.Tensor:
    e = expected.float()
    ulp = torch.from_numpy(np.spacing(np.abs(e.cpu().numpy()).astype(np.float16)).astype(np.float32))
    return (actual.float().cpu() - e.cpu()).abs() / ulp


def within_gemm_bound(out, a, b, k, transpose_b=True):
    """out vs fp64 truth of a @ b^T (or a @ b) with the bound in the module docstring."""
    a64, b64 = a.double().cpu(), b.double().cpu()
    bt = b64.t() if transpose_b else b64
    truth = a64 @ bt
    scale = a64.abs() @ bt.abs()
    ulp = torch.from_numpy(np.spacing(np.abs(truth.numpy()).astype(np.float16)).astype(np.float64))
    err = (out.double().cpu() - truth).abs()
    bound = ulp + k * 2.0 ** -24 * scale
    worst = float((err / bound).max())
    print(f"  worst error / bound = {worst:.3f}, rel_l2 = {rel_l2(out, truth):.2e}", flush=True)
    return worst <= 1.0 and rel_l2(out, truth) < 1e-3


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def weights(d, f, dev, seed=1337):
    g = torch.Generator().manual_seed(seed)
    up = 0.02 * torch.randn(2 * f, d, generator=g)
    down = 0.02 / 14 ** 0.5 * torch.randn(d, f, generator=g)
    return up.to(dev), down.to(dev)


SHAPES = [(8192, 256, 1024), (6656, 256, 1024), (17, 256, 1024), (1000, 1024, 4096)]


@pytest.mark.parametrize("rows,d,f", SHAPES)
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16])
def test_up_swiglu(cuda_device, rows, d, f, xdt):
    up, _ = weights(d, f, cuda_device)
    x = torch.randn(rows, d, generator=torch.Generator().manual_seed(1), dtype=torch.float32).to(cuda_device).to(xdt)
    o, u = mlp.up_swiglu(x, up, keep_u=True)
    assert within_gemm_bound(u, x.half(), up.half(), d)
    u_ref = (x.half().float() @ up.half().float().t()).half()
    o_ref = torch.from_numpy(oracle.swiglu_fwd(u_ref.cpu().numpy()))
    assert rel_l2(o, o_ref) < 2e-3
    # given the kernel's own u, o is the SwiGLU of it (same epilogue rounding)
    o_own = torch.from_numpy(oracle.swiglu_fwd(u.cpu().numpy()))
    assert float(ulps(o, o_own).max()) <= 2.0
    o2, _ = mlp.up_swiglu(x, up)
    assert torch.equal(o, o2)  # deterministic, u output optional


@pytest.mark.parametrize("rows,d,f", SHAPES)
def test_down(cuda_device, rows, d, f):
    _, down = weights(d, f, cuda_device)
    o = (0.5 * torch.randn(rows, f, generator=torch.Generator().manual_seed(2))).half().to(cuda_device)
    y = torch.empty(rows, d, device=cuda_device, dtype=torch.float16)
    mlp.down(o, down, y)
    assert within_gemm_bound(y, o, down.half(), f)


@pytest.mark.parametrize("rows,d,f", SHAPES)
def test_dgate(cuda_device, rows, d, f):
    up, down = weights(d, f, cuda_device)
    g = torch.Generator().manual_seed(3)
    dy = torch.randn(rows, d, generator=g).half().to(cuda_device)
    u = torch.randn(rows, 2 * f, generator=g).half().to(cuda_device)
    du = mlp.dgate(dy, down, u)
    d_o = (dy.float() @ down.half().float()).half()
    du_ref = torch.from_numpy(oracle.swiglu_bwd(u.cpu().numpy(), d_o.cpu().numpy()))
    print(f"  rel_l2 = {rel_l2(du, du_ref):.2e}, >2ulp frac = {float((ulps(du, du_ref) > 2).float().mean()):.2e}")
    assert rel_l2(du, du_ref) < 2e-3
    assert (ulps(du, du_ref) > 2).float().mean() < 0.01


@pytest.mark.parametrize("rows,d,f", SHAPES)
def test_dx(cuda_device, rows, d, f):
    up, _ = weights(d, f, cuda_device)
    du = (0.3 * torch.randn(rows, 2 * f, generator=torch.Generator().manual_seed(4))).half().to(cuda_device)
    dx = torch.empty(rows, d, device=cuda_device)
    mlp.dx(du, up, dx)
    assert dx.dtype == torch.float32
    assert torch.equal(dx, dx.half().float())  # an fp16 value widened
    assert within_gemm_bound(dx, du, up.half(), 2 * f, transpose_b=False)


@pytest.mark.parametrize("rows,d,f", SHAPES)
def test_wgrad_and_accumulate(cuda_device, rows, d, f):
    g = torch.Generator().manual_seed(5)
    dy = torch.randn(rows, d, generator=g).half().to(cuda_device)
    o = torch.randn(rows, f, generator=g).half().to(cuda_device)
    du = (0.3 * torch.randn(rows, 2 * f, generator=g)).half().to(cuda_device)
    x = torch.randn(rows, d, generator=g).to(cuda_device)
    ddown = torch.empty(d, f, device=cuda_device)
    dup = torch.empty(2 * f, d, device=cuda_device)
    mlp.wgrad(dy, o, du, x, ddown, dup, accumulate=False)
    assert within_gemm_bound(ddown, dy.t(), o.t(), rows)
    assert within_gemm_bound(dup, du.t(), x.half().t(), rows)
    first = (ddown.clone(), dup.clone())
    mlp.wgrad(dy, o, du, x, ddown, dup, accumulate=True)
    assert torch.equal(ddown, first[0] + first[0]) and torch.equal(dup, first[1] + first[1])
