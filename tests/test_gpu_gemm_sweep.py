"""A seeded sweep of the MFMA GEMM entry points over shapes the fixed-shape
tests do not pick: model widths 128..1280 and hidden widths 128..4096 (any
multiple of 128, so tiles of 128 columns where 256 do not divide), row counts
from 1 to 40000.  Each product against the fp64 contraction of the same fp16
operands within the fp32-accumulation bound of tests/gemm_bounds.py; the
SwiGLU epilogues against the oracle on the kernel's own pre-activations.
"""
from __future__ import annotations

import math
import random

import numpy as np
import pytest
import torch

import oracle
from gemm_bounds import rel_l2, within_gemm_bound
from reversability_amd import mlp
from reversability_amd._hip import RV_F16, _check, _stream, library

pytestmark = pytest.mark.gpu


def _mlp_shapes(seed: int, count: int):
    rng = random.Random(seed)
    return [(max(1, int(math.exp(rng.uniform(0, math.log(20000))))),
             rng.choice([128, 256, 384, 512, 768, 1024, 1280]),
             rng.choice([128, 256, 384, 640, 1024, 1536, 2048, 4096])) for _ in range(count)]


def _linear_shapes(seed: int, count: int):
    rng = random.Random(seed)
    return [(max(1, int(math.exp(rng.uniform(0, math.log(40000))))),
             rng.choice([128, 256, 512, 768, 1024, 2048]),
             rng.choice([128, 256, 384, 768, 1024, 3072])) for _ in range(count)]


def _ulps(actual: torch.Tensor, expected: torch.Tensor) -> torch.Tensor:
    e = expected.float()
    ulp = torch.from_numpy(np.spacing(np.abs(e.cpu().numpy()).astype(np.float16))
                           .astype(np.float32))
    return (actual.float().cpu() - e.cpu()).abs() / ulp


@pytest.mark.parametrize("rows,d,f", _mlp_shapes(5, 10))
def test_mlp_gemms_sweep(cuda_device, rows, d, f):
    g = torch.Generator().manual_seed(rows * 7 + d * 3 + f)
    up = (0.02 * torch.randn(2 * f, d, generator=g)).to(cuda_device)
    down = (0.02 * torch.randn(d, f, generator=g)).to(cuda_device)
    x16 = mlp.cast_f16(torch.randn(rows, d, generator=g).to(cuda_device))
    up16, down16 = mlp.cast_f16(up), mlp.cast_f16(down)
    o, u = mlp.up_swiglu(x16, up16, keep_u=True)
    assert within_gemm_bound(u, x16, up16, d)
    assert float(_ulps(o, torch.from_numpy(oracle.swiglu_fwd(u.cpu().numpy()))).max()) <= 2.0
    y = torch.empty(rows, d, device=cuda_device, dtype=torch.float16)
    mlp.down(o, down16, y)
    assert within_gemm_bound(y, o, down16, f)
    dy = torch.randn(rows, d, generator=g).half().to(cuda_device)
    du = mlp.dgate(dy, down16, u)
    d_o = (dy.float() @ down16.float()).half()
    du_ref = torch.from_numpy(oracle.swiglu_bwd(u.cpu().numpy(), d_o.cpu().numpy()))
    assert rel_l2(du.cpu(), du_ref) < 2e-3
    assert float((_ulps(du, du_ref) > 2).float().mean()) < 0.01
    dx = torch.empty(rows, d, device=cuda_device)
    mlp.dx(du, up16, dx)
    assert within_gemm_bound(dx, du, up16, 2 * f, transpose_b=False)
    ddown = torch.empty(d, f, device=cuda_device)
    dup = torch.empty(2 * f, d, device=cuda_device)
    mlp.wgrad(dy, o, du, x16, ddown, dup, accumulate=False)
    assert within_gemm_bound(ddown, dy.t(), o.t(), rows)
    assert within_gemm_bound(dup, du.t(), x16.t(), rows)


@pytest.mark.parametrize("rows,in_f,out_f", _linear_shapes(7, 10))
def test_linear_gemms_sweep(cuda_device, rows, in_f, out_f):
    g = torch.Generator().manual_seed(rows * 7 + in_f * 3 + out_f)
    x = torch.randn(rows, in_f, generator=g).half().to(cuda_device)
    w16 = mlp.cast_f16((0.02 * torch.randn(out_f, in_f, generator=g)).to(cuda_device))
    dy = torch.randn(rows, out_f, generator=g).half().to(cuda_device)
    lib = library()
    y = torch.empty(rows, out_f, device=cuda_device, dtype=torch.float16)
    _check(lib.rv_linear_fwd(x.data_ptr(), in_f, w16.data_ptr(), rows, in_f, out_f, y.data_ptr(),
                             _stream(x)), "rv_linear_fwd")
    assert within_gemm_bound(y, x, w16, in_f)
    dx = torch.empty(rows, in_f, device=cuda_device, dtype=torch.float16)
    _check(lib.rv_linear_dx(dy.data_ptr(), w16.data_ptr(), rows, in_f, out_f, dx.data_ptr(),
                            RV_F16, _stream(x)), "rv_linear_dx")
    assert within_gemm_bound(dx, dy, w16, out_f, transpose_b=False)
    nbytes = lib.rv_linear_dw_workspace_bytes(rows, in_f, out_f)
    ws = torch.empty(max(nbytes, 4) // 4, device=cuda_device)
    dw = torch.empty(out_f, in_f, device=cuda_device)
    _check(lib.rv_linear_dw(dy.data_ptr(), x.data_ptr(), in_f, rows, in_f, out_f, dw.data_ptr(),
                            0, ws.data_ptr(), nbytes, _stream(x)), "rv_linear_dw")
    assert within_gemm_bound(dw, dy.t(), x.t(), rows)
