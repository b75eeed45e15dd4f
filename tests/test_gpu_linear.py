"""GPU parity of the attention projections on the MFMA kernels (linear.py).

rv_linear_fwd / rv_linear_dx / rv_linear_dw against the fp64 contraction of
the same fp16 operands, within the fp32-accumulation bound of
tests/gemm_bounds.py; FusedLinear against autocast's F.linear (forward and
both gradients); enable_linear leaves unsupported calls on F.linear.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from gemm_bounds import rel_l2, within_gemm_bound
from reversability_amd import mlp
from reversability_amd._hip import RV_F16, RV_F32, _check, _stream, library
from reversability_amd.linear import FusedLinear, enable_linear, linear, supported

pytestmark = pytest.mark.gpu

# (rows, in, out): configs[3] qkv / proj over the batch, a ragged row count,
# configs[4] qkv / proj
SHAPES = [(16896, 256, 768), (16896, 256, 256), (1000, 256, 768), (32768, 1024, 3072),
          (32768, 1024, 1024)]


def _data(rows, in_f, out_f, dev, seed=7):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, in_f, generator=g).half().to(dev)
    w = (0.02 * torch.randn(out_f, in_f, generator=g)).to(dev)
    dy = torch.randn(rows, out_f, generator=g).half().to(dev)
    return x, w, dy


@pytest.mark.parametrize("rows,in_f,out_f", SHAPES)
def test_linear_kernels_vs_fp64(cuda_device, rows, in_f, out_f):
    x, w, dy = _data(rows, in_f, out_f, cuda_device)
    w16 = mlp.cast_f16(w)
    lib = library()
    y = torch.empty(rows, out_f, device=cuda_device, dtype=torch.float16)
    _check(lib.rv_linear_fwd(x.data_ptr(), in_f, w16.data_ptr(), rows, in_f, out_f, y.data_ptr(),
                             _stream(x)), "fwd")
    assert within_gemm_bound(y, x, w16, in_f)
    for dt, code in ((torch.float32, RV_F32), (torch.float16, RV_F16)):
        dx = torch.empty(rows, in_f, device=cuda_device, dtype=dt)
        _check(lib.rv_linear_dx(dy.data_ptr(), w16.data_ptr(), rows, in_f, out_f, dx.data_ptr(),
                                code, _stream(x)), "dx")
        assert within_gemm_bound(dx, dy, w16, out_f, transpose_b=False)
        if dt == torch.float32:
            assert torch.equal(dx, dx.half().float())
    nbytes = lib.rv_linear_dw_workspace_bytes(rows, in_f, out_f)
    ws = torch.empty(max(nbytes, 4) // 4, device=cuda_device)
    dw = torch.empty(out_f, in_f, device=cuda_device)
    _check(lib.rv_linear_dw(dy.data_ptr(), x.data_ptr(), in_f, rows, in_f, out_f, dw.data_ptr(), 0,
                            ws.data_ptr(), nbytes, _stream(x)), "dw")
    assert torch.equal(dw, dw.half().float())
    assert within_gemm_bound(dw, dy.t(), x.t(), rows)
    first = dw.clone()
    _check(lib.rv_linear_dw(dy.data_ptr(), x.data_ptr(), in_f, rows, in_f, out_f, dw.data_ptr(), 1,
                            ws.data_ptr(), nbytes, _stream(x)), "dw acc")
    assert torch.equal(dw, first + first)


@pytest.mark.parametrize("xdtype", [torch.float32, torch.float16])
def test_fused_linear_matches_autocast_linear(cuda_device, xdtype):
    g = torch.Generator().manual_seed(11)
    x = torch.randn(33, 512, 256, generator=g).to(cuda_device).to(xdtype)
    w = (0.02 * torch.randn(768, 256, generator=g)).to(cuda_device)
    gy = torch.randn(33, 512, 768, generator=g).half().to(cuda_device)
    xa, wa = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    xb, wb = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.float16):
        assert supported(xb, wb, None)
        ya = F.linear(xa, wa)
        yb = FusedLinear.apply(xb, wb)
    assert ya.dtype == yb.dtype == torch.float16 and yb.shape == ya.shape
    ya.backward(gy)
    yb.backward(gy)
    assert xb.grad.dtype == xdtype and wb.grad.dtype == torch.float32
    assert rel_l2(yb, ya) < 1e-3
    assert rel_l2(xb.grad, xa.grad) < 1e-3
    assert rel_l2(wb.grad, wa.grad) < 1e-3


def test_enable_linear_falls_back_outside_fp16_autocast(cuda_device):
    from reversability_amd import build_model
    torch.manual_seed(0)
    model = build_model({"model": {"vocab_size": 97, "max_sequence_length": 32, "n_layers": 1,
                                   "n_heads": 8, "d_model": 256, "d_ff": 1024},
                         "method": "midpoint"}).to(cuda_device)
    enable_linear(model)
    x = torch.randn(2, 32, 256, device=cuda_device)
    layer = model.blocks[0].attn.qkv
    # no autocast: plain fp32 F.linear
    assert torch.equal(layer(x), F.linear(x, layer.weight))
    with torch.autocast("cuda", dtype=torch.bfloat16):
        assert not supported(x, layer.weight, None)
        assert layer(x).dtype == torch.bfloat16
    with torch.autocast("cuda", dtype=torch.float16):
        assert supported(x, layer.weight, None)
        assert linear(x, layer.weight).dtype == torch.float16
