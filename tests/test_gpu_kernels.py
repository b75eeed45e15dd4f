"""GPU parity of the fused kernels against the CPU oracle and torch eager.

Tolerances
----------
RMSNorm (FP32): max |gpu - oracle| <= 1e-5 * max |oracle| for y, dx and dw
    (north-star bar "fp32 within max-abs 1e-5 relative to scale"); against
    torch eager F.rms_norm on the GPU the reference's own test tolerances
    (tests/test_optimized_v3.py:82-84: rtol 5e-5, atol 5e-6; dw atol 5e-5).
SwiGLU (FP16 I/O): at most 2 fp16 ulps from the oracle on every element and
    any difference on under 1% of elements.  The sigmoid uses the hardware
    exp2/rcp, whose last fp32 bit can flip the fp16 rounding of the
    intermediate silu (or dy*value) by 1 ulp; the following fp16 product then
    moves by up to 2 ulps of the output when it sits low in its binade.
    Against eager F.silu(g)*v: the reference's rtol = atol = 3e-3
    (tests/test_kernels.py:49-51).  FP32 I/O: 2e-5.
Residual updates: bit-exact against the oracle and against torch's eager
    expression (same IEEE operations and rounding points).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from reversability_amd import _hip
from reversability_amd._hip import ops
from reversability_amd.kernels import FusedSwiGLU
from reversability_amd.kernels_v3 import FusedRMSNorm

pytestmark = pytest.mark.gpu
EPS32 = float(torch.finfo(torch.float32).eps)


def gen(seed=1337):
    return torch.Generator().manual_seed(seed)


def rel_max(a: np.ndarray, b: np.ndarray) -> float:
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


# --------------------------------------------------------------------------
# RMSNorm
# --------------------------------------------------------------------------

RMS_SHAPES = [(3, 23, 256), (14848, 256), (1, 256), (17, 8), (5, 1024), (7, 33), (9, 4096),
              (1000, 512), (4, 100)]


@pytest.mark.parametrize("shape", RMS_SHAPES)
def test_rmsnorm_matches_oracle(cuda_device, shape):
    g = gen()
    x = torch.randn(shape, generator=g)
    w = 1 + 0.02 * torch.randn(shape[-1], generator=g)
    dy = torch.randn(shape, generator=g)
    y, rstd = ops.rmsnorm_fwd(x.to(cuda_device), w.to(cuda_device), EPS32)
    dx, dw = ops.rmsnorm_bwd(x.to(cuda_device), w.to(cuda_device), dy.to(cuda_device), rstd)
    oy, orstd = oracle.rmsnorm_fwd(x.numpy(), w.numpy(), EPS32)
    odx, odw = oracle.rmsnorm_bwd(x.numpy(), w.numpy(), dy.numpy(), EPS32)
    assert rel_max(y.cpu().numpy(), oy) <= 1e-5
    assert rel_max(rstd.cpu().numpy(), orstd) <= 1e-5
    assert rel_max(dx.cpu().numpy(), odx) <= 1e-5
    assert rel_max(dw.cpu().numpy(), odw) <= 1e-5


def test_rmsnorm_golden_vectors(cuda_device):
    data = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "kernels_golden.npz")
    x = torch.from_numpy(data["rms_x"]).to(cuda_device)
    w = torch.from_numpy(data["rms_w"]).to(cuda_device)
    dy = torch.from_numpy(data["rms_dy"]).to(cuda_device)
    y, rstd = ops.rmsnorm_fwd(x, w, float(data["rms_eps"]))
    dx, dw = ops.rmsnorm_bwd(x, w, dy, rstd)
    assert rel_max(y.cpu().numpy(), data["rms_y"]) <= 1e-5
    assert rel_max(dx.cpu().numpy(), data["rms_dx"]) <= 1e-5
    assert rel_max(dw.cpu().numpy(), data["rms_dw"]) <= 1e-5


def test_fused_rmsnorm_autograd_vs_eager(cuda_device):
    # tests/test_optimized_v3.py:73-84 restated
    torch.manual_seed(74)
    x = torch.randn(3, 23, 256, device=cuda_device, requires_grad=True)
    w = torch.randn(256, device=cuda_device, requires_grad=True)
    u = x.detach().clone().requires_grad_(True)
    v = w.detach().clone().requires_grad_(True)
    expected = F.rms_norm(x, (256,), w, eps=EPS32)
    actual = FusedRMSNorm.apply(u, v, EPS32)
    g = torch.randn_like(actual)
    expected.backward(g)
    actual.backward(g)
    torch.testing.assert_close(expected, actual, rtol=5e-5, atol=5e-6)
    torch.testing.assert_close(x.grad, u.grad, rtol=5e-5, atol=5e-6)
    torch.testing.assert_close(w.grad, v.grad, rtol=5e-5, atol=5e-5)


def test_rmsnorm_is_deterministic(cuda_device):
    g = gen(3)
    x = torch.randn(14848, 256, generator=g).to(cuda_device)
    w = torch.randn(256, generator=g).to(cuda_device)
    dy = torch.randn(14848, 256, generator=g).to(cuda_device)
    y1, r1 = ops.rmsnorm_fwd(x, w, EPS32)
    dx1, dw1 = ops.rmsnorm_bwd(x, w, dy, r1)
    y2, r2 = ops.rmsnorm_fwd(x, w, EPS32)
    dx2, dw2 = ops.rmsnorm_bwd(x, w, dy, r2)
    assert torch.equal(y1, y2) and torch.equal(r1, r2)
    assert torch.equal(dx1, dx2) and torch.equal(dw1, dw2)


@pytest.mark.parametrize("shape", [(14848, 256), (32768, 1024), (7, 100), (3, 4096)])
def test_rmsnorm_fp16_operand_paths_bitwise(cuda_device, shape):
    """The fp16-output forward equals the fp32 forward followed by autocast's
    cast, and the fp16-gradient backward equals the fp32 backward on the same
    (widened) gradient -- bit for bit."""
    rows, width = shape
    g = gen(4)
    x = torch.randn(rows, width, generator=g).to(cuda_device)
    w = (1 + 0.02 * torch.randn(width, generator=g)).to(cuda_device)
    dy16 = torch.randn(rows, width, generator=g).half().to(cuda_device)
    y32, r32 = ops.rmsnorm_fwd(x, w, EPS32)
    y16, r16 = ops.rmsnorm_fwd(x, w, EPS32, True)
    assert y16.dtype == torch.float16 and torch.equal(r16, r32)
    assert torch.equal(y16, y32.half())
    dx32, dw32 = ops.rmsnorm_bwd(x, w, dy16.float(), r32)
    dx16, dw16 = ops.rmsnorm_bwd(x, w, dy16, r32)
    assert torch.equal(dx16, dx32) and torch.equal(dw16, dw32)


def test_fused_rmsnorm_fp16_out_under_autocast(cuda_device):
    g = gen(5)
    x = torch.randn(4, 64, 256, generator=g).to(cuda_device).requires_grad_(True)
    w = torch.ones(256, device=cuda_device, requires_grad=True)
    lin = (0.05 * torch.randn(512, 256, generator=g)).to(cuda_device)
    outs = []
    for flag in (False, True):
        x.grad = w.grad = None
        with torch.autocast("cuda", dtype=torch.float16):
            y = FusedRMSNorm.apply(x, w, EPS32, flag)
            assert y.dtype == (torch.float16 if flag else torch.float32)
            z = F.linear(y, lin)
        z.float().square().sum().backward()
        outs.append((z.detach(), x.grad.clone(), w.grad.clone()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    # outside autocast the flag changes nothing
    assert FusedRMSNorm.apply(x.detach(), w.detach(), EPS32, True).dtype == torch.float32


def test_rmsnorm_rejects_cpu_and_dtype(cuda_device):
    with pytest.raises(ValueError, match="CUDA FP32"):
        FusedRMSNorm.apply(torch.ones(3, 8, device=cuda_device, dtype=torch.float16),
                           torch.ones(8, device=cuda_device), 1e-7)
    with pytest.raises(ValueError, match="Contiguous"):
        FusedRMSNorm.apply(torch.ones(8, 3, device=cuda_device).t(), torch.ones(8, device=cuda_device), 1e-7)


def test_add_rmsnorm_matches_oracle(cuda_device):
    g = gen(5)
    x = torch.randn(4096, 256, generator=g)
    f = (0.5 * torch.randn(4096, 256, generator=g)).half()
    w = 1 + 0.02 * torch.randn(256, generator=g)
    h, y, rstd = ops.add_rmsnorm_fwd(x.to(cuda_device), f.to(cuda_device), w.to(cuda_device), EPS32)
    href = x + f  # eager fp32 + fp16 -> fp32
    assert torch.equal(h.cpu(), href)
    oy, _ = oracle.rmsnorm_fwd(href.numpy(), w.numpy(), EPS32)
    assert rel_max(y.cpu().numpy(), oy) <= 1e-5


# --------------------------------------------------------------------------
# SwiGLU
# --------------------------------------------------------------------------

SWIGLU_SHAPES = [(3, 7, 66), (14848, 2048), (4, 8192), (1, 16), (33, 1000), (2, 3, 2050)]


def _ulp_check(actual: np.ndarray, expected: np.ndarray, max_frac=0.01, max_ulp=2):
    a = actual.astype(np.float32)
    e = expected.astype(np.float32)
    diff = np.abs(a - e)
    ulp = np.spacing(np.abs(expected).astype(np.float16)).astype(np.float32)
    assert np.all(diff <= max_ulp * ulp), float((diff / ulp).max())
    assert (diff > 0).mean() <= max_frac, float((diff > 0).mean())


@pytest.mark.parametrize("shape", SWIGLU_SHAPES)
def test_swiglu_fp16_matches_oracle(cuda_device, shape):
    g = gen()
    u = torch.randn(shape, generator=g).half()
    dy = torch.randn((*shape[:-1], shape[-1] // 2), generator=g).half()
    o = ops.swiglu_fwd(u.to(cuda_device))
    du = ops.swiglu_bwd(u.to(cuda_device), dy.to(cuda_device))
    _ulp_check(o.cpu().numpy(), oracle.swiglu_fwd(u.numpy()))
    _ulp_check(du.cpu().numpy(), oracle.swiglu_bwd(u.numpy(), dy.numpy()))


def test_swiglu_golden_vectors(cuda_device):
    data = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "kernels_golden.npz")
    u = torch.from_numpy(data["sw_u"]).to(cuda_device)
    dy = torch.from_numpy(data["sw_dy"]).to(cuda_device)
    _ulp_check(ops.swiglu_fwd(u).cpu().numpy(), data["sw_o"], max_frac=0.02)
    _ulp_check(ops.swiglu_bwd(u, dy).cpu().numpy(), data["sw_du"], max_frac=0.02)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_fused_swiglu_tail_and_backward_vs_eager(cuda_device, dtype):
    # tests/test_kernels.py:37-51 restated
    torch.manual_seed(42)
    a = torch.randn(3, 7, 66, device=cuda_device, dtype=dtype, requires_grad=True)
    b = a.detach().clone().requires_grad_(True)
    gate, value = a.chunk(2, dim=-1)
    expected = F.silu(gate) * value
    actual = FusedSwiGLU.apply(b)
    upstream = torch.randn_like(actual)
    expected.backward(upstream)
    actual.backward(upstream)
    tol = 3e-3 if dtype == torch.float16 else 2e-5
    torch.testing.assert_close(actual, expected, rtol=tol, atol=tol)
    torch.testing.assert_close(b.grad, a.grad, rtol=tol, atol=tol)


def test_swiglu_fp32_matches_oracle(cuda_device):
    g = gen(9)
    u = torch.randn(1000, 512, generator=g)
    dy = torch.randn(1000, 256, generator=g)
    o = ops.swiglu_fwd(u.to(cuda_device)).cpu().numpy()
    du = ops.swiglu_bwd(u.to(cuda_device), dy.to(cuda_device)).cpu().numpy()
    np.testing.assert_allclose(o, oracle.swiglu_fwd(u.numpy()), rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(du, oracle.swiglu_bwd(u.numpy(), dy.numpy()), rtol=2e-5, atol=2e-5)


def test_swiglu_rejects(cuda_device):
    with pytest.raises(ValueError, match="CUDA"):
        FusedSwiGLU.apply(torch.zeros(3, 32, device=cuda_device, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="CUDA"):
        FusedSwiGLU.apply(torch.zeros(3, 31, device=cuda_device, dtype=torch.float16))


def test_swiglu_special_values(cuda_device):
    gte = torch.tensor([0.0, 30.0, -30.0, -100.0, 12.0, float("inf"), float("-inf"), float("nan")])
    val = torch.tensor([1.5, 2.0, 2.0, 3.0, -1.0, 1.0, 1.0, 1.0])
    u = torch.cat([gte, val]).half()[None]
    o = ops.swiglu_fwd(u.to(cuda_device)).cpu()
    ref = (F.silu(gte).half().float() * val).half()
    assert torch.equal(o[0, :5], ref[:5])
    assert o[0, 5] == float("inf") and torch.isnan(o[0, 6]) and torch.isnan(o[0, 7])


# --------------------------------------------------------------------------
# Residual updates
# --------------------------------------------------------------------------

@pytest.mark.parametrize("force", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("h", [0.5, 0.25, 0.3])
@pytest.mark.parametrize("sign", [1, -1])
def test_midpoint_update_bitwise(cuda_device, force, h, sign):
    g = gen(21)
    n = 33 * 512 * 256 + 3  # tail beyond the 4-element groups
    p = torch.randn(n, generator=g)
    a = (0.3 * torch.randn(n, generator=g)).to(force)
    m = (0.3 * torch.randn(n, generator=g)).to(force)
    scale = 2 * h
    out = ops.midpoint_update(p.to(cuda_device), a.to(cuda_device), m.to(cuda_device), scale, sign).cpu()
    eager = p + scale * (a + m) if sign > 0 else p - scale * (a + m)
    assert torch.equal(out, eager)
    dout = torch.randn(n, generator=g)
    da = ops.midpoint_update_bwd(dout.to(cuda_device), scale, sign, force).cpu()
    name = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}[force]
    assert np.array_equal(da.float().numpy(), oracle.midpoint_bwd(dout.numpy(), scale, sign, name))


def test_midpoint_update_fp64_and_unaligned(cuda_device):
    g = gen(22)
    p, a, m = (torch.randn(1003, generator=g, dtype=torch.float64) for _ in range(3))
    out = ops.midpoint_update(p.to(cuda_device), a.to(cuda_device), m.to(cuda_device), 0.5, 1).cpu()
    assert torch.equal(out, p + 0.5 * (a + m))
    # views starting one element in: the kernel falls back to its scalar path
    pb = torch.randn(4097, generator=g)
    ab = torch.randn(4097, generator=g).half()
    mb = torch.randn(4097, generator=g).half()
    dev = [t.to(cuda_device)[1:] for t in (pb, ab, mb)]
    out = ops.midpoint_update(*dev, 1.0, -1).cpu()
    assert torch.equal(out, pb[1:] - 1.0 * (ab[1:] + mb[1:]))


@pytest.mark.parametrize("sign", [1, -1])
def test_residual_axpy_bitwise(cuda_device, sign):
    g = gen(23)
    x = torch.randn(16896 * 256 + 1, generator=g)
    f = torch.randn(16896 * 256 + 1, generator=g).half()
    out = ops.residual_axpy(x.to(cuda_device), f.to(cuda_device), sign).cpu()
    assert np.array_equal(out.numpy(), oracle.euler(x.numpy(), f.numpy(), sign))


@pytest.mark.parametrize("rows,width,f_dtype", [(1000, 256, torch.float16), (777, 1024, torch.float16),
                                                (33, 1024, torch.float32), (5, 4096, torch.float16)])
def test_sub_rmsnorm_matches_composition_bitwise(cuda_device, rows, width, f_dtype):
    """rv_sub_rmsnorm_fwd_f16: d = x - f with the fp16 norm of d (readd off) or
    of h = d + f (readd on) equals rv_residual_axpy(x, f, -1) followed by the
    fp16 RMSNorm (or the fused add + norm of d and f), bit for bit."""
    g = gen(31)
    eps = float(torch.finfo(torch.float32).eps)
    x = torch.randn(rows, width, generator=g).to(cuda_device)
    f = torch.randn(rows, width, generator=g).to(f_dtype).to(cuda_device)
    w = (1 + 0.02 * torch.randn(width, generator=g)).to(cuda_device)
    d_ref = ops.residual_axpy(x, f, -1)
    y_ref, rstd_ref = ops.rmsnorm_fwd(d_ref, w, eps, True)
    d, h, y, rstd = ops.sub_rmsnorm_fwd16(x, f, w, eps, False)
    assert h.numel() == 0
    assert torch.equal(d, d_ref) and torch.equal(y, y_ref) and torch.equal(rstd, rstd_ref)
    h_ref, y2_ref, rstd2_ref = ops.add_rmsnorm_fwd16(d_ref, f, w, eps)
    d2, h2, y2, rstd2 = ops.sub_rmsnorm_fwd16(x, f, w, eps, True)
    assert torch.equal(d2, d_ref) and torch.equal(h2, h_ref)
    assert torch.equal(y2, y2_ref) and torch.equal(rstd2, rstd2_ref)


@pytest.mark.parametrize("rows,width,scale,sign", [(1000, 256, 1.0, 1), (777, 1024, 0.5, -1),
                                                   (33, 256, 0.3, -1), (5, 4096, 0.5, 1)])
def test_midpoint_rmsnorm_matches_composition_bitwise(cuda_device, rows, width, scale, sign):
    """rv_midpoint_rmsnorm_fwd_f16 equals rv_midpoint_update followed by the
    fp16 RMSNorm of its result, bit for bit."""
    g = gen(37)
    eps = float(torch.finfo(torch.float32).eps)
    p = torch.randn(rows, width, generator=g).to(cuda_device)
    a = torch.randn(rows, width, generator=g).half().to(cuda_device)
    m = torch.randn(rows, width, generator=g).half().to(cuda_device)
    w = (1 + 0.02 * torch.randn(width, generator=g)).to(cuda_device)
    out_ref = ops.midpoint_update(p, a, m, scale, sign)
    y_ref, rstd_ref = ops.rmsnorm_fwd(out_ref, w, eps, True)
    out, y, rstd = ops.midpoint_rmsnorm_fwd16(p, a, m, w, eps, scale, sign)
    assert torch.equal(out, out_ref) and torch.equal(y, y_ref) and torch.equal(rstd, rstd_ref)


def test_sub_rmsnorm_rejects(cuda_device):
    lib = _hip.library()
    x = torch.zeros(4, 6, device=cuda_device)
    f = torch.zeros(4, 6, device=cuda_device, dtype=torch.float16)
    w = torch.ones(6, device=cuda_device)
    d, y, r = torch.empty_like(x), torch.empty_like(f), torch.empty(4, device=cuda_device)
    stream = torch.cuda.current_stream().cuda_stream
    # width 6 is not a multiple of 4: the vector-only entry point refuses it
    assert lib.rv_sub_rmsnorm_fwd_f16(x.data_ptr(), f.data_ptr(), _hip.RV_F16, 0, w.data_ptr(),
                                      d.data_ptr(), None, y.data_ptr(), r.data_ptr(), 4, 6,
                                      1e-6, stream) == 3  # RV_ERR_UNSUPPORTED
    # readd needs h
    assert lib.rv_sub_rmsnorm_fwd_f16(x.data_ptr(), f.data_ptr(), _hip.RV_F16, 1, w.data_ptr(),
                                      d.data_ptr(), None, y.data_ptr(), r.data_ptr(), 4, 6,
                                      1e-6, stream) == 1  # RV_ERR_NULL_POINTER


def test_empty_inputs_match_eager(cuda_device):
    """Zero rows through the autograd Functions: the same shapes and gradients
    as eager torch (dweight zero, no kernel launched)."""
    from reversability_amd.residual import euler_step, midpoint_step
    eps = float(torch.finfo(torch.float32).eps)
    x = torch.zeros(0, 256, device=cuda_device, requires_grad=True)
    w = torch.ones(256, device=cuda_device, requires_grad=True)
    y = FusedRMSNorm.apply(x, w, eps)
    assert y.shape == (0, 256)
    y.sum().backward()
    assert x.grad.shape == (0, 256) and torch.equal(w.grad, torch.zeros_like(w))
    for dtype in (torch.float16, torch.float32):
        u = torch.zeros(2, 0, 2048, device=cuda_device, dtype=dtype, requires_grad=True)
        o = FusedSwiGLU.apply(u)
        ref = F.silu(u[..., :1024]) * u[..., 1024:]
        assert o.shape == ref.shape and o.dtype == ref.dtype
        o.sum().backward()
        assert u.grad.shape == u.shape
    p = torch.zeros(0, 256, device=cuda_device)
    f = torch.zeros(0, 256, device=cuda_device, dtype=torch.float16)
    assert euler_step(p, f, +1).shape == (0, 256)
    assert midpoint_step(p, f, f, 0.5, -1).shape == (0, 256)


@pytest.mark.parametrize("sign", [1, -1])
def test_graph_only_residual_steps_have_the_same_gradients(cuda_device, sign):
    """A residual step built with graph_only=True (value not evaluated) back-
    propagates exactly what the evaluated step does, for the Euler and the
    midpoint update, through a downstream op that reads the input too."""
    from reversability_amd.residual import euler_step, midpoint_step
    g = gen(29)
    x = torch.randn(333, 256, generator=g).to(cuda_device)
    a = torch.randn(333, 256, generator=g).half().to(cuda_device)
    m = torch.randn(333, 256, generator=g).half().to(cuda_device)
    dout = torch.randn(333, 256, generator=g).to(cuda_device)

    def grads(step):
        leaves = [t.detach().clone().requires_grad_(True) for t in (x, a, m)]
        out = step(*leaves)
        torch.autograd.backward((out, leaves[0] * 3.0), (dout, dout))
        return [t.grad for t in leaves]

    for build in (lambda gonly: lambda p, f, h: euler_step(p, f + h, sign, graph_only=gonly),
                  lambda gonly: lambda p, f, h: midpoint_step(p, f, h, 0.5, sign,
                                                              graph_only=gonly)):
        for got, ref in zip(grads(build(True)), grads(build(False))):
            assert torch.equal(got, ref)


@pytest.mark.parametrize("rows,width,f_dtype,use_h", [(1000, 256, torch.float16, True),
                                                      (777, 1024, torch.float16, False),
                                                      (777, 1024, torch.float16, True),
                                                      (64, 256, torch.float32, True)])
def test_fused_add_rmsnorm_matches_composition_bitwise(cuda_device, rows, width, f_dtype, use_h):
    """FusedAddRMSNorm = residual add (euler_step) + FusedRMSNorm(fp16 out) +
    autograd's accumulation of h's gradients and the fp16 cast of f's, bit for
    bit: h, y, dx, df, with and without another use of h.  dweight too, except
    where the accumulating backward runs fewer waves per block (width > 256
    with another use of h: 4 instead of 8 at width 1024, to keep its larger
    register tiles unspilled), which sums the same per-row terms in another
    fixed order: there within fp32 summation error."""
    from reversability_amd.kernels_v3 import FusedAddRMSNorm
    from reversability_amd.residual import euler_step
    g = torch.Generator().manual_seed(rows + width)
    x0 = torch.randn(rows, width, generator=g).to(cuda_device)
    f0 = torch.randn(rows, width, generator=g).to(f_dtype).to(cuda_device)
    w0 = (1 + 0.02 * torch.randn(width, generator=g)).to(cuda_device)
    gy = torch.randn(rows, width, generator=g).half().to(cuda_device)
    gh = torch.randn(rows, width, generator=g).to(cuda_device)
    eps = float(torch.finfo(torch.float32).eps)
    outs = []
    for fused in (True, False):
        x, f, w = (t.clone().requires_grad_(True) for t in (x0, f0, w0))
        with torch.autocast("cuda", dtype=torch.float16):
            if fused:
                h, y = FusedAddRMSNorm.apply(x, f, w, eps)
            else:
                h = euler_step(x, f, +1)
                y = FusedRMSNorm.apply(h, w, eps, True)
        assert y.dtype == torch.float16
        loss = (y.float() * gy.float()).sum() + ((h * gh).sum() if use_h else 0)
        loss.backward()
        outs.append((h.detach(), y.detach(), x.grad, f.grad, w.grad))
    for i, (a, b) in enumerate(zip(*outs)):
        assert a.dtype == b.dtype
        if i == 4 and use_h and width > 256:
            assert torch.allclose(a, b, rtol=1e-5, atol=1e-6)
        else:
            assert torch.equal(a, b), i


@pytest.mark.parametrize("rows,width,fp16_out", [(1000, 256, True), (777, 1024, True),
                                                 (300, 256, False)])
def test_rmsnorm_pass_matches_composition(cuda_device, rows, width, fp16_out):
    """FusedRMSNormPass = the norm + autograd's sum of x's two gradients (the
    norm's and the pass-through use's): y, dx bit for bit; dweight too except
    at width > 256 (the accumulating backward's 4 waves per block sum the
    same per-row terms in another fixed order: within fp32 summation error).
    The fp16 copy of dx it hands a ``half_grad`` list is dx's cast, bit for
    bit."""
    from reversability_amd.kernels_v3 import FusedRMSNormPass
    g = torch.Generator().manual_seed(rows * 3 + width)
    x0 = torch.randn(rows, width, generator=g).to(cuda_device)
    w0 = (1 + 0.02 * torch.randn(width, generator=g)).to(cuda_device)
    gy = torch.randn(rows, width, generator=g).to(cuda_device)
    gp = torch.randn(rows, width, generator=g).to(cuda_device)
    eps = float(torch.finfo(torch.float32).eps)
    outs = []
    half: list = []
    for fused in (True, False):
        x, w = x0.clone().requires_grad_(True), w0.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.float16, enabled=fp16_out):
            if fused:
                xp, y = FusedRMSNormPass.apply(x, w, eps, fp16_out, None, half)
            else:
                xp, y = x, FusedRMSNorm.apply(x, w, eps, fp16_out)
        loss = (y.float() * gy).sum() + (xp * gp).sum()
        loss.backward()
        outs.append((y.detach(), x.grad, w.grad))
    (y1, dx1, dw1), (y2, dx2, dw2) = outs
    assert torch.equal(y1, y2) and torch.equal(dx1, dx2)
    assert len(half) == 1 and half[0].dtype == torch.float16
    assert torch.equal(half[0], dx1.half())
    if width > 256:
        assert torch.allclose(dw1, dw2, rtol=1e-5, atol=1e-6)
    else:
        assert torch.equal(dw1, dw2)


@pytest.mark.parametrize("rows,width", [(1000, 256), (300, 1024)])
def test_fused_add_rmsnorm_pass_matches_composition(cuda_device, rows, width):
    """FusedAddRMSNormPass = (x as a second use, FusedRMSNorm(x + f)) with
    autograd's sum of x's gradients and the fp16 cast of f's: y, dx, df bit
    for bit; dweight too at width 256 (at 1024 the accumulating backward's
    fewer waves sum it in another fixed order: within fp32 summation error)."""
    from reversability_amd.kernels_v3 import FusedAddRMSNormPass
    from reversability_amd.residual import euler_step
    g = torch.Generator().manual_seed(rows + 7 * width)
    x0 = torch.randn(rows, width, generator=g).to(cuda_device)
    f0 = torch.randn(rows, width, generator=g).half().to(cuda_device)
    w0 = (1 + 0.02 * torch.randn(width, generator=g)).to(cuda_device)
    gy = torch.randn(rows, width, generator=g).half().to(cuda_device)
    gp = torch.randn(rows, width, generator=g).to(cuda_device)
    eps = float(torch.finfo(torch.float32).eps)
    outs = []
    for fused in (True, False):
        x, f, w = (t.clone().requires_grad_(True) for t in (x0, f0, w0))
        with torch.autocast("cuda", dtype=torch.float16):
            if fused:
                xp, y = FusedAddRMSNormPass.apply(x, f, w, eps)
            else:
                xp, y = x, FusedRMSNorm.apply(euler_step(x, f, +1), w, eps, True)
        ((y.float() * gy.float()).sum() + (xp * gp).sum()).backward()
        outs.append((y.detach(), x.grad, f.grad, w.grad))
    for i, (a, b) in enumerate(zip(*outs)):
        assert a.dtype == b.dtype
        if i == 3 and width > 256:
            assert torch.allclose(a, b, rtol=1e-5, atol=1e-6)
        else:
            assert torch.equal(a, b), i


@pytest.mark.parametrize("width", [256, 1024])
def test_fused_norm_paths_with_unaligned_weight_take_the_unfused_path(cuda_device, width):
    """A norm weight that sits 4 bytes past a 16-byte boundary (a view into a
    shared buffer): the fused fp16-output norm paths (inverse_rms_norm,
    inverse_add_rms_norm, midpoint_rms_norm, add_rms_norm, rms_norm_pass) fall
    back to the unfused composition instead of raising, and give its values."""
    from reversability_amd.kernels_v3 import (add_rms_norm, enable_rmsnorm, inverse_add_rms_norm,
                                              inverse_rms_norm, midpoint_rms_norm, rms_norm_pass)
    g = torch.Generator().manual_seed(31)
    buf = torch.randn(width + 4, generator=g).to(cuda_device)
    norm = torch.nn.RMSNorm(width).to(cuda_device)
    norm.weight = torch.nn.Parameter(buf[1:width + 1])
    assert norm.weight.data_ptr() % 16 != 0
    enable_rmsnorm(norm, fp16_out=True)
    x = torch.randn(64, width, generator=g).to(cuda_device)
    f = torch.randn(64, width, generator=g).to(cuda_device).half()
    m = torch.randn(64, width, generator=g).to(cuda_device).half()
    with torch.autocast("cuda", dtype=torch.float16):
        d, pre = inverse_rms_norm(x, f, norm)
        assert pre is None and torch.equal(d, x - f)
        d, pre = inverse_add_rms_norm(x, f, norm)
        assert pre is None and torch.equal(d, x - f)
        out, pre = midpoint_rms_norm(x, f, m, 1.0, 1, norm)
        assert pre is None
        assert torch.equal(out, x + (f + m) * 1.0)
        h, y = add_rms_norm(x, f, norm)
        assert torch.equal(h, x + f)
        ref = F.rms_norm(h, (width,), norm.weight.detach(), eps=torch.finfo(torch.float32).eps)
        assert (y.float() - ref).abs().max() <= 1e-5 * ref.abs().max() + 1e-3
        leaf = x.clone().requires_grad_(True)
        passed, y2 = rms_norm_pass(leaf, norm)
        (passed.sum() + y2.float().sum()).backward()
    assert torch.isfinite(leaf.grad).all()


@pytest.mark.parametrize("rows,width", [(1, 256), (15, 256), (17, 100), (255, 1020),
                                        (257, 1024), (14848, 256), (32768, 1024), (4097, 1028),
                                        (33, 66), (16896, 256), (20000, 256), (24000, 256),
                                        (30000, 256), (40000, 256), (40001, 132),
                                        (70000, 256)])
def test_rmsnorm_bwd_reduction_repeats(cuda_device, rows, width):
    """The backward's fixed-order dweight reduction over its partial rows (one
    to 547 of them -- beyond 256 the reduce sums them in several batches --
    vector and scalar paths, and at width <= 256 every instantiated group
    count: 4, 5 (16896, 20000 rows), 6 (24000), 8 (30000 and above, 128 rows
    per block)): dx and dw match the oracle, and fifty calls on one workspace
    give the same bits."""
    lib = _hip.library()
    g = torch.Generator().manual_seed(rows * 7 + width)
    x = torch.randn(rows, width, generator=g)
    w = 1 + 0.02 * torch.randn(width, generator=g)
    dy = torch.randn(rows, width, generator=g)
    xd, wd, dyd = x.to(cuda_device), w.to(cuda_device), dy.to(cuda_device)
    _, rstd = ops.rmsnorm_fwd(xd, wd, EPS32)
    nbytes = lib.rv_rmsnorm_bwd_workspace_bytes(rows, width)
    ws = torch.empty(nbytes // 4, device=cuda_device)
    stream = _hip._stream(xd)
    first = None
    for i in range(50):
        dx, dw = torch.empty_like(xd), torch.full_like(wd, float("nan"))
        assert lib.rv_rmsnorm_bwd(xd.data_ptr(), wd.data_ptr(), dyd.data_ptr(), rstd.data_ptr(),
                                  dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), nbytes, rows,
                                  width, stream) == 0
        if first is None:
            first = (dx.clone(), dw.clone())
        else:
            assert torch.equal(dx, first[0]) and torch.equal(dw, first[1]), i
    torch.cuda.synchronize()
    odx, odw = oracle.rmsnorm_bwd(x.numpy(), w.numpy(), dy.numpy(), EPS32)
    for got, ref in ((first[0], odx), (first[1], odw)):
        err = np.abs(got.cpu().numpy().astype(np.float64) - ref).max() / np.abs(ref).max()
        assert err <= 1e-5, err


@pytest.mark.parametrize("nin,nout", [(1, 1), (2, 1), (3, 2)])
@pytest.mark.parametrize("vec,hints", [(1, 0), (2, 3), (8, 1)])
def test_stream_floor_kernel_moves_the_bytes(cuda_device, nin, nout, vec, hints):
    """rv_stream_floor (measurement only): every output vector is the xor of the
    inputs' vectors (output k with k xored into its first word), a ragged size
    included, so the timed kernel really reads and writes every byte."""
    import ctypes
    lib = _hip.library()
    n = 1000 * 4 + 4  # int32 words: 1001 vectors of 16 bytes, not a multiple of the block
    g = torch.Generator().manual_seed(nin * 10 + nout)
    ins = [torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), generator=g, dtype=torch.int32).to(cuda_device)
           for _ in range(nin)]
    outs = [torch.zeros(n, dtype=torch.int32, device=cuda_device) for _ in range(nout)]
    ip = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in ins])
    op = (ctypes.c_void_p * 2)(*[t.data_ptr() for t in outs])
    assert lib.rv_stream_floor(ctypes.cast(ip, ctypes.c_void_p), nin, ctypes.cast(op, ctypes.c_void_p),
                               nout, n * 4, vec, hints, _hip._stream(ins[0])) == 0
    torch.cuda.synchronize()
    ref = ins[0].clone()
    for t in ins[1:]:
        ref ^= t
    for k, o in enumerate(outs):
        expect = ref.clone().view(-1, 4)
        expect[:, 0] ^= k
        assert torch.equal(o.view(-1, 4), expect), k
