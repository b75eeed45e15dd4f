"""GPU parity of the MFMA MLP projections (reversability_amd.mlp).

Each GEMM output is compared with the same contraction accumulated in fp64 on
the fp16-rounded operands (the values autocast feeds the GEMM).  Any GEMM that
accumulates in fp32 -- MFMA here, cuBLAS in the reference -- may differ from
that truth by the fp32 accumulation bound K * 2^-24 * sum_k |a_k b_k| before
its final fp16 rounding, so the bar per element is

    |out - truth| <= ulp_fp16(truth) + K * 2^-24 * sum_k |a_k b_k|,

plus relative-L2 agreement (1e-3).  The SwiGLU parts are checked against the
CPU oracle applied to the kernel's own pre-activations.  The bound is in
tests/gemm_bounds.py.

The activation GEMMs take the fastest tile shape measured on their first call;
test_every_tile_shape_gives_identical_bits forces each shape in turn
(rv_gemm_force_shape) so that every shape serves every epilogue, and the
weight gradients take both the direct-accumulate and the split-K path; the
8192 x 1024 x 4096 case is one configs[4] token tile.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from gemm_bounds import rel_l2, within_gemm_bound
from reversability_amd import mlp

pytestmark = pytest.mark.gpu


def ulps(actual: torch.Tensor, expected: torch.Tensor) -> torch.Tensor:
    e = expected.float()
    ulp = torch.from_numpy(np.spacing(np.abs(e.cpu().numpy()).astype(np.float16)).astype(np.float32))
    return (actual.float().cpu() - e.cpu()).abs() / ulp


def weights(d, f, dev, seed=1337):
    g = torch.Generator().manual_seed(seed)
    up = 0.02 * torch.randn(2 * f, d, generator=g)
    down = 0.02 / 14 ** 0.5 * torch.randn(d, f, generator=g)
    return up.to(dev), down.to(dev)


SHAPES = [(8192, 256, 1024), (6656, 256, 1024), (17, 256, 1024), (1000, 1024, 4096),
          (8192, 1024, 4096), (16384, 256, 1024), (16384, 1024, 4096)]


def test_cast_f16_matches_torch(cuda_device):
    g = torch.Generator().manual_seed(9)
    for n in (1, 7, 8, 4096 + 3, 1 << 20):
        x = (torch.randn(n, generator=g) * 1e3).to(cuda_device)
        x[: min(n, 4)] = torch.tensor([65520.0, -65504.0, 6e-8, float("nan")][: min(n, 4)])
        y = mlp.cast_f16(x)
        ref = x.half()
        assert torch.equal(torch.isnan(y), torch.isnan(ref))
        keep = ~torch.isnan(ref)
        assert torch.equal(y[keep], ref[keep]), n


@pytest.mark.parametrize("rows,d,f", SHAPES)
def test_up_swiglu(cuda_device, rows, d, f):
    up, _ = weights(d, f, cuda_device)
    x = torch.randn(rows, d, generator=torch.Generator().manual_seed(1)).to(cuda_device)
    x16, up16 = mlp.cast_f16(x), mlp.cast_f16(up)
    o, u = mlp.up_swiglu(x16, up16, keep_u=True)
    assert within_gemm_bound(u, x16, up16, d)
    u_ref = (x16.float() @ up16.float().t()).half()
    o_ref = torch.from_numpy(oracle.swiglu_fwd(u_ref.cpu().numpy()))
    assert rel_l2(o.cpu(), o_ref) < 2e-3
    # given the kernel's own u, o is the SwiGLU of it (same epilogue rounding)
    o_own = torch.from_numpy(oracle.swiglu_fwd(u.cpu().numpy()))
    assert float(ulps(o, o_own).max()) <= 2.0
    o2, _ = mlp.up_swiglu(x16, up16)
    assert torch.equal(o, o2)  # deterministic, u output optional


@pytest.mark.parametrize("rows,d,f", SHAPES)
def test_down(cuda_device, rows, d, f):
    _, down = weights(d, f, cuda_device)
    o = (0.5 * torch.randn(rows, f, generator=torch.Generator().manual_seed(2))).half().to(cuda_device)
    y = torch.empty(rows, d, device=cuda_device, dtype=torch.float16)
    down16 = mlp.cast_f16(down)
    mlp.down(o, down16, y)
    assert within_gemm_bound(y, o, down16, f)


@pytest.mark.parametrize("rows,d,f", SHAPES)
def test_dgate(cuda_device, rows, d, f):
    _, down = weights(d, f, cuda_device)
    g = torch.Generator().manual_seed(3)
    dy = torch.randn(rows, d, generator=g).half().to(cuda_device)
    u = torch.randn(rows, 2 * f, generator=g).half().to(cuda_device)
    down16 = mlp.cast_f16(down)
    du = mlp.dgate(dy, down16, u)
    d_o = (dy.float() @ down16.float()).half()
    du_ref = torch.from_numpy(oracle.swiglu_bwd(u.cpu().numpy(), d_o.cpu().numpy()))
    frac = float((ulps(du, du_ref) > 2).float().mean())
    print(f"  rel_l2 = {rel_l2(du.cpu(), du_ref):.2e}, >2ulp frac = {frac:.2e}")
    assert rel_l2(du.cpu(), du_ref) < 2e-3
    assert frac < 0.01


@pytest.mark.parametrize("rows,d,f", SHAPES)
def test_dx(cuda_device, rows, d, f):
    up, _ = weights(d, f, cuda_device)
    du = (0.3 * torch.randn(rows, 2 * f, generator=torch.Generator().manual_seed(4))).half().to(cuda_device)
    dx = torch.empty(rows, d, device=cuda_device)
    up16 = mlp.cast_f16(up)
    mlp.dx(du, up16, dx)
    assert dx.dtype == torch.float32
    assert torch.equal(dx, dx.half().float())  # an fp16 value widened
    assert within_gemm_bound(dx, du, up16, 2 * f, transpose_b=False)


@pytest.mark.parametrize("rows,d,f", SHAPES)
def test_wgrad_and_accumulate(cuda_device, rows, d, f):
    g = torch.Generator().manual_seed(5)
    dy = torch.randn(rows, d, generator=g).half().to(cuda_device)
    o = torch.randn(rows, f, generator=g).half().to(cuda_device)
    du = (0.3 * torch.randn(rows, 2 * f, generator=g)).half().to(cuda_device)
    x16 = torch.randn(rows, d, generator=g).half().to(cuda_device)
    ddown = torch.empty(d, f, device=cuda_device)
    dup = torch.empty(2 * f, d, device=cuda_device)
    mlp.wgrad(dy, o, du, x16, ddown, dup, accumulate=False)
    assert torch.equal(ddown, ddown.half().float()) and torch.equal(dup, dup.half().float())
    assert within_gemm_bound(ddown, dy.t(), o.t(), rows)
    assert within_gemm_bound(dup, du.t(), x16.t(), rows)
    first = (ddown.clone(), dup.clone())
    mlp.wgrad(dy, o, du, x16, ddown, dup, accumulate=True)
    assert torch.equal(ddown, first[0] + first[0]) and torch.equal(dup, first[1] + first[1])


def test_rejects_fp32_operands(cuda_device):
    up, down = weights(256, 1024, cuda_device)
    x = torch.randn(64, 256, device=cuda_device)
    with pytest.raises(ValueError, match="fp16"):
        mlp.up_swiglu(x, mlp.cast_f16(up))
    with pytest.raises(ValueError, match="fp16"):
        mlp.up_swiglu(x.half(), up)


@pytest.mark.parametrize("rows,d,f", [(1000, 256, 1024), (2100, 1024, 4096)])
def test_every_tile_shape_gives_identical_bits(cuda_device, rows, d, f):
    """The activation GEMMs sum each output's k blocks in the same order in
    every tile shape (rv_gemm_force_shape; the default picks the fastest), so
    every shape -- 4-wave 256x256 / 128x256 / 128x128 / 64x128 and the 8-wave
    256x256 -- gives the same bits, ragged row tails included; shape 0's
    results also meet the fp64 bound."""
    from reversability_amd._hip import RV_F32, _stream, library
    lib = library()
    up, down = weights(d, f, cuda_device)
    up16, down16 = mlp.cast_f16(up), mlp.cast_f16(down)
    g = torch.Generator().manual_seed(7)
    x16 = torch.randn(rows, d, generator=g).half().to(cuda_device)
    dy = torch.randn(rows, d, generator=g).half().to(cuda_device)
    wq = (0.02 * torch.randn(3 * d, d, generator=g)).half().to(cuda_device)
    gq = torch.randn(rows, 3 * d, generator=g).half().to(cuda_device)

    def run():
        o, u = mlp.up_swiglu(x16, up16, keep_u=True)
        y = mlp.down(o, down16, torch.empty(rows, d, device=cuda_device, dtype=torch.float16))
        du = mlp.dgate(dy, down16, u)
        dx = mlp.dx(du, up16, torch.empty(rows, d, device=cuda_device))
        q = torch.empty(rows, 3 * d, device=cuda_device, dtype=torch.float16)
        assert lib.rv_linear_fwd(x16.data_ptr(), d, wq.data_ptr(), rows, d, 3 * d, q.data_ptr(),
                                 _stream(x16)) == 0
        dq = torch.empty(rows, d, device=cuda_device)
        assert lib.rv_linear_dx(gq.data_ptr(), wq.data_ptr(), rows, d, 3 * d, dq.data_ptr(),
                                RV_F32, _stream(x16)) == 0
        torch.cuda.synchronize()
        return {"o": o, "u": u, "y": y, "du": du, "dx": dx, "q": q, "dq": dq}

    results = []
    try:
        for shape in range(lib.rv_gemm_num_shapes()):
            assert lib.rv_gemm_force_shape(shape) == 0
            results.append(run())
    finally:
        assert lib.rv_gemm_force_shape(-1) == 0
    for shape, res in enumerate(results[1:], 1):
        for k, v in res.items():
            assert torch.equal(v, results[0][k]), (shape, k)
    assert within_gemm_bound(results[0]["q"], x16, wq, d)
    assert lib.rv_gemm_force_shape(lib.rv_gemm_num_shapes()) != 0


def test_dgate_every_shape_repeats(cuda_device):
    """dgate + SwiGLU backward at 8192 x 256 x 1024 (the configuration an
    epilogue variant addressing u through buffer resources once failed in,
    for the tile shapes whose waves own 64 columns) on every tile shape, five
    calls each: identical bits across shapes and calls, and the oracle's bar
    on the kernel's own d_o."""
    from reversability_amd._hip import library
    lib = library()
    rows, d, f = 8192, 256, 1024
    _, down = weights(d, f, cuda_device)
    g = torch.Generator().manual_seed(3)
    dy = torch.randn(rows, d, generator=g).half().to(cuda_device)
    u = torch.randn(rows, 2 * f, generator=g).half().to(cuda_device)
    down16 = mlp.cast_f16(down)
    first = None
    try:
        for shape in range(lib.rv_gemm_num_shapes()):
            assert lib.rv_gemm_force_shape(shape) == 0
            for call in range(5):
                du = mlp.dgate(dy, down16, u)
                torch.cuda.synchronize()
                if first is None:
                    first = du.clone()
                assert torch.equal(du, first), (shape, call)
    finally:
        assert lib.rv_gemm_force_shape(-1) == 0
    d_o = (dy.float() @ down16.float()).half()
    du_ref = torch.from_numpy(oracle.swiglu_bwd(u.cpu().numpy(), d_o.cpu().numpy()))
    assert rel_l2(first.cpu(), du_ref) < 2e-3
    assert float((ulps(first, du_ref) > 2).float().mean()) < 0.01


def test_multi_tensor_cast_and_prefetch(cuda_device):
    """rv_cast_f32_f16_multi equals rv_cast_f32_f16 per tensor, bit for bit
    (ragged sizes, more tensors than one launch takes); prefetch_casts fills
    the weight-cast cache with those values, and cast_weight hands them out."""
    g = torch.Generator().manual_seed(3)
    sizes = [(1,), (7,), (8,), (1001,), (256, 768), (4096, 1024), (33, 65)] * 10
    ws = [(70000 * torch.randn(*s, generator=g)).to(cuda_device) for s in sizes]  # some overflow
    with mlp.weight_cast_cache():
        mlp.prefetch_casts(ws)
        got = [mlp.cast_weight(w) for w in ws]
        cache = mlp._weight_cache
        assert all(cache[id(w)][1] is c for w, c in zip(ws, got))
    for w, c in zip(ws, got):
        ref = mlp.cast_f16(w)
        assert c.shape == w.shape and c.dtype == torch.float16
        assert torch.equal(c.view(torch.int16), ref.view(torch.int16))
    # outside a block it does nothing
    mlp.prefetch_casts(ws)
    assert mlp._weight_cache is None


def test_first_call_under_graph_capture(cuda_device):
    """An activation GEMM whose first call for its shape is made while the
    stream is captured does not tune (tuning synchronises): it takes the rule's
    tile shape, and its replays give the bits of the same call made eagerly
    afterwards (which tunes and may pick another shape: every shape gives the
    same bits).  Replays are checked with eager work and synchronisations
    between them."""
    rows, d, f = 3331, 256, 1024  # a row count no other test uses: a new tuning key
    _, down = weights(d, f, cuda_device, seed=11)
    down16 = mlp.cast_f16(down)
    o = (0.5 * torch.randn(rows, f, generator=torch.Generator().manual_seed(12))).half()
    o = o.to(cuda_device)
    y_graph = torch.empty(rows, d, device=cuda_device, dtype=torch.float16)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream), torch.cuda.graph(graph, stream=stream):
        mlp.down(o, down16, y_graph)
    torch.cuda.current_stream().wait_stream(stream)
    y_eager = mlp.down(o, down16, torch.empty(rows, d, device=cuda_device, dtype=torch.float16))
    torch.cuda.synchronize()
    assert within_gemm_bound(y_eager, o, down16, f)
    for _ in range(3):
        y_graph.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_eager)
        mlp.down(o, down16, torch.empty_like(y_eager))  # eager work between replays
