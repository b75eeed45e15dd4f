"""GPU parity of the fused cross-entropy (rv_ce_fwd / rv_ce_bwd).

* The reference's own test (tests/test_kernels.py:19-37): 17 x 50257 logits
  with labels at both vocabulary ends, a tile edge and an ignored row, against
  eager F.cross_entropy (fp16 under autocast, and fp32), scaled backward;
  rtol = atol = 2e-3 on the loss, gradient relative L2 < 2e-2 (fp16) /
  2e-5 (fp32), the ignored row's gradient exactly zero.
* Against the CPU oracle: row max bit-exact; log-sum-exp within fp32
  summation-order error; per-row loss within one fp16 ulp (the rounding of
  the log-probability can flip when the fp32 log-sum-exp differs in its last
  bit); the backward, given the kernel's own row statistics, within one ulp
  on every element and identical on > 99%.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from reversability_amd.kernels import TiledCrossEntropy, cross_entropy_sum
from reversability_amd._hip import ops

pytestmark = pytest.mark.gpu

LABELS17 = [0, 1023, 1024, 50256, -100] + list(range(12))


def ulp16(v):
    return np.spacing(np.abs(np.asarray(v, np.float64)).astype(np.float16)).astype(np.float64)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_reference_full_vocabulary_tail_mask_and_scaled_backward(cuda_device, dtype):
    torch.manual_seed(41)
    a = torch.randn(17, 50257, device=cuda_device, dtype=dtype, requires_grad=True)
    b = a.detach().clone().requires_grad_(True)
    y = torch.tensor(LABELS17, device=cuda_device)
    with torch.autocast("cuda", enabled=dtype == torch.float16, dtype=torch.float16):
        expected = F.cross_entropy(a, y, reduction="sum", ignore_index=-100)
    actual = cross_entropy_sum(b, y)
    (expected * .03125).backward()
    (actual * .03125).backward()
    torch.testing.assert_close(actual, expected.float(), rtol=.002, atol=.002)
    relative = (a.grad.float() - b.grad.float()).norm() / a.grad.float().norm()
    assert relative < (.02 if dtype == torch.float16 else 2e-5)
    assert torch.count_nonzero(b.grad[4]) == 0


@pytest.mark.parametrize("rows,cols,dtype", [(1024, 50257, torch.float16), (17, 50257, torch.float32),
                                             (5, 7, torch.float16), (33, 1000, torch.float16),
                                             (9, 4096, torch.float32)])
def test_matches_oracle(cuda_device, rows, cols, dtype):
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = (3 * torch.randn(rows, cols, generator=g)).to(dtype)
    y = torch.randint(0, cols, (rows,), generator=g)
    y[::5] = -100
    xd, yd = x.to(cuda_device), y.to(cuda_device)
    rmax, rlse, loss = ops.ce_fwd(xd, yd, -100)
    omax, olse, oloss = oracle.ce_fwd(x.numpy(), y.numpy())
    assert np.array_equal(rmax.cpu().numpy(), omax)
    assert np.all(np.abs(rlse.cpu().numpy() - olse) <= 2e-6 * np.abs(olse) + 2e-6)
    lg = loss.cpu().numpy()
    if dtype == torch.float16:
        assert np.all(np.abs(lg - oloss) <= ulp16(oloss))
        assert np.mean(lg == oloss) > 0.95
    else:
        assert np.all(np.abs(lg - oloss) <= 1e-5 * np.abs(oloss) + 1e-6)
    grad = torch.tensor([0.75], device=cuda_device)
    dx = ops.ce_bwd(xd, yd, rmax, rlse, grad, -100).cpu()
    odx = oracle.ce_bwd(x.numpy(), y.numpy(), rmax.cpu().numpy(), rlse.cpu().numpy(), 0.75)
    dg, do = dx.numpy().astype(np.float64), odx.astype(np.float64)
    if dtype == torch.float16:
        assert np.all(np.abs(dg - do) <= ulp16(do) + 1e-12)
        assert np.mean(dg == do) > 0.99
    else:
        assert np.all(np.abs(dg - do) <= 1e-5 * np.abs(do) + 1e-9)
    assert torch.count_nonzero(dx[::5]) == 0


def test_deterministic_and_bad_labels(cuda_device):
    x = torch.randn(8, 50257, device=cuda_device).half()
    y = torch.tensor([1, 2, 50257, -1, 5, 6, 7, -100], device=cuda_device)
    a = ops.ce_fwd(x, y, -100)
    b = ops.ce_fwd(x, y, -100)
    # bitwise identical, NaN rows included
    assert all(torch.equal(torch.isnan(u), torch.isnan(v)) and torch.equal(u.nan_to_num(), v.nan_to_num())
               for u, v in zip(a, b))
    loss = a[2].cpu()
    assert torch.isnan(loss[2]) and torch.isnan(loss[3]) and torch.isfinite(loss[[0, 1, 4, 5, 6]]).all()
    assert loss[7] == 0


def test_rejects_cpu_and_bad_inputs(cuda_device):
    with pytest.raises(ValueError, match="CUDA"):
        cross_entropy_sum(torch.zeros(3, 31), torch.tensor([0, 1, -100]))
    x = torch.zeros(3, 31, device=cuda_device, dtype=torch.float16)
    with pytest.raises(ValueError, match="int64"):
        TiledCrossEntropy.apply(x, torch.tensor([0, 1, 2], device=cuda_device, dtype=torch.int32))
    with pytest.raises(ValueError, match="Contiguous"):
        TiledCrossEntropy.apply(x.t(), torch.tensor([0, 1, 2], device=cuda_device))


@pytest.mark.parametrize("rows,d,vocab", [(1000, 256, 50257), (333, 128, 1001), (64, 256, 64),
                                           (64, 64, 70001)])
def test_tied_head_ce_matches_autograd(cuda_device, rows, d, vocab):
    """The padded-stride head + fused CE (forward and backward in one call;
    two passes above 65536 columns) against autograd of autocast F.linear +
    cross_entropy_sum on the same fp16 operands: the same loss and gradients
    up to the GEMMs' fp32 accumulation order (the padded logits run other
    hipBLASLt kernels)."""
    from reversability_amd.kernels import padded_head, tied_head_ce
    g = torch.Generator().manual_seed(5)
    x16 = torch.randn(rows, d, generator=g).half().to(cuda_device)
    w = (0.05 * torch.randn(vocab, d, generator=g)).to(cuda_device)
    labels = torch.randint(0, vocab, (rows,), generator=g).to(cuda_device)
    labels[::7] = -100
    grad = torch.tensor([0.37], device=cuda_device)
    head16 = padded_head(w)
    assert head16.shape[0] % 64 == 0 and torch.equal(head16[vocab:], torch.zeros_like(head16[vocab:]))
    loss, dx16, dw16 = tied_head_ce(x16, head16, vocab, labels, grad)
    xr = x16.clone().requires_grad_(True)
    hr = w.half().requires_grad_(True)
    ref = cross_entropy_sum(torch.nn.functional.linear(xr, hr), labels)
    (ref * 0.37).backward()
    ref = float(ref.detach())
    assert abs(float(loss) - ref) <= 1e-3 * abs(ref)
    assert dx16.shape == (rows, d) and dw16.shape == (vocab, d) and dw16.is_contiguous()
    for got, want in ((dx16, xr.grad), (dw16, hr.grad)):
        assert got.dtype == torch.float16
        rel = float((got.float() - want.float()).norm() / want.float().norm())
        assert rel < 2e-3, rel


def _fused_vs_two_pass(lib, flat, offset, ld, cols, y, grad, in_place):
    """rv_ce_fused on the rows of stride ld starting at flat[offset] (first cols
    used) against rv_ce_fwd followed by rv_ce_bwd on a copy; returns both
    (row max, lse, loss, dlogits).  Copies keep flat's address modulo 16."""
    from reversability_amd._hip import RV_F16, _stream
    rows = y.numel()
    dev = flat.device
    outs = []
    for fused in (True, False):
        xs = flat.clone()
        x = xs[offset:offset + rows * ld]
        st = [torch.full((rows,), 7.0, device=dev) for _ in range(3)]
        d = x if (fused and in_place) else torch.full_like(xs, 3.0)[offset:offset + rows * ld]
        assert (x.data_ptr() - d.data_ptr()) % 16 == 0
        ptrs = [t.data_ptr() for t in st]
        if fused:
            rc = lib.rv_ce_fused(x.data_ptr(), RV_F16, ld, y.data_ptr(), rows, cols, -100,
                                 grad.data_ptr(), *ptrs, d.data_ptr(), _stream(xs))
            assert rc == 0
        else:
            assert lib.rv_ce_fwd(x.data_ptr(), RV_F16, ld, y.data_ptr(), rows, cols, -100,
                                 *ptrs, _stream(xs)) == 0
            assert lib.rv_ce_bwd(x.data_ptr(), RV_F16, ld, y.data_ptr(), ptrs[0], ptrs[1],
                                 grad.data_ptr(), rows, cols, -100, d.data_ptr(),
                                 _stream(xs)) == 0
        torch.cuda.synchronize()
        outs.append((*st, d.view(rows, ld)))
    return outs


def _same_bits(a, b):
    return torch.equal(a.view(torch.int16) if a.dtype == torch.float16 else a.view(torch.int32),
                       b.view(torch.int16) if b.dtype == torch.float16 else b.view(torch.int32))


@pytest.mark.parametrize("rows,cols,ld,offset", [
    (64, 50257, 50304, 0),     # the tied head's padded stride
    (37, 50257, 50257, 0),     # odd stride: every row has a scalar head and tail
    (19, 65536, 65536, 0),     # widest row the registers hold
    (11, 65535, 65536, 3),     # misaligned base, 16 vectors per thread
    (23, 2048, 2051, 5),
    (9, 7, 8, 1),              # no vector part
    (5, 1, 1, 0),
    (256, 3000, 3072, 0),
])
@pytest.mark.parametrize("in_place", [False, True])
def test_fused_matches_two_pass_bitwise(cuda_device, rows, cols, ld, offset, in_place):
    """rv_ce_fused = rv_ce_fwd then rv_ce_bwd, bit for bit (row max, lse,
    loss, every written dlogits element incl. ignored and bad-label rows);
    the padding past cols is left as it was."""
    from reversability_amd._hip import library
    g = torch.Generator().manual_seed(rows + cols)
    flat = (4 * torch.randn(rows * ld + offset, generator=g)).half().to(cuda_device)
    y = torch.randint(0, cols, (rows,), generator=g)
    y[::4] = -100
    if rows > 5:
        y[1], y[2], y[3] = cols - 1, cols, -7   # last column; two bad labels
    y = y.to(cuda_device)
    if rows > 5 and cols > 64:
        # a row spanning the fp16 range: exp(logp) underflows (zero-signed gradients)
        flat[offset + 5 * ld:offset + 5 * ld + cols] = torch.linspace(
            -60000.0, 8.0, cols, device=cuda_device).half()
    grad = torch.tensor([0.3125], device=cuda_device)
    (fm, fl, floss, fd), (tm, tl, tloss, td) = _fused_vs_two_pass(library(), flat, offset, ld, cols,
                                                                   y, grad, in_place)
    assert _same_bits(fm, tm) and _same_bits(fl, tl) and _same_bits(floss, tloss)
    assert _same_bits(fd[:, :cols], td[:, :cols])
    if ld > cols and not in_place:
        assert bool((fd[:, cols:] == 3.0).all())
    if rows > 5:
        assert torch.isnan(floss[2]) and torch.isnan(floss[3])
        assert torch.isnan(fd[2, :cols].float()).all()
    assert torch.count_nonzero(fd[::4, :cols]) == 0


def test_fused_matches_oracle_and_rejects_wide_rows(cuda_device):
    """Against the CPU oracle (loss within one fp16 ulp, dlogits within one ulp
    given the kernel's own statistics), and RV_ERR_UNSUPPORTED for fp32 and
    rows wider than 65536 (the caller takes the two-pass kernels)."""
    from reversability_amd._hip import RV_F16, RV_F32, _stream, library
    lib = library()
    rows, cols = 200, 50257
    g = torch.Generator().manual_seed(9)
    x = (3 * torch.randn(rows, cols, generator=g)).half()
    y = torch.randint(0, cols, (rows,), generator=g)
    y[::5] = -100
    xd, yd = x.to(cuda_device), y.to(cuda_device)
    grad = torch.tensor([0.75], device=cuda_device)
    rmax, rlse, loss = (torch.empty(rows, device=cuda_device) for _ in range(3))
    dx = torch.empty_like(xd)
    assert lib.rv_ce_fused(xd.data_ptr(), RV_F16, cols, yd.data_ptr(), rows, cols, -100,
                           grad.data_ptr(), rmax.data_ptr(), rlse.data_ptr(), loss.data_ptr(),
                           dx.data_ptr(), _stream(xd)) == 0
    omax, olse, oloss = oracle.ce_fwd(x.numpy(), y.numpy())
    assert np.array_equal(rmax.cpu().numpy(), omax)
    lg = loss.cpu().numpy()
    assert np.all(np.abs(lg - oloss) <= ulp16(oloss))
    odx = oracle.ce_bwd(x.numpy(), y.numpy(), rmax.cpu().numpy(), rlse.cpu().numpy(), 0.75)
    dg, do = dx.cpu().numpy().astype(np.float64), odx.astype(np.float64)
    assert np.all(np.abs(dg - do) <= ulp16(do) + 1e-12)
    assert np.mean(dg == do) > 0.99
    RV_ERR_UNSUPPORTED = 3  # include/reversibility_hip.h
    wide = torch.zeros(2, 65544, device=cuda_device, dtype=torch.float16)
    y2 = torch.zeros(2, device=cuda_device, dtype=torch.int64)
    args = (y2.data_ptr(), 2, 65544, -100, grad.data_ptr(), rmax.data_ptr(), rlse.data_ptr(),
            loss.data_ptr(), wide.data_ptr(), _stream(wide))
    assert lib.rv_ce_fused(wide.data_ptr(), RV_F16, 65544, *args) == RV_ERR_UNSUPPORTED
    assert lib.rv_ce_fused(wide.data_ptr(), RV_F32, 65544, *args) == RV_ERR_UNSUPPORTED
