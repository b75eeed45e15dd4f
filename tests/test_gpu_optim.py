"""GPU parity of FusedAdamW (rv_adamw_step) against torch.optim.AdamW.

torch's foreach AdamW on the same device and inputs is the reference
arithmetic: decoupled decay, lerp for the first moment, mul + addcmul for the
second, sqrt / bias-correction + eps, addcdiv.  The kernel follows that order
in fp32 (its lerp, addcmul and addcdiv as fused multiply-adds), so
parameters and moments agree to a few fp32 ulps (bar after 5 steps: relative
1e-6 plus 8 ulps of the tensor's largest magnitude; parameters that cancel to
~0 keep an absolute error).  Also: the
GradScaler sequence of the reference's update (unscale_, clip_grad_norm_,
step, update), an overflow step that must change nothing (parameters, moments
and the step count), the grad_scale path (step without unscale_), and more
tensors than one launch takes.
"""
from __future__ import annotations

import pytest
import torch

from reversability_amd.optim import FusedAdamW

pytestmark = pytest.mark.gpu

SHAPES = [(256,), (768, 256), (50257, 256), (13,), (1031, 7), (512, 256), (3,)]


def _params(dev, shapes=SHAPES, seed=3):
    g = torch.Generator().manual_seed(seed)
    return [(0.02 * torch.randn(*s, generator=g)).to(dev) for s in shapes]


def _close(a, b, rtol=1e-6, ulps=8):
    """|a - b| <= rtol |b| + ulps fp32 ulps of the tensor's largest magnitude
    (parameters that cancel to ~0 keep an absolute, not a relative, error)."""
    atol = ulps * torch.finfo(torch.float32).eps * float(b.abs().max())
    return bool(((a - b).abs() <= atol + rtol * b.abs()).all())


def _grads(params, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(p.shape, generator=g).to(p.device) * 1e-2 for p in params]


@pytest.mark.parametrize("wd,lr", [(0.1, 6e-4), (0.0, 1e-3)])
def test_matches_torch_adamw(cuda_device, wd, lr):
    base = _params(cuda_device)
    a = [p.clone().requires_grad_(True) for p in base]
    b = [p.clone().requires_grad_(True) for p in base]
    ta = torch.optim.AdamW(a, lr=lr, betas=(0.9, 0.95), weight_decay=wd, foreach=True)
    fb = FusedAdamW(b, lr=lr, betas=(0.9, 0.95), weight_decay=wd)
    equal = total = 0
    for step in range(5):
        for pa, pb, gr in zip(a, b, _grads(base, step)):
            pa.grad, pb.grad = gr.clone(), gr.clone()
        ta.step()
        fb.step()
        for pa, pb in zip(a, b):
            assert _close(pb.detach(), pa.detach()), step
            equal += int((pa == pb).sum())
            total += pa.numel()
    for pa, pb in zip(a, b):
        sa, sb = ta.state[pa], fb.state[pb]
        assert _close(sb["exp_avg"], sa["exp_avg"]) and _close(sb["exp_avg_sq"], sa["exp_avg_sq"])
        assert float(sb["step"]) == float(sa["step"]) == 5.0
    print(f"  bitwise-equal parameters: {equal / total:.4f}", flush=True)


def test_grad_scaler_sequence_and_overflow_skip(cuda_device):
    """The reference's update sequence under GradScaler.  Both optimizers get
    the same scaled gradients each step (a forward/backward of one copy), so
    the comparison isolates the optimizer: independent fp16 forwards of two
    copies that differ by one ulp diverge through Adam's sensitivity to tiny
    second moments, not through the optimizer."""
    torch.manual_seed(0)
    net = torch.nn.Sequential(torch.nn.Linear(256, 512, bias=False), torch.nn.ReLU(),
                              torch.nn.Linear(512, 256, bias=False)).to(cuda_device)
    a = [p.detach().clone().requires_grad_(True) for p in net.parameters()]
    b = [p.detach().clone().requires_grad_(True) for p in net.parameters()]
    opt_a = torch.optim.AdamW(a, lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)
    opt_b = FusedAdamW(b, lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)
    sc_a, sc_b = (torch.amp.GradScaler("cuda", init_scale=2.0 ** 12) for _ in range(2))
    x = torch.randn(64, 256, device=cuda_device)
    for step in range(5):
        with torch.no_grad():
            for p, q in zip(net.parameters(), a):
                p.copy_(q)
        net.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            loss = net(x).float().square().mean()
        sc_a.scale(loss).backward()
        sc_b.scale(loss.detach())  # sc_b holds the same scale as sc_a
        grads = [p.grad.detach().clone() for p in net.parameters()]
        if step == 2:  # overflow: this update must be skipped
            grads[0][0, 0] = float("inf")
        for params, opt, sc in ((a, opt_a, sc_a), (b, opt_b, sc_b)):
            for p, g in zip(params, grads):
                p.grad = g.clone()
            sc.unscale_(opt)
            torch.nn.utils.clip_grad_norm_(params, 1.0)
            sc.step(opt)
            sc.update()
        for pa, pb in zip(a, b):
            assert _close(pb.detach(), pa.detach(), rtol=1e-5, ulps=16), step
        assert sc_a.get_scale() == sc_b.get_scale()
    assert float(opt_b.state[b[0]]["step"]) == float(opt_a.state[a[0]]["step"]) == 4.0


def test_grad_scale_path_without_unscale(cuda_device):
    base = _params(cuda_device, SHAPES[:3])
    a = [p.clone().requires_grad_(True) for p in base]
    b = [p.clone().requires_grad_(True) for p in base]
    ta = torch.optim.AdamW(a, lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)
    fb = FusedAdamW(b, lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)
    sa, sb = (torch.amp.GradScaler("cuda", init_scale=1024.0) for _ in range(2))
    for step in range(3):
        one = torch.ones((), device=cuda_device)
        sa.scale(one), sb.scale(one)  # the scalers' scale tensors exist from here on
        for pa, pb, gr in zip(a, b, _grads(base, 10 + step)):
            pa.grad, pb.grad = gr * 1024.0, gr * 1024.0
        sa.step(ta)
        sa.update()
        sb.step(fb)  # no unscale_: the scaler hands grad_scale to the optimizer
        sb.update()
    for pa, pb in zip(a, b):
        assert _close(pb.detach(), pa.detach(), rtol=1e-5, ulps=16)


def test_many_tensors_and_rejects(cuda_device):
    shapes = [(17 * (i + 1),) for i in range(130)]
    base = _params(cuda_device, shapes)
    a = [p.clone().requires_grad_(True) for p in base]
    b = [p.clone().requires_grad_(True) for p in base]
    ta = torch.optim.AdamW(a, lr=1e-3)
    fb = FusedAdamW(b, lr=1e-3)
    for pa, pb, gr in zip(a, b, _grads(base, 1)):
        pa.grad, pb.grad = gr.clone(), gr.clone()
    ta.step()
    fb.step()
    for pa, pb in zip(a, b):
        assert _close(pb.detach(), pa.detach())
    with pytest.raises(ValueError, match="CUDA"):
        q = torch.zeros(4, requires_grad=True)
        q.grad = torch.ones(4)
        FusedAdamW([q]).step()
    with pytest.raises(ValueError):
        FusedAdamW(a, amsgrad=True)


@pytest.mark.parametrize("max_norm,shapes", [(1.0, SHAPES), (1e9, SHAPES),
                                             (0.5, [(17 * (i + 1),) for i in range(60)])])
def test_unscale_clip_matches_reference_sequence(cuda_device, max_norm, shapes):
    """opt.unscale_clip_(scaler, max_norm) + scaler.step/update equals the
    reference's scaler.unscale_ + clip_grad_norm_ + step/update (on FusedAdamW
    both): the total norm within fp32 summation-order error, parameters within
    a few ulps (the clip coefficient may differ in its last bit), bit for bit
    when the clip is inactive (coefficient 1); an overflowing step is skipped
    by both (parameters, step count) and lowers both scales alike; more
    tensors than one launch takes (60 > 48)."""
    base = _params(cuda_device, shapes)
    a = [p.clone().requires_grad_(True) for p in base]
    b = [p.clone().requires_grad_(True) for p in base]
    opt_a = FusedAdamW(a, lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)
    opt_b = FusedAdamW(b, lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)
    sc_a, sc_b = (torch.amp.GradScaler("cuda", init_scale=2.0 ** 10) for _ in range(2))
    one = torch.ones((), device=cuda_device)
    for step in range(4):
        sc_a.scale(one), sc_b.scale(one)
        grads = [g * 100 * 2.0 ** 10 for g in _grads(base, 20 + step)]
        if step == 2:
            grads[1].view(-1)[0] = float("nan")
        for params, g_ in ((a, grads), (b, grads)):
            for p, g in zip(params, g_):
                p.grad = g.clone()
        sc_a.unscale_(opt_a)
        norm_a = torch.nn.utils.clip_grad_norm_(a, max_norm)
        sc_a.step(opt_a)
        sc_a.update()
        norm_b = opt_b.unscale_clip_(sc_b, max_norm)
        sc_b.step(opt_b)
        sc_b.update()
        torch.cuda.synchronize()
        if step != 2:
            assert abs(float(norm_b) - float(norm_a)) <= 1e-5 * float(norm_a), step
        for pa, pb in zip(a, b):
            if max_norm >= 1e9:
                assert torch.equal(pb, pa), step
            else:
                assert _close(pb.detach(), pa.detach(), rtol=2e-6, ulps=8), step
        assert sc_a.get_scale() == sc_b.get_scale()
    assert float(opt_b.state[b[0]]["step"]) == float(opt_a.state[a[0]]["step"]) == 3.0


def test_clip_without_scaler(cuda_device):
    base = _params(cuda_device, SHAPES[:4])
    a = [p.clone().requires_grad_(True) for p in base]
    b = [p.clone().requires_grad_(True) for p in base]
    opt_a = FusedAdamW(a, lr=1e-3)
    opt_b = FusedAdamW(b, lr=1e-3)
    for pa, pb, g in zip(a, b, _grads(base, 5)):
        pa.grad, pb.grad = g * 50, g * 50
    norm_a = torch.nn.utils.clip_grad_norm_(a, 1.0)
    opt_a.step()
    norm_b = opt_b.unscale_clip_(None, 1.0)
    opt_b.step()
    assert abs(float(norm_b) - float(norm_a)) <= 1e-5 * float(norm_a)
    for pa, pb in zip(a, b):
        assert _close(pb.detach(), pa.detach(), rtol=2e-6, ulps=8)
    with pytest.raises(RuntimeError, match="already been called"):
        sc = torch.amp.GradScaler("cuda")
        sc.scale(torch.ones((), device=cuda_device))
        for p in b:
            p.grad = torch.zeros_like(p)
        opt_b.unscale_clip_(sc, 1.0)
        opt_b.unscale_clip_(sc, 1.0)
