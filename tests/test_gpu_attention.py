"""GPU parity of the fused causal attention (reversability_amd.attention).

Reference: the same attention in fp64 (on the fp16 qkv the kernels read), as
torch computes F.scaled_dot_product_attention(is_causal=True) by its
definition.  Forward bar, per element: the kernels round P to fp16 before the
P V product (rel. error 2^-11 per term) and round the output to fp16
(2^-11), so

    |out - ref| <= 2^-10 * (P |V|) + 2^-10 * |ref| + 1e-6

(twice those terms as slack for the fp32 softmax).  Backward: relative L2 of
dq, dk, dv against fp64 autograd, at most 2e-3 or 3x the error of torch's own
fp16 scaled_dot_product_attention backward on the same device, whichever is
larger.  Also: base-2 log-sum-exp, determinism (bitwise repeatability),
sequence lengths that are not multiples of the tiles, every head size.
"""
from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from reversability_amd import attention

pytestmark = pytest.mark.gpu

CASES = [  # batch, seq, heads, head_dim
    (1, 1, 1, 32),
    (3, 100, 2, 64),
    (2, 130, 3, 128),
    (4, 512, 8, 32),
    (2, 2048, 16, 64),
    (1, 1000, 2, 128),
]


def make_qkv(batch, seq, heads, hd, device, seed=0, spread=1.0):
    g = torch.Generator().manual_seed(seed)
    qkv = spread * torch.randn(batch, seq, 3 * heads * hd, generator=g)
    return qkv.half().to(device)


def ref_parts(qkv, heads):
    batch, seq, width = qkv.shape
    hd = width // 3 // heads
    q, k, v = qkv.double().view(batch, seq, 3, heads, hd).permute(2, 0, 3, 1, 4).unbind(0)
    return q, k, v


def ref_forward(q, k, v):
    hd = q.shape[-1]
    s = (q @ k.transpose(-1, -2).contiguous()) / math.sqrt(hd)
    seq = q.shape[2]
    mask = torch.ones(seq, seq, dtype=torch.bool, device=q.device).triu(1)
    s = s.masked_fill(mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return p @ v, p, s


def to_packed(o):  # [B, H, T, hd] -> [B, T, H*hd]
    batch, heads, seq, hd = o.shape
    return o.transpose(1, 2).reshape(batch, seq, heads * hd)


@pytest.mark.parametrize("batch,seq,heads,hd", CASES)
def test_forward_within_fp16_bound(cuda_device, batch, seq, heads, hd):
    qkv = make_qkv(batch, seq, heads, hd, cuda_device)
    out = attention.causal_attention(qkv, heads)
    assert out.shape == (batch, seq, heads * hd) and out.dtype == torch.float16
    q, k, v = ref_parts(qkv, heads)
    ref, p, s = ref_forward(q, k, v)
    bound = 2.0 ** -10 * to_packed(p @ v.abs()) + 2.0 ** -10 * to_packed(ref).abs() + 1e-6
    err = (out.double() - to_packed(ref)).abs()
    worst = float((err / bound).max())
    sdpa = attention.reference_attention(qkv, heads)
    sdpa_err = float((sdpa.double() - to_packed(ref)).abs().max())
    print(f"  max err {float(err.max()):.3e} (torch sdpa {sdpa_err:.3e}), worst/bound {worst:.3f}")
    assert worst <= 1.0
    # log-sum-exp (base 2, scaled scores) kept for the backward
    lse = torch.empty(batch * heads, seq, device=cuda_device)
    out2 = torch.empty_like(out)
    from reversability_amd._hip import _stream, library
    assert library().rv_attn_fwd(qkv.data_ptr(), batch, seq, heads, hd, out2.data_ptr(),
                                 lse.data_ptr(), _stream(qkv)) == 0
    ref_lse = torch.logsumexp(s, dim=-1).reshape(batch * heads, seq) / math.log(2.0)
    assert torch.allclose(lse.double(), ref_lse, rtol=1e-5, atol=1e-4)
    assert torch.equal(out, out2)  # deterministic


@pytest.mark.parametrize("batch,seq,heads,hd", CASES)
def test_backward_matches_fp64_autograd(cuda_device, batch, seq, heads, hd):
    qkv = make_qkv(batch, seq, heads, hd, cuda_device, seed=1)
    g = torch.Generator().manual_seed(2)
    dout = torch.randn(batch, seq, heads * hd, generator=g).half().to(cuda_device)
    x = qkv.clone().requires_grad_(True)
    attention.causal_attention(x, heads).backward(dout)
    got = x.grad
    # fp64 reference gradient
    r = qkv.double().requires_grad_(True)
    q, k, v = r.view(batch, seq, 3, heads, hd).permute(2, 0, 3, 1, 4).unbind(0)
    ref, _, _ = ref_forward(q, k, v)
    to_packed(ref).backward(dout.double())
    want = r.grad
    # torch's own fp16 attention backward on the same inputs
    t = qkv.clone().requires_grad_(True)
    attention.reference_attention(t, heads).backward(dout)
    lib_grad = t.grad
    for i, name in enumerate("qkv"):
        sl = slice(i * heads * hd, (i + 1) * heads * hd)
        ref_part = want[..., sl]
        denom = float(ref_part.norm()) or 1.0
        ours = float((got[..., sl].double() - ref_part).norm()) / denom
        theirs = float((lib_grad[..., sl].double() - ref_part).norm()) / denom
        print(f"  d{name}: rel L2 {ours:.3e} (torch sdpa {theirs:.3e})")
        assert ours <= max(2e-3, 3 * theirs), name
    # deterministic
    x2 = qkv.clone().requires_grad_(True)
    attention.causal_attention(x2, heads).backward(dout)
    assert torch.equal(x2.grad, got)


def test_large_logits_stay_finite(cuda_device):
    # scores of magnitude ~100: the online max must keep every exponent <= 0
    qkv = make_qkv(2, 300, 2, 64, cuda_device, seed=3, spread=4.0)
    out = attention.causal_attention(qkv, 2)
    assert torch.isfinite(out).all()
    q, k, v = ref_parts(qkv, 2)
    ref, p, _ = ref_forward(q, k, v)
    bound = 2.0 ** -10 * to_packed(p @ v.abs()) + 2.0 ** -10 * to_packed(ref).abs() + 1e-6
    assert ((out.double() - to_packed(ref)).abs() <= bound).all()


def test_enable_attention_matches_reference_module(cuda_device):
    from reversability_amd import build_model
    torch.manual_seed(0)
    cfg = {"model": {"vocab_size": 512, "max_sequence_length": 256, "n_layers": 2, "n_heads": 4,
                     "d_model": 256, "d_ff": 512}, "method": "midpoint", "step_size": 0.5}
    ref_model = build_model(cfg).to(cuda_device)
    cand = build_model(cfg).to(cuda_device)
    cand.load_state_dict(ref_model.state_dict())
    attention.enable_attention(cand)
    ids = torch.randint(0, 512, (3, 256), device=cuda_device)
    losses, grads = [], []
    for m in (ref_model, cand):
        m.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            logits = m(ids)
            loss = F.cross_entropy(logits.flatten(0, 1).float(), ids.flatten())
        loss.backward()
        losses.append(float(loss.detach()))
        grads.append({n: p.grad.float() for n, p in m.named_parameters()})
    assert abs(losses[0] - losses[1]) <= 1e-3 * abs(losses[0])
    for n, g in grads[0].items():
        rel = float((grads[1][n] - g).norm() / (g.norm() + 1e-30))
        assert rel < 2e-2, (n, rel)


def test_rejects_uncovered_inputs(cuda_device):
    qkv = make_qkv(1, 8, 2, 16, cuda_device)  # head size 16
    with pytest.raises(ValueError, match="head size"):
        attention.causal_attention(qkv, 2)
    with pytest.raises(ValueError):
        attention.causal_attention(qkv.float(), 1)
