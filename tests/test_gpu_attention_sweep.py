"""A seeded sweep of the causal attention kernels over sequence lengths on
both sides of the 64-row tiles and 128-row blocks (1..1600), head sizes 32,
64 and 128, and small batch / head counts: the forward within the fp16 bound
and the backward within the relative-L2 bar of test_gpu_attention, against
the fp64 attention on the same fp16 qkv."""
from __future__ import annotations

import random

import pytest
import torch

from reversability_amd import attention
from test_gpu_attention import make_qkv, ref_forward, ref_parts, to_packed

pytestmark = pytest.mark.gpu


def _cases(seed: int, count: int):
    rng = random.Random(seed)
    out = []
    for _ in range(count):
        seq = rng.choice([2, 31, 63, 64, 65, 127, 128, 129, 191, 255, 257, 383, 511, 513, 777,
                          1023, 1600])
        out.append((rng.randint(1, 3), seq, rng.randint(1, 4), rng.choice([32, 64, 128])))
    return out


@pytest.mark.parametrize("batch,seq,heads,hd", _cases(13, 12))
def test_attention_sweep(cuda_device, batch, seq, heads, hd):
    qkv = make_qkv(batch, seq, heads, hd, cuda_device, seed=seq + hd)
    x = qkv.clone().requires_grad_(True)
    out = attention.causal_attention(x, heads)
    q, k, v = ref_parts(qkv, heads)
    ref, p, _ = ref_forward(q, k, v)
    bound = 2.0 ** -10 * to_packed(p @ v.abs()) + 2.0 ** -10 * to_packed(ref).abs() + 1e-6
    assert float(((out.detach().double() - to_packed(ref)).abs() / bound).max()) <= 1.0
    g = torch.Generator().manual_seed(seq)
    dout = torch.randn(batch, seq, heads * hd, generator=g).half().to(cuda_device)
    out.backward(dout)
    r = qkv.double().requires_grad_(True)
    rq, rk, rv = r.view(batch, seq, 3, heads, hd).permute(2, 0, 3, 1, 4).unbind(0)
    to_packed(ref_forward(rq, rk, rv)[0]).backward(dout.double())
    t = qkv.clone().requires_grad_(True)
    attention.reference_attention(t, heads).backward(dout)
    for i in range(3):
        sl = slice(i * heads * hd, (i + 1) * heads * hd)
        want = r.grad[..., sl]
        denom = float(want.norm()) or 1.0
        ours = float((x.grad[..., sl].double() - want).norm()) / denom
        theirs = float((t.grad[..., sl].double() - want).norm()) / denom
        assert ours <= max(2e-3, 3 * theirs), ("qkv"[i], ours, theirs)
