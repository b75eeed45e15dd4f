"""Error bounds shared by the GEMM parity tests.

Any GEMM that accumulates in fp32 -- MFMA here, cuBLAS in the reference --
may differ from the fp64 contraction of the same fp16 operands by the fp32
accumulation bound K * 2^-24 * sum_k |a_k b_k| before its final fp16
rounding, so the bar per element is

    |out - truth| <= ulp_fp16(truth) + K * 2^-24 * sum_k |a_k b_k|,

plus relative-L2 agreement (1e-3).
"""
from __future__ import annotations

import torch


def fp16_ulp(t: torch.Tensor) -> torch.Tensor:
    """Spacing of fp16 at |t| (2^-24 below the normal range), on t's device."""
    a = t.abs().double()
    e = torch.floor(torch.log2(a.clamp_min(2.0 ** -14))).clamp_min(-14)
    return torch.pow(2.0, e - 10)


def rel_l2(a, b):
    a, b = a.detach().double(), b.detach().double().to(a.device)
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def within_gemm_bound(out, a, b, k, transpose_b=True):
    """out vs the fp64 truth of a @ b^T (or a @ b), computed on out's device."""
    a64, b64 = a.double().to(out.device), b.double().to(out.device)
    bt = b64.t() if transpose_b else b64
    truth = a64 @ bt
    scale = a64.abs() @ bt.abs()
    err = (out.double() - truth).abs()
    bound = fp16_ulp(truth) + k * 2.0 ** -24 * scale
    worst = float((err / bound).max())
    r = rel_l2(out, truth)
    print(f"  worst error / bound = {worst:.3f}, rel_l2 = {r:.2e}", flush=True)
    return worst <= 1.0 and r < 1e-3
