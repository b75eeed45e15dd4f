"""Fused RMSNorm on gfx950, behind the reference's v3 RMSNorm operator surface.

Mirrors ``FusedRMSNorm`` / ``enable_rmsnorm`` of
src/reversibility/kernels_v3.py:51-83: same ``apply(x, weight, eps)``
signature, same saved tensors (x, weight, per-row rstd), same ValueError
contract (CUDA FP32 only, contiguous input, 1-D matching weight; no dtype
substitution and no CPU fallback).  The three Triton backward launches of the
reference (dx, dweight tile partials, column reduce) become one fused
dx + dweight-partial pass plus a small deterministic reduce
(``rv_rmsnorm_bwd``).
"""
from __future__ import annotations

import types

import torch
from torch.autograd.function import once_differentiable

from ._hip import ops


def _validate(x: torch.Tensor, weight: torch.Tensor) -> None:
    # kernels_v3.py:54-57
    if x.device.type != "cuda" or x.dtype != torch.float32 or weight.dtype != torch.float32:
        raise ValueError("RMSNorm v3 requires CUDA FP32 (ROCm device) residuals and weights; "
                         "no dtype substitution")
    if (not x.is_contiguous() or weight.ndim != 1 or x.shape[-1] != weight.numel()
            or weight.device != x.device):
        raise ValueError("Contiguous input and one-dimensional matching norm weight required")


class FusedRMSNorm(torch.autograd.Function):
    """``y = x * rsqrt(mean(x^2) + eps) * weight`` over the last dimension."""

    @staticmethod
    def forward(ctx, x, weight, eps):
        _validate(x, weight)
        output, rstd = ops.rmsnorm_fwd(x, weight.contiguous(), float(eps))
        ctx.save_for_backward(x, weight, rstd)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, gradient):
        x, weight, rstd = ctx.saved_tensors
        dx, dweight = ops.rmsnorm_bwd(x, weight.contiguous(), gradient.contiguous(), rstd)
        return dx, dweight, None


def rms_norm_eps(module: torch.nn.RMSNorm, x: torch.Tensor) -> float:
    """The eps nn.RMSNorm uses: its own, else finfo(x.dtype).eps (kernels_v3.py:79)."""
    return module.eps if module.eps is not None else torch.finfo(x.dtype).eps


def enable_rmsnorm(model: torch.nn.Module) -> None:
    """Route every nn.RMSNorm of ``model`` through FusedRMSNorm (kernels_v3.py:77-83)."""
    def forward(self, x):
        return FusedRMSNorm.apply(x, self.weight, rms_norm_eps(self, x))
    for module in model.modules():
        if isinstance(module, torch.nn.RMSNorm):
            module.forward = types.MethodType(forward, module)
            module._rv_fused = True
