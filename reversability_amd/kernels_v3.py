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


def _fp16_out(x: torch.Tensor) -> bool:
    """fp16 output applies under fp16 autocast on rows the vector kernels cover."""
    return (torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.float16
            and x.shape[-1] % 4 == 0 and x.data_ptr() % 16 == 0)


class FusedRMSNorm(torch.autograd.Function):
    """``y = x * rsqrt(mean(x^2) + eps) * weight`` over the last dimension.

    ``fp16_out=True`` (a fourth, optional argument; the reference's three-argument
    call is unchanged) is for norms whose only consumers are fp16-autocast GEMMs:
    under fp16 autocast y is returned as the fp16 value autocast would feed
    those GEMMs, and the incoming fp16 gradient is taken as is -- bit-identical
    results without the fp32 y, its cast, or the fp32 gradient."""

    @staticmethod
    def forward(ctx, x, weight, eps, fp16_out=False):
        _validate(x, weight)
        half = bool(fp16_out) and _fp16_out(x)
        output, rstd = ops.rmsnorm_fwd(x, weight.contiguous(), float(eps), half)
        ctx.save_for_backward(x, weight, rstd)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, gradient):
        x, weight, rstd = ctx.saved_tensors
        if gradient.dtype not in (torch.float32, torch.float16):
            gradient = gradient.float()
        dx, dweight = ops.rmsnorm_bwd(x, weight.contiguous(), gradient.contiguous(), rstd)
        return dx, dweight, None, None


def rms_norm_eps(module: torch.nn.RMSNorm, x: torch.Tensor) -> float:
    """The eps nn.RMSNorm uses: its own, else finfo(x.dtype).eps (kernels_v3.py:79)."""
    return module.eps if module.eps is not None else torch.finfo(x.dtype).eps


def enable_rmsnorm(model: torch.nn.Module, fp16_out: bool = False) -> None:
    """Route every nn.RMSNorm of ``model`` through FusedRMSNorm (kernels_v3.py:77-83).
    ``fp16_out``: every norm output of the model feeds only fp16-autocast GEMMs
    (true of the decoder blocks and the final norm before the tied head)."""
    def forward(self, x):
        return FusedRMSNorm.apply(x, self.weight, rms_norm_eps(self, x), fp16_out)
    for module in model.modules():
        if isinstance(module, torch.nn.RMSNorm):
            module.forward = types.MethodType(forward, module)
            module._rv_fused = True
