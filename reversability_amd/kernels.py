"""Fused SwiGLU on gfx950, behind the reference's operator surface.

Mirrors ``FusedSwiGLU`` / ``enable_swiglu`` of src/reversibility/kernels.py:113-138:
``apply(up)`` takes the packed up-projection ``[..., 2W]`` (gate = first W
columns, value = last W), returns ``[..., W]`` in the input dtype, and its
backward returns the packed gradient.  Same ValueError contract (contiguous
CUDA FP16/FP32, even final width; no CPU fallback).  Rounding points follow
the reference: silu is rounded to the I/O dtype before the multiply, and
``dy * value`` before the sigmoid-derivative product.
"""
from __future__ import annotations

import types

import torch
from torch.autograd.function import once_differentiable

from ._hip import ops


def _validate(up: torch.Tensor) -> None:
    # kernels.py:116-117
    if (up.device.type != "cuda" or up.dtype not in (torch.float16, torch.float32)
            or not up.is_contiguous() or up.shape[-1] % 2):
        raise ValueError("Fused SwiGLU requires contiguous CUDA (ROCm device) FP16/FP32 "
                         "and even final width")


class FusedSwiGLU(torch.autograd.Function):
    """``silu(gate) * value`` over a packed ``[..., 2W]`` tensor."""

    @staticmethod
    def forward(ctx, up):
        _validate(up)
        output = ops.swiglu_fwd(up)
        ctx.save_for_backward(up)
        return output

    @staticmethod
    @once_differentiable
    def backward(ctx, gradient):
        up, = ctx.saved_tensors
        return ops.swiglu_bwd(up, gradient.contiguous())


def enable_swiglu(model: torch.nn.Module) -> None:
    """Patch every block's MLP to ``down(FusedSwiGLU(up(x)))`` (kernels.py:134-138)."""
    def forward(mlp, x):
        return mlp.down(FusedSwiGLU.apply(mlp.up(x)))
    for block in model.blocks:
        block.mlp.forward = types.MethodType(forward, block.mlp)
