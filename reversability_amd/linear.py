"""Attention projections on the MFMA kernels under fp16 autocast.

The decoder's attention has two bias-free ``nn.Linear`` layers, the fused
``qkv`` and the output ``proj`` (src/reversibility/model.py:26-45), run under
``torch.autocast(dtype=float16)`` inside ``midpoint_force`` / ``forward_pair``
and again in every reconstruction backward (src/reversibility/reversible.py,
optimized.py, optimized_v3.py).  ``FusedLinear`` computes what autocast's
``F.linear`` computes -- fp16 casts of the input and of the fp32 weight, an
fp16 GEMM with fp32 accumulation, an fp16 output; backward: ``dx`` as the
fp16 product widened to the input's dtype, ``dW`` as the fp16 product widened
to fp32 -- with the gfx950 GEMM kernels of ``csrc/mlp_gemm.hip``
(``rv_linear_fwd``, ``rv_linear_dx``, ``rv_linear_dw``; the weight gradient
reduces over all tokens in a fixed order, split-K when the output is small).

``enable_linear(model)`` patches every block's ``attn.qkv`` and ``attn.proj``;
calls the kernels do not cover (no fp16 autocast, a bias, widths that are not
multiples of 128, CPU tensors) keep ``F.linear``, recorded in ``paths.report()``
(or raising under ``paths.strict()``).
"""
from __future__ import annotations

import types

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from . import paths
from ._hip import RV_F16, RV_F32, _check, _stream, library
from .mlp import cast_f16, cast_weight


def supported(x: torch.Tensor, weight: torch.Tensor, bias) -> bool:
    return (bias is None and x.is_cuda and x.dtype in (torch.float32, torch.float16)
            and weight.dtype == torch.float32 and weight.is_contiguous() and weight.ndim == 2
            and x.shape[-1] == weight.shape[1] and weight.shape[0] % 128 == 0
            and weight.shape[1] % 128 == 0
            and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.float16)


class FusedLinear(torch.autograd.Function):
    """``F.linear(x, weight)`` under fp16 autocast, bias-free."""

    @staticmethod
    def forward(ctx, x, weight):
        out_f, in_f = weight.shape
        flat = x.reshape(-1, in_f)
        rows = flat.shape[0]
        x16 = cast_f16(flat.contiguous())
        y = torch.empty(rows, out_f, device=x.device, dtype=torch.float16)
        if rows:
            w16 = cast_weight(weight)
            _check(library().rv_linear_fwd(x16.data_ptr(), in_f, w16.data_ptr(), rows, in_f,
                                           out_f, y.data_ptr(), _stream(x)), "rv_linear_fwd")
        ctx.save_for_backward(x16, weight)
        ctx.x_dtype, ctx.x_shape = x.dtype, x.shape
        return y.reshape(*x.shape[:-1], out_f)

    @staticmethod
    @once_differentiable
    def backward(ctx, gradient):
        x16, weight = ctx.saved_tensors
        out_f, in_f = weight.shape
        dy = gradient.reshape(-1, out_f).to(torch.float16).contiguous()
        rows = dy.shape[0]
        lib = library()
        dx = dw = None
        if not rows:
            return (torch.zeros(ctx.x_shape, device=dy.device, dtype=ctx.x_dtype),
                    torch.zeros_like(weight))
        if ctx.needs_input_grad[0]:
            w16 = cast_weight(weight)
            dx = torch.empty(rows, in_f, device=dy.device, dtype=ctx.x_dtype)
            code = RV_F32 if ctx.x_dtype == torch.float32 else RV_F16
            _check(lib.rv_linear_dx(dy.data_ptr(), w16.data_ptr(), rows, in_f, out_f,
                                    dx.data_ptr(), code, _stream(dy)), "rv_linear_dx")
            dx = dx.reshape(ctx.x_shape)
        if ctx.needs_input_grad[1]:
            dw = torch.empty_like(weight)
            nbytes = lib.rv_linear_dw_workspace_bytes(rows, in_f, out_f)
            if nbytes < 0:
                _check(-nbytes, "rv_linear_dw_workspace_bytes")
            ws = torch.empty(max(nbytes, 4) // 4, device=dy.device, dtype=torch.float32)
            _check(lib.rv_linear_dw(dy.data_ptr(), x16.data_ptr(), in_f, rows, in_f, out_f,
                                    dw.data_ptr(), 0, ws.data_ptr(), nbytes, _stream(dy)),
                   "rv_linear_dw")
        return dx, dw


def linear(x: torch.Tensor, weight: torch.Tensor, bias=None) -> torch.Tensor:
    """``F.linear`` with the MFMA path where it applies."""
    if supported(x, weight, bias):
        paths.took("linear", "mfma")
        return FusedLinear.apply(x, weight)
    if x.is_cuda:
        paths.took("linear", "torch",
                   "MFMA projections need fp16 autocast, no bias and widths that are multiples "
                   f"of 128 (weight {tuple(weight.shape)}, input {x.dtype})")
    else:
        paths.took("linear", "torch")
    return F.linear(x, weight, bias)


def enable_linear(model: torch.nn.Module) -> None:
    """Route every block's attention ``qkv`` and ``proj`` through ``linear``."""
    def forward(layer, x):
        return linear(x, layer.weight, layer.bias)
    for block in model.blocks:
        for layer in (block.attn.qkv, block.attn.proj):
            layer.forward = types.MethodType(forward, layer)
            layer._rv_linear = True  # its weight is cast by mlp.cast_weight
