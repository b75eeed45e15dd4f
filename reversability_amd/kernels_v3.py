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


def _fp16_out(x: torch.Tensor, weight: torch.Tensor | None = None) -> bool:
    """fp16 output applies under fp16 autocast on rows the vector kernels cover
    (16-byte aligned rows, and a contiguous, 16-byte aligned weight)."""
    return (torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.float16
            and x.shape[-1] % 4 == 0 and x.data_ptr() % 16 == 0
            and (weight is None or (weight.is_contiguous() and weight.data_ptr() % 16 == 0)))


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
        half = bool(fp16_out) and _fp16_out(x, weight)
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


class FusedAddRMSNorm(torch.autograd.Function):
    """``(h, y) = (x + f, RMSNorm(x + f))`` for the fp32 residual stream x and
    a force term f (fp16 or fp32), y as FusedRMSNorm's fp16 output: the
    residual add that feeds a norm (the midpoint force's ``x + A(x)``, the
    Euler step's ``q + A(p)``; src/reversibility/reversible.py:16-25) in the
    norm's own pass (``rv_add_rmsnorm_fwd_f16``).  Backward in one pass too
    (``rv_rmsnorm_bwd_acc``): the input gradient is the norm backward plus
    the gradient of h's other uses -- the sum autograd would form -- written
    in fp32 for x and rounded to fp16 for f.  Same values as the add, the
    norm and autograd's accumulation and cast."""

    @staticmethod
    def forward(ctx, x, f, weight, eps, pre=None):
        ctx.set_materialize_grads(False)
        if pre is None:
            h, y, rstd = ops.add_rmsnorm_fwd16(x, f, weight.contiguous(), float(eps))
        else:  # (h, y, rstd) already computed from these inputs (inverse_add_rms_norm)
            h, y, rstd = pre
        ctx.save_for_backward(h, weight, rstd)
        ctx.f_dtype = f.dtype
        return h, y

    @staticmethod
    @once_differentiable
    def backward(ctx, dh, dy):
        h, weight, rstd = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(h, dtype=torch.float16)
        elif dy.dtype not in (torch.float32, torch.float16):
            dy = dy.float()
        dx, dx16, dweight = ops.rmsnorm_bwd_acc(h, weight.contiguous(), dy.contiguous(), rstd,
                                                dh.contiguous() if dh is not None else None)
        df = dx16 if ctx.f_dtype == torch.float16 else dx.to(ctx.f_dtype)
        return dx, df, dweight, None, None


class FusedRMSNormPass(torch.autograd.Function):
    """``(x, RMSNorm(x))`` -- the normalized input passed through as a second
    output, for an x that also feeds something else (the Euler step's
    ``p0 + M(...)`` beside ``attn_norm(p0)``; the split midpoint's MLP graph
    beside the attention graph).  Backward in one pass: the norm backward plus
    the pass-through output's gradient (``rv_rmsnorm_bwd_acc``), the sum
    autograd would otherwise form in a separate kernel.  y as FusedRMSNorm's
    (fp16 under fp16 autocast with ``fp16_out``).  ``half_grad``: a list that
    receives fp16(x's gradient), written by the same backward pass, for a
    caller that also needs that gradient in fp16 (the Euler reconstruction
    hands the next layer's fp16 force its output gradient without a cast)."""

    @staticmethod
    def forward(ctx, x, weight, eps, fp16_out=False, pre=None, half_grad=None):
        ctx.set_materialize_grads(False)
        if pre is None:
            half = bool(fp16_out) and _fp16_out(x, weight)
            y, rstd = ops.rmsnorm_fwd(x, weight.contiguous(), float(eps), half)
        else:  # (y, rstd) already computed from x (inverse_rms_norm)
            y, rstd = pre
        ctx.save_for_backward(x, weight, rstd)
        ctx.half_grad = half_grad
        return x.view_as(x), y

    @staticmethod
    @once_differentiable
    def backward(ctx, dpass, dy):
        x, weight, rstd = ctx.saved_tensors
        if dy is None:
            return dpass, None, None, None, None, None
        if dy.dtype not in (torch.float32, torch.float16):
            dy = dy.float()
        want16 = ctx.half_grad is not None
        dx, dx16, dweight = ops.rmsnorm_bwd_acc(x, weight.contiguous(), dy.contiguous(), rstd,
                                                dpass.contiguous() if dpass is not None else None,
                                                want16)
        if want16:
            ctx.half_grad.append(dx16)
        return dx, dweight, None, None, None, None


def rms_norm_pass(x: torch.Tensor, norm: torch.nn.Module, pre=None, half_grad=None):
    """``(x', norm(x))`` with x' = x for x's other use (see FusedRMSNormPass), on the
    fused kernels when ``norm`` is routed by ``enable_rmsnorm`` and x is a
    contiguous fp32 GPU tensor whose rows the vector kernels cover; otherwise
    ``(x, norm(x))`` (also for a norm weight that is not 16-byte aligned).  ``pre``:
    the (y, rstd) ``inverse_rms_norm`` returned for x.  ``half_grad``: a list
    that the fused backward appends fp16(x's gradient) to (nothing is appended
    on the unfused path or when the norm output gets no gradient)."""
    if (getattr(norm, "_rv_fused", False) and x.is_cuda and x.dtype == torch.float32
            and x.is_contiguous() and x.shape[-1] % 4 == 0 and x.data_ptr() % 16 == 0
            and norm.weight.is_contiguous() and norm.weight.data_ptr() % 16 == 0):
        return FusedRMSNormPass.apply(x, norm.weight, rms_norm_eps(norm, x),
                                      getattr(norm, "_rv_fp16_out", False), pre, half_grad)
    return x, norm(x)


def _fp16_norm_input(norm: torch.nn.Module, x: torch.Tensor) -> bool:
    """Whether ``norm`` (routed by ``enable_rmsnorm(..., fp16_out=True)``) hands
    its consumers the fp16 value of the fused kernels for this x."""
    return (getattr(norm, "_rv_fp16_out", False) and x.is_cuda and x.dtype == torch.float32
            and x.is_contiguous() and _fp16_out(x, norm.weight))


def _sub_fusable(x: torch.Tensor, f: torch.Tensor, norm: torch.nn.Module) -> bool:
    """Whether rv_sub_rmsnorm_fwd_f16 gives what the fused fp16-output norm
    paths (rms_norm_pass / add_rms_norm) would compute after ``x - f``."""
    return (getattr(norm, "_rv_fused", False) and getattr(norm, "_rv_fp16_out", False)
            and x.is_cuda and x.dtype == torch.float32
            and f.dtype in (torch.float16, torch.float32) and x.shape == f.shape
            and x.is_contiguous() and f.is_contiguous() and f.data_ptr() % 16 == 0
            and _fp16_out(x, norm.weight))


def inverse_rms_norm(x: torch.Tensor, f: torch.Tensor, norm: torch.nn.Module):
    """``(d, pre)`` with d = x - f (a residual step inverted, no graph) and
    ``pre`` the (y, rstd) of ``norm(d)`` made in the same pass -- to hand to
    ``rms_norm_pass(d, norm, pre)`` -- where the fused kernels apply; else
    ``(euler_step(x, f, -1), None)``.  Same values either way."""
    with torch.no_grad():
        if _sub_fusable(x, f, norm):
            d, _, y, rstd = ops.sub_rmsnorm_fwd16(x, f, norm.weight.contiguous(),
                                                  rms_norm_eps(norm, x), False)
            return d, (y, rstd)
        from .residual import euler_step
        return euler_step(x, f, -1), None


def midpoint_rms_norm(p: torch.Tensor, a: torch.Tensor, m: torch.Tensor, scale: float,
                      sign: int, norm: torch.nn.Module):
    """``(out, pre)`` with out = ``residual.midpoint_step(p, a, m, scale, sign)``
    (no graph) and ``pre`` the (y, rstd) of ``norm(out)`` made in the same pass
    -- the value the next layer's attention norm reads, to use directly or hand
    to ``rms_norm_pass(out, norm, pre)`` -- where the fused kernels apply (fp16
    force terms); else ``(midpoint_step(...), None)``.  Same values either way."""
    with torch.no_grad():
        if (_sub_fusable(p, a, norm) and a.dtype == torch.float16
                and m.dtype == torch.float16 and m.shape == p.shape and m.is_contiguous()
                and m.data_ptr() % 16 == 0):
            out, y, rstd = ops.midpoint_rmsnorm_fwd16(p, a, m, norm.weight.contiguous(),
                                                      rms_norm_eps(norm, p), float(scale),
                                                      int(sign))
            return out, (y, rstd)
        from .residual import midpoint_step
        return midpoint_step(p, a, m, scale, sign), None


def inverse_add_rms_norm(x: torch.Tensor, f: torch.Tensor, norm: torch.nn.Module):
    """``(d, pre)`` with d = x - f (no graph) and ``pre`` the (h, y, rstd) of
    ``add_rms_norm(d, f, norm)`` -- h = d + f and its norm -- made in the same
    pass, to hand to ``add_rms_norm(d, f, norm, pre)``; else
    ``(euler_step(x, f, -1), None)``.  Same values either way."""
    with torch.no_grad():
        if _sub_fusable(x, f, norm):
            d, h, y, rstd = ops.sub_rmsnorm_fwd16(x, f, norm.weight.contiguous(),
                                                  rms_norm_eps(norm, x), True)
            return d, (h, y, rstd)
        from .residual import euler_step
        return euler_step(x, f, -1), None


class FusedAddRMSNormPass(torch.autograd.Function):
    """FusedAddRMSNorm whose residual input x also passes through unchanged as a
    third output (the split midpoint's q: an output of the rebuilt step and
    the input of ``q + proxy``): backward sums x's gradients -- the norm's and
    the pass-through's -- in the norm's backward pass
    (``rv_rmsnorm_bwd_acc_pass``); the force term's fp16 gradient excludes the
    pass-through share.  The sum's other output h must have no other use."""

    @staticmethod
    def forward(ctx, x, f, weight, eps):
        ctx.set_materialize_grads(False)
        h, y, rstd = ops.add_rmsnorm_fwd16(x, f, weight.contiguous(), float(eps))
        ctx.save_for_backward(h, weight, rstd)
        ctx.f_dtype = f.dtype
        return x.view_as(x), y

    @staticmethod
    @once_differentiable
    def backward(ctx, dpass, dy):
        h, weight, rstd = ctx.saved_tensors
        if dy is None:
            dy = torch.zeros_like(h, dtype=torch.float16)
        elif dy.dtype not in (torch.float32, torch.float16):
            dy = dy.float()
        dpass = dpass.contiguous() if dpass is not None else None
        dx, dx16, dweight = ops.rmsnorm_bwd_acc(h, weight.contiguous(), dy.contiguous(), rstd,
                                                None, True, dpass)
        df = dx16 if ctx.f_dtype == torch.float16 else dx.to(ctx.f_dtype)
        return dx, df, dweight, None


def add_rms_norm_pass(x: torch.Tensor, f: torch.Tensor, norm: torch.nn.Module):
    """``(x', norm(x + f))`` for a residual input x with a pass-through use x'
    (and no other use of the sum), on the fused kernels where ``add_rms_norm``
    would take them (f fp16 there); otherwise ``(x, norm(x + f))``."""
    if (getattr(norm, "_rv_fp16_out", False) and x.is_cuda and x.dtype == torch.float32
            and f.dtype == torch.float16 and x.shape == f.shape
            and x.is_contiguous() and f.is_contiguous() and f.data_ptr() % 16 == 0
            and _fp16_out(x, norm.weight)):
        return FusedAddRMSNormPass.apply(x, f, norm.weight, rms_norm_eps(norm, x))
    return x.view_as(x), add_rms_norm(x, f, norm)[1]


def add_rms_norm(x: torch.Tensor, f: torch.Tensor, norm: torch.nn.Module, pre=None):
    """``(h, norm(h))`` with ``h = x + f``.  On the fused kernels when ``norm``
    is an RMSNorm routed by ``enable_rmsnorm(..., fp16_out=True)`` and the
    call runs under fp16 autocast on the GPU; otherwise the residual add
    (``residual.euler_step``) followed by ``norm``.  ``pre``: the (h, y, rstd)
    ``inverse_add_rms_norm`` returned for these inputs."""
    if (getattr(norm, "_rv_fp16_out", False) and x.is_cuda and x.dtype == torch.float32
            and f.dtype in (torch.float16, torch.float32) and x.shape == f.shape
            and x.is_contiguous() and f.is_contiguous() and f.data_ptr() % 16 == 0
            and _fp16_out(x, norm.weight)):
        return FusedAddRMSNorm.apply(x, f, norm.weight, rms_norm_eps(norm, x), pre)
    from .residual import euler_step
    h = euler_step(x, f, +1)
    return h, norm(h)


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
            module._rv_fp16_out = bool(fp16_out)
