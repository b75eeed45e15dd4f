"""Reversible residual updates: the fused HIP kernels plus their autograd rules.

``midpoint_step(p, a, m, scale, sign)`` evaluates ``p + sign * scale * (a + m)``
with the eager expression's rounding points (the force ``a + m`` and the
product with ``scale = 2h`` are rounded to the force dtype before the add into
the wider residual state) -- the arithmetic of forward_pair / inverse_pair,
src/reversibility/reversible.py:16-32.  ``euler_step(x, f, sign)`` is the
Hamiltonian-Euler ``x + sign * f`` of reversible.py:24-25, 31-32.

ROCm tensors go through one HIP kernel per update (``rv_midpoint_update`` /
``rv_residual_axpy``); a missing library raises.  CPU tensors (the fp64 / fp32
host-logic tests, and the reference's own CPU runs) evaluate the reference's
eager expression, which is what the reference computes on CPU.

``eager_updates()`` makes every update inside it (on this thread or task) the
eager torch expression on any device: a model with its modules unpatched and
``backward_mode='autograd'`` then runs as plain torch end to end -- the
independent comparator the GPU parity tests hold the HIP path against.
"""
from __future__ import annotations

import contextlib
import contextvars

import torch
from torch.autograd.function import once_differentiable

from ._hip import ops


def _state_force(p: torch.Tensor, a: torch.Tensor, m: torch.Tensor | None = None):
    """Validate dtypes for the kernels; promote mixed force dtypes like eager ``a + m``."""
    if m is not None and a.dtype != m.dtype:
        common = torch.promote_types(a.dtype, m.dtype)
        a, m = a.to(common), m.to(common)
    force = a.dtype
    if p.dtype == torch.float32 and force in (torch.float16, torch.bfloat16, torch.float32):
        pass
    elif p.dtype == torch.float64 and force == torch.float64:
        pass
    else:
        raise ValueError(f"unsupported residual/force dtypes {p.dtype}/{force} for the HIP "
                         "residual kernels")
    if p.shape != a.shape or (m is not None and m.shape != a.shape):
        raise ValueError("residual state and force terms must have the same shape")
    return p.contiguous(), a.contiguous(), (m.contiguous() if m is not None else None)


class MidpointStep(torch.autograd.Function):
    """out = p + sign * round(round(a + m) * scale); grads: dp = dout,
    da = dm = sign * round(round(dout) * scale) (autograd through the eager form).
    The backward needs no forward value: with ``graph_only`` the output is
    allocated but not computed (for a rebuilt graph whose output value is
    never read, only differentiated)."""

    @staticmethod
    def forward(ctx, p, a, m, scale, sign, graph_only=False):
        p, a, m = _state_force(p, a, m)
        ctx.scale, ctx.sign, ctx.force_dtype = float(scale), int(sign), a.dtype
        if graph_only:
            return torch.empty_like(p)
        return ops.midpoint_update(p, a, m, float(scale), int(sign))

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        dout = dout.contiguous()
        da = ops.midpoint_update_bwd(dout, ctx.scale, ctx.sign, ctx.force_dtype)
        return dout, da, da, None, None, None


class EulerStep(torch.autograd.Function):
    """out = x + sign * f; grads: dx = dout, df = sign * dout cast to f's dtype.
    ``graph_only``: as MidpointStep's."""

    @staticmethod
    def forward(ctx, x, f, sign, graph_only=False):
        x, f, _ = _state_force(x, f)
        ctx.sign, ctx.force_dtype = int(sign), f.dtype
        if graph_only:
            return torch.empty_like(x)
        return ops.residual_axpy(x, f, int(sign))

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        df = dout if ctx.sign > 0 else -dout
        return dout, df.to(ctx.force_dtype), None, None


_EAGER = contextvars.ContextVar("reversability_amd_eager_updates", default=False)


@contextlib.contextmanager
def eager_updates(enabled: bool = True):
    """Inside this block, ``midpoint_step`` / ``euler_step`` evaluate the
    reference's eager torch expression on every device (no HIP kernel).
    The reversible stack Functions record the mode of their forward and
    re-enter it in their backward, which autograd runs on another thread."""
    token = _EAGER.set(bool(enabled))
    try:
        yield
    finally:
        _EAGER.reset(token)


def eager_active() -> bool:
    """Whether ``eager_updates`` is in effect here."""
    return _EAGER.get()


def midpoint_step(p, a, m, scale, sign, graph_only=False):
    """p + sign * scale * (a + m) with the eager rounding points.  ``graph_only``
    (GPU only): the caller differentiates the result but never reads it, so the
    value is not computed (its memory is left as allocated)."""
    if p.device.type == "cuda" and not _EAGER.get():
        return MidpointStep.apply(p, a, m, scale, sign, graph_only)
    force = a + m
    return p + scale * force if sign > 0 else p - scale * force


def euler_step(x, f, sign, graph_only=False):
    """x + sign * f (state dtype = x's); ``graph_only`` as midpoint_step's."""
    if x.device.type == "cuda" and not _EAGER.get():
        return EulerStep.apply(x, f, sign, graph_only)
    return x + f if sign > 0 else x - f
