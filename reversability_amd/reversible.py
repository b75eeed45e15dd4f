"""Reversible integrators and the stack-level reconstruction backward.

Restates src/reversibility/reversible.py:16-118 (paper Eq. 2.4/2.5 midpoint,
Eq. 2.8/2.9 Hamiltonian Euler):

* midpoint:  (p, q) -> (q, p + 2h f(q)),   f(x) = A(x) + M(x + A(x)),
  inverse    (p, q) -> (q - 2h f(p), p);
* Euler:     q' = q + A(p), p' = p + M(q');  inverse p = p' - M(q'), q = q' - A(p);
  A = attn . attn_norm, M = mlp . mlp_norm.

``_InverseStack`` keeps only the final pair and parameter references; its
backward walks the layers in reverse, reconstructs each layer's input under
no_grad, rebuilds that one layer's graph with the forward's autocast mode and
takes its VJP (for Euler the inversion's evaluation of A(p0) is itself the
graph's, computed once instead of twice; same values).  Parameter gradients are returned through autograd (never
written to ``.grad``).  On ROCm tensors the residual updates run as fused HIP
kernels (``residual.midpoint_step`` / ``residual.euler_step``) with the eager
expression's rounding points.
"""
from __future__ import annotations

import contextlib
import math

import torch
from torch.autograd.function import once_differentiable

from . import paths
from ._hip import ops
from .kernels_v3 import (FusedAddRMSNorm, _fp16_norm_input, add_rms_norm, inverse_add_rms_norm,
                         inverse_rms_norm, rms_norm_eps, rms_norm_pass)
from .mlp import output_unused
from .model import BaselineLM, Block, ModelConfig
from .residual import eager_active, eager_updates, euler_step, midpoint_step


def midpoint_terms(block: Block, x: torch.Tensor):
    """(A(x), M(x + A(x))) -- the two summands of the midpoint force (the add
    and M's norm in one pass where the fused norm applies)."""
    attention = block.attn(block.attn_norm(x))
    return attention, block.mlp(add_rms_norm(x, attention, block.mlp_norm)[1])


def midpoint_force(block: Block, x: torch.Tensor) -> torch.Tensor:
    """f(x) = A(x) + M(x + A(x))  (reversible.py:16-18)."""
    attention, mlp = midpoint_terms(block, x)
    return attention + mlp


def forward_pair(block, p, q, method, h):
    """One integrator step (reversible.py:21-25)."""
    if method == "midpoint":
        attention, mlp = midpoint_terms(block, q)
        return q, midpoint_step(p, attention, mlp, 2 * h, +1)
    next_q, normed = add_rms_norm(q, block.attn(block.attn_norm(p)), block.mlp_norm)
    return euler_step(p, block.mlp(normed), +1), next_q


def euler_forward(blocks, p, q):
    """forward_pair's Euler steps over a stack, each p' = p + M(q') made in one
    pass with the next block's attn_norm(p') (add_rms_norm: the residual add
    and the norm where the fused kernels apply, else the add and the norm), so
    the next block reads its normalized input instead of normalizing p' again.
    The same values as calling forward_pair block by block."""
    normed = None
    for i, block in enumerate(blocks):
        if normed is None:
            normed = block.attn_norm(p)
        next_q, mlp_in = add_rms_norm(q, block.attn(normed), block.mlp_norm)
        force = block.mlp(mlp_in)
        if i + 1 < len(blocks):
            p, normed = add_rms_norm(p, force, blocks[i + 1].attn_norm)
        else:
            p = euler_step(p, force, +1)
        q = next_q
    return p, q


def inverse_pair(block, p, q, method, h):
    """Algebraic inverse of forward_pair (reversible.py:28-32)."""
    if method == "midpoint":
        attention, mlp = midpoint_terms(block, p)
        return midpoint_step(q, attention, mlp, 2 * h, -1), p
    previous_p = euler_step(p, block.mlp(block.mlp_norm(q)), -1)
    return previous_p, euler_step(q, block.attn(block.attn_norm(previous_p)), -1)


# The model's switches of the reconstruction backward (paths.ReconstructionPaths):
#   reuse_euler_attention   the Euler reconstruction evaluates A(p0) on the
#       recovered p0 twice -- to invert the step and again in the recompute for
#       the VJP -- on identical bits; the inversion keeps that evaluation's
#       graph for the VJP (_euler_inverse_for_vjp);
#   fuse_euler_inverse      the inversion's subtractions p - M(q) and q - A(p0)
#       computed in the passes of the norms that read their results;
#   skip_unused_mlp_output  the Euler VJP's rebuilt MLP output feeds only the
#       graph-only next_p, so install_v3's tiled MLP does not compute it;
#   euler_mlp_at_stored_q   the inversion's M(q) is made with its graph and
#       serves the VJP (_euler_layer_vjp): M is linearised at the stored q,
#       where the forward evaluated it, instead of at the rebuilt q0 + A(p0).
# The first three give the same values as the plain inverse-then-recompute;
# the last changes the gradients within the rounding of q0 + A(p0).


def _grads_in_order(block, params, grads):
    by_id = {id(w): g for w, g in zip(params, grads)}
    return [by_id[id(w)] for w in block.parameters()]


def _euler_layer_vjp(block, p, q, dp, dq, settings, dp16=None, lower=None, pre_q=None):
    """Invert one Euler step -- (p, q) = (p0 + M(q), q0 + A(p0)) -- and take its
    VJP with one evaluation of each force, both with their graphs: M at the
    stored q (it inverts the step and, linearised there, serves the VJP) and
    A at the recovered p0.  The VJP runs in two phases: the MLP's, giving the
    gradient at M's input, then the step's rest (A, both norms and the
    residual sums) with that gradient entering at the rebuilt q0 + A(p0).
    ``dp16``: fp16(dp) if the caller has it (the layer above's p0 gradient,
    written by its norm backward), handed to an fp16 force as is -- the value
    autograd's cast of dp would give.  ``lower``: the block below, whose M
    input -- its mlp_norm of q0 -- is made with q0 = q - A(p0) in one pass
    when ``fuse_euler_inverse`` is set and the fused norms apply; ``pre_q``:
    that (y, rstd) of this block's q, made by the layer above.  Returns (p0,
    q0, dp0, dq0, parameter gradients in block.parameters() order, fp16(dp0)
    or None, the (y, rstd) for ``lower`` or None)."""
    # the states may be the stack's own saved outputs: nothing here may extend
    # their history (a graph reaching the stack node would re-enter its backward)
    p, q = p.detach(), q.detach()
    fused = _fp16_norm_input(block.mlp_norm, q)
    with torch.enable_grad():
        if fused:  # M's input is the fp16 norm of the stored q (graph from its leaf)
            y_q, rstd_q = pre_q if pre_q is not None else ops.rmsnorm_fwd(
                q, block.mlp_norm.weight.contiguous(), rms_norm_eps(block.mlp_norm, q), True)
            m_in = y_q.requires_grad_(True)
            force = block.mlp(m_in)
        else:  # M's input is the stored state itself
            m_in = q.detach().requires_grad_(True)
            force = block.mlp(block.mlp_norm(m_in))
    with torch.no_grad():
        if settings.fuse_euler_inverse:  # p0 and attn_norm(p0) in one pass
            p0, pre_p0 = inverse_rms_norm(p, force.detach(), block.attn_norm)
        else:
            p0, pre_p0 = euler_step(p, force.detach(), -1), None
    # fp16(dp0) from p0's norm backward when the fused path runs, for the lower
    # layer's force -- fp16 like this one's (asked only then)
    half_dp0: list = []
    with torch.enable_grad():
        p0 = p0.detach().requires_grad_(True)
        p0_pass, normed_p0 = rms_norm_pass(p0, block.attn_norm, pre_p0,
                                           half_dp0 if force.dtype == torch.float16 else None)
        attention = block.attn(normed_p0)
    with torch.no_grad():
        if settings.fuse_euler_inverse and lower is not None:
            q0, pre_lower = inverse_rms_norm(q, attention.detach(), lower.mlp_norm)
        else:
            q0, pre_lower = euler_step(q, attention.detach(), -1), None
    q0.requires_grad_(True)
    mlp_params = tuple(block.mlp.parameters()) if fused else (*block.mlp_norm.parameters(),
                                                              *block.mlp.parameters())
    attn_params = (*block.attn_norm.parameters(), *block.attn.parameters())
    with torch.enable_grad():
        grad_force = dp16 if dp16 is not None and force.dtype == torch.float16 else dp
        first = torch.autograd.grad(force, (m_in, *mlp_params), grad_force)
        del force
        if fused:  # next_q = q0 + A(p0) carrying the value q and its norm
            next_q, y = FusedAddRMSNorm.apply(q0, attention, block.mlp_norm.weight,
                                              rms_norm_eps(block.mlp_norm, q), (q, y_q, rstd_q))
            norm_params = tuple(block.mlp_norm.parameters())
            rest = torch.autograd.grad((next_q, y, p0_pass), (p0, q0, *attn_params, *norm_params),
                                       (dq, first[0], dp))
            grads = _grads_in_order(block, (*attn_params, *norm_params, *mlp_params),
                                    (*rest[2:], *first[1:]))
        else:  # next_q = q0 + A(p0), its gradient dq plus M's input gradient
            next_q = euler_step(q0, attention, +1, graph_only=True)
            rest = torch.autograd.grad((next_q, p0_pass), (p0, q0, *attn_params),
                                       (dq + first[0], dp))
            grads = _grads_in_order(block, (*attn_params, *mlp_params), (*rest[2:], *first[1:]))
    return (p0.detach(), q0.detach(), rest[0], rest[1], grads,
            half_dp0[0] if half_dp0 else None, pre_lower)


def _euler_inverse_for_vjp(block, p, q, settings):
    """Invert one Euler step and rebuild its graph with one evaluation of
    A(p0): p0 = p - M(q) (no graph), a = A(p0) with its graph, q0 = q - a, then
    next_q = q0 + a and next_p = p0 + M(next_q) as forward_pair computes them.
    Returns (next_p, next_q, p0, q0) with p0, q0 the graph's leaves; next_p is
    for differentiation only (on the GPU its value is not computed)."""
    fuse = settings.fuse_euler_inverse
    with torch.no_grad():
        force = block.mlp(block.mlp_norm(q))
        if fuse:  # p0 and attn_norm(p0) in one pass
            p0, pre_p0 = inverse_rms_norm(p, force, block.attn_norm)
        else:
            p0, pre_p0 = euler_step(p, force, -1), None
        del force
    with torch.enable_grad():
        p0 = p0.detach().requires_grad_(True)
        # p0 feeds attn_norm and next_p: its two gradients are summed in the
        # norm's backward pass (rms_norm_pass)
        p0_pass, normed_p0 = rms_norm_pass(p0, block.attn_norm, pre_p0)
        attention = block.attn(normed_p0)
        if fuse:  # q0, q0 + A(p0) and its norm in one pass
            q0, pre_q = inverse_add_rms_norm(q, attention.detach(), block.mlp_norm)
        else:
            with torch.no_grad():
                q0 = euler_step(q, attention.detach(), -1)
            pre_q = None
        q0 = q0.detach().requires_grad_(True)
        next_q, normed = add_rms_norm(q0, attention, block.mlp_norm, pre_q)
        # next_p is only differentiated (its value is never read), and so is
        # the MLP output it adds: a tiled MLP skips its down projection
        with output_unused() if settings.skip_unused_mlp_output else contextlib.nullcontext():
            force = block.mlp(normed)
        next_p = euler_step(p0_pass, force, +1, graph_only=True)
    return next_p, next_q, p0, q0


class _InverseStack(torch.autograd.Function):
    """Whole-stack Function; backward reconstructs inputs layer by layer."""

    @staticmethod
    def forward(ctx, p, q, blocks, method, h, *parameters):
        ctx.blocks, ctx.method, ctx.h = blocks, method, h
        ctx.eager = eager_active()
        ctx.device_type = p.device.type
        ctx.amp_enabled = torch.is_autocast_enabled(ctx.device_type)
        ctx.amp_dtype = torch.get_autocast_dtype(ctx.device_type)
        if method == "euler":
            p, q = euler_forward(blocks, p, q)
        else:
            for block in blocks:
                p, q = forward_pair(block, p, q, method, h)
        ctx.save_for_backward(p, q, *parameters)
        return p, q

    @staticmethod
    @once_differentiable
    def backward(ctx, dp, dq):
        p, q, *_ = ctx.saved_tensors
        p, q = p.detach(), q.detach()  # the forward's outputs: no history of this node
        grads: list = []
        settings = paths.of(ctx.blocks)
        # cache_enabled=False: torch <= 2.10 caches autocast weight casts made
        # under no_grad (the inverse below) and hands them, without autograd
        # history, to the grad-enabled recompute.  Casts are deterministic, so
        # skipping the cache changes no value.
        with torch.autocast(ctx.device_type, enabled=ctx.amp_enabled, dtype=ctx.amp_dtype,
                            cache_enabled=False), eager_updates(ctx.eager):
            dp16 = pre_q = None
            for index in reversed(range(len(ctx.blocks))):
                block = ctx.blocks[index]
                if ctx.method == "euler" and settings.euler_mlp_at_stored_q:
                    lower = ctx.blocks[index - 1] if index > 0 else None
                    p, q, dp, dq, layer, dp16, pre_q = _euler_layer_vjp(
                        block, p, q, dp, dq, settings, dp16, lower, pre_q)
                    grads[0:0] = layer
                    continue
                dp16 = pre_q = None
                if ctx.method == "euler" and settings.reuse_euler_attention:
                    next_p, next_q, p0, q0 = _euler_inverse_for_vjp(block, p, q, settings)
                else:
                    with torch.no_grad():
                        p0, q0 = inverse_pair(block, p, q, ctx.method, ctx.h)
                    with torch.enable_grad():
                        p0 = p0.detach().requires_grad_(True)
                        q0 = q0.detach().requires_grad_(True)
                        next_p, next_q = forward_pair(block, p0, q0, ctx.method, ctx.h)
                with torch.enable_grad():
                    local = torch.autograd.grad((next_p, next_q), (p0, q0, *block.parameters()),
                                                (dp, dq))
                dp, dq = local[0], local[1]
                grads[0:0] = local[2:]
                p, q = p0.detach(), q0.detach()
        return (dp, dq, None, None, None, *grads)


class ReversibleLM(BaselineLM):
    """BaselineLM whose block stack is a reversible integrator (reversible.py:72-107)."""

    def __init__(self, config: ModelConfig, method: str, step_size: float = 0.5,
                 backward_mode: str = "reconstruct") -> None:
        if method not in {"midpoint", "euler"}:
            raise ValueError("method must be midpoint or euler")
        if not math.isfinite(step_size) or step_size <= 0:
            raise ValueError("step size must be finite and positive")
        if method == "euler" and step_size != 0.5:
            raise ValueError("Euler has unit coefficients; step_size applies only to midpoint")
        if backward_mode not in {"reconstruct", "autograd"}:
            raise ValueError("unsupported backward mode")
        if config.dropout != 0:
            raise ValueError("reconstruction requires dropout=0; RNG replay is not implemented")
        super().__init__(config)
        self.method, self.step_size, self.backward_mode = method, step_size, backward_mode

    def core(self, x):
        # Boundary: p = q = embedding for both integrators.  The head reads q
        # (midpoint) or p (Euler).
        p = q = x
        if self.backward_mode == "reconstruct" and torch.is_grad_enabled():
            p, q = _InverseStack.apply(p, q, self.blocks, self.method, self.step_size,
                                       *self.blocks.parameters())
        else:
            for block in self.blocks:
                p, q = forward_pair(block, p, q, self.method, self.step_size)
        return q if self.method == "midpoint" else p

    def forward(self, input_ids):
        return self.lm_head(self.final_norm(self.core(self.embed(input_ids))))


def build_model(config: dict):
    """Model factory over a study config dict (reversible.py:110-118)."""
    model_config = ModelConfig(**config["model"])
    method = config.get("method", "baseline")
    if method == "baseline":
        return BaselineLM(model_config)
    if config.get("compile"):
        raise ValueError("compiled inverse backward is not validated")
    return ReversibleLM(model_config, method, config.get("step_size", 0.5),
                        config.get("backward_mode", "reconstruct"))
