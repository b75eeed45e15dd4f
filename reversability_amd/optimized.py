"""Optimized midpoint training paths (src/reversibility/optimized.py:9-101).

``ReusedMidpoint`` builds one force graph per layer in backward that serves both
the inversion and the VJP: the current ``p`` IS the previous ``q``, so
``F = 2h f(p)`` reconstructs ``previous_p = q - F`` and, through
``previous_p + F``, differentiates the layer -- one force evaluation per layer
instead of the reference stack's two.  On ROCm tensors both residual updates
are the fused ``rv_midpoint_update`` kernel.
"""
from __future__ import annotations

import contextlib

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from .residual import eager_active, eager_updates, midpoint_step
from .reversible import midpoint_terms


class ReusedMidpoint(torch.autograd.Function):
    @staticmethod
    def forward(ctx, p, q, blocks, h, *parameters):
        ctx.blocks, ctx.h = blocks, h
        ctx.eager = eager_active()
        ctx.device = p.device.type
        ctx.amp = torch.is_autocast_enabled(ctx.device)
        ctx.dtype = torch.get_autocast_dtype(ctx.device)
        for block in blocks:
            attention, mlp = midpoint_terms(block, q)
            p, q = q, midpoint_step(p, attention, mlp, 2 * h, +1)
        ctx.save_for_backward(p, q, *parameters)
        return p, q

    @staticmethod
    @once_differentiable
    def backward(ctx, dp, dq):
        p, q, *_ = ctx.saved_tensors
        grads: list = []
        scale = 2 * ctx.h
        # No autocast weight-cast cache: see _InverseStack.backward.
        with torch.autocast(ctx.device, enabled=ctx.amp, dtype=ctx.dtype,
                            cache_enabled=False), eager_updates(ctx.eager):
            for block in reversed(ctx.blocks):
                with torch.enable_grad():
                    previous_q = p.detach().requires_grad_(True)
                    attention, mlp = midpoint_terms(block, previous_q)
                    with torch.no_grad():
                        previous_p = midpoint_step(q, attention.detach(), mlp.detach(), scale, -1)
                    previous_p.requires_grad_(True)
                    # only differentiated: its value is never read
                    next_q = midpoint_step(previous_p, attention, mlp, scale, +1, graph_only=True)
                    # (previous_q, next_q) are the layer's outputs (next_p, next_q).
                    local = torch.autograd.grad((previous_q, next_q),
                                                (previous_p, previous_q, *block.parameters()),
                                                (dp, dq))
                dp, dq = local[0], local[1]
                grads[0:0] = local[2:]
                p, q = previous_p.detach(), previous_q.detach()
                del attention, mlp, next_q, local
        return (dp, dq, None, None, *grads)


def hidden_states(model, ids, reuse=False):
    """embedding -> core -> final_norm (optimized.py:44-61)."""
    if ids.ndim != 2 or ids.shape[1] > model.config.max_sequence_length:
        raise ValueError("Invalid input shape/context")
    x = model.embed(ids)  # token + position embedding (fused once enable_embedding ran)
    if hasattr(model, "core"):
        if reuse:
            if model.method != "midpoint" or model.backward_mode != "reconstruct":
                raise ValueError("Force reuse requires reconstructed midpoint")
            _, x = ReusedMidpoint.apply(x, x, model.blocks, model.step_size,
                                        *model.blocks.parameters())
        else:
            x = model.core(x)
    else:
        if reuse:
            raise ValueError("Force reuse requires midpoint")
        for block in model.blocks:
            x = block(x)
    return model.final_norm(x)


_AMP_DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


def amp_context(device, precision, cache=True):
    """Autocast on GPU for fp16/bf16, a no-op on CPU (optimized.py:64-67)."""
    if device.type == "cuda" and precision != "fp32":
        return torch.autocast("cuda", dtype=_AMP_DTYPES[precision], cache_enabled=cache)
    return contextlib.nullcontext()


def chunked_backward(model, ids, labels, denominator, chunk_tokens, scaler=None,
                     precision="fp32", reuse=False, loss_backend="torch"):
    """One core forward/backward, head + loss in token chunks (optimized.py:70-101).

    Each chunk's vocabulary graph is released right after its backward; the
    tied head/embedding weight accumulates its gradient across chunks; the
    core backward runs once on the accumulated hidden-state gradient.
    """
    if chunk_tokens <= 0 or denominator <= 0:
        raise ValueError("Chunk size and normalization denominator must be positive")
    from .mlp import prefetch_casts, weight_cast_cache
    from .optimized_v3 import castable_weights
    with weight_cast_cache():  # weights are constant until the optimizer step
        if precision == "fp16" and ids.device.type == "cuda":
            prefetch_casts(castable_weights(model))
        return _chunked_backward(model, ids, labels, denominator, chunk_tokens, scaler,
                                 precision, reuse, loss_backend)


def _chunked_backward(model, ids, labels, denominator, chunk_tokens, scaler, precision, reuse,
                      loss_backend):
    with amp_context(ids.device, precision):
        hidden = hidden_states(model, ids, reuse)
    leaf = hidden.detach().reshape(-1, hidden.shape[-1]).requires_grad_(True)
    targets = labels.reshape(-1)
    total = torch.zeros((), device=ids.device, dtype=torch.float32)
    for start in range(0, len(targets), chunk_tokens):
        with amp_context(ids.device, precision, cache=False):
            logits = F.linear(leaf[start:start + chunk_tokens], model.lm_head.weight)
            loss = _chunk_loss(logits, targets[start:start + chunk_tokens], loss_backend)
            normalized = loss / denominator
            (normalized if scaler is None else scaler.scale(normalized)).backward()
        total += loss.detach().float()
        del logits, loss, normalized
    with amp_context(ids.device, precision):
        hidden.backward(leaf.grad.reshape_as(hidden))
    return total


def _chunk_loss(logits, targets, loss_backend):
    """Summed chunk loss.  ``"torch"`` is eager F.cross_entropy; ``"triton"``
    (the reference's name for its fused loss, optimized.py:91-93) and
    ``"hip"`` select the fused HIP cross-entropy."""
    if loss_backend == "torch":
        return F.cross_entropy(logits, targets, ignore_index=-100, reduction="sum")
    if loss_backend in ("triton", "hip"):
        from .kernels import cross_entropy_sum
        return cross_entropy_sum(logits, targets)
    raise ValueError("Unknown loss backend")

