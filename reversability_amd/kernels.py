"""Fused cross-entropy and SwiGLU on gfx950, behind the reference's operator surface.

``TiledCrossEntropy`` / ``cross_entropy_sum`` mirror src/reversibility/kernels.py:56-85:
``apply(logits, labels)`` takes contiguous ``[tokens, vocab]`` fp16/fp32 logits
and int64 labels on the same device and returns the summed loss (fp32); rows
labelled -100 contribute nothing.  It keeps the reference's Half-logsoftmax ->
fp32 NLL policy: the log-probability at the target is rounded to the logits
dtype before it is negated and summed, and the backward rounds the
log-probability again before the exponential.  One HIP kernel reads each row
once per pass (rv_ce_fwd / rv_ce_bwd).

``FusedSwiGLU`` / ``enable_swiglu`` mirror src/reversibility/kernels.py:113-138:
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


IGNORE_INDEX = -100


class TiledCrossEntropy(torch.autograd.Function):
    """Summed cross-entropy over vocabulary rows (kernels.py:56-80)."""

    @staticmethod
    def forward(ctx, logits, labels):
        if logits.device.type != "cuda" or logits.dtype not in (torch.float16, torch.float32):
            raise ValueError("Fused CE requires CUDA (ROCm device) FP16/FP32 logits; "
                             "no silent fallback")
        if (logits.ndim != 2 or not logits.is_contiguous() or labels.device != logits.device
                or labels.dtype != torch.int64 or labels.numel() != logits.shape[0]):
            raise ValueError("Contiguous [tokens,vocab] logits and matching CUDA int64 labels "
                             "required")
        labels = labels.contiguous()
        row_max, row_lse, losses = ops.ce_fwd(logits, labels, IGNORE_INDEX)
        ctx.save_for_backward(logits, labels, row_max, row_lse)
        return losses.sum()

    @staticmethod
    @once_differentiable
    def backward(ctx, gradient):
        logits, labels, row_max, row_lse = ctx.saved_tensors
        grad = gradient.detach().to(torch.float32).reshape(1).contiguous()
        return ops.ce_bwd(logits, labels, row_max, row_lse, grad, IGNORE_INDEX), None


def cross_entropy_sum(logits, labels):
    """Sum of per-token cross-entropy losses (kernels.py:83-84)."""
    return TiledCrossEntropy.apply(logits, labels)


VOCAB_ALIGN = 64  # padded logits row stride (in elements) of tied_head_ce
# widest row rv_ce_fused keeps in registers (32 16-byte vectors per thread)
FUSED_CE_MAX_COLS = 65536


def tied_head_ce(x16: torch.Tensor, head16: torch.Tensor, vocab: int, labels: torch.Tensor,
                 grad: torch.Tensor, dx_out: torch.Tensor | None = None):
    """One chunk of the tied head and its summed cross-entropy, forward and
    backward, with the logits stored at a padded row stride.

    The same computation as ``cross_entropy_sum(F.linear(x16, head16[:vocab]),
    labels)`` under fp16 autocast followed by its backward with upstream
    gradient ``grad`` (a device fp32 scalar): logits = fp16(x16 W^T); loss and
    dlogits from one pass of rv_ce_fused over each logits row (the two-pass
    rv_ce_fwd / rv_ce_bwd above FUSED_CE_MAX_COLS, same bits); dx = dlogits W and
    dW = dlogits^T x16 (fp16, as autocast's linear produces them).  ``head16`` is
    the fp16 head with its rows padded to a multiple of VOCAB_ALIGN (the pad
    rows zero), so every logits row starts 16-byte aligned: with the odd
    vocabulary (50257) as the row stride, hipBLASLt's GEMMs over the logits
    run 15-25% slower on MI355X.  Returns (loss sum, dx16, dW16 [vocab, d]);
    dx16 is written into ``dx_out`` (contiguous fp16 [rows, d]) when given.
    """
    rows, d = x16.shape
    padded = head16.shape[0]
    if (x16.dtype != torch.float16 or head16.dtype != torch.float16 or not x16.is_contiguous()
            or not head16.is_contiguous() or head16.shape[1] != d or padded % VOCAB_ALIGN
            or not 0 < vocab <= padded or labels.dtype != torch.int64
            or labels.numel() != rows or not x16.is_cuda):
        raise ValueError("tied_head_ce needs contiguous CUDA fp16 x [rows, d], a padded fp16 "
                         "head [padded, d] and int64 labels [rows]")
    from ._hip import RV_F16, _check, _stream, library
    lib = library()
    labels = labels.contiguous()
    logits = torch.mm(x16, head16.t())                       # [rows, padded] fp16
    rmax, rlse, losses = (torch.empty(rows, device=x16.device, dtype=torch.float32)
                          for _ in range(3))
    st = _stream(x16)
    if rows and vocab <= FUSED_CE_MAX_COLS:
        # one pass: loss and gradient, written over the logits
        dlogits = logits
        _check(lib.rv_ce_fused(logits.data_ptr(), RV_F16, padded, labels.data_ptr(), rows, vocab,
                               IGNORE_INDEX, grad.data_ptr(), rmax.data_ptr(), rlse.data_ptr(),
                               losses.data_ptr(), dlogits.data_ptr(), st), "rv_ce_fused")
    else:
        dlogits = torch.empty_like(logits)
        if rows:
            _check(lib.rv_ce_fwd(logits.data_ptr(), RV_F16, padded, labels.data_ptr(), rows,
                                 vocab, IGNORE_INDEX, rmax.data_ptr(), rlse.data_ptr(),
                                 losses.data_ptr(), st), "rv_ce_fwd")
            _check(lib.rv_ce_bwd(logits.data_ptr(), RV_F16, padded, labels.data_ptr(),
                                 rmax.data_ptr(), rlse.data_ptr(), grad.data_ptr(), rows, vocab,
                                 IGNORE_INDEX, dlogits.data_ptr(), st), "rv_ce_bwd")
    del logits
    d_view = dlogits[:, :vocab]
    if dx_out is not None:
        dx16 = torch.mm(d_view, head16[:vocab], out=dx_out)
    else:
        dx16 = torch.mm(d_view, head16[:vocab])
    dw16 = torch.mm(d_view.t(), x16)
    return losses.sum(), dx16, dw16


def padded_head(weight: torch.Tensor) -> torch.Tensor:
    """fp16 copy of a [vocab, d] head with zero rows up to a multiple of VOCAB_ALIGN."""
    vocab, d = weight.shape
    padded = -(-vocab // VOCAB_ALIGN) * VOCAB_ALIGN
    head = torch.empty(padded, d, device=weight.device, dtype=torch.float16)
    head[:vocab].copy_(weight)
    head[vocab:].zero_()
    return head


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
