"""Causal self-attention on the gfx950 MFMA kernels (src/reversibility/model.py:26-45).

The reference's ``CausalSelfAttention`` projects to a packed ``qkv`` of width
``3 d``, views it as ``[B, T, 3, H, hd]``, permutes it into three strided
``[B, H, T, hd]`` tensors for ``F.scaled_dot_product_attention(is_causal=True)``,
and transposes the result back to ``[B, T, d]`` for the output projection;
autograd then stacks ``dq, dk, dv`` back into the packed layout.  Here the
kernels read ``qkv`` in the layout the qkv GEMM wrote, write the output in the
layout the output GEMM reads, and write the gradient straight into a packed
``dqkv`` (``rv_attn_fwd`` / ``rv_attn_bwd``, csrc/attention.hip): no permute,
transpose or concatenation copies.  Forward keeps the base-2 log-sum-exp per
query; backward is deterministic (no atomics).

``enable_attention(model)`` patches every block's ``attn.forward``; calls the
kernels do not cover (no fp16 ``qkv`` -- i.e. not under fp16 autocast --, head
sizes other than 32/64/128, dropout in training mode, CPU tensors) keep the
reference computation, recorded in ``paths.report()`` (or raising under
``paths.strict()``).
"""
from __future__ import annotations

import types

import torch
import torch.nn.functional as F
from torch.autograd.function import once_differentiable

from . import paths
from ._hip import _check, _stream, library

HEAD_DIMS = (32, 64, 128)


def supported(qkv: torch.Tensor, heads: int, dropout: float = 0.0) -> bool:
    if not (qkv.is_cuda and qkv.dtype == torch.float16 and qkv.ndim == 3 and dropout == 0.0):
        return False
    width = qkv.shape[-1]
    return width % (3 * heads) == 0 and width // (3 * heads) in HEAD_DIMS


class CausalAttention(torch.autograd.Function):
    """``qkv`` fp16 ``[B, T, 3 d]`` -> causal attention output fp16 ``[B, T, d]``."""

    @staticmethod
    def forward(ctx, qkv, heads):
        batch, seq, width = qkv.shape
        d = width // 3
        qkv = qkv.contiguous()
        out = torch.empty(batch, seq, d, device=qkv.device, dtype=torch.float16)
        lse = torch.empty(batch * heads, seq, device=qkv.device, dtype=torch.float32)
        _check(library().rv_attn_fwd(qkv.data_ptr(), batch, seq, heads, d // heads,
                                     out.data_ptr(), lse.data_ptr(), _stream(qkv)), "rv_attn_fwd")
        ctx.save_for_backward(qkv, out, lse)
        ctx.heads = heads
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        qkv, out, lse = ctx.saved_tensors
        batch, seq, width = qkv.shape
        heads = ctx.heads
        lib = library()
        dout = dout.to(torch.float16).contiguous()
        dqkv = torch.empty_like(qkv)
        nbytes = lib.rv_attn_bwd_workspace_bytes(batch, seq, heads)
        if nbytes < 0:
            _check(-nbytes, "rv_attn_bwd_workspace_bytes")
        ws = torch.empty(nbytes // 4, device=qkv.device, dtype=torch.float32)
        _check(lib.rv_attn_bwd(qkv.data_ptr(), out.data_ptr(), dout.data_ptr(), lse.data_ptr(),
                               batch, seq, heads, width // 3 // heads, dqkv.data_ptr(),
                               ws.data_ptr(), nbytes, _stream(qkv)), "rv_attn_bwd")
        return dqkv, None


def causal_attention(qkv: torch.Tensor, heads: int) -> torch.Tensor:
    """Causal attention of a packed fp16 ``qkv`` on the kernels; raises on inputs
    they do not cover."""
    if not supported(qkv, heads):
        raise ValueError("fused attention needs a CUDA fp16 qkv [B, T, 3 d] with head size "
                         f"in {HEAD_DIMS}")
    return CausalAttention.apply(qkv, heads)


def reference_attention(qkv: torch.Tensor, heads: int, dropout: float = 0.0) -> torch.Tensor:
    """The reference's computation (model.py:40-45) on a packed ``qkv``."""
    batch, length, width = qkv.shape
    d = width // 3
    q, k, v = qkv.view(batch, length, 3, heads, d // heads).permute(2, 0, 3, 1, 4).unbind(0)
    mixed = F.scaled_dot_product_attention(q, k, v, dropout_p=dropout, is_causal=True)
    return mixed.transpose(1, 2).reshape(batch, length, d)


def enable_attention(model: torch.nn.Module) -> None:
    """Route every block's attention through the fused kernels where they apply."""
    def forward(attn, x):
        qkv = attn.qkv(x)
        dropout = attn.dropout if attn.training else 0.0
        if supported(qkv, attn.n_heads, dropout):
            paths.took("attention", "hip")
            mixed = CausalAttention.apply(qkv, attn.n_heads)
        else:
            paths.took("attention", "sdpa",
                       f"attention kernels need a CUDA fp16 qkv, head size in {HEAD_DIMS} and no "
                       f"dropout (got {qkv.dtype} on {qkv.device.type}, head size "
                       f"{qkv.shape[-1] // (3 * attn.n_heads)}, dropout {dropout})")
            mixed = reference_attention(qkv, attn.n_heads, dropout)
        return attn.proj(mixed)
    for block in model.blocks:
        block.attn.forward = types.MethodType(forward, block.attn)
