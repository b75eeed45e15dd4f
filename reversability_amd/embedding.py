"""Token + position embedding on the gfx950 kernels: the boundary in front of
the reversible stack, ``p = q = token_embedding(ids) +
position_embedding(arange(T))`` (src/reversibility/reversible.py:105-106;
src/reversibility/model.py, the two ``nn.Embedding`` and the broadcast add).

Forward: one kernel writes ``tok[ids] + pos[:T]`` (``rv_embed_fwd``) instead
of two gathers and an add.  Backward (``rv_embed_bwd``): the position gradient
is the batch sum in order; the token gradient is a deterministic segmented
sum over the id-sorted tokens (no floating-point atomics, bit-identical run to
run).

The token table is tied to the LM head, whose gradient the chunked-head
trainers (``cached_head_backward``) already hold in ``weight.grad`` when the
stack's backward reaches the embedding.  With ``into_grad=True`` the token
gradient is added into that ``weight.grad`` in place -- what ``AccumulateGrad``
does with the returned gradient -- touching only the rows of ids that occur,
instead of materialising a dense ``[vocab, d]`` gradient and adding it.  In
that mode no gradient is returned for the token table, so
``torch.autograd.grad`` with respect to it, and hooks on it, do not see the
embedding's share; when ``weight.grad`` is not set yet a dense gradient is
returned as usual.
"""
from __future__ import annotations

import types

import torch
from torch.autograd.function import once_differentiable

from ._hip import _check, _stream, library


def supported(ids: torch.Tensor, token_weight: torch.Tensor, position_weight: torch.Tensor) -> bool:
    """Whether the kernels cover this call (fp32 CUDA tables, d a multiple of 4)."""
    d = token_weight.shape[-1]
    return (ids.is_cuda and ids.dtype == torch.int64 and ids.ndim == 2
            and token_weight.is_cuda and position_weight.is_cuda
            and token_weight.dtype == torch.float32 and position_weight.dtype == torch.float32
            and token_weight.ndim == 2 and position_weight.ndim == 2
            and position_weight.shape[1] == d and d % 4 == 0
            and token_weight.is_contiguous() and position_weight.is_contiguous()
            and token_weight.data_ptr() % 16 == 0 and position_weight.data_ptr() % 16 == 0)


class TokenPositionEmbedding(torch.autograd.Function):
    """``token_weight[ids] + position_weight[:T]`` as fp32 ``[B, T, d]``."""

    @staticmethod
    def forward(ctx, ids, token_weight, position_weight, into_grad):
        batch, seq = ids.shape
        vocab, d = token_weight.shape
        max_seq = position_weight.shape[0]
        if seq > max_seq:
            raise ValueError("sequence exceeds max_sequence_length")
        ids = ids.contiguous()
        out = torch.empty(batch, seq, d, device=ids.device, dtype=torch.float32)
        _check(library().rv_embed_fwd(ids.data_ptr(), batch, seq, token_weight.data_ptr(), vocab,
                                      position_weight.data_ptr(), max_seq, d, out.data_ptr(),
                                      _stream(ids)), "rv_embed_fwd")
        ctx.save_for_backward(ids)
        ctx.token_weight = token_weight
        ctx.shapes = (vocab, max_seq, d)
        ctx.into_grad = bool(into_grad)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        (ids,) = ctx.saved_tensors
        vocab, max_seq, d = ctx.shapes
        batch, seq = ids.shape
        dout = dout.to(torch.float32).contiguous()
        want_tok, want_pos = ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        lib = library()
        dtok = dpos = None
        tok_accumulate = 0
        returned_tok = want_tok
        if want_tok:
            sink = ctx.token_weight.grad
            if (ctx.into_grad and sink is not None and sink.dtype == torch.float32
                    and sink.is_contiguous() and sink.shape == (vocab, d)
                    and sink.data_ptr() % 16 == 0 and not sink.requires_grad):
                dtok, tok_accumulate, returned_tok = sink, 1, False
            else:
                dtok = torch.empty(vocab, d, device=dout.device, dtype=torch.float32)
        if want_pos:
            dpos = torch.empty(max_seq, d, device=dout.device, dtype=torch.float32)
        nbytes = lib.rv_embed_bwd_workspace_bytes(batch * seq, vocab, d) if want_tok else 0
        if nbytes < 0:
            _check(-nbytes, "rv_embed_bwd_workspace_bytes")
        ws = torch.empty(max(nbytes, 1), device=dout.device, dtype=torch.uint8)
        _check(lib.rv_embed_bwd(ids.data_ptr(), batch, seq, dout.data_ptr(), vocab, max_seq, d,
                                dtok.data_ptr() if dtok is not None else None, tok_accumulate,
                                dpos.data_ptr() if dpos is not None else None, 0,
                                ws.data_ptr(), nbytes, _stream(dout)), "rv_embed_bwd")
        return None, (dtok if returned_tok else None), dpos, None


def embed(ids: torch.Tensor, token_weight: torch.Tensor, position_weight: torch.Tensor,
          into_grad: bool = False) -> torch.Tensor:
    """``token_weight[ids] + position_weight[:T]`` on the kernels; raises on
    inputs they do not cover (no silent torch path)."""
    if not supported(ids, token_weight, position_weight):
        raise ValueError("fused embedding needs int64 CUDA ids [B, T] and contiguous, 16-byte "
                         "aligned fp32 CUDA tables whose width is a multiple of 4")
    return TokenPositionEmbedding.apply(ids, token_weight, position_weight, into_grad)


def enable_embedding(model: torch.nn.Module, into_grad: bool = False) -> None:
    """Route ``model.embed`` (used by ``forward`` and the trainers'
    ``hidden_states``) through the fused kernels."""
    config = model.config

    def fused(self, input_ids):
        if input_ids.ndim != 2:
            raise ValueError("input_ids must have shape [batch, sequence]")
        if input_ids.shape[1] > config.max_sequence_length:
            raise ValueError("sequence exceeds max_sequence_length")
        return embed(input_ids, self.token_embedding.weight, self.position_embedding.weight,
                     into_grad)

    model.embed = types.MethodType(fused, model)
