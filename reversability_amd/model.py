"""Decoder substrate the reversible hot path runs inside.

Same architecture, parameter names, tying and initialisation as
src/reversibility/model.py:10-107, so that ``torch.manual_seed(s)`` followed by
``BaselineLM(config)`` yields the same weights as the reference and state
dicts load across the two:

* blocks are pre-norm: ``x + attn(attn_norm(x))`` then ``x + mlp(mlp_norm(x))``;
  RMSNorm with ``eps=None`` (i.e. ``finfo(dtype).eps``), causal SDPA attention
  with a fused qkv projection, SwiGLU MLP with a packed ``[gate; value]``
  up-projection of width ``2 * d_ff``;
* learned positions, tied token embedding / LM head;
* N(0, 0.02) for every Linear/Embedding weight, then N(0, 0.02/sqrt(2L)) for
  ``attn.proj`` and ``mlp.down``.  Modules are constructed and initialised in
  the reference's order because each constructor and init draws from the
  global RNG.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int = 50_257
    max_sequence_length: int = 512
    n_layers: int = 7
    n_heads: int = 8
    d_model: int = 256
    d_ff: int = 1_024
    dropout: float = 0.0
    bias: bool = False

    def __post_init__(self) -> None:
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads")


class CausalSelfAttention(nn.Module):
    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.n_heads = config.n_heads
        self.head_dim = config.d_model // config.n_heads
        self.qkv = nn.Linear(config.d_model, 3 * config.d_model, bias=config.bias)
        self.proj = nn.Linear(config.d_model, config.d_model, bias=config.bias)
        self.dropout = config.dropout

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        batch, length, width = x.shape
        heads = self.qkv(x).view(batch, length, 3, self.n_heads, self.head_dim)
        # [3, batch, heads, length, head_dim] views of the packed projection
        q, k, v = heads.permute(2, 0, 3, 1, 4).unbind(0)
        mixed = F.scaled_dot_product_attention(
            q, k, v, dropout_p=self.dropout if self.training else 0.0, is_causal=True)
        return self.proj(mixed.transpose(1, 2).reshape(batch, length, width))


class MLP(nn.Module):
    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.up = nn.Linear(config.d_model, 2 * config.d_ff, bias=config.bias)
        self.down = nn.Linear(config.d_ff, config.d_model, bias=config.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, value = self.up(x).chunk(2, dim=-1)
        return self.down(F.silu(gate) * value)


class Block(nn.Module):
    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.attn_norm = nn.RMSNorm(config.d_model)
        self.attn = CausalSelfAttention(config)
        self.mlp_norm = nn.RMSNorm(config.d_model)
        self.mlp = MLP(config)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.attn_norm(x))
        return x + self.mlp(self.mlp_norm(x))


def _init_weights(module: nn.Module) -> None:
    if isinstance(module, (nn.Linear, nn.Embedding)):
        nn.init.normal_(module.weight, mean=0.0, std=0.02)
    if isinstance(module, nn.Linear) and module.bias is not None:
        nn.init.zeros_(module.bias)


class BaselineLM(nn.Module):
    def __init__(self, config: ModelConfig) -> None:
        super().__init__()
        self.config = config
        self.token_embedding = nn.Embedding(config.vocab_size, config.d_model)
        self.position_embedding = nn.Embedding(config.max_sequence_length, config.d_model)
        self.blocks = nn.ModuleList(Block(config) for _ in range(config.n_layers))
        self.final_norm = nn.RMSNorm(config.d_model)
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        self.lm_head.weight = self.token_embedding.weight
        self.apply(_init_weights)
        residual_std = 0.02 / (2 * config.n_layers) ** 0.5
        for block in self.blocks:
            nn.init.normal_(block.attn.proj.weight, mean=0.0, std=residual_std)
            nn.init.normal_(block.mlp.down.weight, mean=0.0, std=residual_std)

    _init_weights = staticmethod(_init_weights)

    def embed(self, input_ids: torch.Tensor) -> torch.Tensor:
        if input_ids.ndim != 2:
            raise ValueError("input_ids must have shape [batch, sequence]")
        if input_ids.shape[1] > self.config.max_sequence_length:
            raise ValueError("sequence exceeds max_sequence_length")
        positions = torch.arange(input_ids.shape[1], device=input_ids.device)
        return self.token_embedding(input_ids) + self.position_embedding(positions)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        x = self.embed(input_ids)
        for block in self.blocks:
            x = block(x)
        return self.lm_head(self.final_norm(x))

    def parameter_count(self) -> int:
        return sum(p.numel() for p in self.parameters() if p.requires_grad)
