"""The chunked tied-head correctness gate on the GPU, from the procedure of the
reference's ``correctness_gate`` (scripts/benchmark_optimized.py:85-161).

For each method (baseline, midpoint) and head chunk size, an *original* model
and a deep copy, the *candidate*, take two updates on the same fresh batches.

* original: plain torch -- unpatched modules, ``backward_mode='autograd'``, the
  residual updates as eager expressions (``residual.eager_updates``); loss =
  summed ``F.cross_entropy`` over the valid targets, divided by their count,
  times a fixed loss scale of 128 (the reference's ``FixedScale``).
* candidate: the measured training step's wiring (install_v3 -- split core for
  midpoint --, fused SwiGLU and RMSNorm, tiled MFMA MLP, MFMA attention
  projections and causal attention, fused embedding adding into the tied
  gradient), head and loss through ``chunked_backward`` or
  ``cached_head_backward`` with ``loss_backend="triton"`` (the fused HIP
  cross-entropy), in chunks of 1024 / 1536 (a short last chunk) / 2048 / 4096
  tokens of the 4096-token batch.
* batch: 8 x 512 uniform ids over the 50257-token vocabulary, labels = ids
  rolled by one with the last 3 positions of every row ignored (-100).

After each update's backward both gradients are divided by the scale and
compared; both models clip at 1.0 and step AdamW (0.9, 0.95), wd 0.1 -- torch's
for the original, ``FusedAdamW`` for the candidate.  Limits (fp16 autocast, the
reference's values): per-parameter gradient relative L2 .02, loss relative
.002, per-step optimizer coordinate difference .0012, whole-update relative
L2 .05.
"""
from __future__ import annotations

import copy
import math

import pytest
import torch
import torch.nn.functional as F

from reversability_amd import build_model
from reversability_amd.attention import enable_attention
from reversability_amd.embedding import enable_embedding
from reversability_amd.linear import enable_linear
from reversability_amd.optim import FusedAdamW
from reversability_amd.optimized import chunked_backward
from reversability_amd.optimized_v3 import cached_head_backward, install_v3
from reversability_amd.residual import eager_updates

pytestmark = pytest.mark.gpu

MODEL = {"vocab_size": 50257, "max_sequence_length": 512, "n_layers": 7, "n_heads": 8,
         "d_model": 256, "d_ff": 1024}
BATCH, LENGTH, SCALE = 8, 512, 128.0
LIMITS = {"gradient_relative_l2": .02, "loss_relative": .002,
          "optimizer_step_max_absolute": .0012, "optimizer_relative_update_l2": .05}


class FixedScale:
    """A loss scaler with one constant factor (scripts/benchmark_optimized.py:110-111)."""

    def scale(self, loss):
        return loss * SCALE


def _wire(model, method):
    install_v3(model, core_mode="split" if method == "midpoint" else "reference",
               mlp_tokens=BATCH * LENGTH, swiglu=True, rmsnorm=True, keep_mlp_tiles=True)
    enable_linear(model)
    enable_attention(model)
    enable_embedding(model, into_grad=True)


def _batch(device):
    ids = torch.randint(MODEL["vocab_size"], (BATCH, LENGTH), device=device)
    labels = ids.roll(-1, 1).clone()
    labels[:, -3:] = -100
    return ids, labels, int((labels != -100).sum())


def _original_loss(model, ids, labels, denominator):
    with torch.autocast("cuda", dtype=torch.float16), eager_updates():
        loss = F.cross_entropy(model(ids).flatten(0, 1), labels.flatten(), ignore_index=-100,
                               reduction="sum")
        (loss * SCALE / denominator).backward()
    return loss.detach().float()


@pytest.mark.parametrize("head", ["chunked_backward", "cached_head_backward"])
@pytest.mark.parametrize("chunk", [1024, 1536, 2048, 4096])
@pytest.mark.parametrize("method", ["baseline", "midpoint"])
def test_chunked_head_gate(cuda_device, method, chunk, head):
    torch.manual_seed(1337)
    original = build_model({"model": MODEL, "method": method}).to(cuda_device)
    candidate = copy.deepcopy(original)
    if method != "baseline":
        original.backward_mode = "autograd"  # plain autograd through the recurrence
    _wire(candidate, method)
    hyper = dict(lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)
    left = torch.optim.AdamW(original.parameters(), **hyper)
    right = FusedAdamW(candidate.parameters(), **hyper)
    run = chunked_backward if head == "chunked_backward" else cached_head_backward
    for update in range(2):
        left.zero_grad(set_to_none=True)
        right.zero_grad(set_to_none=True)
        ids, labels, denominator = _batch(cuda_device)
        expected = _original_loss(original, ids, labels, denominator)
        actual = run(candidate, ids, labels, denominator, chunk, FixedScale(), "fp16", False,
                     "triton")
        assert candidate.lm_head.weight is candidate.token_embedding.weight
        gradient_errors = {}
        for (name, a), b in zip(original.named_parameters(), candidate.parameters()):
            a.grad.div_(SCALE)
            b.grad.div_(SCALE)
            assert torch.isfinite(a.grad).all() and torch.isfinite(b.grad).all(), name
            gradient_errors[name] = float((a.grad - b.grad).norm()
                                          / a.grad.norm().clamp_min(1e-12))
        for model in (original, candidate):
            torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        start_l = [p.detach().clone() for p in original.parameters()]
        start_r = [p.detach().clone() for p in candidate.parameters()]
        left.step()
        right.step()
        gap = moved = 0.0
        step_gap = 0.0
        for a, b, a0, b0 in zip(original.parameters(), candidate.parameters(), start_l, start_r):
            gap += float((a.detach() - b.detach()).double().square().sum())
            moved += float((a.detach() - a0).double().square().sum())
            step_gap = max(step_gap, float(((a.detach() - a0) - (b.detach() - b0)).abs().max()))
        row = {"gradient_relative_l2": max(gradient_errors.values()),
               "loss_relative": float((expected - actual).abs() / expected.abs().clamp_min(1e-12)),
               "optimizer_step_max_absolute": step_gap,
               "optimizer_relative_update_l2": math.sqrt(gap / max(moved, 1e-30))}
        print(f"\n[head gate] {method} {head} chunk {chunk} update {update}: "
              + ", ".join(f"{k} {v:.3e}" for k, v in row.items()), flush=True)
        worst = max(gradient_errors, key=gradient_errors.get)
        for key, limit in LIMITS.items():
            assert row[key] <= limit, (key, row, worst)
