"""Model-level parity at configs[4]'s shape: the 12-layer Hamiltonian-Euler
decoder at width 1024 (16 heads, head size 64, SwiGLU hidden 4096, vocabulary
50257, context 2048), fp16 autocast with the fp32 residual.

The candidate is wired as the measured configs[4] training step (bench.py):
install_v3 with the reconstruction-stack core, one tiled-MLP tile of the whole
batch keeping its tiles, fused SwiGLU and RMSNorm, MFMA attention projections,
the causal attention kernels, the fused embedding adding into the tied
gradient, and ``cached_head_backward`` with the fused cross-entropy.

Comparators, each independent of this repository's kernels (plain torch:
unpatched modules, residual updates as eager expressions via
``residual.eager_updates``):
  * truth: the model in fp32 with plain autograd through the recurrence, on the
    GPU at T = 2048 (and the fp32 CPU oracle, oracle/model_ref.py -- explicit
    causal softmax, its own RMSNorm and SwiGLU -- on short sequences);
  * the reference's algorithm: the same model under fp16 autocast with the
    reconstruction backward of src/reversibility/reversible.py:35-69 (plain
    inverse, then a recomputed step and its VJP), in plain torch;
  * the reference's reconstruction gate (scripts/validate_reversible.py:32-118)
    at width 1024 / 16 heads, and the reconstructed states of the full
    configs[4] batch.

Bars.  fp16 reconstruction at 12 layers x width 1024 is itself inexact: the
reference's algorithm lands 2-3e-2 (relative L2) from the fp32 truth on the
first layer's weight gradients, while plain fp16 autograd stays within 4e-3 --
the inverse's fp16 force evaluations round differently from the forward's.
So every parameter gradient of the candidate must be within
max(2e-2, 1.5 x the reference algorithm's distance) of the truth for that
parameter; the loss within 2e-3 (relative) of the truth (2e-2 for the CPU
oracle); one AdamW update within max(0.05, 1.5 x the reference algorithm's)
relative L2 of the truth's update; every rebuilt state within the gate's fp16
policy (atol 5e-3, rtol 5e-2) and within 1.5 x the reference algorithm's
worst state error on the same batch.
"""
from __future__ import annotations

import copy
import math

import pytest
import torch
import torch.nn.functional as F

from reconstruction_gate import TOLERANCES, run_gate
from reversability_amd import build_model, paths
from reversability_amd.attention import enable_attention
from reversability_amd.embedding import enable_embedding
from reversability_amd.linear import enable_linear
from reversability_amd.optimized_v3 import cached_head_backward, install_v3
from reversability_amd.residual import eager_updates
from reversability_amd.reversible import forward_pair, inverse_pair

pytestmark = pytest.mark.gpu

C5 = {"model": {"vocab_size": 50257, "max_sequence_length": 2048, "n_layers": 12,
                "n_heads": 16, "d_model": 1024, "d_ff": 4096},
      "method": "euler", "step_size": 0.5}


def rel_l2(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _wire(model, tokens):
    install_v3(model, core_mode="reference", mlp_tokens=tokens, swiglu=True, rmsnorm=True,
               keep_mlp_tiles=True)
    enable_linear(model)
    enable_attention(model)
    enable_embedding(model, into_grad=True)


REFERENCE_ALGORITHM = dict(reuse_euler_attention=False, fuse_euler_inverse=False,
                           skip_unused_mlp_output=False)


def _models(device):
    torch.manual_seed(1337)
    plain = build_model(C5).to(device)
    candidate = copy.deepcopy(plain)
    return plain, candidate


def _ids(device, batch, length, seed=1337):
    g = torch.Generator().manual_seed(seed)
    stream = torch.randint(0, 50257, (batch * length + 1,), generator=g)
    x = stream[:-1].reshape(batch, length).to(device)
    y = stream[1:].reshape(batch, length).to(device)
    return x, y


def _plain_step(base, x, y, mode, amp):
    """Loss and unscaled gradients of a plain-torch copy of ``base``:
    ``mode`` 'autograd' or 'reconstruct' (the reference's inverse-then-recompute
    backward), under fp16 autocast with a loss scale when ``amp``."""
    model = copy.deepcopy(base)
    model.backward_mode = mode
    paths.configure(model, **REFERENCE_ALGORITHM)
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 10, enabled=amp)
    with torch.autocast("cuda", dtype=torch.float16, enabled=amp), eager_updates():
        loss = F.cross_entropy(model(x).flatten(0, 1), y.flatten(), reduction="sum") / y.numel()
    scaler.scale(loss).backward()
    inv = 1.0 / scaler.get_scale()
    grads = {n: p.grad.detach() * inv for n, p in model.named_parameters()}
    return loss.detach(), grads


def _candidate_step(model, x, y):
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 10)
    model.zero_grad(set_to_none=True)
    total = cached_head_backward(model, x, y, y.numel(), y.numel(), scaler, "fp16", False,
                                 "triton")
    inv = 1.0 / scaler.get_scale()
    return total / y.numel(), {n: p.grad.detach() * inv for n, p in model.named_parameters()}


def _check_gradients(tag, grads, reference_algorithm, truth):
    """Per parameter: the candidate's distance from the truth within
    max(2e-2, 1.5 x the reference algorithm's)."""
    rows = {}
    for name, g in truth.items():
        mine, theirs = rel_l2(grads[name], g), rel_l2(reference_algorithm[name], g)
        rows[name] = (mine, theirs)
    worst = max(rows, key=lambda n: rows[n][0])
    print(f"[{tag}] worst parameter-gradient relative L2 to the truth: candidate "
          f"{rows[worst][0]:.3e}, reference algorithm {rows[worst][1]:.3e} ({worst}); "
          f"reference algorithm's worst {max(v[1] for v in rows.values()):.3e}", flush=True)
    for name, (mine, theirs) in rows.items():
        assert mine <= max(2e-2, 1.5 * theirs), (name, mine, theirs)


def _adamw_update(base, grads):
    model = copy.deepcopy(base)
    for n, p in model.named_parameters():
        p.grad = grads[n].clone()
    torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
    torch.optim.AdamW(model.parameters(), lr=6e-4, betas=(.9, .95), weight_decay=.1).step()
    return {n: p.detach() - q.detach() for (n, p), q in zip(model.named_parameters(),
                                                              base.parameters())}


def _update_distance(a, b):
    gap = sum(float((a[n] - b[n]).double().square().sum()) for n in b)
    size = sum(float(b[n].double().square().sum()) for n in b)
    return math.sqrt(gap / size), max(float((a[n] - b[n]).abs().max()) for n in b)


def test_c5_step_matches_truth_within_reference_accuracy(cuda_device):
    """Loss, every parameter gradient and one AdamW update of a configs[4]-shaped
    step (B = 2, T = 2048): candidate, reference algorithm and fp32 truth."""
    base, candidate = _models(cuda_device)
    x, y = _ids(cuda_device, 2, 2048)
    loss_t, truth = _plain_step(base, x, y, "autograd", amp=False)
    loss_r, reference_algorithm = _plain_step(base, x, y, "reconstruct", amp=True)
    _wire(candidate, x.numel())
    loss_c, grads = _candidate_step(candidate, x, y)
    print(f"\n[c5] loss candidate {loss_c.item():.6f} reference algorithm {loss_r.item():.6f} "
          f"fp32 truth {loss_t.item():.6f}", flush=True)
    assert abs(loss_c.item() - loss_t.item()) <= 2e-3 * abs(loss_t.item())
    _check_gradients("c5", grads, reference_algorithm, truth)
    step_t = _adamw_update(base, truth)
    mine, mine_max = _update_distance(_adamw_update(base, grads), step_t)
    theirs, theirs_max = _update_distance(_adamw_update(base, reference_algorithm), step_t)
    print(f"[c5] AdamW update relative L2 to the truth's: candidate {mine:.3e} (max coordinate "
          f"{mine_max:.3e}), reference algorithm {theirs:.3e} ({theirs_max:.3e})", flush=True)
    assert mine <= max(0.05, 1.5 * theirs) and mine_max <= 1.2e-3


def test_c5_short_sequences_match_cpu_oracle(cuda_device):
    """Two 256-token sequences through the configs[4] candidate on the GPU
    against the fp32 CPU oracle with the same weights (the reference
    algorithm in fp16 on the GPU sets the gradient bar)."""
    from oracle import model_ref
    base, candidate = _models(cuda_device)
    x, y = _ids(cuda_device, 2, 256, seed=2026)
    loss_o, truth = model_ref.loss_and_grads(base.state_dict(), x, y, 12, 16, "euler")
    _, reference_algorithm = _plain_step(base, x, y, "reconstruct", amp=True)
    _wire(candidate, x.numel())
    loss_c, grads = _candidate_step(candidate, x, y)
    print(f"\n[c5-oracle] loss candidate {loss_c.item():.6f} oracle {loss_o.item():.6f}",
          flush=True)
    assert abs(loss_c.item() - loss_o.item()) <= 2e-2 * abs(loss_o.item())
    truth.pop("lm_head.weight", None)
    _check_gradients("c5-oracle", {n: g for n, g in grads.items() if n in truth},
                     {n: g for n, g in reference_algorithm.items() if n in truth}, truth)


@pytest.mark.parametrize("depth,length", [(3, 64), (12, 256)])
def test_reconstruction_gate_width_1024(cuda_device, depth, length):
    """The reference's gate at configs[4]'s width and head count, candidate with
    the full configs[4] wiring (the gate's small vocabulary)."""
    def prepare(model):
        _wire(model, 2 * length)
    report = run_gate("euler", "fp16", cuda_device, depth, length, width=1024, heads=16,
                      prepare=prepare)
    print(f"\n[gate d1024] depth {depth} length {length}: worst state "
          f"{report.worst_state_error():.3e}, worst gradient "
          f"{max(v['max_abs'] for k, v in report.errors.items() if k.startswith('gradient_')):.3e}",
          flush=True)


def _worst_reconstruction_error(model, x, eager, check=False):
    """Forward 12 Euler steps under no grad recording every state, then invert
    layer by layer; the worst max-abs difference of a rebuilt state from its
    record (``check``: each also held to the gate's fp16 policy)."""
    worst = 0.0
    with torch.autocast("cuda", dtype=torch.float16), torch.no_grad(), eager_updates(eager):
        record = [(model.embed(x),) * 2]
        for block in model.blocks:
            record.append(forward_pair(block, *record[-1], "euler", 0.5))
        pair = record.pop()
        for block in reversed(model.blocks):
            pair = inverse_pair(block, *pair, "euler", 0.5)
            stored = record.pop()
            for rebuilt, kept in zip(pair, stored):
                worst = max(worst, float((rebuilt - kept).abs().max()))
                if check:
                    torch.testing.assert_close(rebuilt, kept, **TOLERANCES["fp16"])
            del stored
    return worst


def test_c5_full_batch_reconstruction_error(cuda_device):
    """All of configs[4] (B = 16, T = 2048): every rebuilt state of the wired
    model within the gate's fp16 policy and within 1.5 x the reference
    algorithm's (plain torch) worst error on the same batch."""
    base, model = _models(cuda_device)
    x, _ = _ids(cuda_device, 16, 2048)
    worst_plain = _worst_reconstruction_error(base, x, eager=True)
    _wire(model, x.numel())
    worst = _worst_reconstruction_error(model, x, eager=False, check=True)
    print(f"\n[c5] worst reconstructed-state max-abs over 12 layers: candidate {worst:.3e}, "
          f"reference algorithm {worst_plain:.3e}", flush=True)
    assert worst <= 1.5 * worst_plain
