"""Reconstruction / gradient gate for the reversible core, written from the
procedure of the reference's gate (scripts/validate_reversible.py:18-118).

A case builds one seeded ``ReversibleLM`` -- the *candidate*: reconstruction
backward, optionally with this repository's fused paths installed by a
``prepare`` hook -- and a deep copy made before ``prepare`` runs -- the
*comparator*: modules unpatched, ``backward_mode='autograd'``, and every
residual update evaluated as the eager torch expression
(``residual.eager_updates``), so it is plain torch end to end.

Four stages compare the two, each quantity against the tolerance tables of the
reference's policy (kept as they are: they are the parity bar):

  states   a no-grad forward records every (p, q); ``inverse_pair`` walks back
           from the last pair and each rebuilt pair must match the record;
  core     the candidate stack's output, input gradient and parameter gradients
           under a random probe, against an equation-level restatement of the
           recurrence (``eager_core``) differentiated by autograd;
  model    logits and mean cross-entropy with one ignored target;
  update   full-model gradients (GradScaler-scaled under fp16), clip at 1.0 and
           one AdamW step: every parameter coordinatewise (optimizer table) and
           the whole update's relative L2.
"""
from __future__ import annotations

import contextlib
import copy
import dataclasses

import torch
import torch.nn.functional as F

from reversability_amd import ModelConfig, ReversibleLM
from reversability_amd.residual import eager_updates
from reversability_amd.reversible import forward_pair, inverse_pair

# scripts/validate_reversible.py:20-29 (policy "reconstruction-gradient-v2")
OPTIMIZER_TOLERANCES = {"fp64": {"atol": 1e-9, "rtol": 1e-8},
                        "fp32": {"atol": 5e-5, "rtol": 3e-4},
                        "fp16": {"atol": 1.2e-3, "rtol": 0.0}}
UPDATE_RELATIVE_L2 = {"fp64": 1e-7, "fp32": .01, "fp16": .05}
TOLERANCES = {"fp64": {"atol": 1e-9, "rtol": 1e-8},
              "fp32": {"atol": 3e-5, "rtol": 3e-4},
              "fp16": {"atol": 5e-3, "rtol": 5e-2}}

# The reference's CUDA case list (scripts/validate_reversible.py:134-141):
# three (depth, length) shapes, midpoint at two step sizes, two seeds, plus the
# architecture-sized probe (7 layers x 512 tokens x width 256, 8 heads).
GRID_SHAPES = ((1, 8), (3, 17), (7, 32))
GRID_SEEDS = (1337, 2026)
MIDPOINT_STEPS = (0.25, 0.5)


def step_sizes(method):
    return MIDPOINT_STEPS if method == "midpoint" else (0.5,)


def eager_core(model, x, method, h):
    """The integrator written as equations over the model's submodules."""
    p = q = x
    for block in model.blocks:
        if method == "euler":
            q = q + block.attn(block.attn_norm(p))
            p = p + block.mlp(block.mlp_norm(q))
            continue
        attention = block.attn(block.attn_norm(q))
        force = attention + block.mlp(block.mlp_norm(q + attention))
        p, q = q, p + (2 * h) * force
    return p if method == "euler" else q


@dataclasses.dataclass
class GateReport:
    method: str
    precision: str
    depth: int
    length: int
    width: int
    step_size: float
    seed: int
    errors: dict = dataclasses.field(default_factory=dict)

    def check(self, name, actual, expected):
        """Record max-abs and relative error of ``actual`` and assert the policy."""
        actual, expected = actual.detach(), expected.detach()
        assert torch.isfinite(actual).all(), f"{name}: non-finite candidate"
        assert torch.isfinite(expected).all(), f"{name}: non-finite comparator"
        worst = (actual - expected).abs().max().item() if actual.numel() else 0.0
        scale = expected.abs().max().item() if expected.numel() else 0.0
        self.errors[name] = {"max_abs": worst,
                             "relative_to_max_reference": worst / max(scale, 1e-12)}
        table = OPTIMIZER_TOLERANCES if name.startswith("optimizer_") else TOLERANCES
        torch.testing.assert_close(actual, expected, **table[self.precision], msg=name)

    def worst_state_error(self) -> float:
        return max(v["max_abs"] for k, v in self.errors.items() if k.startswith("state_"))


def _autocast(precision):
    if precision == "fp16":
        return torch.autocast(device_type="cuda", dtype=torch.float16)
    return contextlib.nullcontext()


def _stage_states(report, model, x, method, h, precision):
    with _autocast(precision), torch.no_grad():
        record = [(x, x)]
        for block in model.blocks:
            record.append(forward_pair(block, *record[-1], method, h))
        pair = record[-1]
        for index in reversed(range(len(model.blocks))):
            pair = inverse_pair(model.blocks[index], *pair, method, h)
            report.check(f"state_{index}_p", pair[0], record[index][0])
            report.check(f"state_{index}_q", pair[1], record[index][1])


def _stage_core(report, candidate, comparator, x, method, h, precision):
    leaves = [x.detach().clone().requires_grad_(True) for _ in range(2)]
    with _autocast(precision):
        out = candidate.core(leaves[0])
        with eager_updates():
            expected = eager_core(comparator, leaves[1], method, h)
        report.check("core_output", out, expected)
        probe = torch.randn_like(out)
        for value, leaf in ((out, leaves[0]), (expected, leaves[1])):
            (value * probe).mean().backward()
    report.check("input_gradient", leaves[0].grad, leaves[1].grad)
    theirs = dict(comparator.named_parameters())
    for name, param in candidate.named_parameters():
        if param.grad is not None:
            report.check("core_gradient_" + name, param.grad, theirs[name].grad)


def _stage_model(report, candidate, comparator, ids, labels, precision):
    losses = []
    with _autocast(precision):
        for model, eager in ((candidate, False), (comparator, True)):
            with eager_updates() if eager else contextlib.nullcontext():
                logits = model(ids)
            losses.append((logits, F.cross_entropy(logits.flatten(0, 1), labels.flatten())))
        report.check("logits", losses[0][0], losses[1][0])
        report.check("loss", losses[0][1], losses[1][1])
    return [loss for _, loss in losses]


def _stage_update(report, candidate, comparator, losses, precision):
    pair = (candidate, comparator)
    optimizers = [torch.optim.AdamW(m.parameters(), lr=6e-4, betas=(.9, .95), weight_decay=.1)
                  for m in pair]
    scalers = ([torch.amp.GradScaler("cuda") for _ in pair] if precision == "fp16"
               else [None, None])
    for loss, opt, scaler in zip(losses, optimizers, scalers):
        if scaler is None:
            loss.backward()
        else:
            scaler.scale(loss).backward()
            scaler.unscale_(opt)
    named = list(zip(candidate.named_parameters(), comparator.named_parameters()))
    for (name, mine), (other_name, theirs) in named:
        assert name == other_name and mine.grad is not None and theirs.grad is not None, name
        report.check("gradient_" + name, mine.grad, theirs.grad)
    start = [p.detach().clone() for p in comparator.parameters()]
    for model, opt, scaler in zip(pair, optimizers, scalers):
        assert torch.isfinite(torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0))
        if scaler is None:
            opt.step()
            continue
        scale = scaler.get_scale()
        scaler.step(opt)
        scaler.update()
        assert scaler.get_scale() >= scale, "loss-scale overflow in the update stage"
    for (name, mine), (_, theirs) in named:
        report.check("optimizer_" + name, mine, theirs)
    gap = sum(float((a.detach() - b.detach()).double().square().sum())
              for a, b in zip(candidate.parameters(), comparator.parameters()))
    moved = sum(float((b.detach() - b0).double().square().sum())
                for b, b0 in zip(comparator.parameters(), start))
    relative = (gap / max(moved, 1e-30)) ** .5
    report.errors["optimizer_relative_update_l2"] = relative
    assert relative <= UPDATE_RELATIVE_L2[report.precision], ("update relative L2", relative)


def run_gate(method, precision, device, depth, length, width=32, heads=2, h=0.5, seed=1337,
             prepare=None) -> GateReport:
    """One gate case; raises AssertionError on the first quantity outside the
    policy.  ``prepare(candidate)`` installs optional paths on the candidate."""
    torch.manual_seed(seed)
    config = ModelConfig(vocab_size=101, max_sequence_length=length, n_layers=depth,
                         n_heads=heads, d_model=width, d_ff=4 * width)
    dtype = torch.float64 if precision == "fp64" else torch.float32
    candidate = ReversibleLM(config, method, h).to(device=device, dtype=dtype)
    comparator = copy.deepcopy(candidate)
    comparator.backward_mode = "autograd"
    if prepare is not None:
        prepare(candidate)
    ids = torch.randint(0, config.vocab_size, (2, length), device=device)
    labels = torch.randint(0, config.vocab_size, (2, length), device=device)
    labels[-1, -1] = -100  # a partial-target normalization
    report = GateReport(method, precision, depth, length, width, h, seed)
    with torch.no_grad():
        x = comparator.token_embedding(ids) + comparator.position_embedding(
            torch.arange(length, device=device))
    _stage_states(report, candidate, x, method, h, precision)
    _stage_core(report, candidate, comparator, x, method, h, precision)
    candidate.zero_grad()
    comparator.zero_grad()
    losses = _stage_model(report, candidate, comparator, ids, labels, precision)
    _stage_update(report, candidate, comparator, losses, precision)
    return report
