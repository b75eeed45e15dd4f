"""Reconstruction / gradient gate, restated from scripts/validate_reversible.py:18-118.

``check_case`` compares, for one (method, precision, device, depth, length):

1. every state reconstructed by ``inverse_pair`` against the state recorded by
   the no-grad forward (validate_reversible.py:55-63);
2. ``ReversibleLM.core`` (reconstruction backward) against an independent
   eager restatement of the recurrence differentiated by ordinary autograd:
   outputs, input gradient and every parameter gradient (:64-83);
3. logits and loss of the two models (:85-90);
4. full-model gradients and one clipped AdamW step, coordinatewise and as a
   relative L2 of the update (:91-116).

The tolerance tables are the reference's (validate_reversible.py:20-29).
``models`` lets a caller pass a candidate built some other way (e.g. with the
fused HIP kernels installed) next to the plain autograd reference.
"""
from __future__ import annotations

import contextlib
import copy

import torch
import torch.nn.functional as F

from reversability_amd import ModelConfig, ReversibleLM
from reversability_amd.reversible import forward_pair, inverse_pair

OPTIMIZER_TOLERANCES = {"fp64": {"atol": 1e-9, "rtol": 1e-8},
                        "fp32": {"atol": 5e-5, "rtol": 3e-4},
                        "fp16": {"atol": 1.2e-3, "rtol": 0.0}}
UPDATE_RELATIVE_L2 = {"fp64": 1e-7, "fp32": .01, "fp16": .05}
TOLERANCES = {"fp64": {"atol": 1e-9, "rtol": 1e-8},
              "fp32": {"atol": 3e-5, "rtol": 3e-4},
              "fp16": {"atol": 5e-3, "rtol": 5e-2}}


def reference_core(model, x, method, h):
    """The recurrence written out with eager torch ops (validate_reversible.py:65-73)."""
    p, q = x, x
    for b in model.blocks:
        if method == "midpoint":
            a = b.attn(b.attn_norm(q))
            force = a + b.mlp(b.mlp_norm(q + a))
            p, q = q, p + (2 * h) * force
        else:
            q = q + b.attn(b.attn_norm(p))
            p = p + b.mlp(b.mlp_norm(q))
    return q if method == "midpoint" else p


def check_case(method, precision, device, depth, length, width=32, heads=2, h=0.5, seed=1337,
               prepare=None):
    """Run the gate; ``prepare(model)`` may install optimized paths on the
    candidate.  Returns the error report; raises AssertionError on failure."""
    torch.manual_seed(seed)
    config = ModelConfig(vocab_size=101, max_sequence_length=length, n_layers=depth,
                         n_heads=heads, d_model=width, d_ff=4 * width)
    dtype = torch.float64 if precision == "fp64" else torch.float32
    candidate = ReversibleLM(config, method, h).to(device=device, dtype=dtype)
    reference = copy.deepcopy(candidate)
    reference.backward_mode = "autograd"
    if prepare is not None:
        prepare(candidate)
    amp = ((lambda: torch.autocast(device_type="cuda", dtype=torch.float16))
           if precision == "fp16" else contextlib.nullcontext)
    errors = {}

    def compare(name, actual, expected):
        assert torch.isfinite(actual).all() and torch.isfinite(expected).all(), name
        delta = (actual.detach() - expected.detach()).abs()
        errors[name] = {"max_abs": delta.max().item(),
                        "relative_to_max_reference":
                            delta.max().item() / max(expected.detach().abs().max().item(), 1e-12)}
        policy = OPTIMIZER_TOLERANCES if name.startswith("optimizer_") else TOLERANCES
        torch.testing.assert_close(actual, expected, **policy[precision], msg=name)

    ids = torch.randint(0, config.vocab_size, (2, length), device=device)
    labels = torch.randint(0, config.vocab_size, (2, length), device=device)
    labels[-1, -1] = -100
    with amp(), torch.no_grad():
        x = candidate.token_embedding(ids) + candidate.position_embedding(
            torch.arange(length, device=device))
        p, q = x, x
        states = [(p, q)]
        for block in candidate.blocks:
            p, q = forward_pair(block, p, q, method, h)
            states.append((p, q))
        for i in range(depth - 1, -1, -1):
            p, q = inverse_pair(candidate.blocks[i], p, q, method, h)
            compare(f"state_{i}_p", p, states[i][0])
            compare(f"state_{i}_q", q, states[i][1])
    with amp():
        x1 = x.detach().requires_grad_(True)
        x2 = x.detach().requires_grad_(True)
        out1 = candidate.core(x1)
        out2 = reference_core(reference, x2, method, h)
        compare("core_output", out1, out2)
        probe = torch.randn_like(out1)
        (out1 * probe).mean().backward()
        (out2 * probe).mean().backward()
        compare("input_gradient", x1.grad, x2.grad)
    ref_params = dict(reference.named_parameters())
    for name, p1 in candidate.named_parameters():
        if p1.grad is not None:
            compare("core_gradient_" + name, p1.grad, ref_params[name].grad)
    candidate.zero_grad()
    reference.zero_grad()
    with amp():
        logits1 = candidate(ids)
        logits2 = reference(ids)
        compare("logits", logits1, logits2)
        loss1 = F.cross_entropy(logits1.flatten(0, 1), labels.flatten())
        loss2 = F.cross_entropy(logits2.flatten(0, 1), labels.flatten())
        compare("loss", loss1, loss2)
    optimizers = [torch.optim.AdamW(m.parameters(), lr=6e-4, betas=(.9, .95), weight_decay=.1)
                  for m in (candidate, reference)]
    scalers = [torch.amp.GradScaler("cuda") for _ in optimizers] if precision == "fp16" else None
    if scalers:
        for scaler, opt, loss in zip(scalers, optimizers, (loss1, loss2)):
            scaler.scale(loss).backward()
            scaler.unscale_(opt)
    else:
        loss1.backward()
        loss2.backward()
    for (name, p1), (name2, p2) in zip(candidate.named_parameters(), reference.named_parameters()):
        assert name == name2 and p1.grad is not None and p2.grad is not None
        compare("gradient_" + name, p1.grad, p2.grad)
    before = {name: p.detach().clone() for name, p in reference.named_parameters()}
    for i, (m, opt) in enumerate(zip((candidate, reference), optimizers)):
        norm = torch.nn.utils.clip_grad_norm_(m.parameters(), 1.0)
        assert torch.isfinite(norm)
        if scalers:
            old = scalers[i].get_scale()
            scalers[i].step(opt)
            scalers[i].update()
            assert scalers[i].get_scale() >= old, "overflow in optimizer gate"
        else:
            opt.step()
    for (name, p1), (_, p2) in zip(candidate.named_parameters(), reference.named_parameters()):
        compare("optimizer_" + name, p1, p2)
    diff_sq = sum((a.detach() - b.detach()).double().square().sum().item()
                  for a, b in zip(candidate.parameters(), reference.parameters()))
    update_sq = sum((p.detach() - before[name]).double().square().sum().item()
                    for name, p in reference.named_parameters())
    relative = (diff_sq / max(update_sq, 1e-30)) ** .5
    errors["optimizer_relative_update_l2"] = relative
    assert relative <= UPDATE_RELATIVE_L2[precision], ("optimizer update L2", relative)
    return {"method": method, "precision": precision, "depth": depth, "length": length,
            "width": width, "errors": errors}
