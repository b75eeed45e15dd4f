"""Model-level GPU parity: reconstruction gate, tiled MLP block and
the full midpoint-reversible training step.

Bars (north star / the reference's own gates)
--------------------------------------------
* reconstruction and gradient gate: scripts/validate_reversible.py:20-29
  tolerance tables (fp16: atol 5e-3, rtol 5e-2; fp32: atol 3e-5, rtol 3e-4;
  fp64: atol 1e-9, rtol 1e-8; update relative L2 0.05 / 0.01 / 1e-7);
* fp16-autocast outputs and gradients: relative L2 <= 2e-2 against the eager
  autograd path on the GPU and against the fp32 CPU oracle;
* tiled MLP boundary: scripts/benchmark_midpoint_v3.py:44-45 limits over two
  AdamW updates.
"""
from __future__ import annotations

import contextlib
import copy
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from reconstruction_gate import (GRID_SEEDS, GRID_SHAPES, TOLERANCES, run_gate,
                                  step_sizes)
from reversability_amd import build_model, paths
from reversability_amd.attention import enable_attention
from reversability_amd.embedding import enable_embedding
from reversability_amd.kernels_v3 import FusedRMSNorm
from reversability_amd.linear import enable_linear
from reversability_amd.optimized_v3 import TiledMLP, cached_head_backward, install_v3
from reversability_amd.residual import eager_updates
from reversability_amd.reversible import forward_pair, inverse_pair

pytestmark = pytest.mark.gpu
EPS32 = float(torch.finfo(torch.float32).eps)


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


# --------------------------------------------------------------------------
# Reconstruction gate on the GPU (validate_reversible --device cuda)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("method", ["midpoint", "euler"])
@pytest.mark.parametrize("precision", ["fp64", "fp32", "fp16"])
def test_reconstruction_gate_plain(cuda_device, method, precision):
    """The reference's CUDA grid (validate_reversible.py:134-139): three shapes,
    midpoint at h = 0.25 and 0.5, seeds 1337 and 2026 -- 54 cases over the
    parametrization; the candidate runs its residual updates on the HIP
    kernels, the comparator is plain torch."""
    for depth, length in GRID_SHAPES:
        for h in step_sizes(method):
            for seed in GRID_SEEDS:
                run_gate(method, precision, cuda_device, depth, length, h=h, seed=seed)


def _install_all(method):
    def prepare(model):
        if method == "midpoint":
            install_v3(model, core_mode="split", mlp_tokens=13, swiglu=True, rmsnorm=True)
        else:
            install_v3(model, core_mode="reference", mlp_tokens=13, swiglu=True, rmsnorm=True)
    return prepare


@pytest.mark.parametrize("method", ["midpoint", "euler"])
@pytest.mark.parametrize("precision", ["fp32", "fp16"])
def test_reconstruction_gate_fused_v3(cuda_device, method, precision):
    for h in step_sizes(method):
        run_gate(method, precision, cuda_device, 3, 17, h=h, prepare=_install_all(method))


@pytest.mark.parametrize("core", ["reuse", "split"])
def test_reconstruction_gate_optimized_cores_fp16(cuda_device, core):
    run_gate("midpoint", "fp16", cuda_device, 3, 17,
             prepare=lambda m: install_v3(m, core_mode=core, swiglu=True, rmsnorm=True))


# Worst reconstructed-state errors the reference recorded on its GPU (T4) for the
# 7 x 512 x 256 probe (results/recorded/reversible-v1/correctness/cuda.json):
# fp16 AMP 7.63e-5 (midpoint) / 9.54e-5 (Euler), fp32 1.30e-7 / 1.36e-7.  The
# seeded inputs differ between CUDA and ROCm generators, so the measured value
# here is held to 4x the recorded one (a tracking bar well inside the gate's
# atol) rather than to equality.
RECORDED_PROBE_STATE_ERROR = {("midpoint", "fp16"): 7.63e-5, ("euler", "fp16"): 9.54e-5,
                              ("midpoint", "fp32"): 1.30e-7, ("euler", "fp32"): 1.36e-7}


@pytest.mark.parametrize("method", ["midpoint", "euler"])
@pytest.mark.parametrize("precision", ["fp64", "fp32", "fp16"])
@pytest.mark.parametrize("wiring", ["plain", "v3"])
def test_architecture_sized_probe(cuda_device, method, precision, wiring):
    """validate_reversible.py:141: 7 layers x 512 tokens x width 256, 8 heads --
    the plain model (HIP residual updates) and the v3 wiring (fused norms,
    SwiGLU, tiled MFMA MLP; fp32/fp16 only: the fused operators are fp32/fp16)."""
    if wiring == "v3" and precision == "fp64":
        pytest.skip("the fused v3 operators take fp32 / fp16 tensors")
    report = run_gate(method, precision, cuda_device, 7, 512, width=256, heads=8,
                      prepare=_install_all(method) if wiring == "v3" else None)
    worst = report.worst_state_error()
    print(f"\n[probe] {method} {precision} {wiring} worst reconstructed-state max-abs "
          f"{worst:.3e}", flush=True)
    assert worst < TOLERANCES[precision]["atol"]
    recorded = RECORDED_PROBE_STATE_ERROR.get((method, precision))
    if recorded is not None:
        assert worst < 4 * recorded, (worst, recorded)


@pytest.mark.parametrize("method", ["midpoint", "euler"])
def test_comparator_is_plain_torch(cuda_device, monkeypatch, method):
    """Under residual.eager_updates an unpatched model in autograd mode (the
    comparator of the gates below) reaches none of the HIP residual kernels:
    with their autograd Functions made to raise, its fp16 forward + backward
    still runs, and its loss equals the same model's under autograd with the
    HIP residual kernels to fp16-autocast tolerance."""
    from reversability_amd import residual
    torch.manual_seed(5)
    cfg = {"model": {"vocab_size": 101, "max_sequence_length": 64, "n_layers": 3,
                     "n_heads": 4, "d_model": 128, "d_ff": 256}, "method": method}
    model = build_model(cfg).to(cuda_device)
    model.backward_mode = "autograd"
    ids = torch.randint(0, 101, (2, 64), device=cuda_device)
    with torch.autocast("cuda", dtype=torch.float16):
        with_kernels = F.cross_entropy(model(ids).flatten(0, 1).float(), ids.flatten())

    def refuse(*args, **kwargs):
        raise AssertionError("the comparator reached a HIP residual kernel")
    monkeypatch.setattr(residual.MidpointStep, "apply", refuse)
    monkeypatch.setattr(residual.EulerStep, "apply", refuse)
    with torch.autocast("cuda", dtype=torch.float16), eager_updates():
        loss = F.cross_entropy(model(ids).flatten(0, 1).float(), ids.flatten())
    loss.backward()
    assert all(p.grad is not None for p in model.parameters())
    assert abs(loss.item() - with_kernels.item()) <= 2e-3 * abs(loss.item())


# --------------------------------------------------------------------------
# tiled SwiGLU MLP block under fp16 autocast, fp32 residual
# --------------------------------------------------------------------------

def _mlp_block_inputs(device, rows_shape=(29, 512)):
    g = torch.Generator().manual_seed(1337)
    d, f = 256, 1024
    x = torch.randn(*rows_shape, d, generator=g)
    w_up = 0.02 * torch.randn(2 * f, d, generator=g)
    w_down = 0.02 / math.sqrt(2 * 7) * torch.randn(d, f, generator=g)
    upstream = torch.randn(*rows_shape, d, generator=g)
    norm_w = torch.ones(d)
    return [t.to(device) for t in (x, norm_w, w_up, w_down, upstream)]


def _block_candidate(x, norm_w, w_up, w_down, tokens):
    with torch.autocast("cuda", dtype=torch.float16):
        h = FusedRMSNorm.apply(x, norm_w, EPS32)
        return TiledMLP.apply(h, w_up, w_down, tokens, True)


def _block_eager(x, norm_w, w_up, w_down):
    with torch.autocast("cuda", dtype=torch.float16):
        h = F.rms_norm(x, (x.shape[-1],), norm_w, eps=EPS32)
        gate, value = F.linear(h, w_up).chunk(2, -1)
        return F.linear(F.silu(gate) * value, w_down)


def test_tiled_mlp_block_matches_eager_and_oracle(cuda_device):
    from oracle import model_ref
    x, norm_w, w_up, w_down, upstream = _mlp_block_inputs(cuda_device)
    leaves = [t.clone().requires_grad_(True) for t in (x, norm_w, w_up, w_down)]
    ref_leaves = [t.clone().requires_grad_(True) for t in (x, norm_w, w_up, w_down)]
    y = _block_candidate(*leaves, 8192)
    ref = _block_eager(*ref_leaves)
    assert y.dtype == ref.dtype == torch.float16
    (y.float() * upstream).sum().backward()
    (ref.float() * upstream).sum().backward()
    assert rel_l2(y, ref) < 2e-3
    for a, b, name in zip(leaves, ref_leaves, ["x", "norm_w", "w_up", "w_down"]):
        assert rel_l2(a.grad, b.grad) < 2e-2, name
    # fp32 CPU oracle on the first 2 sequences (the candidate on the same rows)
    sub = [t[:2].detach().cpu() for t in (x, upstream)]
    cpu = [sub[0].clone().requires_grad_(True)] + [t.detach().cpu().clone().requires_grad_(True)
                                                  for t in (norm_w, w_up, w_down)]
    oy = model_ref.mlp(model_ref.rms_norm(cpu[0], cpu[1]), cpu[2], cpu[3])
    (oy * sub[1]).sum().backward()
    part = [t[:2].clone().requires_grad_(True) if i == 0 else t.clone().requires_grad_(True)
            for i, t in enumerate((x, norm_w, w_up, w_down))]
    py = _block_candidate(*part, 8192)
    (py.float() * upstream[:2]).sum().backward()
    assert rel_l2(py.float(), oy) < 2e-2
    for a, b, name in zip(part, cpu, ["x", "norm_w", "w_up", "w_down"]):
        assert rel_l2(a.grad, b.grad) < 2e-2, name


def test_tiled_mlp_boundary_gate(cuda_device):
    """benchmark_midpoint_v3.tile_gate: configured tile + a 17-row tail vs the
    untiled MLP module, two AdamW updates (fp16 autocast limits)."""
    torch.manual_seed(1337)
    model = build_model({"model": {"vocab_size": 101, "n_layers": 7}, "method": "midpoint"})
    left = copy.deepcopy(model.blocks[0].mlp).to(cuda_device)
    right = copy.deepcopy(left)
    del model
    opt_kw = dict(lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)
    a = torch.optim.AdamW(left.parameters(), **opt_kw)
    b = torch.optim.AdamW(right.parameters(), **opt_kw)
    limits = {"gradient_relative_l2": .02, "loss_relative": .002,
              "optimizer_step_max_absolute": .0012, "optimizer_relative_update_l2": .05}
    tokens, scale = 8192, 128.0
    rows = tokens + 17
    for _ in range(2):
        a.zero_grad(set_to_none=True)
        b.zero_grad(set_to_none=True)
        x = torch.randn(rows, 256, device=cuda_device, requires_grad=True)
        y = x.detach().clone().requires_grad_(True)
        upstream = torch.randn_like(x)
        with torch.autocast("cuda", dtype=torch.float16):
            out = left(x)
            cand = TiledMLP.apply(y, right.up.weight, right.down.weight, tokens, True)
            loss = (out.float() * upstream).sum() / rows
            other = (cand.float() * upstream).sum() / rows
        (loss * scale).backward()
        (other * scale).backward()
        pairs = [(x.grad / scale, y.grad / scale)]
        for p, q in zip(left.parameters(), right.parameters()):
            p.grad.div_(scale)
            q.grad.div_(scale)
            pairs.append((p.grad, q.grad))
        grad = max(rel_l2(v, u) for u, v in pairs)
        torch.nn.utils.clip_grad_norm_(left.parameters(), 1.0)
        torch.nn.utils.clip_grad_norm_(right.parameters(), 1.0)
        old = [p.detach().clone() for p in left.parameters()]
        old_r = [p.detach().clone() for p in right.parameters()]
        a.step()
        b.step()
        diff = sum((p - q).detach().double().square().sum().item()
                   for p, q in zip(left.parameters(), right.parameters()))
        inc = sum((p.detach() - u).double().square().sum().item()
                  for p, u in zip(left.parameters(), old))
        row = {"gradient_relative_l2": grad,
               "loss_relative": float((loss - other).detach().abs()
                                      / loss.detach().abs().clamp_min(1e-12)),
               "optimizer_step_max_absolute": max(
                   float(((p.detach() - u) - (q.detach() - v)).abs().max())
                   for p, q, u, v in zip(left.parameters(), right.parameters(), old, old_r)),
               "optimizer_relative_update_l2": math.sqrt(diff / max(inc, 1e-30))}
        for key, value in limits.items():
            assert row[key] <= value, (key, row)


# --------------------------------------------------------------------------
# full midpoint-reversible step, B=33, T=512, fp16 autocast
# --------------------------------------------------------------------------

C4 = {"model": {"vocab_size": 50257, "max_sequence_length": 512, "n_layers": 7, "n_heads": 8,
                "d_model": 256, "d_ff": 1024}, "method": "midpoint", "step_size": 0.5}


def _c4_batch(device, batch=33, length=512):
    stream = np.random.default_rng(1337).integers(0, 50257, batch * length + 1).astype(np.uint16)
    x = torch.from_numpy(stream[:-1].astype(np.int64).reshape(batch, length)).to(device)
    y = torch.from_numpy(stream[1:].astype(np.int64).reshape(batch, length)).to(device)
    return x, y


def _step_grads(model, x, y, eager=False):
    """Loss and unscaled gradients of one fp16-autocast step; ``eager``: the
    model's residual updates as the eager torch expression (the comparator)."""
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 10)
    model.zero_grad(set_to_none=True)
    with torch.autocast("cuda", dtype=torch.float16):
        with eager_updates() if eager else contextlib.nullcontext():
            logits = model(x)
        loss = F.cross_entropy(logits.flatten(0, 1), y.flatten(), reduction="sum") / y.numel()
    scaler.scale(loss).backward()
    inv = 1.0 / scaler.get_scale()
    return loss.detach(), {n: p.grad.detach() * inv for n, p in model.named_parameters()}


@pytest.mark.parametrize("core", ["split", "reuse", "reference"])
def test_full_midpoint_step_matches_autograd(cuda_device, core):
    torch.manual_seed(1337)
    reference = build_model(C4).to(cuda_device)
    candidate = copy.deepcopy(reference)
    reference.backward_mode = "autograd"
    install_v3(candidate, core_mode=core, mlp_tokens=8192, swiglu=True, rmsnorm=True)
    x, y = _c4_batch(cuda_device)
    loss_r, grads_r = _step_grads(reference, x, y, eager=True)
    loss_c, grads_c = _step_grads(candidate, x, y)
    print(f"\n[c4] core={core} loss candidate {loss_c.item():.6f} eager {loss_r.item():.6f}",
          flush=True)
    assert abs(loss_c.item() - loss_r.item()) <= 2e-3 * abs(loss_r.item())
    worst = 0.0
    for name, g in grads_r.items():
        r = rel_l2(grads_c[name], g)
        worst = max(worst, r)
        assert r < 2e-2, (name, r)
    print(f"[c4] worst parameter-gradient relative L2 {worst:.3e}", flush=True)
    # one AdamW update (fp16 gate: update relative L2 <= 0.05)
    before = {n: p.detach().clone() for n, p in reference.named_parameters()}
    for model, grads in ((reference, grads_r), (candidate, grads_c)):
        for n, p in model.named_parameters():
            p.grad = grads[n].clone()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        torch.optim.AdamW(model.parameters(), lr=6e-4, betas=(.9, .95), weight_decay=.1).step()
    diff = sum((a.detach() - b.detach()).double().square().sum().item()
               for a, b in zip(candidate.parameters(), reference.parameters()))
    inc = sum((p.detach() - before[n]).double().square().sum().item()
              for n, p in reference.named_parameters())
    assert math.sqrt(diff / inc) <= 0.05


def test_bench_path_step_matches_autograd(cuda_device):
    """The measured training step's path -- split core, tiled MLP, fused SwiGLU
    and RMSNorm, MFMA attention projections and causal attention, fused
    embedding adding into the
    tied gradient, cached head with the fused
    cross-entropy over the whole batch -- against eager autograd of the same
    model with F.cross_entropy (loss within 2e-3, every parameter gradient
    within relative L2 2e-2)."""
    torch.manual_seed(1337)
    reference = build_model(C4).to(cuda_device)
    candidate = copy.deepcopy(reference)
    reference.backward_mode = "autograd"
    install_v3(candidate, core_mode="split", mlp_tokens=33 * 512, swiglu=True, rmsnorm=True,
               keep_mlp_tiles=True)  # bench.py: one MLP tile of the whole batch
    enable_linear(candidate)
    enable_attention(candidate)
    enable_embedding(candidate, into_grad=True)
    x, y = _c4_batch(cuda_device)
    loss_r, grads_r = _step_grads(reference, x, y, eager=True)
    scaler = torch.amp.GradScaler("cuda", init_scale=2.0 ** 10)
    candidate.zero_grad(set_to_none=True)
    total = cached_head_backward(candidate, x, y, y.numel(), y.numel(), scaler, "fp16", False,
                                 "triton")
    inv = 1.0 / scaler.get_scale()
    loss_c = total / y.numel()
    print(f"\n[c4 bench path] loss {loss_c.item():.6f} eager {loss_r.item():.6f}", flush=True)
    assert abs(loss_c.item() - loss_r.item()) <= 2e-3 * abs(loss_r.item())
    worst = 0.0
    for name, p in candidate.named_parameters():
        r = rel_l2(p.grad * inv, grads_r[name])
        worst = max(worst, r)
        assert r < 2e-2, (name, r)
    print(f"[c4 bench path] worst parameter-gradient relative L2 {worst:.3e}", flush=True)


def test_full_step_reconstruction_error(cuda_device):
    torch.manual_seed(1337)
    model = build_model(C4).to(cuda_device)
    install_v3(model, core_mode="split", mlp_tokens=8192, swiglu=True, rmsnorm=True)
    x, _ = _c4_batch(cuda_device)
    with torch.autocast("cuda", dtype=torch.float16), torch.no_grad():
        p = q = model.embed(x)
        states = [(p, q)]
        for block in model.blocks:
            p, q = forward_pair(block, p, q, "midpoint", 0.5)
            states.append((p, q))
        worst = 0.0
        for i in range(6, -1, -1):
            p, q = inverse_pair(model.blocks[i], p, q, "midpoint", 0.5)
            worst = max(worst, float((p - states[i][0]).abs().max()),
                        float((q - states[i][1]).abs().max()))
    print(f"\n[c4] worst reconstructed-state max-abs {worst:.3e} (reference T4: 7.63e-5)", flush=True)
    assert worst < 5e-3


def test_full_step_matches_cpu_oracle(cuda_device):
    """Same weights and the first two sequences: the HIP path under fp16
    autocast against the fp32 CPU oracle (autograd through the recurrence)."""
    from oracle import model_ref
    torch.manual_seed(1337)
    model = build_model(C4).to(cuda_device)
    install_v3(model, core_mode="split", mlp_tokens=8192, swiglu=True, rmsnorm=True)
    x, y = _c4_batch(cuda_device, batch=2)
    loss_c, grads_c = _step_grads(model, x, y)
    loss_o, grads_o = model_ref.loss_and_grads(model.state_dict(), x, y, 7, 8, "midpoint")
    print(f"\n[c4-oracle] loss candidate {loss_c.item():.6f} oracle {loss_o.item():.6f}", flush=True)
    assert abs(loss_c.item() - loss_o.item()) <= 2e-2 * abs(loss_o.item())
    for name, g in grads_o.items():
        assert rel_l2(grads_c[name], g) < 2e-2, name


def test_tiled_mlp_kept_tiles_bitwise(cuda_device):
    """TiledMLP keeping its tiles' SwiGLU input/output for the backward gives
    the same output and gradients, bit for bit, as recomputing them."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 7000, 256, generator=g).to(cuda_device)
    up = (0.02 * torch.randn(2048, 256, generator=g)).to(cuda_device)
    down = (0.02 * torch.randn(256, 1024, generator=g)).to(cuda_device)
    gy = torch.randn(3, 7000, 256, generator=g).to(cuda_device)
    res = []
    for keep in (False, True):
        xs, us, ds = (t.clone().requires_grad_(True) for t in (x, up, down))
        with torch.autocast("cuda", dtype=torch.float16):
            out = TiledMLP.apply(xs, us, ds, 8192, True, keep)
        out.backward(gy)
        res.append((out.detach(), xs.grad, us.grad, ds.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_euler_attention_reuse_bitwise(cuda_device):
    """The Euler reconstruction with the inversion's A(p0) reused for the VJP
    gives the same loss and gradients, bit for bit, as inverting and then
    recomputing the step."""
    torch.manual_seed(11)
    cfg = {"model": {"vocab_size": 512, "max_sequence_length": 256, "n_layers": 3, "n_heads": 4,
                     "d_model": 256, "d_ff": 512}, "method": "euler", "step_size": 0.5}
    model = build_model(cfg).to(cuda_device)
    install_v3(model, core_mode="reference", mlp_tokens=256, swiglu=True, rmsnorm=True,
               keep_mlp_tiles=True)
    enable_linear(model)
    enable_attention(model)
    ids = torch.randint(0, 512, (2, 256), device=cuda_device)
    runs = []
    for reuse in (False, True):
        paths.configure(model, reuse_euler_attention=reuse, euler_mlp_at_stored_q=False)
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            loss = F.cross_entropy(model(ids).flatten(0, 1).float(), ids.flatten())
        loss.backward()
        runs.append((loss.detach(), [p.grad.clone() for p in model.parameters()]))
    assert torch.equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("switch", ["skip_unused_mlp_output", "fuse_euler_inverse"])
@pytest.mark.parametrize("keep_tiles", [False, True])
def test_euler_unused_mlp_output_skipped_bitwise(cuda_device, keep_tiles, switch):
    """The Euler VJP's rebuilt MLP output only feeds the graph-only next_p
    (skip_unused_mlp_output), and the inversion's subtractions can run inside
    the norms that read them (fuse_euler_inverse): either switch leaves the
    loss and every gradient unchanged, bit for bit."""
    torch.manual_seed(13)
    cfg = {"model": {"vocab_size": 512, "max_sequence_length": 256, "n_layers": 3, "n_heads": 4,
                     "d_model": 256, "d_ff": 512}, "method": "euler", "step_size": 0.5}
    model = build_model(cfg).to(cuda_device)
    install_v3(model, core_mode="reference", mlp_tokens=256, swiglu=True, rmsnorm=True,
               keep_mlp_tiles=keep_tiles)
    enable_linear(model)
    enable_attention(model)
    ids = torch.randint(0, 512, (2, 256), device=cuda_device)
    runs = []
    for on in (False, True):
        paths.configure(model, **{switch: on}, euler_mlp_at_stored_q=False)
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            loss = F.cross_entropy(model(ids).flatten(0, 1).float(), ids.flatten())
        loss.backward()
        runs.append((loss.detach(), [p.grad.clone() for p in model.parameters()]))
    assert torch.equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("width,heads", [(256, 4), (1024, 16)])
def test_euler_stored_q_fused_inverse_bitwise(cuda_device, width, heads):
    """The Euler VJP at the stored state with fuse_euler_inverse -- p0 made with
    its attention norm, and q0 = q - A(p0) made with the lower block's MLP norm
    (that block's M input) -- gives the loss and every gradient bit for bit as
    the unfused subtractions and norms."""
    torch.manual_seed(19)
    cfg = {"model": {"vocab_size": 512, "max_sequence_length": 256, "n_layers": 3,
                     "n_heads": heads, "d_model": width, "d_ff": 2 * width},
           "method": "euler", "step_size": 0.5}
    model = build_model(cfg).to(cuda_device)
    install_v3(model, core_mode="reference", mlp_tokens=512, swiglu=True, rmsnorm=True,
               keep_mlp_tiles=True)
    enable_linear(model)
    enable_attention(model)
    ids = torch.randint(0, 512, (2, 256), device=cuda_device)
    runs = []
    for on in (False, True):
        paths.configure(model, fuse_euler_inverse=on, euler_mlp_at_stored_q=True)
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            loss = F.cross_entropy(model(ids).flatten(0, 1).float(), ids.flatten())
        loss.backward()
        runs.append((loss.detach(), [p.grad.clone() for p in model.parameters()]))
    assert torch.equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("fused", [True, False])
def test_euler_forward_with_next_norm_bitwise(cuda_device, fused):
    """The Euler stack's forward with each p' = p + M(q') made together with the
    next block's attention norm (euler_forward) returns the same (p, q), bit for
    bit, as forward_pair block by block: on the fused fp16-output norms at
    width 1024 (the configs[4] wiring), and on the plain fp32 path."""
    from reversability_amd.reversible import euler_forward
    torch.manual_seed(17)
    cfg = {"model": {"vocab_size": 512, "max_sequence_length": 256, "n_layers": 3, "n_heads": 16,
                     "d_model": 1024, "d_ff": 2048}, "method": "euler", "step_size": 0.5}
    model = build_model(cfg).to(cuda_device)
    if fused:
        install_v3(model, core_mode="reference", mlp_tokens=512, swiglu=True, rmsnorm=True)
        enable_linear(model)
        enable_attention(model)
    x = torch.randn(2, 256, 1024, device=cuda_device)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.float16, enabled=fused):
        p1, q1 = euler_forward(model.blocks, x, x)
        p2, q2 = x, x
        for block in model.blocks:
            p2, q2 = forward_pair(block, p2, q2, "euler", 0.5)
    assert torch.equal(p1, p2) and torch.equal(q1, q2)


def test_split_midpoint_fused_update_norm_bitwise(cuda_device):
    """The split midpoint core with each midpoint update made together with
    the next layer's attention norm (fuse_midpoint_norm) gives the same loss
    and gradients, bit for bit, as the separate update and norm."""
    torch.manual_seed(17)
    cfg = {"model": {"vocab_size": 512, "max_sequence_length": 256, "n_layers": 3, "n_heads": 4,
                     "d_model": 256, "d_ff": 512}, "method": "midpoint", "step_size": 0.5}
    model = build_model(cfg).to(cuda_device)
    install_v3(model, core_mode="split", mlp_tokens=512, swiglu=True, rmsnorm=True,
               keep_mlp_tiles=True)
    enable_linear(model)
    enable_attention(model)
    ids = torch.randint(0, 512, (2, 256), device=cuda_device)
    runs = []
    for on in (False, True):
        paths.configure(model, fuse_midpoint_norm=on)
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            loss = F.cross_entropy(model(ids).flatten(0, 1).float(), ids.flatten())
        loss.backward()
        runs.append((loss.detach(), [p.grad.clone() for p in model.parameters()]))
    assert torch.equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a, b)


def test_split_midpoint_kept_attention_bitwise(cuda_device):
    """SplitMidpoint with the inversion's attention graph kept for the attention
    VJP gives the same loss and gradients, bit for bit, as recomputing it."""
    torch.manual_seed(12)
    model = build_model(C4).to(cuda_device)
    install_v3(model, core_mode="split", mlp_tokens=8192, swiglu=True, rmsnorm=True,
               keep_mlp_tiles=True)
    enable_linear(model)
    enable_attention(model)
    x, y = _c4_batch(cuda_device, batch=4)
    runs = []
    for keep in (False, True):
        paths.configure(model, keep_split_attention=keep)
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            loss = F.cross_entropy(model(x).flatten(0, 1).float(), y.flatten())
        loss.backward()
        runs.append((loss.detach(), [p.grad.clone() for p in model.parameters()]))
    assert torch.equal(runs[0][0], runs[1][0])
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("config", ["c4", "c5"])
def test_captured_train_step_matches_eager_bitwise(cuda_device, config):
    """The whole configs[3] / configs[4] update (bench.make_train_step: batch cut on the
    device, fp16 core forward and reconstruction backward, tied head and fused
    cross-entropy, GradScaler unscale, clip, FusedAdamW) captured once in a
    HIP graph and replayed equals the eager update of a twin model bit for
    bit -- loss, every parameter, the loss scale -- after each of three
    replays, with the twin's eager updates and host synchronisations between
    the replays.  Replays must also change the parameters (the graph is not
    a no-op)."""
    import bench
    from reversability_amd.graph import CapturedStep
    eager, _, _ = bench.make_train_step(cuda_device, config)
    graphed, _, _ = bench.make_train_step(cuda_device, config)
    captured = CapturedStep(graphed, warmup=3)
    for _ in range(3):  # the capture's warm-up updates
        eager()
    torch.cuda.synchronize()
    before = [p.detach().clone() for p in graphed.model.parameters()]
    for i in range(3):
        print(f"  replay {i}", flush=True)
        loss_g = captured().clone()
        torch.cuda.synchronize()
        loss_e = eager()
        torch.cuda.synchronize()
        assert torch.equal(loss_g, loss_e), (i, float(loss_g), float(loss_e))
        for (name, pe), pg in zip(eager.model.named_parameters(), graphed.model.parameters()):
            assert torch.equal(pe, pg), (i, name)
        assert torch.equal(eager.scaler._scale, graphed.scaler._scale)
    changed = sum(not torch.equal(b, p) for b, p in zip(before, graphed.model.parameters()))
    assert changed == len(before)


def test_euler_mlp_at_stored_state_within_truth(cuda_device):
    """The Euler VJP with M linearised at the stored q (euler_mlp_at_stored_q,
    one MLP evaluation per layer less) against the rebuild at q0 + A(p0): the
    same loss bit for bit (the forward is unchanged) and gradients no farther
    from the fp32 truth than the rebuild's, within 1.25x per parameter (floor
    1e-2 relative L2)."""
    from reversability_amd.residual import eager_updates
    torch.manual_seed(19)
    cfg = {"model": {"vocab_size": 512, "max_sequence_length": 256, "n_layers": 4, "n_heads": 4,
                     "d_model": 256, "d_ff": 512}, "method": "euler", "step_size": 0.5}
    base = build_model(cfg).to(cuda_device)
    ids = torch.randint(0, 512, (4, 256), device=cuda_device)
    truth = copy.deepcopy(base)
    truth.backward_mode = "autograd"
    with eager_updates():
        F.cross_entropy(truth(ids).flatten(0, 1), ids.flatten()).backward()
    model = copy.deepcopy(base)
    install_v3(model, core_mode="reference", mlp_tokens=1024, swiglu=True, rmsnorm=True,
               keep_mlp_tiles=True)
    enable_linear(model)
    enable_attention(model)
    runs = {}
    for on in (False, True):
        paths.configure(model, euler_mlp_at_stored_q=on)
        model.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.float16):
            loss = F.cross_entropy(model(ids).flatten(0, 1).float(), ids.flatten())
        loss.backward()
        runs[on] = (loss.detach(), {n: p.grad.clone() for n, p in model.named_parameters()})
    assert torch.equal(runs[False][0], runs[True][0])
    worst = 0.0
    for name, p in truth.named_parameters():
        stored, rebuilt = rel_l2(runs[True][1][name], p.grad), rel_l2(runs[False][1][name], p.grad)
        worst = max(worst, stored)
        assert stored <= max(1e-2, 1.25 * rebuilt), (name, stored, rebuilt)
    print(f"\n[euler stored-q] worst gradient relative L2 to the fp32 truth {worst:.3e}", flush=True)
