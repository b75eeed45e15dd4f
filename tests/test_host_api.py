"""Host-side behaviour of the reference operator surface, on the CPU.

Restates the reference's CPU tests for this path (tests/test_kernels.py:10-16,
tests/test_optimized_v3.py:14-70, tests/test_reversible.py:12-33,
tests/test_optimized.py:17-50) against this package, plus the CPU-autocast
regression for the reconstruction backward.  No kernel runs here: the fused
operators must refuse CPU tensors, and everything else is torch on the CPU.
"""
from __future__ import annotations

import copy

import pytest
import torch
import torch.nn.functional as F

from reconstruction_gate import run_gate
from reversability_amd import BaselineLM, ModelConfig, ReversibleLM, build_model
from reversability_amd import optimized_v3 as v3
from reversability_amd.kernels import FusedSwiGLU, enable_swiglu
from reversability_amd.kernels_v3 import FusedRMSNorm
from reversability_amd.optimized import ReusedMidpoint, chunked_backward
from reversability_amd.optimized_v3 import SplitMidpoint, TiledMLP, cached_head_backward, install_v3
from reversability_amd.residual import midpoint_step
from reversability_amd.reversible import forward_pair

TINY = {"vocab_size": 31, "max_sequence_length": 8, "n_layers": 3, "n_heads": 2, "d_model": 8,
        "d_ff": 16}


# ---------------------------------------------------------------------------
# No silent CPU fallback (tests/test_kernels.py:10-16, test_optimized_v3.py:66-70)
# ---------------------------------------------------------------------------

def test_kernels_reject_cpu_instead_of_silent_fallback():
    with pytest.raises(ValueError, match="CUDA"):
        FusedSwiGLU.apply(torch.zeros(3, 32))


def test_v3_norm_rejects_cpu():
    with pytest.raises(ValueError, match="CUDA FP32"):
        FusedRMSNorm.apply(torch.ones(3, 8), torch.ones(8), 1e-7)


def test_fused_paths_installed_on_cpu_model_refuse_to_run():
    model = build_model({"model": TINY, "method": "midpoint"})
    install_v3(model, core_mode="split", mlp_tokens=5, swiglu=True, rmsnorm=True)
    with pytest.raises(ValueError, match="CUDA"):
        model(torch.randint(31, (2, 8)))
    other = build_model({"model": TINY, "method": "midpoint"})
    enable_swiglu(other)
    with pytest.raises(ValueError, match="CUDA"):
        other(torch.randint(31, (2, 8)))


# ---------------------------------------------------------------------------
# Reconstruction gate (tests/test_reversible.py:12-15)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("method", ["midpoint", "euler"])
@pytest.mark.parametrize("precision", ["fp64", "fp32"])
def test_reconstruction_gradients_and_update(method, precision):
    report = run_gate(method, precision, "cpu", 3, 17)
    if precision == "fp64":  # algebraic inverse: reconstruction exact to rounding
        assert report.worst_state_error() < 1e-13


@pytest.mark.parametrize("core", ["reuse", "split"])
def test_reconstruction_gate_with_optimized_core(core):
    run_gate("midpoint", "fp64", "cpu", 3, 17, prepare=lambda m: install_v3(m, core_mode=core))


# ---------------------------------------------------------------------------
# Structure (tests/test_reversible.py:17-33)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("method", ["midpoint", "euler"])
def test_initialization_mapping_and_parameter_count(method):
    config = ModelConfig(vocab_size=101, n_layers=3, d_model=32, n_heads=2, d_ff=64)
    torch.manual_seed(1337)
    base = BaselineLM(config)
    torch.manual_seed(1337)
    rev = ReversibleLM(config, method)
    assert base.parameter_count() == rev.parameter_count()
    for name, p in base.state_dict().items():
        torch.testing.assert_close(p, rev.state_dict()[name], rtol=0, atol=0)


def test_default_architecture_parameter_count_and_names():
    model = ReversibleLM(ModelConfig(), "midpoint")
    assert model.parameter_count() == 20_340_736  # README.md:31 of the reference
    names = [n for n, _ in model.named_parameters()]
    assert names[:2] == ["token_embedding.weight", "position_embedding.weight"]
    assert names[2:8] == ["blocks.0.attn_norm.weight", "blocks.0.attn.qkv.weight",
                          "blocks.0.attn.proj.weight", "blocks.0.mlp_norm.weight",
                          "blocks.0.mlp.up.weight", "blocks.0.mlp.down.weight"]
    assert model.lm_head.weight is model.token_embedding.weight
    assert tuple(model.blocks[0].mlp.up.weight.shape) == (2048, 256)


def test_initialization_statistics():
    torch.manual_seed(0)
    model = BaselineLM(ModelConfig(n_layers=7))
    std = lambda t: float(t.detach().std())  # noqa: E731
    assert abs(std(model.token_embedding.weight) - 0.02) < 5e-4
    assert abs(std(model.blocks[0].attn.qkv.weight) - 0.02) < 5e-4
    assert abs(std(model.blocks[3].mlp.down.weight) - 0.02 / 14 ** 0.5) < 2e-4
    assert abs(std(model.blocks[6].attn.proj.weight) - 0.02 / 14 ** 0.5) < 4e-4
    assert torch.equal(model.blocks[0].attn_norm.weight, torch.ones(256))


@pytest.mark.parametrize("method", ["midpoint", "euler"])
def test_inverse_stack_retains_only_final_pair_and_parameters(method):
    model = ReversibleLM(ModelConfig(vocab_size=31, n_layers=7, n_heads=1, d_model=8, d_ff=16), method)
    x = torch.randn(2, 4, 8, requires_grad=True)
    y = model.core(x)
    saved = y.grad_fn.saved_tensors
    assert len(saved) == 2 + len(tuple(model.blocks.parameters()))
    assert [tuple(t.shape) for t in saved[:2]] == [(2, 4, 8), (2, 4, 8)]


def test_constructor_validation():
    config = ModelConfig(vocab_size=31, n_layers=1, n_heads=1, d_model=8, d_ff=16)
    for kwargs in [dict(method="leapfrog"), dict(method="midpoint", step_size=0.0),
                   dict(method="euler", step_size=0.25),
                   dict(method="midpoint", backward_mode="checkpoint")]:
        with pytest.raises(ValueError):
            ReversibleLM(config, **kwargs)
    with pytest.raises(ValueError):
        ReversibleLM(ModelConfig(vocab_size=31, n_layers=1, n_heads=1, d_model=8, d_ff=16,
                                 dropout=0.1), "midpoint")
    with pytest.raises(ValueError):
        ModelConfig(d_model=10, n_heads=3)
    with pytest.raises(ValueError):
        build_model({"model": TINY, "method": "midpoint", "compile": True})


# ---------------------------------------------------------------------------
# Optimized cores vs the unrolled recurrence, fp64 (tests/test_optimized.py:36-50,
# tests/test_optimized_v3.py:38-51)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("h", [.25, .5, .75])
@pytest.mark.parametrize("function", [ReusedMidpoint, SplitMidpoint])
def test_optimized_core_state_and_vjp_vs_unrolled(h, function):
    torch.manual_seed(73)
    a = build_model({"model": {**TINY, "max_sequence_length": 512}, "method": "midpoint"}).double()
    b = copy.deepcopy(a)
    p = torch.randn(3, 4, 8, dtype=torch.float64, requires_grad=True)
    q = torch.randn_like(p, requires_grad=True)
    rp = p.detach().clone().requires_grad_(True)
    rq = q.detach().clone().requires_grad_(True)
    x, y = p, q
    for block in a.blocks:
        x, y = forward_pair(block, x, y, "midpoint", h)
    u, v = function.apply(rp, rq, b.blocks, h, *b.blocks.parameters())
    gp, gq = torch.randn_like(p), torch.randn_like(q)
    torch.autograd.backward((x, y), (gp, gq))
    torch.autograd.backward((u, v), (gp, gq))
    torch.testing.assert_close(x, u, rtol=0, atol=0)
    torch.testing.assert_close(y, v, rtol=0, atol=0)
    pairs = [(p.grad, rp.grad), (q.grad, rq.grad)]
    pairs += [(s.grad, t.grad) for s, t in zip(a.parameters(), b.parameters()) if s.grad is not None]
    for left, right in pairs:
        torch.testing.assert_close(left, right, rtol=1e-10, atol=1e-11)


# ---------------------------------------------------------------------------
# Tiled MLP (tests/test_optimized_v3.py:54-64)
# ---------------------------------------------------------------------------

def test_tiled_mlp_tiles_and_entire_input(monkeypatch):
    sizes = []
    original = v3.tile_forward

    def observe(x, *args, **kwargs):
        sizes.append(x.shape[0])
        return original(x, *args, **kwargs)
    monkeypatch.setattr(v3, "tile_forward", observe)
    x = torch.randn(50, 8, 8, requires_grad=True)
    up = torch.randn(32, 8, requires_grad=True)
    down = torch.randn(8, 16, requires_grad=True)
    y = TiledMLP.apply(x, up, down, 37, False)
    y.square().mean().backward()
    assert y.shape == (50, 8, 8)
    assert len(sizes) == 2 * ((400 + 36) // 37) and max(sizes) <= 37
    assert x.grad.shape == x.shape


@pytest.mark.parametrize("tokens", [1, 7, 37, 400, 1000])
def test_tiled_mlp_matches_untiled_fp64(tokens):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(50, 8, 8, generator=g, dtype=torch.float64, requires_grad=True)
    up = torch.randn(32, 8, generator=g, dtype=torch.float64, requires_grad=True)
    down = torch.randn(8, 16, generator=g, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(50, 8, 8, generator=g, dtype=torch.float64)
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, up, down)]
    y = TiledMLP.apply(x, up, down, tokens, False)
    ref = v3.mlp_value(*leaves, False)
    torch.testing.assert_close(y, ref, rtol=1e-12, atol=1e-12)
    y.backward(dy)
    ref.backward(dy)
    for a, b in zip((x, up, down), leaves):
        torch.testing.assert_close(a.grad, b.grad, rtol=1e-10, atol=1e-11)


def test_tiled_mlp_rejects_nonpositive_tile():
    with pytest.raises(ValueError):
        TiledMLP.apply(torch.randn(4, 8), torch.randn(32, 8), torch.randn(8, 16), 0, False)


def test_tiled_mlp_under_cpu_autocast_matches_autograd():
    # bf16 CPU autocast exercises the explicit backward's casts (the GPU runs fp16)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(40, 16, generator=g, requires_grad=True)
    up = (0.1 * torch.randn(64, 16, generator=g)).requires_grad_(True)
    down = (0.1 * torch.randn(16, 32, generator=g)).requires_grad_(True)
    dy = torch.randn(40, 16, generator=g).bfloat16()
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, up, down)]
    with torch.autocast("cpu", dtype=torch.bfloat16):
        y = TiledMLP.apply(x, up, down, 9, False)
        ref = v3.mlp_value(*leaves, False)
    assert y.dtype == ref.dtype == torch.bfloat16
    torch.testing.assert_close(y, ref, rtol=0, atol=0)
    y.backward(dy)
    ref.backward(dy)
    for a, b in zip((x, up, down), leaves):
        assert a.grad.dtype == b.grad.dtype == torch.float32
        torch.testing.assert_close(a.grad, b.grad, rtol=2e-2, atol=2e-2)


# ---------------------------------------------------------------------------
# install_v3 wiring (tests/test_optimized_v3.py:14-35)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("core", ["reference", "reuse", "split"])
@pytest.mark.parametrize("tile", [0, 5])
def test_full_batch_v3_tied_gradients_masks_and_two_updates(dtype, core, tile):
    config = {"model": TINY, "method": "midpoint"}
    torch.manual_seed(71)
    reference = build_model(config).to(dtype)
    candidate = copy.deepcopy(reference)
    install_v3(candidate, core_mode=core, mlp_tokens=tile)
    a = torch.optim.AdamW(reference.parameters(), lr=.0006)
    b = torch.optim.AdamW(candidate.parameters(), lr=.0006)
    for _ in range(2):
        a.zero_grad(set_to_none=True)
        b.zero_grad(set_to_none=True)
        ids = torch.randint(31, (5, 8))
        labels = ids.roll(-1, 1)
        labels[-1, :] = -100
        labels[0, -1] = -100
        denominator = int((labels != -100).sum())
        expected = F.cross_entropy(reference(ids).flatten(0, 1), labels.flatten(),
                                   ignore_index=-100, reduction="sum")
        (expected / denominator).backward()
        actual = cached_head_backward(candidate, ids, labels, denominator, 7)
        torch.testing.assert_close(actual, expected.detach().float(), rtol=2e-6, atol=2e-5)
        tolerance = 1e-10 if dtype == torch.float64 else 5e-5
        for p, q in zip(reference.parameters(), candidate.parameters()):
            assert torch.isfinite(q.grad).all()
            torch.testing.assert_close(p.grad, q.grad, rtol=tolerance, atol=tolerance * .01)
        a.step()
        b.step()
    assert candidate.lm_head.weight is candidate.token_embedding.weight


def test_install_v3_is_idempotent_and_rejects_conflicts():
    model = build_model({"model": TINY, "method": "midpoint"})
    assert install_v3(model, core_mode="reuse", mlp_tokens=5) is model
    assert install_v3(model, core_mode="reuse", mlp_tokens=5) is model
    with pytest.raises(ValueError):
        install_v3(model, core_mode="split", mlp_tokens=5)
    with pytest.raises(ValueError):
        install_v3(build_model({"model": TINY, "method": "euler"}), core_mode="reuse")
    biased = build_model({"model": {**TINY, "bias": True}, "method": "midpoint"})
    with pytest.raises(ValueError):
        install_v3(biased, mlp_tokens=4)


# ---------------------------------------------------------------------------
# Chunked head (tests/test_optimized.py:17-33)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("method", ["baseline", "midpoint"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("chunk", [1, 7, 100])
def test_chunked_tied_weight_gradients_masks_accumulation(method, dtype, chunk):
    config = {"model": TINY, "method": method}
    torch.manual_seed(23)
    original = build_model(config).to(dtype)
    candidate = copy.deepcopy(original)
    for _ in range(2):
        ids = torch.randint(31, (3, 8))
        labels = ids.roll(-1, 1).clone()
        labels[-1, :] = -100
        labels[0, -1] = -100
        loss = F.cross_entropy(original(ids).flatten(0, 1), labels.flatten(), ignore_index=-100,
                               reduction="sum")
        (loss / 91).backward()
        actual = chunked_backward(candidate, ids, labels, 91, chunk, reuse=method == "midpoint")
        torch.testing.assert_close(actual, loss.detach().float(), rtol=2e-6, atol=2e-5)
    tolerance = 2e-5 if dtype == torch.float32 else 1e-10
    for a, b in zip(original.parameters(), candidate.parameters()):
        torch.testing.assert_close(a.grad, b.grad, rtol=tolerance, atol=tolerance * .01)
    assert candidate.lm_head.weight is candidate.token_embedding.weight


# ---------------------------------------------------------------------------
# Residual update on CPU = the reference's eager expression, bit for bit
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("sign", [1, -1])
def test_midpoint_step_cpu_is_the_eager_expression(sign):
    g = torch.Generator().manual_seed(3)
    p = torch.randn(1000, generator=g)
    a = torch.randn(1000, generator=g).bfloat16()
    m = torch.randn(1000, generator=g).bfloat16()
    out = midpoint_step(p, a, m, 2 * 0.3, sign)
    ref = p + 2 * 0.3 * (a + m) if sign > 0 else p - 2 * 0.3 * (a + m)
    assert torch.equal(out, ref)


# ---------------------------------------------------------------------------
# Reconstruction backward under autocast with the backward outside the
# autocast context (CPU bf16 stands in for the GPU's fp16): weight casts made
# under no_grad must not be reused without autograd history.
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("core", ["reference", "reuse", "split"])
def test_reconstruction_under_autocast_backward_outside_context(core):
    torch.manual_seed(5)
    config = {"model": {**TINY, "d_model": 16, "d_ff": 32}, "method": "midpoint"}
    reference = build_model(config)
    candidate = copy.deepcopy(reference)
    reference.backward_mode = "autograd"
    install_v3(candidate, core_mode=core, mlp_tokens=5 if core == "split" else 0)
    ids = torch.randint(31, (2, 8))
    for model in (reference, candidate):
        with torch.autocast("cpu", dtype=torch.bfloat16):
            loss = F.cross_entropy(model(ids).flatten(0, 1).float(), ids.flatten())
        loss.backward()
    for (name, a), b in zip(reference.named_parameters(), candidate.parameters()):
        assert b.grad is not None, name
        rel = float((a.grad - b.grad).norm() / a.grad.norm().clamp_min(1e-12))
        assert rel < 2e-2, (name, rel)


def test_weight_cast_cache_scope():
    """cast_weight reuses a cast only inside weight_cast_cache, keyed on the
    tensor object itself (CPU: the cast's launcher is replaced by a stub)."""
    import torch
    from reversability_amd import mlp
    calls = []
    original = mlp.cast_f16
    mlp.cast_f16 = lambda t: calls.append(t) or t.half()
    try:
        w, v = torch.ones(4, 4), torch.ones(4, 4)
        mlp.cast_weight(w), mlp.cast_weight(w)
        assert len(calls) == 2          # no cache outside the block
        with mlp.weight_cast_cache():
            a = mlp.cast_weight(w)
            with mlp.weight_cast_cache():   # nested blocks share the cache
                assert mlp.cast_weight(w) is a
            assert mlp.cast_weight(v) is not a
            assert mlp.cast_weight(w) is a
        assert len(calls) == 4
        mlp.cast_weight(w)
        assert len(calls) == 5          # the cache ends with the outer block
    finally:
        mlp.cast_f16 = original


def test_mlp_output_unused_is_per_thread_and_gpu_only():
    """mlp.output_unused() marks only the opening thread's GPU MLP calls (the
    autograd device thread that runs a reconstruction backward); CPU inputs and
    other threads always get their output computed."""
    import threading
    from reversability_amd import mlp
    cpu = torch.zeros(2, 4)
    meta_cuda = torch.empty(2, 4, device="meta")
    assert mlp.output_wanted(cpu) and mlp.output_wanted(meta_cuda)
    with mlp.output_unused():
        with mlp.output_unused():
            assert mlp.output_wanted(cpu)
        other = []
        worker = threading.Thread(target=lambda: other.append(getattr(mlp._output_unused,
                                                                      "depth", 0)))
        worker.start()
        worker.join()
        assert other == [0] and mlp._output_unused.depth == 1
    assert mlp._output_unused.depth == 0


# ---------------------------------------------------------------------------
# Path selection: per-model switches and the path record
# ---------------------------------------------------------------------------

def test_reconstruction_switches_are_per_model():
    from reversability_amd import paths
    a = build_model({"model": TINY, "method": "euler"})
    b = build_model({"model": TINY, "method": "euler"})
    assert paths.of(a.blocks) == paths.DEFAULT
    paths.configure(a, fuse_euler_inverse=False)
    assert not paths.of(a.blocks).fuse_euler_inverse
    assert paths.of(b.blocks).fuse_euler_inverse  # the other model is untouched
    assert not paths.of(copy.deepcopy(a).blocks).fuse_euler_inverse
    c = build_model({"model": TINY, "method": "midpoint"})
    off = paths.ReconstructionPaths(keep_split_attention=False)
    install_v3(c, core_mode="split", paths=off)
    assert paths.of(c.blocks) == off
    assert install_v3(c, core_mode="split", paths=off) is c
    with pytest.raises(ValueError):
        install_v3(c, core_mode="split")  # another configuration: the default switches


@pytest.mark.parametrize("switches", [dict(keep_split_attention=False),
                                      dict(fuse_midpoint_norm=False), {}])
def test_split_core_switches_keep_values_fp64(switches):
    """Every switch setting gives the same fp64 loss and gradients on the CPU."""
    from reversability_amd import paths
    torch.manual_seed(5)
    ref = build_model({"model": TINY, "method": "midpoint"}).double()
    cand = copy.deepcopy(ref)
    install_v3(cand, core_mode="split")
    paths.configure(cand, **switches)
    ids = torch.randint(31, (2, 8))
    for model in (ref, cand):
        F.cross_entropy(model(ids).flatten(0, 1), ids.flatten()).backward()
    for p, q in zip(ref.parameters(), cand.parameters()):
        torch.testing.assert_close(p.grad, q.grad, rtol=1e-10, atol=1e-12)


def test_path_record_and_strict_mode():
    from reversability_amd import paths
    paths.reset()
    paths.took("attention", "hip")
    paths.took("attention", "hip")
    paths.took("attention", "sdpa", "head size 48")
    assert paths.report() == {"attention": {"hip": 2, "sdpa": 1}}
    with paths.strict():
        paths.took("attention", "hip")  # the HIP path never raises
        with pytest.raises(paths.UnsupportedPathError, match="head size 48"):
            paths.took("attention", "sdpa", "head size 48")
    paths.took("attention", "sdpa", "outside strict() a fallback only counts")
    assert paths.report()["attention"] == {"hip": 3, "sdpa": 2}
    paths.reset()
    assert paths.report() == {}


def test_tiled_mlp_records_its_path_on_cpu():
    from reversability_amd import paths
    paths.reset()
    x = torch.randn(2, 5, 8, dtype=torch.float64, requires_grad=True)
    up = torch.randn(32, 8, dtype=torch.float64, requires_grad=True)
    down = torch.randn(8, 16, dtype=torch.float64, requires_grad=True)
    with paths.strict():  # the unfused CPU computation is what was asked for: no fallback
        TiledMLP.apply(x, up, down, 3, False).sum().backward()
    assert paths.report() == {"tiled_mlp": {"torch-gemm": 1}}
    paths.reset()
