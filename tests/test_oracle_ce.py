"""Pins of the cross-entropy oracle (oracle.ce_fwd / oracle.ce_bwd), CPU only.

The oracle restates src/reversibility/kernels.py:14-77 (TiledCrossEntropy):
the log-probability at the target is rounded to the logits dtype before the
fp32 NLL, and the backward rounds the log-probability again before exp.
What fixes it here, independently of its own formula:

* fp64 cross-entropy (torch, library) per row, within the one rounding of
  the log-probability to the logits dtype;
* the uniform-logits closed form loss = log V, rounded as the reference does;
* torch's eager fp16 log_softmax gathered at the target (the reference's
  Half-logsoftmax policy; torch accumulates in fp32, so <= 1 fp16 ulp);
* the fp64 gradient g (softmax - onehot), within the effect of rounding the
  log-probability before exp, and its zero row sums;
* ignore_index rows (zero loss, zero gradient) and out-of-range labels (NaN).
A dropped max-subtraction, a missing rounding point, or a sign error in the
gradient each fails one of these (tests below plant two of them).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

LABELS17 = [0, 1023, 1024, 50256, -100] + list(range(12))  # tests/test_kernels.py:25


def ulp16(v):
    return np.spacing(np.abs(np.asarray(v, np.float64)).astype(np.float16)).astype(np.float64)


def logits(rows, cols, dtype, seed=41, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(rows, cols, generator=g)).to(dtype).numpy()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_ce_oracle_matches_fp64(dtype):
    x = logits(17, 50257, dtype)
    y = np.array(LABELS17, np.int64)
    _, _, loss = oracle.ce_fwd(x, y)
    ref = F.cross_entropy(torch.from_numpy(x).double(), torch.from_numpy(y), reduction="none",
                          ignore_index=-100).numpy()
    bound = ulp16(ref) if dtype == torch.float16 else 1e-6 * np.abs(ref) + 1e-7
    assert np.all(np.abs(loss - ref) <= bound)
    assert loss[4] == 0.0
    assert abs(loss.sum() - ref.sum()) <= 2e-3 * abs(ref.sum())


def test_ce_oracle_uniform_closed_form():
    for v in (7, 1000, 50257):
        x = np.zeros((3, v), np.float16)
        _, lse, loss = oracle.ce_fwd(x, np.array([0, v - 1, v // 2], np.int64))
        expect = -float(np.float16(-np.float32(np.log(v))))
        assert np.all(lse == np.float32(np.log(v)))
        assert np.all(loss == np.float32(expect))


def test_ce_oracle_matches_torch_half_log_softmax():
    x = logits(64, 4099, torch.float16, seed=3, scale=4.0)
    y = np.random.default_rng(3).integers(0, 4099, 64).astype(np.int64)
    _, _, loss = oracle.ce_fwd(x, y)
    logp = torch.log_softmax(torch.from_numpy(x), -1)  # fp16 out, fp32 accumulation
    ref = -logp[torch.arange(64), torch.from_numpy(y)].float().numpy()
    diff = np.abs(loss - ref)
    assert np.all(diff <= ulp16(ref))
    assert np.mean(diff == 0) > 0.9


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_ce_oracle_backward_vs_fp64_gradient(dtype):
    x = logits(17, 50257, dtype, seed=5)
    y = np.array(LABELS17, np.int64)
    g = 0.03125
    rmax, rlse, _ = oracle.ce_fwd(x, y)
    dx = oracle.ce_bwd(x, y, rmax, rlse, g).astype(np.float64)
    xt = torch.from_numpy(x).double().requires_grad_(True)
    F.cross_entropy(xt, torch.from_numpy(y), reduction="sum", ignore_index=-100).mul(g).backward()
    ref = xt.grad.numpy()
    p = np.exp(x.astype(np.float64) - rmax[:, None].astype(np.float64) - rlse[:, None].astype(np.float64))
    if dtype == torch.float16:
        # exp of the fp16-rounded log-probability: relative error <= ulp(logp) / 2
        logp = x.astype(np.float64) - rmax[:, None] - rlse[:, None]
        tol = g * p * (np.exp(ulp16(logp) / 2) - 1) * 1.01 + ulp16(ref) + 1e-12
    else:
        tol = 1e-5 * np.abs(ref) + 1e-9
    tol[4] = 0.0
    assert np.all(np.abs(dx - ref) <= tol)
    assert np.all(dx[4] == 0.0)
    # rows of a softmax gradient sum to zero (up to the output rounding)
    assert np.all(np.abs(dx.sum(1)) <= 2e-3 * g)


def test_ce_oracle_bad_label_is_nan():
    x = logits(3, 10, torch.float16)
    rmax, rlse, loss = oracle.ce_fwd(x, np.array([10, -1, 2], np.int64))
    assert np.isnan(loss[0]) and np.isnan(loss[1]) and not np.isnan(loss[2])
    dx = oracle.ce_bwd(x, np.array([10, -1, 2], np.int64), rmax, rlse, 1.0)
    assert np.all(np.isnan(dx[:2].astype(np.float32))) and np.all(np.isfinite(dx[2].astype(np.float32)))


def test_ce_pins_catch_planted_mistakes():
    """A restatement without the max subtraction overflows in fp32-range
    logits, and one that skips the fp16 rounding of logp disagrees with the
    eager Half log_softmax: the pins above would reject either."""
    x = logits(8, 3000, torch.float16, seed=9, scale=30.0)
    y = np.arange(8, dtype=np.int64)
    xf = x.astype(np.float32)
    with np.errstate(over="ignore"):
        no_max = np.log(np.exp(xf).sum(1)) - xf[np.arange(8), y]  # overflows: inf
    ref = F.cross_entropy(torch.from_numpy(x).double(), torch.from_numpy(y), reduction="none").numpy()
    assert not np.all(np.abs(no_max - ref) <= ulp16(ref))
    _, lse, loss = oracle.ce_fwd(x, y)
    m = xf.max(1)
    unrounded = -((xf[np.arange(8), y] - m) - lse)
    torch_ref = -torch.log_softmax(torch.from_numpy(x), -1)[torch.arange(8), torch.from_numpy(y)].float().numpy()
    assert np.any(unrounded != torch_ref) and np.all(np.abs(loss - torch_ref) <= ulp16(torch_ref))
