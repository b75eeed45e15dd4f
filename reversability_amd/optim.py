"""AdamW on one multi-tensor HIP kernel, a drop-in for torch.optim.AdamW.

The training step of the reference (scripts/benchmark_optimized.py:38-40,
66-80; scripts/train_baseline.py:270-284) runs ``torch.optim.AdamW(params,
lr, betas=(0.9, 0.95), weight_decay=0.1)`` behind ``torch.amp.GradScaler``:
``unscale_``, ``clip_grad_norm_``, ``scaler.step``, ``scaler.update``.
``FusedAdamW`` keeps that constructor and that driving sequence and replaces
torch's per-operation multi-tensor kernels with one pass over parameters,
gradients and both moments (``rv_adamw_step``), in torch's arithmetic order.

It declares ``_step_supports_amp_scaling``: ``GradScaler.step`` then hands it
the device ``found_inf`` flag (and ``grad_scale`` when gradients were not
unscaled first) instead of synchronising on the host; an overflowing step
changes no parameter, moment or step count.  The step count is a device
tensor per parameter group (shared by the group's ``state[p]["step"]``).
Supported: fp32 dense CUDA parameters, amsgrad=False, maximize=False; other
configurations raise.

``unscale_clip_(scaler, max_norm)`` stands for the reference's
``scaler.unscale_(opt); torch.nn.utils.clip_grad_norm_(params, max_norm)``
(scripts/train_baseline.py:278-280) in one read of the gradients: it computes
the norm of the unscaled gradients and the clip coefficient on the device
(``rv_grad_sq_partials`` / ``rv_grad_clip_coef``), records the overflow flag
with the scaler as ``unscale_`` does, and leaves both multiplies to the next
``step()``, which applies them as it reads each gradient
(``rv_adamw_step_clipped``) -- the values the two passes would have written.
Between the two calls ``p.grad`` still holds the scaled, unclipped gradient.
"""
from __future__ import annotations

import ctypes

import torch
from torch.optim import Optimizer

from ._hip import _check, _stream, library


class FusedAdamW(Optimizer):
    _step_supports_amp_scaling = True

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2,
                 amsgrad=False, *, maximize=False, foreach=None, capturable=False,
                 differentiable=False, fused=None):
        if amsgrad or maximize or differentiable:
            raise ValueError("FusedAdamW supports amsgrad=False, maximize=False, "
                             "differentiable=False")
        if not 0.0 <= lr or not 0.0 <= eps or not 0.0 <= weight_decay:
            raise ValueError("Invalid learning rate, epsilon or weight decay")
        if not (0.0 <= betas[0] < 1.0 and 0.0 <= betas[1] < 1.0):
            raise ValueError(f"Invalid betas: {betas}")
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))

    def _group_state(self, group):
        params = [p for p in group["params"] if p.grad is not None]
        for p in params:
            if p.dtype != torch.float32 or not p.is_cuda or p.grad.is_sparse:
                raise ValueError("FusedAdamW requires dense CUDA (ROCm device) FP32 parameters")
        if not params:
            return None, []
        step = None
        for p in group["params"]:
            st = self.state[p]
            if "step" in st:
                step = st["step"]
                break
        if step is None:
            step = torch.zeros((), device=params[0].device, dtype=torch.float32)
        for p in params:
            st = self.state[p]
            if "exp_avg" not in st:
                st["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
            st["step"] = step
        return step, params

    @torch.no_grad()
    def unscale_clip_(self, scaler, max_norm: float) -> torch.Tensor:
        """``scaler.unscale_(self)`` + ``clip_grad_norm_(all parameters with a
        gradient, max_norm)`` (norm type 2); returns the total norm of the
        unscaled gradients (a device scalar).  ``scaler`` may be None (clip
        only)."""
        from torch.amp.grad_scaler import OptState
        lib = library()
        params = [p for group in self.param_groups for p in group["params"] if p.grad is not None]
        if not params:
            return torch.zeros(())
        dev = params[0].device
        for p in params:
            if p.grad.dtype != torch.float32 or not p.grad.is_contiguous() or p.grad.device != dev:
                raise ValueError("unscale_clip_ requires contiguous fp32 gradients on one device")
        state = None
        inv = None
        if scaler is not None and scaler.is_enabled():
            state = scaler._per_optimizer_states[id(self)]
            if state["stage"] is OptState.UNSCALED:
                raise RuntimeError("unscale_() has already been called on this optimizer since "
                                   "the last update().")
            if state["stage"] is OptState.STEPPED:
                raise RuntimeError("unscale_() is being called after step().")
            inv = scaler._scale.double().reciprocal().float()
        limit = lib.rv_adamw_max_tensors()
        groups = [params[i:i + limit] for i in range(0, len(params), limit)]
        numels = [(ctypes.c_int64 * len(g))(*[p.numel() for p in g]) for g in groups]
        counts = [lib.rv_grad_chunks(n, len(g)) for n, g in zip(numels, groups)]
        for c in counts:
            if c < 0:
                _check(-c, "rv_grad_chunks")
        total_chunks = sum(counts)
        work = torch.empty(2 * total_chunks + 3, device=dev, dtype=torch.float32)
        partials, flags = work[:total_chunks], work[total_chunks:2 * total_chunks]
        total, coef, found = (work[2 * total_chunks + i:2 * total_chunks + i + 1]
                              for i in range(3))
        stream = _stream(params[0])
        first = 0
        for g, n, c in zip(groups, numels, counts):
            ptrs = (ctypes.c_void_p * len(g))(*[p.grad.data_ptr() for p in g])
            _check(lib.rv_grad_sq_partials(len(g), ptrs, n,
                                           inv.data_ptr() if inv is not None else None,
                                           partials.data_ptr(), flags.data_ptr(), first, stream),
                   "rv_grad_sq_partials")
            first += c
        _check(lib.rv_grad_clip_coef(partials.data_ptr(), flags.data_ptr(), total_chunks,
                                     float(max_norm), total.data_ptr(), coef.data_ptr(),
                                     found.data_ptr(), stream), "rv_grad_clip_coef")
        if state is not None:
            state["found_inf_per_device"] = {dev: found.reshape(())}
            state["stage"] = OptState.UNSCALED
        self._pending = (inv, coef)
        return total.reshape(())

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        lib = library()
        found_inf = getattr(self, "found_inf", None)
        grad_scale = getattr(self, "grad_scale", None)
        pending_inv, clip = getattr(self, "_pending", (None, None))
        self._pending = (None, None)
        for group in self.param_groups:
            step, params = self._group_state(group)
            if not params:
                continue
            dev = params[0].device
            stream = _stream(params[0])
            fi = found_inf.to(dev, torch.float32) if found_inf is not None else None
            inv = (grad_scale.to(dev, torch.float64).reciprocal().to(torch.float32)
                   if grad_scale is not None else pending_inv)
            _check(lib.rv_adamw_advance(step.data_ptr(), fi.data_ptr() if fi is not None else None,
                                        stream), "rv_adamw_advance")
            beta1, beta2 = group["betas"]
            limit = lib.rv_adamw_max_tensors()
            for start in range(0, len(params), limit):
                chunk = params[start:start + limit]
                n = len(chunk)
                for p in chunk:
                    if not (p.is_contiguous() and p.grad.is_contiguous()):
                        raise ValueError("FusedAdamW requires contiguous parameters and gradients")
                P = ctypes.c_void_p * n
                ptrs = [P(*[t.data_ptr() for t in ts]) for ts in (
                    chunk, [p.grad for p in chunk], [self.state[p]["exp_avg"] for p in chunk],
                    [self.state[p]["exp_avg_sq"] for p in chunk])]
                numel = (ctypes.c_int64 * n)(*[p.numel() for p in chunk])
                _check(lib.rv_adamw_step_clipped(
                    n, ptrs[0], ptrs[1], ptrs[2], ptrs[3], numel, float(group["lr"]),
                    float(beta1), float(beta2), float(group["eps"]), float(group["weight_decay"]),
                    step.data_ptr(), fi.data_ptr() if fi is not None else None,
                    inv.data_ptr() if inv is not None else None,
                    clip.data_ptr() if clip is not None else None, stream),
                    "rv_adamw_step_clipped")
        return loss
