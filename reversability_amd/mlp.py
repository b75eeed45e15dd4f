"""MFMA MLP projections with fused SwiGLU epilogues (the HIP path of TiledMLP).

Thin launchers over the C ABI (``rv_mlp_*`` in include/reversibility_hip.h) for
one token tile of the SwiGLU MLP under fp16 autocast.  All operands are fp16:

    cast_f16(t)                 fp16 copy of an fp32 tensor (autocast's cast)
    up_swiglu(x, W_up)          o = fp16(silu(fp16 u_g)) * fp16 u_v, u = x W_up^T
    down(o, W_down, out)        out = fp16(o W_down^T)
    dgate(dy, W_down, u)        du = swiglu_bwd(u, fp16(dy W_down))
    dx(du, W_up, out)           out = fp32(fp16(du W_up))
    wgrad(dy, o, du, x, ...)    dW_down (+)= fp32(fp16(dy^T o)), dW_up (+)= fp32(fp16(du^T x))

The weights passed here are the fp16 casts of the fp32 masters (one cast per
TiledMLP call: autocast's F.linear casts the same fp32 weight to the same fp16
values on every call).  Outputs are written into caller-provided slices where
the tiled caller owns the buffer.  ``supported`` says whether a shape is
covered (model width and hidden width multiples of 128); the caller uses
torch's GEMMs otherwise.
"""
from __future__ import annotations

import contextlib
import ctypes
import threading

import torch

from ._hip import RV_F16, _check, _stream, library


def supported(x: torch.Tensor, up: torch.Tensor, down: torch.Tensor) -> bool:
    d, f = x.shape[-1], down.shape[1]
    return (x.is_cuda and x.dtype in (torch.float32, torch.float16)
            and up.dtype == torch.float32 and down.dtype == torch.float32
            and up.is_contiguous() and down.is_contiguous()
            and tuple(up.shape) == (2 * f, d) and tuple(down.shape) == (d, f)
            and d % 128 == 0 and f % 128 == 0)


def cast_f16(t: torch.Tensor) -> torch.Tensor:
    """fp16 copy of a contiguous fp32 tensor (round to nearest even); fp16 passes through."""
    if t.dtype == torch.float16:
        return t.contiguous()
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError("cast_f16 needs a contiguous fp32 or fp16 CUDA (ROCm device) tensor")
    out = torch.empty(t.shape, device=t.device, dtype=torch.float16)
    _check(library().rv_cast_f32_f16(t.data_ptr(), out.data_ptr(), t.numel(), _stream(t)),
           "rv_cast_f32_f16")
    return out


# Call-scoped cache of fp16 weight casts (see weight_cast_cache).
_weight_cache: dict | None = None

# Depth of the output_unused blocks open on each thread (autograd runs a CUDA
# backward on its own device thread; another thread's forward is unaffected).
_output_unused = threading.local()


@contextlib.contextmanager
def output_unused():
    """Inside this block (on this thread) the tiled MLP's output is only
    differentiated, never read: ``install_v3``'s MLP forward on a GPU tensor
    keeps its tiles for the backward but skips the down projection (the
    output tensor is allocated, not computed).  For an MLP evaluation that
    only feeds a rebuilt ``graph_only`` residual step.  The backward is
    unchanged."""
    _output_unused.depth = getattr(_output_unused, "depth", 0) + 1
    try:
        yield
    finally:
        _output_unused.depth -= 1


def output_wanted(x: torch.Tensor) -> bool:
    """False inside ``output_unused`` (on this thread) for a GPU input."""
    return not (getattr(_output_unused, "depth", 0) and x.is_cuda)


@contextlib.contextmanager
def weight_cast_cache():
    """Reuse fp16 casts of the same fp32 weight inside this block.

    A training step evaluates each layer's force several times -- forward,
    the reconstruction's inverse, the recompute for the VJP -- and each
    evaluation cast every weight again.  Inside the block, ``cast_weight``
    casts a given weight tensor once and hands out that copy afterwards
    (what autocast's own cast cache does within one autocast region).  The
    weights must not be modified inside the block; the trainers open it
    around one forward + backward, before the optimizer step.  Nested blocks
    share the outer cache.
    """
    global _weight_cache
    if _weight_cache is not None:
        yield
        return
    _weight_cache = {}
    try:
        yield
    finally:
        _weight_cache = None


def cast_weight(w: torch.Tensor) -> torch.Tensor:
    """``cast_f16(w)``, reused inside a ``weight_cast_cache`` block."""
    cache = _weight_cache
    if cache is None:
        return cast_f16(w)
    hit = cache.get(id(w))
    if hit is not None and hit[0] is w:
        return hit[1]
    w16 = cast_f16(w)
    cache[id(w)] = (w, w16)  # the strong reference keeps id(w) unique in the block
    return w16


def prefetch_casts(weights) -> None:
    """Inside a ``weight_cast_cache`` block, make the fp16 casts of all of
    ``weights`` (contiguous fp32 CUDA tensors; others are skipped) in one
    launch per rv_cast_f32_f16_max_tensors() tensors, into one buffer, so
    that the block's ``cast_weight`` calls find them.  Same values as
    ``cast_f16`` per weight.  No effect outside a block."""
    cache = _weight_cache
    if cache is None:
        return
    todo, seen = [], set()
    for w in weights:
        if (w.is_cuda and w.dtype == torch.float32 and w.is_contiguous() and w.numel()
                and id(w) not in cache and id(w) not in seen):
            todo.append(w)
            seen.add(id(w))
    if not todo:
        return
    lib = library()
    limit = lib.rv_cast_f32_f16_max_tensors()
    for start in range(0, len(todo), limit):
        group = todo[start:start + limit]
        sizes = [-(-w.numel() // 8) * 8 for w in group]  # 16-byte aligned slices
        flat = torch.empty(sum(sizes), device=group[0].device, dtype=torch.float16)
        outs, offset = [], 0
        for w, size in zip(group, sizes):
            outs.append(flat[offset:offset + w.numel()].view(w.shape))
            offset += size
        n = len(group)
        src = (ctypes.c_void_p * n)(*[w.data_ptr() for w in group])
        dst = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
        numel = (ctypes.c_int64 * n)(*[w.numel() for w in group])
        _check(lib.rv_cast_f32_f16_multi(n, src, dst, numel, _stream(group[0])),
               "rv_cast_f32_f16_multi")
        for w, o in zip(group, outs):
            cache[id(w)] = (w, o)


def _f16(t: torch.Tensor, what: str) -> None:
    if t.dtype != torch.float16:
        raise ValueError(f"{what} must be fp16 (cast with mlp.cast_f16)")


def up_swiglu(x: torch.Tensor, up: torch.Tensor, keep_u: bool = False):
    """x [rows, d] fp16 (contiguous rows), up [2f, d] fp16 -> (o, u or None)."""
    _f16(x, "x"), _f16(up, "W_up")
    rows, d = x.shape
    f = up.shape[0] // 2
    o = torch.empty(rows, f, device=x.device, dtype=torch.float16)
    u = torch.empty(rows, 2 * f, device=x.device, dtype=torch.float16) if keep_u else None
    _check(library().rv_mlp_up_swiglu(x.data_ptr(), x.stride(0), up.data_ptr(), rows, d, f,
                                      o.data_ptr(), u.data_ptr() if keep_u else None,
                                      _stream(x)), "rv_mlp_up_swiglu")
    return o, u


def down(o: torch.Tensor, w: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    _f16(o, "o"), _f16(w, "W_down")
    rows, f = o.shape
    d = w.shape[0]
    _check(library().rv_mlp_down(o.data_ptr(), w.data_ptr(), rows, d, f, out.data_ptr(),
                                 _stream(o)), "rv_mlp_down")
    return out


def dgate(dy: torch.Tensor, w_down: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    _f16(dy, "dy"), _f16(w_down, "W_down"), _f16(u, "u")
    rows, d = dy.shape
    f = w_down.shape[1]
    du = torch.empty(rows, 2 * f, device=dy.device, dtype=torch.float16)
    _check(library().rv_mlp_dgate(dy.data_ptr(), w_down.data_ptr(), u.data_ptr(), rows, d, f,
                                  du.data_ptr(), _stream(dy)), "rv_mlp_dgate")
    return du


def dx(du: torch.Tensor, w_up: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out [rows, d] = du W_up rounded to fp16; stored as fp32 (the widened
    value, for an fp32 input x) or as fp16 (for an fp16 input x)."""
    _f16(du, "du"), _f16(w_up, "W_up")
    rows, two_f = du.shape
    d = w_up.shape[1]
    if tuple(out.shape) != (rows, d) or not out.is_contiguous():
        raise ValueError("dx output must be a contiguous [rows, d] tensor")
    if out.dtype == torch.float32:
        _check(library().rv_mlp_dx(du.data_ptr(), w_up.data_ptr(), rows, d, two_f // 2,
                                   out.data_ptr(), _stream(du)), "rv_mlp_dx")
    elif out.dtype == torch.float16:  # the same contraction as a linear layer's dx
        _check(library().rv_linear_dx(du.data_ptr(), w_up.data_ptr(), rows, d, two_f,
                                      out.data_ptr(), RV_F16, _stream(du)), "rv_linear_dx")
    else:
        raise ValueError("dx output must be fp32 or fp16")
    return out


def wgrad(dy, o, du, x, ddown, dup, accumulate: bool) -> None:
    for t, what in ((dy, "dy"), (o, "o"), (du, "du"), (x, "x")):
        _f16(t, what)
    rows, d = dy.shape
    f = o.shape[1]
    lib = library()
    nbytes = lib.rv_mlp_wgrad_workspace_bytes(rows, d, f)
    if nbytes < 0:
        _check(-nbytes, "rv_mlp_wgrad_workspace_bytes")
    ws = torch.empty(max(nbytes, 4) // 4, device=dy.device, dtype=torch.float32)
    _check(lib.rv_mlp_wgrad(dy.data_ptr(), o.data_ptr(), du.data_ptr(), x.data_ptr(),
                            x.stride(0), rows, d, f, ddown.data_ptr(), dup.data_ptr(),
                            int(accumulate), ws.data_ptr(), nbytes, _stream(dy)), "rv_mlp_wgrad")
