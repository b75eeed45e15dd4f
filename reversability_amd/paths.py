"""Path selection: per-model switches of the reconstruction backward and a
record of which implementation each hot-path operation took.

Switches (``ReconstructionPaths``).  The reconstruction backward has six
optional restructurings; the first five leave every value unchanged (the GPU
tests compare each one on and off bit for bit), the sixth moves one
linearisation point by a rounding (compared to fp32 truth).  They are settings of a model, kept
on its ``blocks`` (the ``nn.ModuleList`` the stack Functions receive), so two
models in one process can differ and nothing process-wide is mutated:

    reuse_euler_attention   Euler VJP builds its graph from the inversion's A(p0)
    fuse_euler_inverse      Euler inversion's p - M(q), q - A(p0) inside the norms
    skip_unused_mlp_output  Euler VJP's rebuilt MLP output (graph-only) not computed
    keep_split_attention    split midpoint keeps the inversion's attention graph
    fuse_midpoint_norm      midpoint update made with the next layer's attention norm
    euler_mlp_at_stored_q   Euler VJP reuses the inversion's M(q) graph, made at the
                            stored state q (the point the forward evaluated M at)
                            instead of at the rebuilt q0 + A(p0): one MLP evaluation
                            per layer less; the linearisation point moves by the
                            rounding of q0 + A(p0) (at most an ulp of fp32), so the
                            gradients change within that rounding, not bit for bit

``configure(model, **flags)`` sets them; ``install_v3(..., paths=...)``
records them at installation.  Models that never had them set use the
defaults (all on).

Record (``took`` / ``report``).  Where a fused operator can only cover some
calls (the MFMA MLP and attention projections need widths that are multiples
of 128, the attention kernels head sizes 32/64/128 and fp16 autocast), the
dispatching code records the path each call took.  ``report()`` returns the
counts; under ``strict()`` (or with ``RV_STRICT_PATHS=1`` in the environment)
a call that would leave the HIP path raises ``UnsupportedPathError`` instead.
"""
from __future__ import annotations

import collections
import contextlib
import dataclasses
import os
import threading


@dataclasses.dataclass(frozen=True)
class ReconstructionPaths:
    reuse_euler_attention: bool = True
    fuse_euler_inverse: bool = True
    skip_unused_mlp_output: bool = True
    keep_split_attention: bool = True
    fuse_midpoint_norm: bool = True
    euler_mlp_at_stored_q: bool = True


DEFAULT = ReconstructionPaths()


def of(blocks) -> ReconstructionPaths:
    """The settings recorded on a model's ``blocks`` (defaults if none)."""
    return getattr(blocks, "_rv_paths", DEFAULT)


def configure(model, paths: ReconstructionPaths | None = None, **flags) -> ReconstructionPaths:
    """Set ``model``'s reconstruction switches: ``paths`` as a whole, or the named
    ``flags`` over the current settings.  Returns the new settings."""
    current = paths if paths is not None else of(model.blocks)
    new = dataclasses.replace(current, **flags)
    model.blocks._rv_paths = new
    return new


class UnsupportedPathError(RuntimeError):
    """A call would leave the HIP path while strict path checking is on."""


_lock = threading.Lock()
_counts: collections.Counter = collections.Counter()
_strict_depth = 0


def strict_enabled() -> bool:
    return _strict_depth > 0 or os.environ.get("RV_STRICT_PATHS", "") == "1"


@contextlib.contextmanager
def strict():
    """Inside this block a fallback off the HIP path raises instead of running."""
    global _strict_depth
    with _lock:
        _strict_depth += 1
    try:
        yield
    finally:
        with _lock:
            _strict_depth -= 1


def took(op: str, path: str, fallback: str | None = None) -> None:
    """Record that ``op`` ran on ``path``; ``fallback`` is the reason when that
    path is not the HIP one (raises under ``strict()``)."""
    if fallback is not None and strict_enabled():
        raise UnsupportedPathError(f"{op}: {fallback}")
    with _lock:
        _counts[(op, path)] += 1


def report() -> dict:
    """``{op: {path: calls}}`` since the last ``reset()``."""
    with _lock:
        items = list(_counts.items())
    out: dict = {}
    for (op, path), n in sorted(items):
        out.setdefault(op, {})[path] = n
    return out


def reset() -> None:
    with _lock:
        _counts.clear()
