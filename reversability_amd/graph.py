"""Whole-update HIP graph capture of a training step.

The reference launches every kernel of an update from Python
(scripts/benchmark_optimized.py:54-82, scripts/train_baseline.py:256-284); at
configs[3] that is ~390 launches per update, and the host needs about as long
to enqueue them as the GPU needs to run them.  ``CapturedStep`` records one
call of a step function into a HIP graph (``torch.cuda.CUDAGraph``) and then
replays it: the same kernels on the same buffers, in the same order, for one
host call per update.

What a step must satisfy to be captured (the bench's ``make_train_step``
does): static shapes and input buffers (the batch is cut on the device from a
resident token stream), no host synchronisation (``FusedAdamW`` takes the
GradScaler's device ``found_inf`` flag instead of reading it; the step counter
and bias corrections live on the device), gradients set to ``None`` at the
start of the step (so the captured backward writes them rather than adding
to stale ones), and no ``hipMemsetAsync`` inside (none of this library's entry
points records one; the embedding backward's rocPRIM sort takes its
memset-free merge path up to 2^20 tokens).  The GEMM tile-shape tuner never
runs during capture: captured calls use the shapes the warm-up calls chose.

Everything the graph touches must outlive it: the step's parameters,
optimizer state, scaler and token stream are kept by the closure; the
intermediate tensors live in the graph's private memory pool.
"""
from __future__ import annotations

from typing import Callable, Optional

import torch


class CapturedStep:
    """``step()`` captured once after ``warmup`` eager calls on a side stream
    (which also run first-call work: GEMM tile tuning, library handles,
    optimizer and scaler state); calling the object replays the graph on the
    current stream and returns the tensor the captured call returned (its
    storage is rewritten by every replay)."""

    def __init__(self, step: Callable[[], torch.Tensor], warmup: int = 3,
                 device: Optional[torch.device] = None):
        if not torch.cuda.is_available():
            raise RuntimeError("CapturedStep requires a ROCm GPU")
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(warmup):
                step()
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.output = step()
        self.step = step

    def __call__(self) -> torch.Tensor:
        self.graph.replay()
        return self.output
