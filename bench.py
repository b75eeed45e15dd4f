"""Benchmark of the reversible-training hot path on one MI355X.

Headline (``value``): fused RMSNorm + SwiGLU forward+backward throughput in
algorithmic HBM GB/s.  One step = RMSNorm fwd over configs[0] (x fp32
[14848, 256]), SwiGLU fwd + bwd over configs[1] (gate/up fp16 [14848, 1024]),
RMSNorm bwd over configs[0] -- the order the ops run in a training step's MLP
block -- launched through the C ABI; the timed steps are captured in one HIP
graph and replayed (the eagerly launched step is reported beside it).  Algorithmic bytes per step (each tensor read or written
once):

    RMSNorm fwd  x r, w r, y w, rstd w             30,469,120 B
    RMSNorm bwd  x r, dy r, rstd r, w r, dx w, dw w 45,674,496 B
    SwiGLU fwd   gate r, up r, out w               91,226,112 B
    SwiGLU bwd   gate r, up r, dy r, dgate w, dup w 152,043,520 B
    step total                                    319,413,248 B

Inputs are already resident in HBM when the timed region starts.  The
256 MB Infinity Cache would hold one step's working set, so each kernel
family rotates through its own distinct buffer sets (> 1.5 GB each) and every
launch reads data last touched a full rotation earlier.

Also reported, on the same line:
  roofline      the dominant kernel (SwiGLU backward): its algorithmic bytes
                divided by its average duration (HIP events around replays
                of a HIP graph of back-to-back launches of that kernel),
                against the 8 TB/s HBM peak; ``traffic`` is the HBM bytes per
                launch from rocprofv3 FETCH_SIZE/WRITE_SIZE runs
                (profiles/traffic.json) when the kernel's sources are the ones
                it was measured on (``traffic_measured_on``), else null.
  kernels       the same per-kernel timing for every kernel of the step
                (rms_bwd includes its small dw-reduce launch).
  stream_floor  per kernel, the fastest hand-written streaming kernel
                (rv_stream_floor) moving the same arrays' bytes with the same
                read/write shape, swept over vectors per thread and cache
                hints; the RMSNorm backward's bytes also followed by an empty
                launch (the floor of a two-launch backward); configs[0]'s
                forward and backward arrays in one kernel; the step's sum.
  mlp_block     configs[2]: RMSNorm + tiled SwiGLU MLP block fwd+bwd, GEMM
                TFLOP/s against the 2.5 PFLOP/s dense fp16 MFMA peak and
                algorithmic HBM GB/s (mlp_block_bytes) against 8 TB/s.
  mlp_gemms     each MFMA MLP GEMM entry point alone at one 8192-token tile
                of configs[2] and of configs[4], TFLOP/s and peak fraction.
  train_step    configs[3]: midpoint-reversible 7-layer decoder step
                (B=33, T=512, fp16 autocast, GradScaler, clip 1.0, AdamW)
                on the reference's v3 probe path (install_v3 split core,
                a whole-batch MLP tile, fused SwiGLU + RMSNorm, cached head
                with the fused cross-entropy), in tokens/s: the update
                captured once in a HIP graph and replayed (``launch``), the
                same update launched eagerly beside it (``eager_*``).
  train_step_c5 configs[4]: the 12-layer Hamiltonian-Euler d1024 step on
                the same kernels (reconstruction-stack core), tokens/s.
  copy_ceiling  the same bytes moved by torch's own elementwise kernels (a
                plain streaming kernel per config): mul (1 read, 1 write)
                for RMSNorm fwd, add (2 reads, 1 write) for RMSNorm bwd and
                SwiGLU fwd, mul over tensors of SwiGLU bwd's total bytes for
                SwiGLU bwd; per kernel and for the whole step.
  cpu_baseline  the reference's CPU path for the same step -- eager fp32
                torch (nn.RMSNorm and F.silu(g) * v, forward and autograd
                backward) -- on every CPU of the host this process may use,
                with lscpu's description of the host; ``cpu_baseline_oracle``
                is the C oracle (oracle/kernels_ref.c, OpenMP) on the same
                step.  The train step carries its own: the reference's CPU
                training path (fp32, reconstruction backward, AdamW) restated
                in oracle/model_ref.py, on a bounded sample of configs[3].

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "RMSNorm+SwiGLU fwd/bwd HBM GB/s (% of peak); reversible train step tokens/s"
HBM_PEAK_GBS = 8000.0
ROWS, D_MODEL, D_FF = 14848, 256, 1024
RMS_FWD_BYTES = ROWS * D_MODEL * 4 * 2 + D_MODEL * 4 + ROWS * 4
RMS_BWD_BYTES = ROWS * D_MODEL * 4 * 3 + ROWS * 4 + D_MODEL * 4 * 2
SW_FWD_BYTES = ROWS * D_FF * 2 * 3
SW_BWD_BYTES = ROWS * D_FF * 2 * 5
STEP_BYTES = RMS_FWD_BYTES + RMS_BWD_BYTES + SW_FWD_BYTES + SW_BWD_BYTES
assert STEP_BYTES == 319_413_248
RMS_SETS = 26  # 26 x 61 MB (x, dy, y, dx) > 1.5 GB
SW_SETS = 9    # 9 x 182 MB (u, dy, o, du) > 1.5 GB
COPY_BYTES = 256 << 20
COPY_CALIBRATION_LAUNCHES = 10


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--train-steps", type=int, default=10)
    p.add_argument("--train-warmup", type=int, default=3)
    p.add_argument("--no-train-step", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="bounded CPU-baseline sample length (0 disables)")
    p.add_argument("--kernels-only", action="store_true",
                   help="only the kernel loop (used under rocprofv3)")
    p.add_argument("--mlp-only", action="store_true",
                   help="only the MLP block and MLP GEMM measurements (used under rocprofv3)")
    p.add_argument("--train-only", choices=sorted(TRAIN_CONFIGS),
                   help="only the named training step (--train-steps / --train-warmup)")
    p.add_argument("--attn-only", action="store_true",
                   help="only the attention and embedding measurements (used under rocprofv3)")
    return p.parse_args()


class KernelStep:
    """Preallocated buffers and direct C-ABI launches for one bench step.

    RMSNorm and SwiGLU each rotate through their own buffer sets, > 1.5 GB of
    distinct memory per kernel family, so neither a whole step nor a run of
    one kernel alone finds its inputs in the 256 MB Infinity Cache.
    """

    def __init__(self, dev):
        import torch
        from reversability_amd import _hip
        self.lib = _hip.library()
        eps = float(torch.finfo(torch.float32).eps)
        g = torch.Generator().manual_seed(1337)
        x = torch.randn(ROWS, D_MODEL, generator=g)
        w = 1 + 0.02 * torch.randn(D_MODEL, generator=g)
        gy = torch.randn(ROWS, D_MODEL, generator=g)
        gate = torch.randn(ROWS, D_FF, generator=g).half()
        up = torch.randn(ROWS, D_FF, generator=g).half()
        sdy = torch.randn(ROWS, D_FF, generator=g).half()
        u = torch.cat([gate, up], 1)  # packed [gate | up], the reference layout
        ws_bytes = _hip.rmsnorm_workspace_bytes(ROWS, D_MODEL)
        self.rms_sets, self.sw_sets = [], []
        for _ in range(RMS_SETS):
            s = {"x": x.to(dev), "w": w.to(dev), "gy": gy.to(dev),
                 "y": torch.empty(ROWS, D_MODEL, device=dev),
                 "rstd": torch.empty(ROWS, device=dev),
                 "dx": torch.empty(ROWS, D_MODEL, device=dev),
                 "dw": torch.empty(D_MODEL, device=dev),
                 "ws": torch.empty(ws_bytes // 4, device=dev)}
            p = {k: v.data_ptr() for k, v in s.items()}
            s["args"] = {
                "rms_fwd": (p["x"], p["w"], p["y"], p["rstd"], ROWS, D_MODEL, eps),
                "rms_bwd": (p["x"], p["w"], p["gy"], p["rstd"], p["dx"], p["dw"], p["ws"],
                            ws_bytes, ROWS, D_MODEL),
            }
            self.rms_sets.append(s)
        for _ in range(SW_SETS):
            s = {"u": u.to(dev), "sdy": sdy.to(dev),
                 "o": torch.empty(ROWS, D_FF, device=dev, dtype=torch.float16),
                 "du": torch.empty(ROWS, 2 * D_FF, device=dev, dtype=torch.float16)}
            p = {k: v.data_ptr() for k, v in s.items()}
            s["args"] = {
                "sw_fwd": (p["u"], 2 * D_FF, p["o"], ROWS, D_FF, _hip.RV_F16),
                "sw_bwd": (p["u"], 2 * D_FF, p["sdy"], p["du"], ROWS, D_FF, _hip.RV_F16),
            }
            self.sw_sets.append(s)
        self.fns = {"rms_fwd": self.lib.rv_rmsnorm_fwd, "rms_bwd": self.lib.rv_rmsnorm_bwd,
                    "sw_fwd": self.lib.rv_swiglu_fwd, "sw_bwd": self.lib.rv_swiglu_bwd}
        # the order the ops run in a training step's MLP block: RMSNorm forward,
        # SwiGLU forward, then the backward in reverse order
        self.order = ["rms_fwd", "sw_fwd", "sw_bwd", "rms_bwd"]
        self.stream = torch.cuda.current_stream(dev).cuda_stream

    def set_for(self, name: str, i: int) -> dict:
        sets = self.rms_sets if name.startswith("rms") else self.sw_sets
        return sets[i % len(sets)]

    def run_one(self, name: str, i: int, stream=None) -> None:
        """One launch of ``name`` on set i, on ``stream`` (a hipStream_t value;
        default: the stream torch had at construction)."""
        rc = self.fns[name](*self.set_for(name, i)["args"][name],
                            self.stream if stream is None else stream)
        if rc:
            raise RuntimeError(f"{name} failed with status {rc}")

    def run(self, i: int) -> None:
        for name in self.order:
            self.run_one(name, i)


def graph_time_ms(launch, count: int, replays: int = 3) -> float:
    """Average device time (ms) of one launch: ``count`` calls of
    ``launch(i, stream)`` captured back to back in one HIP graph, replayed
    ``replays`` times between two HIP events on the replay stream.  Kernels a
    few microseconds long launched one by one from Python are bound by the
    host's launch rate (ctypes call + hipLaunchKernel, ~7-8 us per call on the
    MI355X boxes); a replayed graph issues them back to back, so the average
    is the kernels' own duration, the quantity rocprofv3 --kernel-trace
    reports."""
    import torch
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stream = torch.cuda.current_stream().cuda_stream
        for i in range(count):
            launch(i, stream)
    graph.replay()  # warm-up replay (clocks, caches, code objects)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(replays):
        graph.replay()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / (replays * count)
    del graph
    return ms


def time_kernels(dev, steps: int, warmup: int):
    """Headline step timing plus per-kernel averages.

    Step: ``steps`` steps (each the four ops over its rotating buffer sets)
    captured in one HIP graph and replayed, wall clock of the replays between
    two synchronizations -- the way the training steps below are launched --
    and, beside it, the same steps launched one by one from Python on torch's
    current stream (``eager``).  Per kernel: the kernel alone, ``steps``
    launches over the rotating buffer sets captured in a HIP graph and
    replayed (``graph_time_ms``).
    """
    import torch
    step = KernelStep(dev)
    for i in range(warmup):
        step.run(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step.run(i)
    torch.cuda.synchronize()
    eager = (time.perf_counter() - t0) / steps
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stream = torch.cuda.current_stream().cuda_stream
        for i in range(steps):
            for name in step.order:
                step.run_one(name, i, stream)
    graph.replay()  # untimed replay: the warm-up of the captured steps
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    graph.replay()  # exactly ``steps`` timed steps
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    del graph
    per_kernel = {}
    for name in step.order:
        for i in range(max(warmup, 20)):
            step.run_one(name, i)
        per_kernel[name] = graph_time_ms(
            lambda i, stream, name=name: step.run_one(name, i, stream), steps)
    ceiling = copy_ceilings(dev, steps)
    # determinism spot check: relaunch the last sets, compare outputs bitwise
    r, w = step.set_for("rms_bwd", steps - 1), step.set_for("sw_bwd", steps - 1)
    step.run(steps - 1)
    torch.cuda.synchronize()
    ref_dx, ref_du, ref_dw = r["dx"].clone(), w["du"].clone(), r["dw"].clone()
    step.run(steps - 1)
    torch.cuda.synchronize()
    if not (torch.equal(ref_dx, r["dx"]) and torch.equal(ref_du, w["du"])
            and torch.equal(ref_dw, r["dw"])):
        raise RuntimeError("kernel outputs are not run-to-run deterministic")
    return wall, eager, per_kernel, ceiling


def copy_ceilings(dev, launches: int) -> dict:
    """Average duration (ms) of torch's own elementwise kernels moving each
    kernel's bytes, on rotating buffers (> 1.5 GB per shape), timed like the
    kernels (``graph_time_ms``): RMSNorm fwd = mul [14848, 256] fp32 (1 read,
    1 write); RMSNorm bwd = add [14848, 256] fp32 (2 reads, 1 write); SwiGLU
    fwd = add [14848, 1024] fp16 (2 reads, 1 write); SwiGLU bwd = mul
    [14848, 2560] fp16 (1 read, 1 write of 76 MB each: its 152 MB total)."""
    import torch
    shapes = {"rms_fwd": ((ROWS, D_MODEL), torch.float32, 1),
              "rms_bwd": ((ROWS, D_MODEL), torch.float32, 2),
              "sw_fwd": ((ROWS, D_FF), torch.float16, 2),
              "sw_bwd": ((ROWS, 5 * D_FF // 2), torch.float16, 1)}
    out = {}
    for name, (shape, dtype, reads) in shapes.items():
        one = shape[0] * shape[1] * torch.tensor([], dtype=dtype).element_size()
        nsets = max(3, int(1.6e9 // ((reads + 1) * one)))
        sets = [[torch.ones(shape, device=dev, dtype=dtype) for _ in range(reads + 1)]
                for _ in range(nsets)]

        def run(i, stream=None, sets=sets, reads=reads):
            t = sets[i % len(sets)]
            if reads == 1:
                torch.mul(t[0], 2.0, out=t[1])
            else:
                torch.add(t[0], t[1], out=t[2])
        for i in range(20):
            run(i)
        out[name] = graph_time_ms(run, launches)
        del sets
    torch.cuda.empty_cache()
    return out


STREAM_SHAPES = {  # kernel: (arrays read, arrays written, bytes per array)
    "rms_fwd": (1, 1, ROWS * D_MODEL * 4),
    "rms_bwd": (2, 1, ROWS * D_MODEL * 4),
    "sw_fwd": (2, 1, ROWS * D_FF * 2),
    "sw_bwd": (3, 2, ROWS * D_FF * 2),
    # configs[0]'s forward and backward bytes in one launch: x (read by both), dy; y, dx
    "c1_one_kernel": (3, 2, ROWS * D_MODEL * 4),
}


def stream_floors(dev, launches: int) -> dict:
    """The streaming floor of each kernel's read/write shape at its exact
    byte count: rv_stream_floor (a hand-written kernel that only moves the
    bytes: NR arrays read, NW written, 16 bytes per access, every load issued
    before the first wait) swept over 1/2/4/8 vectors per thread and the four
    load/store cache-hint combinations, each timed like the kernels
    (graph_time_ms over rotating buffers, > 1.5 GB per shape), fastest kept.
    ``rms_bwd_two_launch`` adds an empty 4-workgroup launch after each
    2-read-1-write stream: the floor of any backward that finishes dweight in
    a second launch.  ``c1_one_kernel`` moves configs[0]'s forward and
    backward arrays (3 reads, 2 writes) in one kernel."""
    import ctypes
    import torch
    from reversability_amd import _hip
    lib = _hip.library()
    out = {}
    for name, (nr, nw, nbytes) in STREAM_SHAPES.items():
        nsets = max(3, int(1.6e9 // ((nr + nw) * nbytes)))
        sets, ptrs = [], []
        for _ in range(nsets):
            arrays = [torch.ones(nbytes // 4, device=dev) for _ in range(nr + nw)]
            ins = (ctypes.c_void_p * 3)(*[a.data_ptr() for a in arrays[:nr]])
            outs = (ctypes.c_void_p * 2)(*[a.data_ptr() for a in arrays[nr:]])
            sets.append(arrays)
            ptrs.append((ctypes.cast(ins, ctypes.c_void_p), ctypes.cast(outs, ctypes.c_void_p),
                         ins, outs))
        best = None
        for vec in (1, 2, 4, 8):
            for hints in range(4):
                def run(i, stream=None, vec=vec, hints=hints):
                    p = ptrs[i % len(ptrs)]
                    rc = lib.rv_stream_floor(p[0], nr, p[1], nw, nbytes, vec, hints, stream)
                    if rc:
                        raise RuntimeError(f"rv_stream_floor failed with status {rc}")
                for i in range(5):
                    run(i)
                ms = graph_time_ms(run, launches)
                if best is None or ms < best[0]:
                    best = (ms, vec, hints, run)
        ms, vec, hints, run = best
        moved = (nr + nw) * nbytes
        out[name] = {"us": round(ms * 1e3, 2), "bytes": moved,
                     "GBps": round(moved / (ms * 1e-3) / 1e9, 1),
                     "frac_of_peak": round(moved / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "vec": vec, "nt_loads": bool(hints & 1), "nt_stores": bool(hints & 2)}
        if name == "rms_bwd":
            def two(i, stream=None, run=run):
                run(i, stream)
                rc = lib.rv_empty_kernel(4, stream)
                if rc:
                    raise RuntimeError(f"rv_empty_kernel failed with status {rc}")
            ms2 = graph_time_ms(two, launches)
            out["rms_bwd_two_launch"] = {
                "us": round(ms2 * 1e3, 2), "bytes": moved,
                "GBps": round(moved / (ms2 * 1e-3) / 1e9, 1),
                "frac_of_peak": round(moved / (ms2 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del sets, ptrs
    torch.cuda.empty_cache()
    return out


def kernel_loop_only(dev, steps: int, warmup: int) -> None:
    """The kernel loop alone (rocprofv3 --kernel-trace / --pmc target), preceded
    by COPY_CALIBRATION_LAUNCHES elementwise copies (dst = 2 * src) of
    COPY_BYTES each: a plain streaming kernel that reads and writes exactly
    COPY_BYTES, whose FETCH_SIZE / WRITE_SIZE per dispatch calibrate the
    counters against a known byte count."""
    import torch
    src = torch.ones(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(COPY_CALIBRATION_LAUNCHES):
        torch.mul(src, 2.0, out=dst)  # a kernel (device copies go to the DMA engines)
    torch.cuda.synchronize()
    del src, dst
    step = KernelStep(dev)
    for i in range(warmup + steps):
        step.run(i)
    torch.cuda.synchronize()
    print(json.dumps({"kernels_only": True, "steps": steps, "warmup": warmup,
                      "copy_bytes": COPY_BYTES, "copy_launches": COPY_CALIBRATION_LAUNCHES}),
          flush=True)


def step_flop(model: dict, batch: int) -> int:
    """Baseline-equivalent algorithmic FLOP of one training update: 6 per
    token per matrix parameter (block projections and the tied head; forward
    2, backward 4) plus the attention products, 3 x 4 T^2 d per sequence and
    layer without the causal discount."""
    d, f, layers = model["d_model"], model["d_ff"], model["n_layers"]
    t, vocab = model["max_sequence_length"], model["vocab_size"]
    block = layers * (3 * d * d + d * d + 2 * f * d + f * d)
    tokens = batch * t
    return 6 * tokens * (block + vocab * d) + 3 * layers * batch * 4 * t * t * d


TRAIN_CONFIGS = {
    # midpoint 7 layers, d 256, split core, whole-batch MLP tile (MLP_TOKENS)
    "c4": {"model": {"vocab_size": 50257, "max_sequence_length": 512, "n_layers": 7,
                     "n_heads": 8, "d_model": 256, "d_ff": 1024},
           "method": "midpoint", "step_size": 0.5, "batch": 33, "core_mode": "split",
           "workload": "configs[3] midpoint 7L d256 h8 ff1024 vocab50257"},
    # Hamiltonian-Euler 12 layers, d 1024, reconstruction stack
    "c5": {"model": {"vocab_size": 50257, "max_sequence_length": 2048, "n_layers": 12,
                     "n_heads": 16, "d_model": 1024, "d_ff": 4096},
           "method": "euler", "step_size": 0.5, "batch": 16, "core_mode": "reference",
           "workload": "configs[4] euler 12L d1024 h16 ff4096 vocab50257"},
}
assert step_flop(TRAIN_CONFIGS["c4"]["model"], 33) == 2_234_411_384_832
assert step_flop(TRAIN_CONFIGS["c5"]["model"], 16) == 59_596_093_784_064


# Cached-head token chunk: the reference probes 1024 on a 16 GB T4
# (scripts/benchmark_midpoint_v3.py:174); on a 288 GB MI355X one chunk covers
# the whole batch (C4 logits: 1.7 GB fp16), measured fastest (C4 6.84 ms vs
# 7.23 ms at 8448 tokens and 9.01 ms at 2048).  None = the whole batch.
HEAD_CHUNK = None

# TiledMLP token tile: the reference probes 8192 (scripts/benchmark_midpoint_v3.py),
# a memory setting for a 16 GB T4; at configs[3] (16896 tokens) it leaves a
# 512-token third tile whose GEMMs are pure launch latency.  None = one tile of
# the whole batch (C5's widest tile intermediates: 0.8 GB).
MLP_TOKENS = None


def make_train_step(dev, name: str):
    """One full training update of a TRAIN_CONFIGS entry, on the reference's
    v3 probe path (scripts/benchmark_midpoint_v3.py:78-83 over
    scripts/benchmark_optimized.py:54-82): install_v3 (split core for the
    midpoint config, tiled MLP (MLP_TOKENS) keeping its tiles for its backward,
    fused SwiGLU and RMSNorm), the
    attention projections and the causal attention itself on the MFMA kernels
    (enable_linear, enable_attention), the fused token +
    position embedding adding its token gradient into the tied weight's
    gradient (enable_embedding), the batch cut from a uint16 token stream
    resident in HBM (batch_at over DeviceTokens), then
    cached_head_backward -- fp16 autocast core forward, the tied head and the
    fused cross-entropy in HEAD_CHUNK-token chunks, sum loss / valid targets, one
    core backward -- then GradScaler unscale, clip 1.0 and AdamW (0.9, 0.95),
    wd 0.1 (FusedAdamW.unscale_clip_: one gradient-norm pass; the update applies
    unscale and clip as it reads each gradient; no host synchronisation).
    Returns (step function returning the summed loss, targets per step,
    config)."""
    import numpy as np
    import torch
    from reversability_amd import build_model
    from reversability_amd.attention import enable_attention
    from reversability_amd.data import DeviceTokens, batch_at
    from reversability_amd.embedding import enable_embedding
    from reversability_amd.linear import enable_linear
    from reversability_amd.optim import FusedAdamW
    from reversability_amd.optimized_v3 import cached_head_backward, install_v3

    cfg = TRAIN_CONFIGS[name]
    batch, length = cfg["batch"], cfg["model"]["max_sequence_length"]
    vocab = cfg["model"]["vocab_size"]
    torch.manual_seed(1337)
    model = build_model({"model": cfg["model"], "method": cfg["method"],
                         "step_size": cfg["step_size"]}).to(dev)
    install_v3(model, core_mode=cfg["core_mode"], mlp_tokens=MLP_TOKENS or batch * length,
               swiglu=True, rmsnorm=True,
               keep_mlp_tiles=True)
    enable_linear(model)
    enable_attention(model)
    enable_embedding(model, into_grad=True)
    opt = FusedAdamW(model.parameters(), lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)
    scaler = torch.amp.GradScaler("cuda")
    # one uint16 stream of B*T+1 uniform ids, resident in HBM; each step cuts
    # x = stream[:-1], y = stream[1:] from it (batch_at)
    stream = np.random.default_rng(1337).integers(0, vocab, batch * length + 1).astype(np.uint16)
    tokens = DeviceTokens(stream, dev)
    targets = batch * length

    def step():
        x, y, _ = batch_at(tokens, 0, batch, length, targets)
        opt.zero_grad(set_to_none=True)
        loss = cached_head_backward(model, x, y, targets, HEAD_CHUNK or targets, scaler, "fp16",
                                    False, "triton")
        opt.unscale_clip_(scaler, 1.0)  # scaler.unscale_(opt) + clip_grad_norm_(params, 1.0)
        scaler.step(opt)
        scaler.update()
        return loss

    step.model, step.opt, step.scaler = model, opt, scaler
    return step, targets, cfg


def train_step_bench(dev, steps: int, warmup: int, name: str = "c4", graph: bool = True):
    """Tokens/s of one TRAIN_CONFIGS entry's full training update: ``steps``
    replays of the update captured in a HIP graph (reversability_amd.graph;
    ``warmup`` eager updates precede the capture), and the same number of
    eager updates of a second copy for comparison (host-launched, every
    kernel enqueued from Python)."""
    import gc
    import torch
    from reversability_amd.graph import CapturedStep

    def timed(fn):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            out = fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps, out

    from reversability_amd import paths
    step, targets, cfg = make_train_step(dev, name)
    for _ in range(warmup):
        step()
    paths.reset()  # which implementation each dispatching op took, over one update
    step()
    taken = paths.report()
    dt_eager, loss_eager = timed(step)
    loss_eager = float(loss_eager.item())
    dt, loss = dt_eager, loss_eager
    if graph:
        del step
        gc.collect()
        torch.cuda.empty_cache()
        step, targets, cfg = make_train_step(dev, name)
        captured = CapturedStep(step, warmup)
        dt, out = timed(captured)
        loss = float(out.item())
    flop = step_flop(cfg["model"], cfg["batch"])
    return {"tokens_per_s": targets / dt, "ms_per_step": dt * 1e3,
            "algorithmic_flop_per_step": flop,
            "TFLOPs": round(flop / dt / 1e12, 1),
            "frac_of_mfma_peak": round(flop / dt / 1e12 / MFMA_PEAK_TFLOPS, 4),
            "paths": taken,
            "launch": "HIP graph of the whole update, replayed" if graph else "eager",
            "eager_tokens_per_s": targets / dt_eager, "eager_ms_per_step": dt_eager * 1e3,
            "loss": loss / targets, "steps": steps, "warmup": warmup,
            "config": {"workload": cfg["workload"], "global_batch": cfg["batch"],
                       "seq_len": cfg["model"]["max_sequence_length"],
                       "core_mode": cfg["core_mode"],
                       "mlp_tokens": MLP_TOKENS or cfg["batch"] * cfg["model"]["max_sequence_length"],
                       "head": f"cached head, {HEAD_CHUNK or 'whole-batch'} token chunks, "
                               "fused CE",
                       "precision": "fp16-autocast"},
            "data": "synthetic uniform token ids (seed 1337)"}


MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16


def _event_time_us(fn, reps: int, warmup: int = 3) -> float:
    """Average duration of fn's launches (HIP events on the current stream)."""
    import torch
    for _ in range(warmup):
        fn()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / reps * 1e3


def mlp_gemm_bench(dev, reps: int = 20):
    """MFMA MLP GEMMs alone, per entry point, at one token tile of configs[2]
    (8192 x d256 x f1024) and of configs[4] (8192 x d1024 x f4096): TFLOP/s
    of the algorithmic contraction and the fraction of the dense fp16 peak.
    Epilogues (SwiGLU and its backward, fp16 rounding, accumulation) are
    inside the measured kernels."""
    import torch
    from reversability_amd import mlp
    out = {}
    for rows, d, f in ((8192, 256, 1024), (8192, 1024, 4096)):
        g = torch.Generator(device=dev).manual_seed(1337)
        x16 = torch.randn(rows, d, device=dev, generator=g).half()
        up16 = (0.02 * torch.randn(2 * f, d, device=dev, generator=g)).half()
        down16 = (0.02 * torch.randn(d, f, device=dev, generator=g)).half()
        dy = torch.randn(rows, d, device=dev, generator=g).half()
        o, u = mlp.up_swiglu(x16, up16, keep_u=True)
        du = mlp.dgate(dy, down16, u)
        y = torch.empty(rows, d, device=dev, dtype=torch.float16)
        dx = torch.empty(rows, d, device=dev)
        ddown, dup = torch.empty(d, f, device=dev), torch.empty(2 * f, d, device=dev)
        cases = {
            "up_swiglu": (lambda: mlp.up_swiglu(x16, up16), 2 * rows * 2 * f * d),
            "down": (lambda: mlp.down(o, down16, y), 2 * rows * d * f),
            "dgate_swiglu_bwd": (lambda: mlp.dgate(dy, down16, u), 2 * rows * f * d),
            "dx": (lambda: mlp.dx(du, up16, dx), 2 * rows * 2 * f * d),
            "wgrad": (lambda: mlp.wgrad(dy, o, du, x16, ddown, dup, True),
                      2 * rows * d * f + 2 * rows * 2 * f * d),
        }
        line = {}
        for name, (fn, flops) in cases.items():
            us = _event_time_us(fn, reps)
            tf = flops / us / 1e6
            line[name] = {"us": round(us, 1), "TFLOPs": round(tf, 1),
                          "frac": round(tf / MFMA_PEAK_TFLOPS, 4)}
        out[f"tile{rows}_d{d}_f{f}"] = line
    return out


def mlp_block_bench(dev, steps: int = 20):
    """RMSNorm + token-tiled SwiGLU MLP block (TiledMLP, 8192-token
    tiles: rows [0, 8192) and [8192, 14848)) under fp16 autocast with an fp32
    residual input, forward + backward against a random fp32 upstream
    gradient.  Algorithmic GEMM work fwd+bwd: 70,061,654,016 flop."""
    import torch
    from reversability_amd.kernels_v3 import FusedRMSNorm
    from reversability_amd.optimized_v3 import TiledMLP
    g = torch.Generator().manual_seed(1337)
    x = torch.randn(29, 512, 256, generator=g).to(dev).requires_grad_(True)
    up = (0.02 * torch.randn(2048, 256, generator=g)).to(dev).requires_grad_(True)
    down = (0.02 / 14 ** 0.5 * torch.randn(256, 1024, generator=g)).to(dev).requires_grad_(True)
    w = torch.ones(256, device=dev, requires_grad=True)
    gy = torch.randn(29, 512, 256, generator=g).to(dev)
    eps = float(torch.finfo(torch.float32).eps)

    def step():
        with torch.autocast("cuda", dtype=torch.float16):
            out = TiledMLP.apply(FusedRMSNorm.apply(x, w, eps), up, down, 8192, True)
        torch.autograd.backward(out, gy)

    us = _event_time_us(step, steps)
    flops = 70_061_654_016
    moved = mlp_block_bytes()
    return {"workload": "configs[2] tiled MLP block 29x512 d256 f1024 tile 8192, fp16 autocast",
            "ms_per_step": round(us / 1e3, 4), "gemm_TFLOPs": round(flops / us / 1e6, 1),
            "frac_of_mfma_peak": round(flops / us / 1e6 / MFMA_PEAK_TFLOPS, 4),
            "algorithmic_flop": flops, "algorithmic_bytes": moved,
            "GBps": round(moved / us / 1e3, 1),
            "frac_of_hbm_peak": round(moved / us / 1e3 / HBM_PEAK_GBS, 4)}


def mlp_block_bytes(rows: int = 29 * 512, d: int = 256, f: int = 1024) -> int:
    """Algorithmic HBM bytes of configs[2]'s block forward + backward: each
    tensor of the dataflow read or written once at its stored precision (the
    per-GEMM accounting of the up projection's arithmetic intensity, 224
    FLOP/B: fp16 operands and fp16 outputs), the tiles' SwiGLU input u kept
    from the forward for the backward (no recompute), the weights' fp16 casts
    once per call:

      weight casts    W_up, W_down fp32 r, fp16 w
      RMSNorm fwd     x fp32 r, w r, y fp16 w, rstd w
      up + SwiGLU     y r, W_up16 r, u = [gate | value] fp16 w, o fp16 w
      down            o r, W_down16 r, out fp16 w
      grad cast       dout fp32 r, fp16 w
      dgate + SwiGLU' dout16 r, W_down16 r, u r, du fp16 w
      dx              du r, W_up16 r, dy fp32 w
      dW_down         dout16 r, o r, dW_down fp32 w
      dW_up           du r, y r, dW_up fp32 w
      RMSNorm bwd     x r, dy r, rstd r, w r, dx fp32 w, dw w"""
    h, s = 2, 4  # fp16, fp32 bytes
    wup, wdown = 2 * f * d, d * f
    total = (wup + wdown) * (s + h)                               # weight casts
    total += rows * d * s + d * s + rows * d * h + rows * s       # RMSNorm fwd
    total += rows * d * h + wup * h + rows * 2 * f * h + rows * f * h  # up + SwiGLU
    total += rows * f * h + wdown * h + rows * d * h              # down
    total += rows * d * (s + h)                                   # grad cast
    total += rows * d * h + wdown * h + 2 * rows * 2 * f * h      # dgate + SwiGLU bwd
    total += rows * 2 * f * h + wup * h + rows * d * s            # dx
    total += rows * d * h + rows * f * h + wdown * s              # dW_down
    total += rows * 2 * f * h + rows * d * h + wup * s            # dW_up
    total += 3 * rows * d * s + rows * s + 2 * d * s              # RMSNorm bwd
    return total


ATTN_SHAPES = {  # (batch, seq, heads, head_dim) of the attention inside configs[3] / [4]
    "c4_b33_t512_h8_d32": (33, 512, 8, 32),
    "c5_b16_t2048_h16_d64": (16, 2048, 16, 64),
}


def attention_bench(dev, reps: int = 20):
    """Causal attention kernels alone (rv_attn_fwd, rv_attn_bwd on the packed
    qkv) at the configs' shapes, with torch's scaled_dot_product_attention on
    the same inputs beside them.  Algorithmic flop, causal: forward
    4 B H hd T (T + 1) / 2 (the two products over the lower triangle),
    backward 2.5x that (dV, dP, dQ, dK and one recomputation of S)."""
    import torch
    from reversability_amd import attention
    from reversability_amd._hip import _stream, library
    lib = library()
    out = {}
    for name, (b, t, h, hd) in ATTN_SHAPES.items():
        g = torch.Generator(device=dev).manual_seed(1337)
        qkv = (0.5 * torch.randn(b, t, 3 * h * hd, device=dev, generator=g)).half()
        dout = torch.randn(b, t, h * hd, device=dev, generator=g).half()
        o = torch.empty(b, t, h * hd, device=dev, dtype=torch.float16)
        lse = torch.empty(b * h, t, device=dev)
        dqkv = torch.empty_like(qkv)
        ws = torch.empty(lib.rv_attn_bwd_workspace_bytes(b, t, h) // 4, device=dev)
        st = _stream(qkv)

        def fwd():
            lib.rv_attn_fwd(qkv.data_ptr(), b, t, h, hd, o.data_ptr(), lse.data_ptr(), st)

        def bwd():
            lib.rv_attn_bwd(qkv.data_ptr(), o.data_ptr(), dout.data_ptr(), lse.data_ptr(), b, t,
                            h, hd, dqkv.data_ptr(), ws.data_ptr(), ws.numel() * 4, st)

        fwd()
        f_us, b_us = _event_time_us(fwd, reps), _event_time_us(bwd, reps)
        x = qkv.clone().requires_grad_(True)

        def torch_fb():
            x.grad = None
            attention.reference_attention(x, h).backward(dout)

        def torch_f():
            attention.reference_attention(qkv, h)

        tf_us, tfb_us = _event_time_us(torch_f, reps), _event_time_us(torch_fb, reps)
        flop = 4 * b * h * hd * t * (t + 1) // 2
        out[name] = {
            "fwd_us": round(f_us, 1), "bwd_us": round(b_us, 1),
            "fwd_TFLOPs": round(flop / f_us / 1e6, 1),
            "bwd_TFLOPs": round(2.5 * flop / b_us / 1e6, 1),
            "fwd_frac": round(flop / f_us / 1e6 / MFMA_PEAK_TFLOPS, 4),
            "bwd_frac": round(2.5 * flop / b_us / 1e6 / MFMA_PEAK_TFLOPS, 4),
            "torch_sdpa_fwd_us": round(tf_us, 1), "torch_sdpa_fwd_bwd_us": round(tfb_us, 1),
            "algorithmic_fwd_flop": flop}
    return out


def embedding_bench(dev, reps: int = 20):
    """Token pipeline and embedding kernels alone at configs[4]'s shape
    (16 x 2048 tokens, d 1024, vocab 50257, uniform ids): batch_at from an
    HBM-resident uint16 stream, forward (token rows read, output written:
    8 d bytes per token) and backward adding into an existing token-table
    gradient (dout read twice -- token and position sums -- and each touched
    token row read and written: at most 16 d bytes per token)."""
    import numpy as np
    import torch
    from reversability_amd import data, embedding
    b, t, d, vocab = 16, 2048, 1024, 50257
    stream = np.random.default_rng(1337).integers(0, vocab, b * t + 1).astype(np.uint16)
    tokens = data.DeviceTokens(stream, dev)
    x, _, _ = data.batch_at(tokens, 0, b, t, b * t)
    g = torch.Generator(device=dev).manual_seed(1337)
    tok = (0.02 * torch.randn(vocab, d, device=dev, generator=g)).requires_grad_(True)
    pos = (0.02 * torch.randn(t, d, device=dev, generator=g)).requires_grad_(True)
    dout = torch.randn(b, t, d, device=dev, generator=g)
    tok.grad = torch.zeros_like(tok)
    n = b * t
    fwd_us = _event_time_us(lambda: embedding.embed(x, tok.detach(), pos.detach()), reps)
    y = embedding.embed(x, tok, pos, into_grad=True)

    def bwd():
        pos.grad = None
        torch.autograd.backward(y, dout, retain_graph=True)

    bwd_us = _event_time_us(bwd, reps)
    batch_us = _event_time_us(lambda: data.batch_at(tokens, 0, b, t, b * t), reps)
    return {"workload": "configs[4] embedding 16x2048 d1024 vocab 50257",
            "batch_at_us": round(batch_us, 1),
            "fwd_us": round(fwd_us, 1), "fwd_GBps": round(8 * d * n / fwd_us / 1e3, 1),
            "bwd_us": round(bwd_us, 1), "bwd_GBps_upper": round(16 * d * n / bwd_us / 1e3, 1)}


def host_cpu() -> dict:
    """The host's CPU as lscpu reports it (model, sockets, cores per socket,
    threads per core, logical CPUs) and the CPUs this process may run on."""
    import subprocess
    info = {"affinity_cpus": len(os.sched_getaffinity(0))}
    keys = {"Model name": "model", "Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
            "Thread(s) per core": "threads_per_core", "CPU(s)": "logical_cpus"}
    try:
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        text = ""
    for line in text.splitlines():
        key, _, value = line.partition(":")
        if key.strip() in keys:
            value = value.strip()
            info[keys[key.strip()]] = int(value) if value.isdigit() else value
    return info


def cpu_baseline_torch(seconds: float, reps_min: int = 5):
    """The reference's CPU path for configs[0] + configs[1], timed on this
    host: eager torch in fp32 -- nn.RMSNorm (eps from finfo, the module
    src/reversibility/model.py:62,64,79 builds) forward and its autograd
    backward (dx, dweight), then F.silu(gate) * value (model.py:55-56) forward
    and backward.  The reference's fused ops refuse CPU tensors
    (kernels_v3.py:54-55, kernels.py:116-117) and its CPU path runs without
    autocast (optimized.py:64-67), so configs[1] is fp32 here.  Threads: every
    CPU this process may use (torch.set_num_threads).  Median of the timed
    repetitions after two warm-ups, repeated for about ``seconds`` (at least
    ``reps_min``); the value is the step's algorithmic bytes (STEP_BYTES, the
    GPU step's unit of work) per second."""
    import statistics
    import torch
    threads = len(os.sched_getaffinity(0))
    saved = torch.get_num_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(1337)
    norm = torch.nn.RMSNorm(D_MODEL)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.02 * torch.randn(D_MODEL, generator=g))
    x = torch.randn(ROWS, D_MODEL, generator=g).requires_grad_(True)
    gy = torch.randn(ROWS, D_MODEL, generator=g)
    gate = torch.randn(ROWS, D_FF, generator=g).requires_grad_(True)
    value = torch.randn(ROWS, D_FF, generator=g).requires_grad_(True)
    sdy = torch.randn(ROWS, D_FF, generator=g)

    def one():
        y = norm(x)
        torch.autograd.grad(y, (x, norm.weight), gy)
        o = torch.nn.functional.silu(gate) * value
        torch.autograd.grad(o, (gate, value), sdy)

    for _ in range(2):
        one()
    times, t_start = [], time.perf_counter()
    while len(times) < reps_min or time.perf_counter() - t_start < seconds:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    torch.set_num_threads(saved)
    per = statistics.median(times)
    return {"value": round(STEP_BYTES / per / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "ms_per_step": round(per * 1e3, 3), "host": host_cpu(),
            "sample": f"median of {len(times)} full steps (RMSNorm [14848,256] fwd+bwd + "
                      f"SwiGLU [14848,1024] fwd+bwd) in eager fp32 torch on the CPU -- the "
                      f"reference's CPU path -- after 2 warm-ups, "
                      f"torch.set_num_threads({threads}); GB/s = the GPU step's algorithmic "
                      f"bytes per second"}


def cpu_baseline(seconds: float):
    """Oracle (C, OpenMP) on this host's cores: the same RMSNorm+SwiGLU step."""
    import numpy as np
    import oracle
    threads = len(os.sched_getaffinity(0))
    oracle.set_num_threads(threads)
    r = np.random.default_rng(1337)
    x = r.standard_normal((ROWS, D_MODEL)).astype(np.float32)
    w = (1 + 0.02 * r.standard_normal(D_MODEL)).astype(np.float32)
    gy = r.standard_normal((ROWS, D_MODEL)).astype(np.float32)
    u = r.standard_normal((ROWS, 2 * D_FF)).astype(np.float16)
    sdy = r.standard_normal((ROWS, D_FF)).astype(np.float16)
    eps = float(np.finfo(np.float32).eps)

    def one():
        oracle.rmsnorm_fwd(x, w, eps)
        oracle.rmsnorm_bwd(x, w, gy, eps)
        oracle.swiglu_fwd(u)
        oracle.swiglu_bwd(u, sdy)

    one()
    n, t0 = 0, time.perf_counter()
    while True:
        one()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    per = dt / n
    return {"value": STEP_BYTES / per / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "ms_per_step": per * 1e3,
            "sample": f"{n} full steps (RMSNorm [14848,256] fwd+bwd + SwiGLU [14848,1024] "
                      f"fwd+bwd) of oracle/kernels_ref.c with OpenMP, {dt:.1f} s"}


def cpu_train_baseline(seconds: float, batch: int = 2):
    """The reference's CPU training path -- fp32 (the reference disables
    autocast on the CPU, src/reversibility/optimized.py:64-67), the
    reconstruction backward, torch's AdamW (0.9, 0.95), wd 0.1 -- restated in
    oracle/model_ref.py, on a bounded sample of configs[3]: ``batch`` of its
    33 sequences per update (512 tokens each), updates repeated for about
    ``seconds``; tokens/s on this host's cores."""
    import numpy as np
    import torch
    from oracle import model_ref
    from reversability_amd import build_model
    threads = len(os.sched_getaffinity(0))
    saved = torch.get_num_threads()
    torch.set_num_threads(threads)
    cfg = TRAIN_CONFIGS["c4"]
    model, length = cfg["model"], cfg["model"]["max_sequence_length"]
    torch.manual_seed(1337)
    state = build_model({"model": model, "method": cfg["method"]}).state_dict()
    params = {k: v for k, v in state.items() if k != "lm_head.weight"}
    stream = np.random.default_rng(1337).integers(0, model["vocab_size"], batch * length + 1)
    x = torch.from_numpy(stream[:-1].reshape(batch, length))
    y = torch.from_numpy(stream[1:].reshape(batch, length))
    leaves = {k: v.clone().requires_grad_(True) for k, v in params.items()}
    opt = torch.optim.AdamW(leaves.values(), lr=6e-4, betas=(0.9, 0.95), weight_decay=0.1)

    def update():
        loss, grads = model_ref.loss_and_grads_reconstruct(
            {k: v.detach() for k, v in leaves.items()}, x, y, model["n_layers"],
            model["n_heads"], cfg["method"], cfg["step_size"])
        for k, v in leaves.items():
            v.grad = grads[k]
        torch.nn.utils.clip_grad_norm_(leaves.values(), 1.0)
        opt.step()
        return loss

    update()  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        update()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    torch.set_num_threads(saved)
    per = dt / n
    return {"value": round(batch * length / per, 1), "unit": "tokens/s", "cores": threads,
            "kind": "port", "ms_per_step": round(per * 1e3, 1),
            "sample": f"{n} updates of {batch} x {length} tokens of configs[3] (7L d256, vocab "
                      f"50257): oracle/model_ref.py loss_and_grads_reconstruct in fp32, "
                      f"clip 1.0, torch AdamW, {dt:.1f} s, torch.set_num_threads({threads})"}


def load_traffic():
    """HBM bytes per launch of the roofline kernel from profiles/traffic.json
    (rocprofv3 FETCH_SIZE / WRITE_SIZE runs), and where they were measured:
    the commit and the sha256 of the kernel's sources then.  A recorded
    figure whose sources differ from the ones built now is stale: None."""
    import hashlib
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None, None
    try:
        data = json.loads(path.read_text())
    except (OSError, ValueError):
        return None, None
    where = data.get("measured_on") or {}
    for name, digest in (where.get("sources_sha256") or {}).items():
        try:
            current = hashlib.sha256((ROOT / name).read_bytes()).hexdigest()
        except OSError:
            current = None
        if current != digest:
            return None, {"stale": True, **where}
    if not where:
        return None, None
    return data.get("swiglu_bwd_bytes_per_launch"), where


def main() -> int:
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(collectives, sharding and rank code are out of scope); run with --gpus 1.",
              file=sys.stderr, flush=True)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    if args.kernels_only:
        kernel_loop_only(dev, args.steps, args.warmup)
        return 0
    if args.mlp_only:
        print(json.dumps({"mlp_block": mlp_block_bench(dev), "mlp_gemms": mlp_gemm_bench(dev)}),
              flush=True)
        return 0
    if args.train_only:
        print(json.dumps({f"train_step_{args.train_only}": train_step_bench(
            dev, args.train_steps, args.train_warmup, args.train_only)}), flush=True)
        return 0
    if args.attn_only:
        print(json.dumps({"attention": attention_bench(dev), "embedding": embedding_bench(dev)}),
              flush=True)
        return 0
    ms_step_s, eager_s, per_kernel, ceiling = time_kernels(dev, args.steps, args.warmup)
    value = STEP_BYTES / ms_step_s / 1e9
    bytes_by = {"rms_fwd": RMS_FWD_BYTES, "rms_bwd": RMS_BWD_BYTES,
                "sw_fwd": SW_FWD_BYTES, "sw_bwd": SW_BWD_BYTES}
    kernels = {n: {"avg_us": round(per_kernel[n] * 1e3, 2), "algorithmic_bytes": bytes_by[n],
                   "GBps": round(bytes_by[n] / (per_kernel[n] * 1e-3) / 1e9, 1),
                   "frac_of_peak": round(bytes_by[n] / (per_kernel[n] * 1e-3) / 1e9
                                         / HBM_PEAK_GBS, 4),
                   "copy_ceiling_us": round(ceiling[n] * 1e3, 2),
                   "frac_of_copy_ceiling": round(ceiling[n] / per_kernel[n], 4)}
               for n in per_kernel}
    ceiling_gbs = STEP_BYTES / (sum(ceiling.values()) * 1e-3) / 1e9
    floors = stream_floors(dev, args.steps)
    for n in per_kernel:
        kernels[n]["stream_floor_us"] = floors[n]["us"]
        kernels[n]["frac_of_stream_floor"] = round(floors[n]["us"] / kernels[n]["avg_us"], 4)
    floor_step_us = sum(floors[n]["us"] for n in per_kernel)
    floors["step"] = {"us": round(floor_step_us, 2),
                      "GBps": round(STEP_BYTES / (floor_step_us * 1e-6) / 1e9, 1),
                      "frac_of_peak": round(STEP_BYTES / (floor_step_us * 1e-6) / 1e9
                                            / HBM_PEAK_GBS, 4),
                      "value_over_floor": round(value / (STEP_BYTES / (floor_step_us * 1e-6)
                                                         / 1e9), 4)}
    achieved = kernels["sw_bwd"]["GBps"]
    traffic, traffic_where = load_traffic()
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step_s * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 (RMSNorm) + fp16 I/O, fp32 math (SwiGLU)",
        "data": "synthetic, seed 1337 (x, dy ~N(0,1); w = 1 + N(0, 0.02))",
        "config": {"workload": "configs[0] RMSNorm fwd+bwd [14848,256] fp32 + "
                               "configs[1] SwiGLU fwd+bwd [14848,1024] fp16",
                   "buffer_sets": {"rmsnorm": RMS_SETS, "swiglu": SW_SETS},
                   "step_bytes": STEP_BYTES},
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "launch": "HIP graph of the timed steps, replayed",
        "eager": {"GBps": round(STEP_BYTES / eager_s / 1e9, 2), "ms_per_step": eager_s * 1e3,
                  "what": "the same steps launched one by one from Python (ctypes) on "
                          "torch's current stream"},
        "copy_ceiling": {"GBps": round(ceiling_gbs, 1),
                         "frac_of_peak": round(ceiling_gbs / HBM_PEAK_GBS, 4),
                         "value_over_ceiling": round(value / ceiling_gbs, 4),
                         "what": "the step's bytes moved by torch's elementwise mul/add "
                                 "kernels of the same read/write shape, summed over the "
                                 "four kernels (copy_ceiling_us per kernel)"},
        "stream_floor": floors,
        "roofline": {"bound": "hbm", "kernel": "swiglu_once<__half, true, 1> (SwiGLU bwd)",
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_measured_on": traffic_where,
                     "algorithmic_bytes": SW_BWD_BYTES},
        "kernels": kernels,
    }
    if not args.no_train_step:
        line["mlp_block"] = mlp_block_bench(dev)
        line["mlp_gemms"] = mlp_gemm_bench(dev)
        line["attention"] = attention_bench(dev)
        line["embedding"] = embedding_bench(dev)
        line["train_step"] = train_step_bench(dev, args.train_steps, args.train_warmup)
        line["train_step_c5"] = train_step_bench(dev, args.train_steps, args.train_warmup, "c5")
        if args.cpu_seconds > 0:
            line["train_step"]["cpu_baseline"] = cpu_train_baseline(args.cpu_seconds)
    if args.cpu_seconds > 0:
        line["cpu_baseline"] = cpu_baseline_torch(args.cpu_seconds)
        line["cpu_baseline_oracle"] = cpu_baseline(args.cpu_seconds / 2)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
