"""bench.py's contract on the CPU: the algorithmic byte and FLOP counts it
reports against, the one-GPU refusal, and the traffic record's source check.

The byte counts are the per-kernel figures of the configs[0] / configs[1]
workload worked out independently from the tensors each kernel must read and
write (x, dy [14848, 256] fp32, w [256], rstd [14848]; gate, up, dy
[14848, 1024] fp16); the FLOP counts are 6 * tokens * (block + head
parameters) + 3 * layers * B * 4 T^2 D for configs[3] and configs[4].
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_headline_bytes_per_kernel():
    rows, d, f = 14848, 256, 1024
    # forward: x read, y written (fp32), w read, rstd written
    assert bench.RMS_FWD_BYTES == 30_469_120 == rows * d * 8 + d * 4 + rows * 4
    # backward: x, dy read, dx written (fp32), rstd and w read, dw written
    assert bench.RMS_BWD_BYTES == 45_674_496 == rows * d * 12 + rows * 4 + d * 8
    # SwiGLU forward: gate, up read, out written (fp16)
    assert bench.SW_FWD_BYTES == 91_226_112 == rows * f * 2 * 3
    # SwiGLU backward: gate, up, dy read, dgate, dup written (fp16)
    assert bench.SW_BWD_BYTES == 152_043_520 == rows * f * 2 * 5
    assert bench.STEP_BYTES == 319_413_248


def test_train_step_flop_counts():
    c4, c5 = bench.TRAIN_CONFIGS["c4"]["model"], bench.TRAIN_CONFIGS["c5"]["model"]
    assert bench.step_flop(c4, 33) == 2_234_411_384_832
    assert bench.step_flop(c5, 16) == 59_596_093_784_064
    # the parameter split behind configs[3]'s figure: 7 blocks of the matrix
    # parameters 4 d^2 (attention projections) + 3 d f (MLP) and the tied
    # head V d (norm weights and the position table carry no matmul FLOPs)
    d, f, layers, vocab, t = 256, 1024, 7, 50257, 512
    blocks = layers * (4 * d * d + 3 * d * f)
    assert blocks == 7_340_032
    assert vocab * d == 12_865_792
    tokens = 33 * t
    assert 6 * tokens * (blocks + vocab * d) + 3 * layers * 33 * 4 * t * t * d \
        == bench.step_flop(c4, 33)


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}),
                                      ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_is_refused(argv, env):
    """Refused before torch is imported or a GPU is touched."""
    run_env = dict(os.environ, **env)
    out = subprocess.run([sys.executable, str(ROOT / "bench.py"), *argv], capture_output=True,
                         text=True, env=run_env, timeout=120)
    assert out.returncode == 2
    assert "one GPU" in out.stderr and out.stdout == ""


def test_traffic_record_matches_its_sources():
    """roofline.traffic comes from profiles/traffic.json only while the SwiGLU
    kernel's sources hash to what the counters were measured on; the counted
    bytes then equal the algorithmic bytes within 1%."""
    traffic, where = bench.load_traffic()
    assert traffic is not None, where
    assert abs(traffic / bench.SW_BWD_BYTES - 1) < 0.01
    assert where["kernel"] == "swiglu_once<__half, true, 1>"
    assert set(where["sources_sha256"]) == {"reversability_amd/csrc/swiglu.hip",
                                            "reversability_amd/csrc/rv_device.h"}


def test_mlp_block_bytes():
    """configs[2]'s algorithmic HBM bytes, counted here by tensor (how many
    times each is written or read, at its stored width) rather than by op as
    bench.mlp_block_bytes does."""
    rows, d, f = 29 * 512, 256, 1024
    per_rows_d = (2 * 4      # x fp32: RMSNorm fwd, RMSNorm bwd
                  + 3 * 2    # y fp16: written, read by up, read by dW_up
                  + 1 * 2    # block output fp16: written
                  + 1 * 4    # upstream gradient fp32: read by its cast
                  + 3 * 2    # its fp16 cast: written, read by dgate and dW_down
                  + 2 * 4    # gradient of y fp32: written by dx, read by RMSNorm bwd
                  + 1 * 4)   # dx fp32: written
    per_rows_2f = 2 * 2 + 3 * 2  # u: written, read; du: written, read by dx and dW_up
    per_rows_f = 3 * 2           # o: written, read by down and dW_down
    per_weight = 4 + 3 * 2 + 4   # fp32 read by the cast; fp16 written, read twice; grad written
    total = (rows * d * per_rows_d + rows * 2 * f * per_rows_2f + rows * f * per_rows_f
             + rows * 2 * 4               # rstd: written, read
             + d * (2 * 4 + 4)            # norm weight read twice, its gradient written
             + (2 * f * d + d * f) * per_weight)
    assert total == 550_886_400
    assert bench.mlp_block_bytes() == total


def test_host_cpu_description():
    info = bench.host_cpu()
    assert info["affinity_cpus"] == len(os.sched_getaffinity(0)) >= 1
