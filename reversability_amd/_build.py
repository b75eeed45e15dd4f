"""Compile the gfx950 HIP kernels into the in-tree C-ABI shared library.

The library is built with hipcc directly (no JIT, no cache outside the tree):
each ``csrc/*.hip`` file is compiled to an object under ``csrc/_build`` and the
objects are linked into ``libreversibility_hip.so`` next to this file, which
is what :mod:`reversability_amd._hip` loads.
"""
from __future__ import annotations

import concurrent.futures as _futures
import os
import shutil
import subprocess
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = CSRC / "_build"
LIBRARY = PACKAGE_DIR / "libreversibility_hip.so"
ARCH = "gfx950"

# -ffp-contract=off: no FMA contraction (the reference's Triton kernels are
# launched with enable_fp_fusion=False).  -packed-fp32-ops: keep the compiler
# from emitting packed FP32 VALU instructions.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the gfx950 kernels cannot be built")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every kernel source and link the shared library; return its path."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    workers = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", "8"))))
    with _futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
