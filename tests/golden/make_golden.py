"""Write tests/golden/kernels_golden.npz: seeded small inputs and the oracle's
outputs for the fused kernels.

Shapes follow the reference's own kernel tests: RMSNorm [3, 23, 256]
(tests/test_optimized_v3.py:73-84) and SwiGLU [3, 7, 66] with its odd tail
(tests/test_kernels.py:37-51); the midpoint update uses an fp16 force with
h = 0.5.  Inputs come from numpy's PCG64 with seed 1337, so they are
reproducible without torch.  Run from the repository root:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402

EPS32 = float(np.finfo(np.float32).eps)


def main() -> Path:
    r = np.random.default_rng(1337)
    rms_x = r.standard_normal((3, 23, 256)).astype(np.float32)
    rms_w = (1 + 0.02 * r.standard_normal(256)).astype(np.float32)
    rms_dy = r.standard_normal((3, 23, 256)).astype(np.float32)
    rms_y, rms_rstd = oracle.rmsnorm_fwd(rms_x, rms_w, EPS32)
    rms_dx, rms_dw = oracle.rmsnorm_bwd(rms_x, rms_w, rms_dy, EPS32)

    sw_u = r.standard_normal((3, 7, 66)).astype(np.float16)
    sw_dy = r.standard_normal((3, 7, 33)).astype(np.float16)
    sw_o = oracle.swiglu_fwd(sw_u)
    sw_du = oracle.swiglu_bwd(sw_u, sw_dy)

    mp_p = r.standard_normal(1000).astype(np.float32)
    mp_a = (0.3 * r.standard_normal(1000)).astype(np.float16)
    mp_m = (0.3 * r.standard_normal(1000)).astype(np.float16)
    mp_scale = np.float32(1.0)
    mp_out = oracle.midpoint(mp_p, mp_a, mp_m, float(mp_scale), 1)

    out = Path(__file__).resolve().parent / "kernels_golden.npz"
    np.savez_compressed(out, rms_x=rms_x, rms_w=rms_w, rms_dy=rms_dy, rms_eps=np.float64(EPS32),
                        rms_y=rms_y, rms_rstd=rms_rstd, rms_dx=rms_dx, rms_dw=rms_dw,
                        sw_u=sw_u, sw_dy=sw_dy, sw_o=sw_o, sw_du=sw_du,
                        mp_p=mp_p, mp_a=mp_a, mp_m=mp_m, mp_scale=mp_scale, mp_out=mp_out)
    return out


if __name__ == "__main__":
    print(main())
