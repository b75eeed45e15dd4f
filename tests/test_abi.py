"""The C-ABI library: it loads, exports every entry point include/*.h declares,
and rejects bad arguments with the documented status codes before touching a
device (no kernel is launched here)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from reversability_amd import _hip

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions() -> list[str]:
    names = []
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"\b(rv_\w+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ["rv_rmsnorm_fwd", "rv_rmsnorm_bwd", "rv_rmsnorm_bwd_workspace_bytes",
                     "rv_swiglu_fwd", "rv_swiglu_bwd", "rv_midpoint_update",
                     "rv_midpoint_update_bwd", "rv_residual_axpy", "rv_add_rmsnorm_fwd"]:
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = _hip.library()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding declares a signature for each of them
    assert set(declared_functions()) <= set(_hip.SIGNATURES)


def test_status_strings_and_version():
    lib = _hip.library()
    assert lib.rv_abi_version() == _hip.ABI_VERSION
    assert lib.rv_status_string(0) == b"ok"
    for code in range(1, 6):
        assert lib.rv_status_string(code) not in (b"ok", b"unknown status")


def test_argument_validation_without_device():
    lib = _hip.library()
    fake = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    assert lib.rv_rmsnorm_fwd(None, fake, fake, fake, 4, 256, 1e-7, None) == 1
    assert lib.rv_rmsnorm_fwd(fake, fake, fake, fake, 0, 256, 1e-7, None) == 2
    assert lib.rv_rmsnorm_fwd(fake, fake, fake, fake, 4, 8192, 1e-7, None) == 3
    assert lib.rv_rmsnorm_bwd(fake, fake, fake, fake, fake, fake, fake, 0, 4, 256, None) == 4
    assert lib.rv_rmsnorm_bwd(fake, fake, fake, fake, fake, fake, None, 1 << 20, 4, 256, None) == 4
    assert lib.rv_swiglu_fwd(fake, 10, fake, 4, 8, _hip.RV_F16, None) == 2  # ld < 2*width
    assert lib.rv_swiglu_fwd(fake, 16, fake, 4, 8, _hip.RV_F64, None) == 3
    assert lib.rv_swiglu_bwd(None, 16, fake, fake, 4, 8, _hip.RV_F16, None) == 1
    assert lib.rv_midpoint_update(fake, fake, fake, fake, 1.0, 2, 16, 0, 1, None) == 2
    assert lib.rv_midpoint_update(fake, fake, fake, fake, 1.0, 1, 16, _hip.RV_F16, _hip.RV_F32, None) == 3
    assert lib.rv_residual_axpy(fake, fake, fake, 1, -1, 0, 1, None) == 2
    assert lib.rv_add_rmsnorm_fwd(fake, fake, _hip.RV_F64, fake, fake, fake, fake, 4, 256, 1e-7, None) == 3
    ptrs = (ctypes.c_void_p * 3)(4096, 4096, 4096)
    arr = ctypes.cast(ptrs, ctypes.c_void_p)
    assert lib.rv_stream_floor(None, 1, arr, 1, 64, 1, 0, None) == 1
    assert lib.rv_stream_floor(arr, 4, arr, 1, 64, 1, 0, None) == 2  # at most 3 inputs
    assert lib.rv_stream_floor(arr, 1, arr, 3, 64, 1, 0, None) == 2  # at most 2 outputs
    assert lib.rv_stream_floor(arr, 1, arr, 1, 24, 1, 0, None) == 2  # whole 16-byte vectors
    assert lib.rv_stream_floor(arr, 1, arr, 1, 64, 1, 4, None) == 3  # hint bits 0..1
    assert lib.rv_empty_kernel(0, None) == 2


@pytest.mark.parametrize("rows,width", [(1, 8), (14848, 256), (32768, 1024), (69, 33),
                                        (16896, 256), (24000, 256), (27000, 256),
                                        (40000, 256), (300, 260)])
def test_workspace_size_is_device_independent(rows, width):
    """Partial rows: one per block of ceil(rows / 256) rows -- for width <= 256
    at least 16 and at most 128 rows per block."""
    n = _hip.rmsnorm_workspace_bytes(rows, width)
    per_block = -(-rows // 256)
    if width <= 256:
        per_block = min(max(per_block, 16), 128)
    parts = -(-rows // per_block)
    assert n == parts * width * 4


def test_embedding_entry_points_validate_without_device():
    lib = _hip.library()
    fake = ctypes.c_void_p(4096)
    odd = ctypes.c_void_p(4100)  # not 16-byte aligned
    assert lib.rv_batch_from_tokens(None, 4, 2, fake, fake, None) == 1
    assert lib.rv_batch_from_tokens(fake, 0, 2, fake, fake, None) == 2
    assert lib.rv_batch_from_tokens(fake, 4, 0, fake, fake, None) == 2
    assert lib.rv_embed_fwd(fake, 2, 4, fake, 10, fake, 8, 6, fake, None) == 2   # d % 4
    assert lib.rv_embed_fwd(fake, 2, 9, fake, 10, fake, 8, 8, fake, None) == 2   # seq > max_seq
    assert lib.rv_embed_fwd(fake, 2, 4, odd, 10, fake, 8, 8, fake, None) == 3
    assert lib.rv_embed_fwd(None, 2, 4, fake, 10, fake, 8, 8, fake, None) == 1
    assert lib.rv_embed_bwd_workspace_bytes(-1, 10, 8) == -2
    assert lib.rv_embed_bwd_workspace_bytes(16, 10, 6) == -2
    assert lib.rv_embed_bwd_workspace_bytes(0, 10, 8) == 0
    assert lib.rv_embed_bwd(fake, 2, 4, odd, 10, 8, 8, fake, 0, fake, 0, fake, 0, None) == 3
    assert lib.rv_embed_bwd(fake, 2, 4, fake, 0, 8, 8, fake, 0, fake, 0, fake, 0, None) == 2


def test_attention_entry_points_validate_without_device():
    lib = _hip.library()
    fake = ctypes.c_void_p(4096)
    odd = ctypes.c_void_p(4104)
    assert lib.rv_attn_fwd(None, 2, 16, 2, 32, fake, fake, None) == 1
    assert lib.rv_attn_fwd(fake, 0, 16, 2, 32, fake, fake, None) == 2
    assert lib.rv_attn_fwd(fake, 2, 16, 2, 16, fake, fake, None) == 3   # head_dim 16
    assert lib.rv_attn_fwd(odd, 2, 16, 2, 64, fake, fake, None) == 3
    assert lib.rv_attn_bwd_workspace_bytes(2, 16, 3) == 2 * 16 * 3 * 4
    assert lib.rv_attn_bwd_workspace_bytes(0, 16, 3) == -2
    assert lib.rv_attn_bwd(fake, fake, fake, fake, 2, 16, 2, 64, fake, fake, 4, None) == 4
    assert lib.rv_attn_bwd(fake, fake, fake, fake, 2, 16, 2, 48, fake, fake, 1 << 20, None) == 3


def test_rmsnorm_fp16_entry_points_validate_without_device():
    lib = _hip.library()
    fake = ctypes.c_void_p(4096)
    assert lib.rv_rmsnorm_fwd_f16(None, fake, fake, fake, 4, 256, 1e-7, None) == 1
    assert lib.rv_rmsnorm_fwd_f16(fake, fake, fake, fake, 0, 256, 1e-7, None) == 2
    assert lib.rv_rmsnorm_fwd_f16(fake, fake, fake, fake, 4, 8192, 1e-7, None) == 3
    assert lib.rv_rmsnorm_fwd_f16(fake, fake, ctypes.c_void_p(4098), fake, 4, 256, 1e-7,
                                  None) == 3  # fp16 output must be 8-byte aligned
    assert lib.rv_rmsnorm_bwd_f16(fake, fake, fake, fake, fake, fake, None, 0, 4, 256, None) == 4


def test_gemm_entry_points_validate_without_device():
    """The MFMA GEMM entry points refuse null pointers (1), bad sizes (2),
    widths the tiles do not cover and any operand or output that is not
    16-byte aligned (3), and a missing workspace (4), before any launch."""
    lib = _hip.library()
    fake = ctypes.c_void_p(4096)
    odd = ctypes.c_void_p(4104)  # 8-byte, not 16-byte, aligned
    rows, d, f = 64, 256, 1024
    assert lib.rv_mlp_up_swiglu(None, d, fake, rows, d, f, fake, None, None) == 1
    assert lib.rv_mlp_up_swiglu(fake, d, fake, 0, d, f, fake, None, None) == 2
    assert lib.rv_mlp_up_swiglu(fake, d, fake, rows, 100, f, fake, None, None) == 3
    assert lib.rv_mlp_up_swiglu(fake, d, fake, rows, d, f, odd, None, None) == 3
    assert lib.rv_mlp_up_swiglu(fake, d, fake, rows, d, f, fake, odd, None) == 3
    assert lib.rv_mlp_down(fake, fake, rows, d, f, odd, None) == 3
    assert lib.rv_mlp_down(fake, fake, rows, 192, f, fake, None) == 3  # d % 128
    for which in range(4):  # dy, w_down, u, du
        ptrs = [fake] * 4
        ptrs[which] = odd
        assert lib.rv_mlp_dgate(ptrs[0], ptrs[1], ptrs[2], rows, d, f, ptrs[3], None) == 3
    assert lib.rv_mlp_dgate(fake, fake, None, rows, d, f, fake, None) == 1
    for which in range(3):  # du, w_up, dx
        ptrs = [fake] * 3
        ptrs[which] = odd
        assert lib.rv_mlp_dx(ptrs[0], ptrs[1], rows, d, f, ptrs[2], None) == 3
    need = lib.rv_mlp_wgrad_workspace_bytes(rows, d, f)
    assert need >= 0
    if need:
        assert lib.rv_mlp_wgrad(fake, fake, fake, fake, d, rows, d, f, fake, fake, 0, None, 0,
                                None) == 4
    assert lib.rv_mlp_wgrad(fake, fake, fake, fake, d, rows, d, f, odd, fake, 0, fake, 1 << 30,
                            None) == 3
    assert lib.rv_linear_fwd(fake, 256, fake, rows, 256, 768, odd, None) == 3
    assert lib.rv_linear_fwd(fake, 100, fake, rows, 256, 768, fake, None) == 2  # ldx < in
    assert lib.rv_linear_dx(fake, fake, rows, 256, 768, fake, _hip.RV_F64, None) == 3
    assert lib.rv_linear_dx(fake, fake, rows, 256, 768, odd, _hip.RV_F16, None) == 3
    assert lib.rv_linear_dw(fake, fake, 256, rows, 256, 768, odd, 0, fake, 1 << 30, None) == 3


def test_fused_cross_entropy_validates_without_device():
    lib = _hip.library()
    fake = ctypes.c_void_p(4096)
    args = lambda x, dt, ld, rows, cols, d: (x, dt, ld, fake, rows, cols, -100, fake, fake, fake,
                                             fake, d, None)
    assert lib.rv_ce_fused(*args(None, _hip.RV_F16, 8, 4, 8, fake)) == 1
    assert lib.rv_ce_fused(*args(fake, _hip.RV_F16, 8, 4, 8, None)) == 1
    assert lib.rv_ce_fused(*args(fake, _hip.RV_F16, 7, 4, 8, fake)) == 2   # ld < cols
    assert lib.rv_ce_fused(*args(fake, _hip.RV_F16, 8, -1, 8, fake)) == 2
    assert lib.rv_ce_fused(*args(fake, _hip.RV_F16, 8, 0, 8, fake)) == 0   # nothing to do
    assert lib.rv_ce_fused(*args(fake, _hip.RV_F32, 8, 4, 8, fake)) == 3   # fp16 only
    assert lib.rv_ce_fused(*args(fake, _hip.RV_F16, 65544, 4, 65544, fake)) == 3  # too wide
    # logits and dlogits must share their address modulo 16
    assert lib.rv_ce_fused(*args(fake, _hip.RV_F16, 8, 4, 8, ctypes.c_void_p(4098))) == 3


def test_multi_cast_validates_without_device():
    lib = _hip.library()
    n = lib.rv_cast_f32_f16_max_tensors()
    assert n >= 32
    fake = ctypes.c_void_p(4096)
    P = ctypes.c_void_p * 2
    numel = (ctypes.c_int64 * 2)(8, 8)
    assert lib.rv_cast_f32_f16_multi(0, None, None, None, None) == 0
    assert lib.rv_cast_f32_f16_multi(-1, None, None, None, None) == 2
    assert lib.rv_cast_f32_f16_multi(2, None, P(fake, fake), numel, None) == 1
    assert lib.rv_cast_f32_f16_multi(2, P(fake, None), P(fake, fake), numel, None) == 1
    assert lib.rv_cast_f32_f16_multi(2, P(fake, fake), P(fake, ctypes.c_void_p(4098)), numel,
                                     None) == 3  # 16-byte alignment
    assert lib.rv_cast_f32_f16_multi(n + 1, P(fake, fake), P(fake, fake), numel, None) == 3
    bad = (ctypes.c_int64 * 2)(8, -1)
    assert lib.rv_cast_f32_f16_multi(2, P(fake, fake), P(fake, fake), bad, None) == 2


def test_grad_clip_entry_points_validate_without_device():
    lib = _hip.library()
    fake = ctypes.c_void_p(4096)
    n = (ctypes.c_int64 * 3)(16384, 16385, 1)  # 16384-element chunks
    assert lib.rv_grad_chunks(n, 3) == 1 + 2 + 1
    assert lib.rv_grad_chunks(n, 0) == 0
    assert lib.rv_grad_chunks(n, -1) < 0
    P = ctypes.c_void_p * 3
    assert lib.rv_grad_sq_partials(0, None, None, None, None, None, 0, None) == 0
    assert lib.rv_grad_sq_partials(3, P(fake, fake, None), n, None, fake, fake, 0, None) == 1
    assert lib.rv_grad_sq_partials(3, P(fake, fake, fake), n, None, fake, fake, -1, None) == 2
    assert lib.rv_grad_sq_partials(lib.rv_adamw_max_tensors() + 1, P(fake, fake, fake), n, None,
                                   fake, fake, 0, None) == 3
    assert lib.rv_grad_clip_coef(fake, fake, 0, 1.0, fake, fake, fake, None) == 2
    assert lib.rv_grad_clip_coef(fake, None, 4, 1.0, fake, fake, fake, None) == 1
