"""ctypes binding of ``libreversibility_hip.so`` and the ``torch.library`` ops over it.

The shared library exports the C ABI declared in ``include/reversibility_hip.h``
(device pointers, int64 sizes, a dtype code and a hipStream_t).  This module

* loads it (once, lazily) and declares every entry point's signature;
* registers one ``reversability_amd::<name>`` operator per kernel family for the
  ``CUDA`` dispatch key (ROCm tensors are ``device.type == 'cuda'``), plus a
  fake (meta) kernel for shape propagation;
* launches on torch's current stream of the tensors' device, so the kernels
  order correctly with torch's own work and can be captured in a HIP graph.

There is no fallback: a missing library or a non-zero status raises.  The ops
allocate their outputs with torch (the caching allocator), never inside the
library.  Operators are registered with ``torch.library.Library`` rather than
``torch.library.custom_op``: the latter adds ~15 us of Python dispatch per call,
more than several of these kernels take on an MI355X.
"""
from __future__ import annotations

import ctypes
from typing import Optional
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().with_name("libreversibility_hip.so")

RV_F32, RV_F16, RV_BF16, RV_F64 = 0, 1, 2, 3
_DTYPE_CODE = {
    torch.float32: RV_F32,
    torch.float16: RV_F16,
    torch.bfloat16: RV_BF16,
    torch.float64: RV_F64,
}

# Every symbol include/reversibility_hip.h declares, with (restype, argtypes).
_P, _I64, _I, _F, _D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_double
SIGNATURES = {
    "rv_status_string": (ctypes.c_char_p, [_I]),
    "rv_last_error": (ctypes.c_char_p, []),
    "rv_abi_version": (_I, []),
    "rv_rmsnorm_fwd": (_I, [_P, _P, _P, _P, _I64, _I64, _F, _P]),
    "rv_rmsnorm_bwd_workspace_bytes": (_I64, [_I64, _I64]),
    "rv_rmsnorm_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "rv_rmsnorm_bwd_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _P]),
    "rv_rmsnorm_fwd_f16": (_I, [_P, _P, _P, _P, _I64, _I64, _F, _P]),
    "rv_rmsnorm_bwd_f16": (_I, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "rv_swiglu_fwd": (_I, [_P, _I64, _P, _I64, _I64, _I, _P]),
    "rv_swiglu_bwd": (_I, [_P, _I64, _P, _P, _I64, _I64, _I, _P]),
    "rv_midpoint_update": (_I, [_P, _P, _P, _P, _D, _I, _I64, _I, _I, _P]),
    "rv_midpoint_update_bwd": (_I, [_P, _P, _D, _I, _I64, _I, _I, _P]),
    "rv_residual_axpy": (_I, [_P, _P, _P, _I, _I64, _I, _I, _P]),
    "rv_add_rmsnorm_fwd": (_I, [_P, _P, _I, _P, _P, _P, _P, _I64, _I64, _F, _P]),
    "rv_cast_f32_f16": (_I, [_P, _P, _I64, _P]),
    "rv_cast_f32_f16_max_tensors": (_I, []),
    "rv_cast_f32_f16_multi": (_I, [_I, _P, _P, _P, _P]),
    "rv_linear_fwd": (_I, [_P, _I64, _P, _I64, _I64, _I64, _P, _P]),
    "rv_linear_dx": (_I, [_P, _P, _I64, _I64, _I64, _P, _I, _P]),
    "rv_linear_dw_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "rv_linear_dw": (_I, [_P, _P, _I64, _I64, _I64, _I64, _P, _I, _P, _I64, _P]),
    "rv_adamw_max_tensors": (_I, []),
    "rv_adamw_advance": (_I, [_P, _P, _P]),
    "rv_adamw_step": (_I, [_I, _P, _P, _P, _P, _P, _D, _D, _D, _D, _D, _P, _P, _P, _P]),
    "rv_adamw_step_clipped": (_I, [_I, _P, _P, _P, _P, _P, _D, _D, _D, _D, _D, _P, _P, _P, _P,
                                   _P]),
    "rv_grad_chunks": (_I, [_P, _I]),
    "rv_grad_sq_partials": (_I, [_I, _P, _P, _P, _P, _P, _I, _P]),
    "rv_grad_clip_coef": (_I, [_P, _P, _I, _D, _P, _P, _P, _P]),
    "rv_ce_fwd": (_I, [_P, _I, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P]),
    "rv_ce_bwd": (_I, [_P, _I, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P]),
    "rv_gemm_num_shapes": (_I, []),
    "rv_gemm_force_shape": (_I, [_I]),
    "rv_add_rmsnorm_fwd_f16": (_I, [_P, _P, _I, _P, _P, _P, _P, _I64, _I64, _F, _P]),
    "rv_sub_rmsnorm_fwd_f16": (_I, [_P, _P, _I, _I, _P, _P, _P, _P, _P, _I64, _I64, _F, _P]),
    "rv_midpoint_rmsnorm_fwd_f16": (_I, [_P, _P, _P, _I, _D, _I, _P, _P, _P, _P, _I64, _I64, _F,
                                         _P]),
    "rv_rmsnorm_bwd_acc": (_I, [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "rv_rmsnorm_bwd_acc_pass": (_I, [_P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                     _I64, _P]),
    "rv_ce_fused": (_I, [_P, _I, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P]),
    "rv_mlp_up_swiglu": (_I, [_P, _I64, _P, _I64, _I64, _I64, _P, _P, _P]),
    "rv_mlp_down": (_I, [_P, _P, _I64, _I64, _I64, _P, _P]),
    "rv_mlp_dgate": (_I, [_P, _P, _P, _I64, _I64, _I64, _P, _P]),
    "rv_mlp_dx": (_I, [_P, _P, _I64, _I64, _I64, _P, _P]),
    "rv_mlp_wgrad_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "rv_mlp_wgrad": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I, _P, _I64, _P]),
    "rv_attn_fwd": (_I, [_P, _I64, _I64, _I64, _I64, _P, _P, _P]),
    "rv_attn_bwd_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "rv_attn_bwd": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "rv_batch_from_tokens": (_I, [_P, _I64, _I64, _P, _P, _P]),
    "rv_embed_fwd": (_I, [_P, _I64, _I64, _P, _I64, _P, _I64, _I64, _P, _P]),
    "rv_embed_bwd_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "rv_embed_bwd": (_I, [_P, _I64, _I64, _P, _I64, _I64, _I64, _P, _I, _P, _I, _P, _I64, _P]),
    "rv_stream_floor": (_I, [_P, _I, _P, _I, _I64, _I, _I, _P]),
    "rv_empty_kernel": (_I, [_I, _P]),
}
ABI_VERSION = 3


class HipExtensionError(RuntimeError):
    """The HIP library is missing, stale, or a kernel launch failed."""


_lib = None


def library() -> ctypes.CDLL:
    """Load the shared library (once) and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY_PATH.exists():
        raise HipExtensionError(
            f"{LIBRARY_PATH.name} is not built; run __graft_entry__.build() "
            "(hipcc --offload-arch=gfx950). There is no non-HIP fallback.")
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    _check_single_hip_runtime()
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.rv_abi_version() != ABI_VERSION:
        raise HipExtensionError("libreversibility_hip.so ABI version mismatch; rebuild it")
    _lib = lib
    return lib


def _check_single_hip_runtime() -> None:
    """torch ships its own libamdhip64 (SONAME libamdhip64.so.7); the kernels'
    library must bind to that same runtime, or stream handles would cross
    runtimes.  Importing torch before loading the library guarantees it (the
    loader matches the SONAME); verify from the process's mappings."""
    try:
        with open("/proc/self/maps") as maps:
            paths = {line.split()[-1] for line in maps if "libamdhip64" in line}
    except OSError:  # pragma: no cover - non-Linux
        return
    if len(paths) > 1:
        raise HipExtensionError(f"two HIP runtimes are mapped: {sorted(paths)}")


def _check(status: int, what: str) -> None:
    if status != 0:
        lib = library()
        text = lib.rv_status_string(status).decode()
        detail = lib.rv_last_error().decode() if status == 5 else ""
        raise HipExtensionError(f"{what}: {text}" + (f" [{detail}]" if detail else ""))


try:  # raw stream handle without constructing a torch.cuda.Stream object
    _raw_stream = torch._C._cuda_getCurrentRawStream
except AttributeError:  # pragma: no cover - older torch
    def _raw_stream(index):
        return torch.cuda.current_stream(index).cuda_stream


def _stream(t: torch.Tensor) -> int:
    return _raw_stream(t.device.index)


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPE_CODE[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}") from None


class _DeviceGuard:
    """Make the tensors' device current for the launch (no-op when it is)."""

    __slots__ = ("index", "prev")

    def __init__(self, t: torch.Tensor):
        self.index = t.device.index
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.index:
            self.prev = cur
            torch.cuda.set_device(self.index)

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)


# ---------------------------------------------------------------------------
# Kernel launchers (CUDA tensors, validated by the callers' autograd Functions)
# ---------------------------------------------------------------------------

def _rmsnorm_fwd(x: torch.Tensor, w: torch.Tensor, eps: float, fp16_out: bool = False):
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    y = torch.empty_like(x, dtype=torch.float16 if fp16_out else x.dtype)
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
    if rows:
        fn = library().rv_rmsnorm_fwd_f16 if fp16_out else library().rv_rmsnorm_fwd
        with _DeviceGuard(x):
            _check(fn(x.data_ptr(), w.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, width,
                      eps, _stream(x)), "rv_rmsnorm_fwd")
    return y, rstd


def rmsnorm_workspace_bytes(rows: int, width: int) -> int:
    n = library().rv_rmsnorm_bwd_workspace_bytes(rows, width)
    if n < 0:
        _check(-n, "rv_rmsnorm_bwd_workspace_bytes")
    return n


def _rmsnorm_bwd(x: torch.Tensor, w: torch.Tensor, dy: torch.Tensor, rstd: torch.Tensor):
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    dx = torch.empty_like(x)
    if not rows:
        return dx, torch.zeros_like(w)
    dw = torch.empty_like(w)
    nbytes = rmsnorm_workspace_bytes(rows, width)
    ws = torch.empty(nbytes // 4, device=x.device, dtype=torch.float32)
    fn = library().rv_rmsnorm_bwd_f16 if dy.dtype == torch.float16 else library().rv_rmsnorm_bwd
    with _DeviceGuard(x):
        _check(fn(x.data_ptr(), w.data_ptr(), dy.data_ptr(),
                                        rstd.data_ptr(), dx.data_ptr(), dw.data_ptr(),
                                        ws.data_ptr(), nbytes, rows, width, _stream(x)),
               "rv_rmsnorm_bwd")
    return dx, dw


def _add_rmsnorm_fwd(x: torch.Tensor, f: torch.Tensor, w: torch.Tensor, eps: float):
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    h = torch.empty_like(x)
    y = torch.empty_like(x)
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
    if rows:
        with _DeviceGuard(x):
            _check(library().rv_add_rmsnorm_fwd(x.data_ptr(), f.data_ptr(), _dtype_code(f),
                                                w.data_ptr(), h.data_ptr(), y.data_ptr(),
                                                rstd.data_ptr(), rows, width, eps, _stream(x)),
                   "rv_add_rmsnorm_fwd")
    return h, y, rstd


def _add_rmsnorm_fwd16(x: torch.Tensor, f: torch.Tensor, w: torch.Tensor, eps: float):
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    h = torch.empty_like(x)
    y = torch.empty_like(x, dtype=torch.float16)
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
    if rows:
        with _DeviceGuard(x):
            _check(library().rv_add_rmsnorm_fwd_f16(x.data_ptr(), f.data_ptr(), _dtype_code(f),
                                                    w.data_ptr(), h.data_ptr(), y.data_ptr(),
                                                    rstd.data_ptr(), rows, width, eps,
                                                    _stream(x)),
                   "rv_add_rmsnorm_fwd_f16")
    return h, y, rstd


def _sub_rmsnorm_fwd16(x: torch.Tensor, f: torch.Tensor, w: torch.Tensor, eps: float,
                       readd: bool):
    """d = x - f and the fp16 RMSNorm of d (readd False) or of h = d + f
    (readd True): (d, h (empty when not readd), y16, rstd)."""
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    d = torch.empty_like(x)
    h = torch.empty_like(x) if readd else x.new_empty(0)
    y = torch.empty_like(x, dtype=torch.float16)
    rstd = torch.empty(rows, device=x.device, dtype=torch.float32)
    if rows:
        with _DeviceGuard(x):
            _check(library().rv_sub_rmsnorm_fwd_f16(x.data_ptr(), f.data_ptr(), _dtype_code(f),
                                                    int(readd), w.data_ptr(), d.data_ptr(),
                                                    h.data_ptr() if readd else None,
                                                    y.data_ptr(), rstd.data_ptr(), rows, width,
                                                    eps, _stream(x)),
                   "rv_sub_rmsnorm_fwd_f16")
    return d, h, y, rstd


def _midpoint_rmsnorm_fwd16(p: torch.Tensor, a: torch.Tensor, m: torch.Tensor, w: torch.Tensor,
                            eps: float, scale: float, sign: int):
    """The midpoint update of p with fp16 a, m and the fp16 RMSNorm of the
    result: (out, y16, rstd)."""
    width = p.shape[-1]
    rows = p.numel() // width if width else 0
    out = torch.empty_like(p)
    y = torch.empty_like(p, dtype=torch.float16)
    rstd = torch.empty(rows, device=p.device, dtype=torch.float32)
    if rows:
        with _DeviceGuard(p):
            _check(library().rv_midpoint_rmsnorm_fwd_f16(p.data_ptr(), a.data_ptr(), m.data_ptr(),
                                                         _dtype_code(a), scale, sign,
                                                         w.data_ptr(), out.data_ptr(),
                                                         y.data_ptr(), rstd.data_ptr(), rows,
                                                         width, eps, _stream(p)),
                   "rv_midpoint_rmsnorm_fwd_f16")
    return out, y, rstd


def _rmsnorm_bwd_acc(x: torch.Tensor, w: torch.Tensor, dy: torch.Tensor, rstd: torch.Tensor,
                     dh: Optional[torch.Tensor], f16: bool = True,
                     dpass: Optional[torch.Tensor] = None):
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    dx = torch.empty_like(x)
    dx16 = (torch.empty_like(x, dtype=torch.float16) if f16
            else x.new_empty(0, dtype=torch.float16))
    if not rows:
        return dx, dx16, torch.zeros_like(w)
    dw = torch.empty_like(w)
    nbytes = rmsnorm_workspace_bytes(rows, width)
    ws = torch.empty(nbytes // 4, device=x.device, dtype=torch.float32)
    with _DeviceGuard(x):
        _check(library().rv_rmsnorm_bwd_acc_pass(x.data_ptr(), w.data_ptr(), dy.data_ptr(),
                                            _dtype_code(dy), rstd.data_ptr(),
                                            dh.data_ptr() if dh is not None else None,
                                            dpass.data_ptr() if dpass is not None else None,
                                            dx.data_ptr(), dx16.data_ptr() if f16 else None,
                                            dw.data_ptr(),
                                            ws.data_ptr(), nbytes, rows, width, _stream(x)),
               "rv_rmsnorm_bwd_acc")
    return dx, dx16, dw


def _swiglu_fwd(u: torch.Tensor):
    packed = u.shape[-1]
    width = packed // 2
    rows = u.numel() // packed if packed else 0
    out = torch.empty((*u.shape[:-1], width), device=u.device, dtype=u.dtype)
    if rows and width:
        with _DeviceGuard(u):
            _check(library().rv_swiglu_fwd(u.data_ptr(), packed, out.data_ptr(), rows, width,
                                           _dtype_code(u), _stream(u)),
                   "rv_swiglu_fwd")
    return out


def _swiglu_bwd(u: torch.Tensor, dy: torch.Tensor):
    packed = u.shape[-1]
    width = packed // 2
    rows = u.numel() // packed if packed else 0
    du = torch.empty_like(u)
    if rows and width:
        with _DeviceGuard(u):
            _check(library().rv_swiglu_bwd(u.data_ptr(), packed, dy.data_ptr(), du.data_ptr(),
                                           rows, width, _dtype_code(u), _stream(u)),
                   "rv_swiglu_bwd")
    return du


def _midpoint_update(p: torch.Tensor, a: torch.Tensor, m: torch.Tensor, scale: float, sign: int):
    out = torch.empty_like(p)
    n = p.numel()
    if n:
        with _DeviceGuard(p):
            _check(library().rv_midpoint_update(p.data_ptr(), a.data_ptr(), m.data_ptr(),
                                                out.data_ptr(), scale, sign, n, _dtype_code(p),
                                                _dtype_code(a), _stream(p)),
                   "rv_midpoint_update")
    return out


def _midpoint_update_bwd(dout: torch.Tensor, scale: float, sign: int, force_dtype: torch.dtype):
    da = torch.empty(dout.shape, device=dout.device, dtype=force_dtype)
    n = dout.numel()
    if n:
        with _DeviceGuard(dout):
            _check(library().rv_midpoint_update_bwd(dout.data_ptr(), da.data_ptr(), scale, sign,
                                                    n, _dtype_code(dout), _DTYPE_CODE[force_dtype],
                                                    _stream(dout)),
                   "rv_midpoint_update_bwd")
    return da


def _residual_axpy(x: torch.Tensor, f: torch.Tensor, sign: int):
    out = torch.empty_like(x)
    n = x.numel()
    if n:
        with _DeviceGuard(x):
            _check(library().rv_residual_axpy(x.data_ptr(), f.data_ptr(), out.data_ptr(), sign, n,
                                              _dtype_code(x), _dtype_code(f), _stream(x)),
                   "rv_residual_axpy")
    return out


def _ce_fwd(logits: torch.Tensor, labels: torch.Tensor, ignore_index: int):
    rows, cols = logits.shape
    rmax, rlse, loss = (torch.empty(rows, device=logits.device, dtype=torch.float32)
                        for _ in range(3))
    if rows:
        with _DeviceGuard(logits):
            _check(library().rv_ce_fwd(logits.data_ptr(), _dtype_code(logits), logits.stride(0),
                                       labels.data_ptr(), rows, cols, ignore_index,
                                       rmax.data_ptr(), rlse.data_ptr(), loss.data_ptr(),
                                       _stream(logits)),
                   "rv_ce_fwd")
    return rmax, rlse, loss


def _ce_bwd(logits: torch.Tensor, labels: torch.Tensor, rmax: torch.Tensor, rlse: torch.Tensor,
            grad: torch.Tensor, ignore_index: int):
    rows, cols = logits.shape
    dx = torch.empty_like(logits)
    if rows:
        with _DeviceGuard(logits):
            _check(library().rv_ce_bwd(logits.data_ptr(), _dtype_code(logits), logits.stride(0),
                                       labels.data_ptr(), rmax.data_ptr(), rlse.data_ptr(),
                                       grad.data_ptr(), rows, cols, ignore_index, dx.data_ptr(),
                                       _stream(logits)),
                   "rv_ce_bwd")
    return dx


# ---------------------------------------------------------------------------
# torch.library registration
# ---------------------------------------------------------------------------
NAMESPACE = "reversability_amd"
_library = torch.library.Library(NAMESPACE, "DEF")
_SCHEMAS = {
    "rmsnorm_fwd": ("rmsnorm_fwd(Tensor x, Tensor weight, float eps, bool fp16_out=False) "
                    "-> (Tensor, Tensor)", _rmsnorm_fwd),
    "rmsnorm_bwd": ("rmsnorm_bwd(Tensor x, Tensor weight, Tensor dy, Tensor rstd) -> (Tensor, Tensor)",
                    _rmsnorm_bwd),
    "add_rmsnorm_fwd": ("add_rmsnorm_fwd(Tensor x, Tensor f, Tensor weight, float eps) -> (Tensor, Tensor, Tensor)",
                        _add_rmsnorm_fwd),
    "add_rmsnorm_fwd16": ("add_rmsnorm_fwd16(Tensor x, Tensor f, Tensor weight, float eps) "
                          "-> (Tensor, Tensor, Tensor)", _add_rmsnorm_fwd16),
    "sub_rmsnorm_fwd16": ("sub_rmsnorm_fwd16(Tensor x, Tensor f, Tensor weight, float eps, "
                          "bool readd) -> (Tensor, Tensor, Tensor, Tensor)", _sub_rmsnorm_fwd16),
    "midpoint_rmsnorm_fwd16": ("midpoint_rmsnorm_fwd16(Tensor p, Tensor a, Tensor m, "
                               "Tensor weight, float eps, float scale, int sign) "
                               "-> (Tensor, Tensor, Tensor)", _midpoint_rmsnorm_fwd16),
    "rmsnorm_bwd_acc": ("rmsnorm_bwd_acc(Tensor x, Tensor weight, Tensor dy, Tensor rstd, "
                        "Tensor? dh, bool f16=True, Tensor? dpass=None) "
                        "-> (Tensor, Tensor, Tensor)",
                        _rmsnorm_bwd_acc),
    "swiglu_fwd": ("swiglu_fwd(Tensor u) -> Tensor", _swiglu_fwd),
    "swiglu_bwd": ("swiglu_bwd(Tensor u, Tensor dy) -> Tensor", _swiglu_bwd),
    "midpoint_update": ("midpoint_update(Tensor p, Tensor a, Tensor m, float scale, int sign) -> Tensor",
                        _midpoint_update),
    "midpoint_update_bwd": ("midpoint_update_bwd(Tensor dout, float scale, int sign, ScalarType force_dtype) -> Tensor",
                            _midpoint_update_bwd),
    "residual_axpy": ("residual_axpy(Tensor x, Tensor f, int sign) -> Tensor", _residual_axpy),
    "ce_fwd": ("ce_fwd(Tensor logits, Tensor labels, int ignore_index) -> (Tensor, Tensor, Tensor)",
               _ce_fwd),
    "ce_bwd": ("ce_bwd(Tensor logits, Tensor labels, Tensor rmax, Tensor rlse, Tensor grad, "
               "int ignore_index) -> Tensor", _ce_bwd),
}
for _name, (_schema, _impl) in _SCHEMAS.items():
    _library.define(_schema)
    _library.impl(_name, _impl, "CUDA")


def _fake_rows(x):
    width = x.shape[-1]
    return x.numel() // width if width else 0


@torch.library.register_fake(f"{NAMESPACE}::rmsnorm_fwd")
def _(x, weight, eps, fp16_out=False):
    return (torch.empty_like(x, dtype=torch.float16 if fp16_out else x.dtype),
            x.new_empty(_fake_rows(x), dtype=torch.float32))


@torch.library.register_fake(f"{NAMESPACE}::rmsnorm_bwd")
def _(x, weight, dy, rstd):
    return torch.empty_like(x), torch.empty_like(weight)


@torch.library.register_fake(f"{NAMESPACE}::add_rmsnorm_fwd")
def _(x, f, weight, eps):
    return torch.empty_like(x), torch.empty_like(x), x.new_empty(_fake_rows(x), dtype=torch.float32)


@torch.library.register_fake(f"{NAMESPACE}::add_rmsnorm_fwd16")
def _(x, f, weight, eps):
    return (torch.empty_like(x), torch.empty_like(x, dtype=torch.float16),
            x.new_empty(_fake_rows(x), dtype=torch.float32))


@torch.library.register_fake(f"{NAMESPACE}::sub_rmsnorm_fwd16")
def _(x, f, weight, eps, readd):
    return (torch.empty_like(x), torch.empty_like(x) if readd else x.new_empty(0),
            torch.empty_like(x, dtype=torch.float16),
            x.new_empty(_fake_rows(x), dtype=torch.float32))


@torch.library.register_fake(f"{NAMESPACE}::midpoint_rmsnorm_fwd16")
def _(p, a, m, weight, eps, scale, sign):
    return (torch.empty_like(p), torch.empty_like(p, dtype=torch.float16),
            p.new_empty(_fake_rows(p), dtype=torch.float32))


@torch.library.register_fake(f"{NAMESPACE}::rmsnorm_bwd_acc")
def _(x, weight, dy, rstd, dh, f16=True, dpass=None):
    return (torch.empty_like(x), torch.empty_like(x, dtype=torch.float16) if f16
            else x.new_empty(0, dtype=torch.float16), torch.empty_like(weight))


@torch.library.register_fake(f"{NAMESPACE}::swiglu_fwd")
def _(u):
    return u.new_empty((*u.shape[:-1], u.shape[-1] // 2))


@torch.library.register_fake(f"{NAMESPACE}::swiglu_bwd")
def _(u, dy):
    return torch.empty_like(u)


@torch.library.register_fake(f"{NAMESPACE}::midpoint_update")
def _(p, a, m, scale, sign):
    return torch.empty_like(p)


@torch.library.register_fake(f"{NAMESPACE}::midpoint_update_bwd")
def _(dout, scale, sign, force_dtype):
    return dout.new_empty(dout.shape, dtype=force_dtype)


@torch.library.register_fake(f"{NAMESPACE}::residual_axpy")
def _(x, f, sign):
    return torch.empty_like(x)


@torch.library.register_fake(f"{NAMESPACE}::ce_fwd")
def _(logits, labels, ignore_index):
    rows = logits.shape[0]
    return tuple(logits.new_empty(rows, dtype=torch.float32) for _ in range(3))


@torch.library.register_fake(f"{NAMESPACE}::ce_bwd")
def _(logits, labels, rmax, rlse, grad, ignore_index):
    return torch.empty_like(logits)


ops = getattr(torch.ops, NAMESPACE)
