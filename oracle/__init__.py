"""CPU oracle for the reversible-training hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product package ``reversability_amd`` never imports it.

Contents
--------
``kernels_ref.c`` (built into ``liboracle.so`` by ``make -C oracle``)
    C restatement of the fused kernels, wrapped here over numpy arrays:
    :func:`rmsnorm_fwd`, :func:`rmsnorm_bwd` (src/reversibility/kernels_v3.py:9-48),
    :func:`swiglu_fwd`, :func:`swiglu_bwd` (src/reversibility/kernels.py:88-110),
    :func:`midpoint`, :func:`midpoint_bwd`, :func:`euler`
    (src/reversibility/reversible.py:16-32), :func:`ce_fwd`, :func:`ce_bwd`
    (src/reversibility/kernels.py:14-77), :func:`embed_fwd`, :func:`embed_bwd`
    (src/reversibility/reversible.py:105-106 with model.py's two nn.Embedding).
:func:`batch_at`
    numpy restatement of scripts/train_baseline.py:50-63.
``model_ref.py``
    torch-CPU functional restatement of the decoder and both integrators
    (src/reversibility/model.py, reversible.py) for model-level checks.

How each function is pinned (tests/test_oracle.py):
    rmsnorm_fwd/bwd -- torch.nn.functional.rms_norm and its autograd in fp64,
        the scale-invariance identity <dx, x> = 0 at eps = 0, constant-row
        closed form, central finite differences on tiny inputs, golden file.
    swiglu_fwd/bwd  -- F.silu in fp32 with explicit fp16 casts (library),
        fp64 autograd of silu(g)*v at fp16 tolerance, special values
        (g = 0, large |g|), golden file.
    midpoint/euler  -- torch's own eager fp16/fp32 expression bit for bit.
    ce_fwd/bwd      -- fp64 cross-entropy and its gradient (library), the
        uniform-logits closed form log V, torch's eager fp16 log_softmax at
        the target (the reference's Half-logsoftmax policy), zero column sums
        of the gradient, ignore_index rows.
    batch_at        -- the reference's own test vector
        (tests/test_baseline.py:30-38), the shift identity x[1:] == y[:-1]
        on its test stream (arange(4097) % 31, tests/test_optimized.py:89),
        target counts of partial batches, StopIteration past the limit.
    embed_fwd       -- numpy gather + broadcast add (library), bit for bit.
    embed_bwd       -- np.add.at / numpy sum over the batch on small-integer
        gradients (exact in any order), fp64 sums at fp32 tolerance, the
        block order changing nothing for runs inside one block, ids outside
        the vocabulary contributing nothing, accumulation.
    f16 conversion  -- all 65536 binary16 patterns round-trip; numpy's
        float16 cast on 2^20 random floats including subnormals/overflow.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
F32, F16, BF16, F64 = 0, 1, 2, 3

_lib = None


def build() -> Path:
    """Compile kernels_ref.c with gcc (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        P, I64, I, F, D = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                           ctypes.c_float, ctypes.c_double)
        sig = {
            "oracle_f32_to_f16": (ctypes.c_uint16, [F]),
            "oracle_f16_to_f32": (F, [ctypes.c_uint16]),
            "oracle_round_bf16": (F, [F]),
            "oracle_num_threads": (I, []),
            "oracle_set_num_threads": (None, [I]),
            "oracle_rmsnorm_fwd": (None, [P, P, P, P, I64, I64, D]),
            "oracle_rmsnorm_bwd": (None, [P, P, P, P, P, I64, I64, D]),
            "oracle_swiglu_fwd": (None, [P, I64, P, I64, I64, I]),
            "oracle_swiglu_bwd": (None, [P, I64, P, P, I64, I64, I]),
            "oracle_midpoint": (None, [P, P, P, P, F, I, I64, I]),
            "oracle_midpoint_bwd": (None, [P, P, F, I, I64, I]),
            "oracle_midpoint_f64": (None, [P, P, P, P, D, I, I64]),
            "oracle_euler": (None, [P, P, P, I, I64, I]),
            "oracle_f32_to_f16_array": (None, [P, P, I64]),
            "oracle_f16_to_f32_array": (None, [P, P, I64]),
            "oracle_ce_fwd": (None, [P, I64, P, I64, I64, I64, I, P, P, P]),
            "oracle_ce_bwd": (None, [P, I64, P, P, P, F, I64, I64, I64, I, P]),
            "oracle_embed_fwd": (None, [P, I64, I64, P, I64, P, I64, P]),
            "oracle_embed_bwd_pos": (None, [P, I64, I64, I64, I64, P, I]),
            "oracle_embed_bwd_tok": (None, [P, I64, P, I64, I64, I64, P, I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def _code(a: np.ndarray) -> int:
    return {np.dtype(np.float16): F16, np.dtype(np.float32): F32}[a.dtype]


def set_num_threads(n: int) -> None:
    lib().oracle_set_num_threads(int(n))


def num_threads() -> int:
    return lib().oracle_num_threads()


def rmsnorm_fwd(x: np.ndarray, w: np.ndarray, eps: float):
    """y, rstd for x [..., W] float32 (rstd flat [rows])."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    width = x.shape[-1]
    rows = x.size // width
    y = np.empty_like(x)
    rstd = np.empty(rows, np.float32)
    lib().oracle_rmsnorm_fwd(_ptr(x), _ptr(w), _ptr(y), _ptr(rstd), rows, width, eps)
    return y, rstd


def rmsnorm_bwd(x: np.ndarray, w: np.ndarray, dy: np.ndarray, eps: float):
    """dx, dw for upstream dy."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    dy = np.ascontiguousarray(dy, np.float32)
    width = x.shape[-1]
    rows = x.size // width
    dx = np.empty_like(x)
    dw = np.empty(width, np.float32)
    lib().oracle_rmsnorm_bwd(_ptr(x), _ptr(w), _ptr(dy), _ptr(dx), _ptr(dw), rows, width, eps)
    return dx, dw


def swiglu_fwd(u: np.ndarray) -> np.ndarray:
    """u [..., 2W] float16/float32 -> [..., W] same dtype."""
    u = np.ascontiguousarray(u)
    packed = u.shape[-1]
    width = packed // 2
    rows = u.size // packed
    o = np.empty((*u.shape[:-1], width), u.dtype)
    lib().oracle_swiglu_fwd(_ptr(u), packed, _ptr(o), rows, width, _code(u))
    return o


def swiglu_bwd(u: np.ndarray, dy: np.ndarray) -> np.ndarray:
    """Packed du [..., 2W] for upstream dy [..., W]."""
    u = np.ascontiguousarray(u)
    dy = np.ascontiguousarray(dy, u.dtype)
    packed = u.shape[-1]
    width = packed // 2
    rows = u.size // packed
    du = np.empty_like(u)
    lib().oracle_swiglu_bwd(_ptr(u), packed, _ptr(dy), _ptr(du), rows, width, _code(u))
    return du


def _force_code(a: np.ndarray, force_dtype: str | None) -> int:
    if force_dtype == "bf16":
        return BF16
    return _code(a)


def midpoint(p, a, m, scale, sign, force_dtype=None):
    """p + sign * round(round(a + m) * scale); p float32 (or float64 with a, m float64).
    For bf16 forces pass a, m as uint16 bit patterns and force_dtype='bf16'."""
    if p.dtype == np.float64:
        p, a, m = (np.ascontiguousarray(t, np.float64) for t in (p, a, m))
        out = np.empty_like(p)
        lib().oracle_midpoint_f64(_ptr(p), _ptr(a), _ptr(m), _ptr(out), scale, sign, p.size)
        return out
    p = np.ascontiguousarray(p, np.float32)
    a, m = np.ascontiguousarray(a), np.ascontiguousarray(m)
    out = np.empty_like(p)
    code = BF16 if force_dtype == "bf16" else _code(a)
    lib().oracle_midpoint(_ptr(p), _ptr(a), _ptr(m), _ptr(out), scale, sign, p.size, code)
    return out


def midpoint_bwd(dout, scale, sign, force_dtype="f16"):
    """sign * round(round(dout) * scale) as float32 values."""
    dout = np.ascontiguousarray(dout, np.float32)
    da = np.empty_like(dout)
    code = {"f16": F16, "bf16": BF16, "f32": F32}[force_dtype]
    lib().oracle_midpoint_bwd(_ptr(dout), _ptr(da), scale, sign, dout.size, code)
    return da


def euler(x, f, sign, force_dtype=None):
    x = np.ascontiguousarray(x, np.float32)
    f = np.ascontiguousarray(f)
    out = np.empty_like(x)
    code = BF16 if force_dtype == "bf16" else _code(f)
    lib().oracle_euler(_ptr(x), _ptr(f), _ptr(out), sign, x.size, code)
    return out


def f32_to_f16_bits(v: np.ndarray) -> np.ndarray:
    """float32 array -> binary16 bit patterns (uint16), round to nearest even."""
    v = np.ascontiguousarray(v, np.float32)
    out = np.empty(v.shape, np.uint16)
    lib().oracle_f32_to_f16_array(_ptr(v), _ptr(out), v.size)
    return out


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    """binary16 bit patterns (uint16) -> float32 array."""
    b = np.ascontiguousarray(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_f16_to_f32_array(_ptr(b), _ptr(out), b.size)
    return out


def ce_fwd(x: np.ndarray, labels: np.ndarray, ignore_index: int = -100):
    """(row_max, row_lse, loss) float32 [rows] for logits x [rows, cols] float16/float32."""
    x = np.ascontiguousarray(x)
    labels = np.ascontiguousarray(labels, np.int64)
    rows, cols = x.shape
    rmax, rlse, loss = (np.empty(rows, np.float32) for _ in range(3))
    lib().oracle_ce_fwd(_ptr(x), cols, _ptr(labels), rows, cols, ignore_index, _code(x),
                        _ptr(rmax), _ptr(rlse), _ptr(loss))
    return rmax, rlse, loss


def ce_bwd(x: np.ndarray, labels: np.ndarray, rmax: np.ndarray, rlse: np.ndarray, grad: float,
           ignore_index: int = -100) -> np.ndarray:
    """d(sum loss)/dx * grad, in x's dtype, given the forward's row statistics."""
    x = np.ascontiguousarray(x)
    labels = np.ascontiguousarray(labels, np.int64)
    rmax = np.ascontiguousarray(rmax, np.float32)
    rlse = np.ascontiguousarray(rlse, np.float32)
    rows, cols = x.shape
    dx = np.empty_like(x)
    lib().oracle_ce_bwd(_ptr(x), cols, _ptr(labels), _ptr(rmax), _ptr(rlse), grad, rows, cols,
                        ignore_index, _code(x), _ptr(dx))
    return dx


IGNORE_INDEX = -100
EMBED_RUN_BLOCK = 16  # sorted entries per block in the device token-gradient reduction


def batch_at(data: np.ndarray, cursor: int, batch_size: int, sequence_length: int,
             target_limit: int):
    """(x, y, count) int64 [sequences, sequence_length] from a uint16 token
    stream (scripts/train_baseline.py:50-63): x = stream[cursor:cursor+count],
    y shifted by one, padded with x = 0 and y = -100."""
    count = min(batch_size * sequence_length, target_limit - cursor)
    if count <= 0:
        raise StopIteration
    sequences = -(-count // sequence_length)
    raw = np.asarray(data[cursor:cursor + count + 1], dtype=np.int64)
    x = np.zeros(sequences * sequence_length, np.int64)
    y = np.full(sequences * sequence_length, IGNORE_INDEX, np.int64)
    x[:count] = raw[:-1]
    y[:count] = raw[1:]
    return x.reshape(sequences, sequence_length), y.reshape(sequences, sequence_length), count


def embed_fwd(ids: np.ndarray, tok: np.ndarray, pos: np.ndarray) -> np.ndarray:
    """tok[ids] + pos[:T] as float32 [B, T, d]; NaN rows for ids outside the table."""
    ids = np.ascontiguousarray(ids, np.int64)
    tok = np.ascontiguousarray(tok, np.float32)
    pos = np.ascontiguousarray(pos, np.float32)
    batch, seq = ids.shape
    d = tok.shape[1]
    out = np.empty((batch, seq, d), np.float32)
    lib().oracle_embed_fwd(_ptr(ids), batch * seq, seq, _ptr(tok), tok.shape[0], _ptr(pos), d,
                           _ptr(out))
    return out


def embed_bwd(ids: np.ndarray, dout: np.ndarray, vocab: int, max_seq: int, dtok=None, dpos=None,
              block: int = EMBED_RUN_BLOCK):
    """(dtok [vocab, d], dpos [max_seq, d]) float32.  Given dtok / dpos arrays
    are accumulated into (in place); otherwise fresh ones are returned."""
    ids = np.ascontiguousarray(ids, np.int64)
    dout = np.ascontiguousarray(dout, np.float32)
    batch, seq = ids.shape
    d = dout.shape[-1]
    tok_acc, pos_acc = dtok is not None, dpos is not None
    if dtok is None:
        dtok = np.empty((vocab, d), np.float32)
    if dpos is None:
        dpos = np.empty((max_seq, d), np.float32)
    assert dtok.flags.c_contiguous and dpos.flags.c_contiguous
    lib().oracle_embed_bwd_tok(_ptr(ids), batch * seq, _ptr(dout), vocab, d, block, _ptr(dtok),
                               int(tok_acc))
    lib().oracle_embed_bwd_pos(_ptr(dout), batch, seq, max_seq, d, _ptr(dpos), int(pos_acc))
    return dtok, dpos
