"""CPU oracle for the int4 weight-only linear path -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
import this package, and only as the checker (or, for the baseline, as the
timed reference algorithm).  The product under ``accel_amd/`` never imports,
links or calls it.

Two independent restatements live here:

* ``oracle.c`` (built to ``liboracle.so``): the reference's algorithm in the
  reference's evaluation order, bitwise equal to the Go CPU backend.  Bound
  through ctypes by the functions below.
* ``oracle_np.py``: a vectorised numpy restatement of the packer, written
  separately, used to cross-check ``orc_int4_quantize`` bit for bit.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_u32 = ctypes.c_uint32


def build() -> str:
    """Compile liboracle.so from oracle.c with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    L.orc_to_f16.argtypes = [ctypes.c_float]
    L.orc_to_f16.restype = ctypes.c_uint16
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f16_to_f32.restype = ctypes.c_float
    L.orc_to_bf16.argtypes = [ctypes.c_float]
    L.orc_to_bf16.restype = ctypes.c_uint16
    L.orc_to_f16_batch.argtypes = [_f32p, _u16p, _i64]
    L.orc_to_bf16_batch.argtypes = [_f32p, _u16p, _i64]
    L.orc_f16_to_f32_batch.argtypes = [_u16p, _f32p, _i64]
    if hasattr(L, "orc_check_f16_range"):
        L.orc_check_f16_range.argtypes = [ctypes.c_uint64, ctypes.c_uint64,
                                          ctypes.POINTER(ctypes.c_int64),
                                          ctypes.POINTER(ctypes.c_uint64)]
        L.orc_check_f16_range.restype = ctypes.c_int64
    L.orc_int4_quantize.argtypes = [_f32p, _i64, _u32p, _u16p, _u16p]
    L.orc_int4_nibble.argtypes = [_u32p, _i64]
    L.orc_int4_nibble.restype = ctypes.c_uint32
    L.orc_int4_dequantize.argtypes = [_u32p, _u16p, _u16p, _i64, _f32p]
    L.orc_ulp16.argtypes = [ctypes.c_uint16]
    L.orc_ulp16.restype = ctypes.c_double
    L.orc_int4_error_bound.argtypes = [_f32p, _i64, _u16p, _i64, _u16p, _i64]
    L.orc_int4_error_bound.restype = ctypes.c_double
    L.orc_int8_quantize.argtypes = [_f32p, _i64, _i8p, _u16p]
    L.orc_int8_dequantize.argtypes = [_i8p, _u16p, _i64, _f32p]
    L.orc_quant_matvec_int4.argtypes = [_u32, _u32, _f32p, _u32p, _u16p, _u16p, _f32p,
                                        ctypes.c_int]
    L.orc_quant_matmul_int4.argtypes = [_u32, _u32, _u32, _f32p, _u32p, _u16p, _u16p,
                                        _f32p, ctypes.c_int]
    L.orc_segment_offsets.argtypes = [_u32, _u32p, _u32p]
    L.orc_grouped_matvec.argtypes = [_u32, _u32, _u32, _u32, _f32p, _f32p, _u32p, _f32p,
                                     ctypes.c_int]
    L.orc_grouped_matmul.argtypes = [_u32, _u32, _u32, _u32, _f32p, _f32p, _u32p, _f32p,
                                     ctypes.c_int]
    L.orc_int4_grouped_matvec.argtypes = [_u32, _u32, _u32, _u32, _f32p, _u32p, _u16p,
                                          _u16p, _u32p, _f32p, ctypes.c_int]
    L.orc_int4_grouped_matmul.argtypes = [_u32, _u32, _u32, _u32, _f32p, _u32p, _u16p,
                                          _u16p, _u32p, _f32p, ctypes.c_int]
    L.orc_swiglu.argtypes = [_f32p, _f32p, _f32p, _i64]
    L.orc_add_rows.argtypes = [_u32, _u32, _f32p, _f32p, _f32p]
    L.orc_foreign_dequant.argtypes = [ctypes.c_int32, _i64, _i64, _i64, _u32p, _u32p, _u16p,
                                      ctypes.c_void_p, _f32p]
    L.orc_rmsnorm.argtypes = [_u32, _u32, ctypes.c_float, _f32p, _f32p, _f32p]
    L.orc_matvec_f32_f16.argtypes = [_u32, _u32, _f32p, _u16p, _f32p]
    L.orc_quant_matvec_i8.argtypes = [_u32, _u32, _f32p, _i8p, _u16p, _f32p]
    L.orc_quant_matmul_i8.argtypes = [_u32, _u32, _u32, _f32p, _i8p, _u16p, _f32p]
    _lib = L
    return L


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# --- conversions (internal/kernel/narrow.go) ---------------------------------

def to_f16(x) -> np.ndarray:
    x = _f32(np.atleast_1d(x)).ravel()
    out = np.empty(x.size, np.uint16)
    lib().orc_to_f16_batch(x, out, x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(np.atleast_1d(h), dtype=np.uint16).ravel()
    out = np.empty(h.size, np.float32)
    lib().orc_f16_to_f32_batch(h, out, h.size)
    return out


def to_bf16(x) -> np.ndarray:
    x = _f32(np.atleast_1d(x)).ravel()
    out = np.empty(x.size, np.uint16)
    lib().orc_to_bf16_batch(x, out, x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x) -> np.ndarray:
    """f32 values rounded to bf16 (RNE) and widened back."""
    x = _f32(x)
    return bf16_to_f32(to_bf16(x).reshape(x.shape))


# --- quant (quant/int4.go, quant/quant.go) -----------------------------------

def int4_quantize(w):
    """Returns (packed u32[ceil(n/8)], scales f16-bits[ceil(n/128)], zeros)."""
    w = _f32(w).ravel()
    n = w.size
    packed = np.zeros((n + 7) // 8, np.uint32)
    groups = (n + 127) // 128
    scales = np.zeros(groups, np.uint16)
    zeros = np.zeros(groups, np.uint16)
    lib().orc_int4_quantize(w, n, packed, scales, zeros)
    return packed, scales, zeros


def int4_nibble(packed, i: int) -> int:
    return int(lib().orc_int4_nibble(np.ascontiguousarray(packed, np.uint32), i))


def int4_dequantize(packed, scales, zeros, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_int4_dequantize(np.ascontiguousarray(packed, np.uint32),
                              np.ascontiguousarray(scales, np.uint16),
                              np.ascontiguousarray(zeros, np.uint16), n, out)
    return out


def ulp16(h: int) -> float:
    return float(lib().orc_ulp16(int(h)))


def int4_error_bound(x, term_scales, term_zeros) -> float:
    x = _f32(x).ravel()
    ts = np.ascontiguousarray(term_scales, np.uint16).ravel()
    tz = np.ascontiguousarray(term_zeros, np.uint16).ravel()
    v = lib().orc_int4_error_bound(x, x.size, ts, ts.size, tz, tz.size)
    if v < 0:
        raise ValueError(
            f"Int4ErrorBound has {x.size} terms, {ts.size} scales and {tz.size} zeros; "
            "it takes one scale and one zero per term")
    return float(v)


def int8_quantize(w):
    w = _f32(w).ravel()
    q = np.zeros(w.size, np.int8)
    s = np.zeros((w.size + 31) // 32, np.uint16)
    lib().orc_int8_quantize(w, w.size, q, s)
    return q, s


def int8_dequantize(q, s) -> np.ndarray:
    q = np.ascontiguousarray(q, np.int8)
    out = np.empty(q.size, np.float32)
    lib().orc_int8_dequantize(q, np.ascontiguousarray(s, np.uint16), q.size, out)
    return out


# --- kernels in reference order ----------------------------------------------

def quant_matvec_int4(a, packed, scales, zeros, K: int, N: int, threads: int = 1):
    a = _f32(a).ravel()
    out = np.zeros(N, np.float32)
    lib().orc_quant_matvec_int4(K, N, a, np.ascontiguousarray(packed, np.uint32),
                                np.ascontiguousarray(scales, np.uint16),
                                np.ascontiguousarray(zeros, np.uint16), out, threads)
    return out


def quant_matmul_int4(a, packed, scales, zeros, M: int, K: int, N: int,
                      threads: int = 1):
    a = _f32(a).ravel()
    out = np.zeros(M * N, np.float32)
    lib().orc_quant_matmul_int4(M, K, N, a, np.ascontiguousarray(packed, np.uint32),
                                np.ascontiguousarray(scales, np.uint16),
                                np.ascontiguousarray(zeros, np.uint16), out, threads)
    return out.reshape(M, N)


def segment_offsets(counts) -> np.ndarray:
    c = np.ascontiguousarray(counts, np.uint32)
    off = np.zeros(c.size + 1, np.uint32)
    lib().orc_segment_offsets(c.size, c, off)
    return off


def grouped_matvec(x, w, offsets, E, T, K, N, threads: int = 1, out=None):
    out = np.zeros(T * N, np.float32) if out is None else _f32(out).ravel().copy()
    lib().orc_grouped_matvec(E, T, K, N, _f32(x).ravel(), _f32(w).ravel(),
                             np.ascontiguousarray(offsets, np.uint32), out, threads)
    return out.reshape(T, N)


def grouped_matmul(x, w, offsets, E, T, K, N, threads: int = 1, out=None):
    out = np.zeros(T * N, np.float32) if out is None else _f32(out).ravel().copy()
    lib().orc_grouped_matmul(E, T, K, N, _f32(x).ravel(), _f32(w).ravel(),
                             np.ascontiguousarray(offsets, np.uint32), out, threads)
    return out.reshape(T, N)


def int4_grouped_matvec(x, packed, scales, zeros, offsets, E, T, K, N,
                        threads: int = 1, out=None):
    out = np.zeros(T * N, np.float32) if out is None else _f32(out).ravel().copy()
    lib().orc_int4_grouped_matvec(E, T, K, N, _f32(x).ravel(),
                                  np.ascontiguousarray(packed, np.uint32),
                                  np.ascontiguousarray(scales, np.uint16),
                                  np.ascontiguousarray(zeros, np.uint16),
                                  np.ascontiguousarray(offsets, np.uint32), out, threads)
    return out.reshape(T, N)


def int4_grouped_matmul(x, packed, scales, zeros, offsets, E, T, K, N,
                        threads: int = 1, out=None):
    out = np.zeros(T * N, np.float32) if out is None else _f32(out).ravel().copy()
    lib().orc_int4_grouped_matmul(E, T, K, N, _f32(x).ravel(),
                                  np.ascontiguousarray(packed, np.uint32),
                                  np.ascontiguousarray(scales, np.uint16),
                                  np.ascontiguousarray(zeros, np.uint16),
                                  np.ascontiguousarray(offsets, np.uint32), out, threads)
    return out.reshape(T, N)


# --- f64 references (no reference order; the mathematics) -------------------

def dequantized(packed, scales, zeros, n: int) -> np.ndarray:
    return int4_dequantize(packed, scales, zeros, n)


def matmul_f64(a, wdq, M: int, K: int, N: int) -> np.ndarray:
    """Exact-ish product of f32 activations and dequantized weights in f64."""
    return (np.asarray(a, np.float64).reshape(M, K) @
            np.asarray(wdq, np.float64).reshape(K, N))


# ---- decode-step neighbours -------------------------------------------------

def foreign_dequant(fmt: int, K: int, N: int, group_size: int, qweight, qzeros, scales,
                    g_idx=None) -> np.ndarray:
    """A published AWQ (fmt 1) / GPTQ (2) / GPTQ v2 (3) layer's weights,
    dequantized exactly, [K, N] f32."""
    qw = np.ascontiguousarray(qweight).view(np.uint32).reshape(-1)
    qz = np.ascontiguousarray(qzeros).view(np.uint32).reshape(-1)
    sc = np.ascontiguousarray(scales).view(np.uint16).reshape(-1)
    gi = None if g_idx is None else np.ascontiguousarray(g_idx, np.int32)
    if gi is not None:
        assert gi.size == K and gi.min() >= 0 and gi.max() < sc.size // N
    w = np.empty(K * N, np.float32)
    lib().orc_foreign_dequant(fmt, K, N, group_size, qw, qz, sc,
                              None if gi is None else gi.ctypes.data, w)
    return w.reshape(K, N)


def int4_repack(fmt: int, K: int, N: int, group_size: int, qweight, qzeros, scales,
                g_idx=None):
    """A published layer in the reference int4 format: the reference's
    Int4Quantize (quant/int4.go:71-138) of its exactly dequantized weights."""
    w = foreign_dequant(fmt, K, N, group_size, qweight, qzeros, scales, g_idx)
    return int4_quantize(w.reshape(-1))


def add_rows(x, v) -> np.ndarray:
    """ElemAdd (internal/kernels/elementwise.go:19-27) of x [rows, cols] and
    v [cols] broadcast over rows."""
    x = _f32(x)
    v = _f32(v).reshape(-1)
    cols = v.size
    rows = x.size // max(cols, 1)
    assert x.size == rows * cols
    out = np.empty_like(x)
    lib().orc_add_rows(rows, cols, x.reshape(-1), v, out.reshape(-1))
    return out


def int4_linear(x, packed, scales, zeros, bias, M: int, K: int, N: int,
                bf16_out: bool = False) -> np.ndarray:
    """The composed form of an int4 Linear, which the reference keeps as the
    fused kernel's reference (tensor/matmul.go:184-188): the int4 product in
    reference order (QuantMatVecInt4 at M = 1, QuantMatMulInt4 otherwise),
    then ElemAdd of the bias broadcast over rows when there is one, then one
    narrowing to bf16 bits (ToBFloat16) for a bf16 result.  Returns [M, N]
    f32, or u16 bf16 bits."""
    if M == 1:
        y = quant_matvec_int4(x, packed, scales, zeros, K, N).reshape(1, N)
    else:
        y = quant_matmul_int4(x, packed, scales, zeros, M, K, N)
    if bias is not None:
        y = add_rows(y, bias)
    return to_bf16(y).reshape(M, N) if bf16_out else y


def swiglu(a, b) -> np.ndarray:
    """SwiGLU (internal/kernels/elementwise.go:85-91), f32 in reference order."""
    a = _f32(a)
    b = _f32(b)
    assert a.shape == b.shape
    out = np.empty_like(a)
    lib().orc_swiglu(a.reshape(-1), b.reshape(-1), out.reshape(-1), a.size)
    return out


def rmsnorm(x, w, eps: float) -> np.ndarray:
    """RMSNorm over the last axis (internal/kernels/norm.go:47-80)."""
    x = _f32(x)
    w = _f32(w)
    width = x.shape[-1]
    assert w.shape == (width,)
    rows = x.size // width
    out = np.empty_like(x)
    lib().orc_rmsnorm(rows, width, eps, x.reshape(-1), w, out.reshape(-1))
    return out


def matvec_f32_f16(a, b_bits, K: int, N: int) -> np.ndarray:
    """MatVecF32F16 (internal/kernels/matvec.go:79-105): a f32 [K], b f16 bits
    [K, N] -> f32 [N]."""
    a = _f32(a).reshape(-1)
    b_bits = np.ascontiguousarray(b_bits, np.uint16).reshape(-1)
    assert a.size == K and b_bits.size == K * N
    out = np.empty(N, np.float32)
    lib().orc_matvec_f32_f16(K, N, a, b_bits, out)
    return out


# ---- int8 weights -------------------------------------------------------------

def quant_matvec_i8(a, quants, scales, K: int, N: int) -> np.ndarray:
    """QuantMatVecF32 (internal/kernels/matvec.go:204-235); pass f16
    activations widened to f32 for QuantMatVec."""
    a = _f32(a).reshape(-1)
    q = np.ascontiguousarray(quants, np.int8).reshape(-1)
    s = np.ascontiguousarray(scales, np.uint16)
    assert a.size == K and q.size == K * N and s.size == (K * N + 31) // 32
    out = np.empty(N, np.float32)
    lib().orc_quant_matvec_i8(K, N, a, q, s, out)
    return out


def quant_matmul_i8(a, quants, scales, M: int, K: int, N: int) -> np.ndarray:
    """QuantMatMulTiledF32 (internal/kernels/quant.go:195-238)."""
    a = _f32(a).reshape(-1)
    q = np.ascontiguousarray(quants, np.int8).reshape(-1)
    s = np.ascontiguousarray(scales, np.uint16)
    assert a.size == M * K and q.size == K * N and s.size == (K * N + 31) // 32
    out = np.empty((M, N), np.float32)
    lib().orc_quant_matmul_i8(M, K, N, a, q, s, out.reshape(-1))
    return out
