"""accel_amd -- Python binding of libaccel_hip.so, the gfx950 backend for
golang-design/accel's int4 weight-only linear path.

The product is the C ABI in ``include/accel_hip.h``; this module binds it
with ctypes for the tests and the benchmark.  Device memory, streams and
events are the library's own (``accel_hip_alloc`` etc.); numpy arrays are
only the host side.  Importing fails loudly when the library has not been
built: there is no other implementation to fall back to.

Names follow the reference: ``Int4MatVec`` / ``Int4MatMul``
(tensor/int4.go:99,168), ``GroupedMatVec`` / ``GroupedMatMul``
(tensor/grouped.go:48,138), ``SegmentOffsets`` (tensor/segment.go:31),
``int4_quantize`` (quant/int4.go:71).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaccel_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is not built; run `python accel_amd/build.py` (hipcc, gfx950). "
        "accel_amd has no other implementation to fall back to.")

_lib = ctypes.CDLL(LIB_PATH)

OK = 0
E_INVALID = -1
E_NO_DEVICE = -2
E_DEVICE_LOST = -3
E_OOM = -4
E_UNSUPPORTED = -5
E_HIP = -6

F32, F16, BF16, U32, I8 = 1, 2, 3, 4, 5
_NP_DTYPE = {F32: np.float32, F16: np.uint16, BF16: np.uint16, U32: np.uint32, I8: np.int8}


class AccelError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


class DeviceLost(AccelError):
    """The sticky loss of internal/driver/plan.go:385-391."""


class Refused(AccelError):
    """A refusal by the operator layer's validation (the tensor builder's b.fail)."""


class HipInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 128), ("arch", ctypes.c_char * 64),
                ("compute_units", ctypes.c_int32), ("wavefront", ctypes.c_int32),
                ("lds_per_block", ctypes.c_int32), ("clock_khz", ctypes.c_int32),
                ("mem_clock_khz", ctypes.c_int32), ("mem_bus_bits", ctypes.c_int32),
                ("hbm_bytes", ctypes.c_uint64), ("l2_bytes", ctypes.c_int32),
                ("pci_bus", ctypes.c_int32)]


class Tensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32),
                ("rank", ctypes.c_int32), ("shape", ctypes.c_int64 * 4)]


class Int4Desc(ctypes.Structure):
    _fields_ = [("codes", ctypes.c_void_p), ("codes_len", ctypes.c_int64),
                ("scales", ctypes.c_void_p), ("scales_len", ctypes.c_int64),
                ("zeros", ctypes.c_void_p), ("zeros_len", ctypes.c_int64),
                ("weights", ctypes.c_int64)]


class Int4G32Desc(ctypes.Structure):
    """accel_int4_g32_t: BASELINE config 1's literal format (32-row groups
    along K, f32 scale, no zero)."""
    _fields_ = [("codes", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("K", ctypes.c_int64), ("N", ctypes.c_int64)]


class SelectionDesc(ctypes.Structure):
    """accel_selection_t: KernelSelection{Op, Kernel, Reason, Rejected}."""
    _fields_ = [("op", ctypes.c_char * 32), ("kernel", ctypes.c_char * 320),
                ("reason", ctypes.c_char * 320), ("rejected", ctypes.c_char * 1024)]


class Selection:
    """Which kernels an int4 product became, and why (tensor/compile.go:36-42):
    ``kernel`` is the launches in order, ``rejected`` the routes turned down,
    each with its reason."""

    def __init__(self, d: SelectionDesc):
        self.op = d.op.decode()
        self.launches = [k for k in d.kernel.decode().split(" + ") if k]
        self.kernel = d.kernel.decode()
        self.reason = d.reason.decode()
        self.rejected = [r for r in d.rejected.decode().split("; ") if r]

    def __repr__(self) -> str:
        return (f"Selection(op={self.op!r}, kernel={self.kernel!r}, reason={self.reason!r}, "
                f"rejected={self.rejected!r})")


SELECT_BIAS, SELECT_BF16_OUT = 1, 2

QFMT_AWQ, QFMT_GPTQ, QFMT_GPTQ_V2 = 1, 2, 3


class ForeignDesc(ctypes.Structure):
    """accel_foreign_int4_t: a published AWQ / GPTQ layer's planes."""
    _fields_ = [("format", ctypes.c_int32), ("group_size", ctypes.c_int32),
                ("K", ctypes.c_int64), ("N", ctypes.c_int64), ("groups", ctypes.c_int64),
                ("qweight", ctypes.c_void_p), ("qzeros", ctypes.c_void_p),
                ("scales", ctypes.c_void_p), ("g_idx", ctypes.c_void_p)]


_vp = ctypes.c_void_p
_i = ctypes.c_int
_sz = ctypes.c_size_t
_P = ctypes.POINTER

# Every symbol include/accel_hip.h declares, with its argument types.
SIGNATURES = {
    "accel_hip_last_error": ([], ctypes.c_char_p),
    "accel_hip_abi_version": ([], _i),
    "accel_hip_probe": ([_P(_i)], _i),
    "accel_hip_info": ([_i, _P(HipInfo)], _i),
    "accel_hip_open": ([_i], _i),
    "accel_hip_close": ([_i], _i),
    "accel_hip_lost": ([_i], _i),
    "accel_hip_inject_loss": ([_i, ctypes.c_int64], _i),
    "accel_hip_alloc": ([_i, _sz, _P(_vp)], _i),
    "accel_hip_free": ([_i, _vp], _i),
    "accel_hip_write": ([_i, _vp, _sz, _vp, _sz], _i),
    "accel_hip_read": ([_i, _vp, _sz, _vp, _sz], _i),
    "accel_hip_copy": ([_i, _vp, _vp, _vp, _sz], _i),
    "accel_hip_stream_create": ([_i, _P(_vp)], _i),
    "accel_hip_stream_destroy": ([_i, _vp], _i),
    "accel_hip_stream_sync": ([_i, _vp], _i),
    "accel_hip_event_create": ([_i, _P(_vp)], _i),
    "accel_hip_event_destroy": ([_i, _vp], _i),
    "accel_hip_event_record": ([_i, _vp, _vp], _i),
    "accel_hip_event_query": ([_i, _vp], _i),
    "accel_hip_event_sync": ([_i, _vp], _i),
    "accel_hip_event_elapsed": ([_i, _vp, _vp, _P(ctypes.c_float)], _i),
    "accel_hip_capture_begin": ([_i, _vp], _i),
    "accel_hip_capture_end": ([_i, _vp, _P(_vp)], _i),
    "accel_hip_exec_launch": ([_i, _vp, _vp], _i),
    "accel_hip_exec_destroy": ([_i, _vp], _i),
    "accel_hip_set_wait_limit": ([_i, ctypes.c_int32], _i),
    "accel_hip_workspace_generation": ([_i, _P(ctypes.c_uint64), _P(ctypes.c_int32)], _i),
    "accel_hip_floor": ([_i, _vp, _i, _vp, _sz, _vp], _i),
    "accel_hip_supports_kernel": ([ctypes.c_char_p], _i),
    "accel_hip_dispatch": ([_i, _vp, ctypes.c_char_p, _P(_vp), _P(ctypes.c_uint64),
                            ctypes.c_int32, _vp, _sz, _P(ctypes.c_uint32)], _i),
    "accel_int4_matvec": ([_i, _vp, _P(Tensor), _P(Int4Desc), _P(Tensor)], _i),
    "accel_int4_matmul": ([_i, _vp, _P(Tensor), _P(Int4Desc), _P(Tensor)], _i),
    "accel_int4_matvec_noalloc": ([_i, _vp, _P(Tensor), _P(Int4Desc), _P(Tensor)], _i),
    "accel_int4_g32_quantize": ([_vp, ctypes.c_int64, ctypes.c_int64, _vp, _vp], _i),
    "accel_int4_g32_matvec": ([_i, _vp, _P(Tensor), _P(Int4G32Desc), _P(Tensor)], _i),
    "accel_int4_linear": ([_i, _vp, _P(Tensor), _P(Int4Desc), _P(Tensor), _P(Tensor)], _i),
    "accel_int4_select": ([_i, ctypes.c_char_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                           ctypes.c_int64, _vp, _P(Int4Desc), ctypes.c_int32,
                           _P(SelectionDesc)], _i),
    "accel_hip_last_selection": ([_i, _P(SelectionDesc)], _i),
    "accel_int4_prepare": ([_i, _vp, _P(Int4Desc), ctypes.c_int64, ctypes.c_int64, _P(_vp)], _i),
    "accel_int4_prepare_tiles": ([_i, _vp, _P(Int4Desc), ctypes.c_int64, ctypes.c_int64,
                                  _P(_vp)], _i),
    "accel_int4_prepare_grouped": ([_i, _vp, _P(Int4Desc), ctypes.c_int64, ctypes.c_int64,
                                    ctypes.c_int64, _P(_vp)], _i),
    "accel_int4_prepare_grouped_panels": ([_i, _vp, _P(Int4Desc), ctypes.c_int64,
                                           ctypes.c_int64, ctypes.c_int64, _P(_vp)], _i),
    "accel_int4_prepared_free": ([_i, _vp], _i),
    "accel_int4_prepared_bytes": ([_vp, _P(ctypes.c_uint64)], _i),
    "accel_int4_matvec_prepared": ([_i, _vp, _P(Tensor), _vp, _P(Tensor)], _i),
    "accel_int4_matvec_prepared_set": ([_i, _vp, _P(Tensor), _P(_vp), _P(Tensor), _i], _i),
    "accel_int4_matvec_prepared_swiglu": ([_i, _vp, _P(Tensor), _vp, _vp, _P(Tensor)], _i),
    "accel_int4_matmul_prepared": ([_i, _vp, _P(Tensor), _vp, _P(Tensor)], _i),
    "accel_int4_matmul_prepared_set": ([_i, _vp, _P(Tensor), _P(_vp), _P(Tensor), _i], _i),
    "accel_int4_matvec_set": ([_i, _vp, _P(Tensor), _P(Int4Desc), _P(Tensor), _i], _i),
    "accel_int4_matmul_set": ([_i, _vp, _P(Tensor), _P(Int4Desc), _P(Tensor), _i], _i),
    "accel_segment_offsets": ([_i, _vp, _P(Tensor), _P(Tensor)], _i),
    "accel_grouped_matvec": ([_i, _vp, _P(Tensor), _P(Tensor), _P(Tensor), _P(Tensor)], _i),
    "accel_grouped_matmul": ([_i, _vp, _P(Tensor), _P(Tensor), _P(Tensor), _P(Tensor)], _i),
    "accel_int4_grouped_matvec": ([_i, _vp, _P(Tensor), _P(Int4Desc), ctypes.c_int64,
                                   _P(Tensor), _P(Tensor)], _i),
    "accel_int4_grouped_matmul": ([_i, _vp, _P(Tensor), _P(Int4Desc), ctypes.c_int64,
                                   _P(Tensor), _P(Tensor)], _i),
    "accel_int4_grouped_matvec_prepared": ([_i, _vp, _P(Tensor), _vp, _P(Tensor), _P(Tensor)],
                                           _i),
    "accel_int4_grouped_matmul_prepared": ([_i, _vp, _P(Tensor), _vp, _P(Tensor), _P(Tensor)],
                                           _i),
    "accel_swiglu": ([_i, _vp, _P(Tensor), _P(Tensor), _P(Tensor)], _i),
    "accel_rmsnorm": ([_i, _vp, _P(Tensor), _P(Tensor), ctypes.c_float, _P(Tensor)], _i),
    "accel_matvec_f32_f16": ([_i, _vp, _P(Tensor), _P(Tensor), _P(Tensor)], _i),
    "accel_quant_matmul": ([_i, _vp, _P(Tensor), _P(Tensor), _P(Tensor), _P(Tensor)], _i),
    "accel_int8_quantize": ([_vp, ctypes.c_int64, _vp, _vp], _i),
    "accel_int8_dequantize": ([_vp, _vp, ctypes.c_int64, _vp], _i),
    "accel_int4_quantize": ([_vp, ctypes.c_int64, _vp, _vp, _vp], _i),
    "accel_int4_dequantize": ([_vp, _vp, _vp, ctypes.c_int64, _vp], _i),
    "accel_int4_repack_host": ([_P(ForeignDesc), _vp, _vp, _vp], _i),
    "accel_int4_repack": ([_i, _vp, _P(ForeignDesc), _P(Int4Desc)], _i),
    "accel_int4_quantize_device": ([_i, _vp, _vp, ctypes.c_int64, _vp, _vp, _vp], _i),
}

for _name, (_args, _ret) in SIGNATURES.items():
    _fn = getattr(_lib, _name)  # AttributeError here means the ABI is incomplete
    _fn.argtypes = _args
    _fn.restype = _ret


def lib():
    return _lib


def last_error() -> str:
    return (_lib.accel_hip_last_error() or b"").decode()


def _check(rc: int) -> int:
    if rc >= 0:
        return rc
    msg = last_error()
    if rc == E_DEVICE_LOST:
        raise DeviceLost(rc, msg)
    if rc == E_INVALID:
        raise Refused(rc, msg)
    raise AccelError(rc, msg)


def select(M: int, K: int, N: int, dtype: int = None, a: int = None, codes: int = None,
           op: str = None, flags: int = 0, dev: int = -1) -> Selection:
    """The kernels an int4 product would become (accel_int4_select), planned
    without running: dev < 0 plans for the modelled MI355X (no GPU needed).
    ``a`` and ``codes`` are addresses whose alignment matters (None: aligned)."""
    dtype = F32 if dtype is None else dtype
    desc = SelectionDesc()
    w = Int4Desc(codes or 0, 0, 0, 0, 0, 0, int(K) * int(N))
    _check(_lib.accel_int4_select(int(dev), op.encode() if op else None, int(dtype), int(M),
                                  int(K), int(N), a, ctypes.byref(w), int(flags),
                                  ctypes.byref(desc)))
    return Selection(desc)


def device_count() -> int:
    n = ctypes.c_int(0)
    _check(_lib.accel_hip_probe(ctypes.byref(n)))
    return n.value


# ---- host-side quantisation (quant/int4.go) --------------------------------

def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def int4_quantize(w: np.ndarray):
    """quant.Int4Quantize on host memory: (packed u32, scales f16 bits, zeros f16 bits)."""
    w = np.ascontiguousarray(w, np.float32).ravel()
    n = w.size
    packed = np.zeros((n + 7) // 8, np.uint32)
    scales = np.zeros((n + 127) // 128, np.uint16)
    zeros = np.zeros((n + 127) // 128, np.uint16)
    if n:
        _check(_lib.accel_int4_quantize(_ptr(w), n, _ptr(packed), _ptr(scales), _ptr(zeros)))
    return packed, scales, zeros


def int4_g32_quantize(w: np.ndarray):
    """BASELINE config 1's literal format on host memory: w f32 [K, N] ->
    (packed u32 [K*N/8], scales f32 [K/32, N])."""
    w = np.ascontiguousarray(w, np.float32)
    K, N = w.shape
    packed = np.zeros(K * N // 8, np.uint32)
    scales = np.zeros((K // 32, N), np.float32)
    _check(_lib.accel_int4_g32_quantize(_ptr(w), K, N, _ptr(packed), _ptr(scales)))
    return packed, scales


def int8_quantize(w: np.ndarray):
    """quant.Int8Quantize through the library's host packer: (quants i8,
    scales f16 bits)."""
    w = np.ascontiguousarray(w, np.float32).reshape(-1)
    n = w.size
    q = np.zeros(n, np.int8)
    s = np.zeros((n + 31) // 32, np.uint16)
    _check(_lib.accel_int8_quantize(_ptr(w), n, _ptr(q), _ptr(s)))
    return q, s


def int8_dequantize(quants, scales) -> np.ndarray:
    q = np.ascontiguousarray(quants, np.int8).reshape(-1)
    s = np.ascontiguousarray(scales, np.uint16)
    out = np.empty(q.size, np.float32)
    _check(_lib.accel_int8_dequantize(_ptr(q), _ptr(s), q.size, _ptr(out)))
    return out


@dataclass
class ForeignInt4:
    """A published 4-bit layer (AWQ or GPTQ) as host arrays: qweight and qzeros
    u32 words, scales f16 bits [groups, N], g_idx int32 [K] or None."""
    format: int
    group_size: int
    K: int
    N: int
    qweight: np.ndarray
    qzeros: np.ndarray
    scales: np.ndarray
    g_idx: np.ndarray = None

    def __post_init__(self):
        self.qweight = np.ascontiguousarray(self.qweight).view(np.uint32)
        self.qzeros = np.ascontiguousarray(self.qzeros).view(np.uint32)
        self.scales = np.ascontiguousarray(self.scales).view(np.uint16)
        if self.g_idx is not None:
            self.g_idx = np.ascontiguousarray(self.g_idx, np.int32)

    def check_lengths(self) -> None:
        """Raises ValueError unless the planes hold what a K x N layer with
        this group size needs.  The repack (host and device) indexes the planes
        from K, N and the group count alone, so this runs before any pointer
        to them crosses the ABI."""
        K, N, G = int(self.K), int(self.N), int(self.group_size)
        if K <= 0 or N <= 0 or G <= 0:
            raise ValueError(f"layer dims K={K} N={N} group_size={G} must be positive")
        if N % 8 or (self.format != QFMT_AWQ and K % 8):
            raise ValueError(f"layer dims K={K} N={N} do not pack eight codes a word")
        groups = -(-K // G)
        want = {"qweight": K * N // 8, "qzeros": groups * N // 8, "scales": groups * N}
        for name, n in want.items():
            got = getattr(self, name).size
            if got != n:
                raise ValueError(f"{name} holds {got} elements; a {K}x{N} layer with "
                                 f"{G}-row groups needs {n}")
        if self.g_idx is not None and self.g_idx.size != K:
            raise ValueError(f"g_idx holds {self.g_idx.size} entries; the layer has {K} rows")

    @property
    def groups(self) -> int:
        return self.scales.size // self.N if self.N else 0

    def desc(self, qweight=None, qzeros=None, scales=None, g_idx=None) -> ForeignDesc:
        """The C descriptor over the host arrays, or over the given pointers."""
        d = ForeignDesc()
        d.format, d.group_size = self.format, self.group_size
        d.K, d.N, d.groups = self.K, self.N, self.groups
        d.qweight = qweight if qweight is not None else self.qweight.ctypes.data
        d.qzeros = qzeros if qzeros is not None else self.qzeros.ctypes.data
        d.scales = scales if scales is not None else self.scales.ctypes.data
        if g_idx is not None:
            d.g_idx = g_idx
        elif self.g_idx is not None:
            d.g_idx = self.g_idx.ctypes.data
        return d


def int4_repack_host(layer: ForeignInt4):
    """A published layer in the reference int4 format, on the host: (codes,
    scales, zeros) over its K*N weights."""
    layer.check_lengths()
    n = layer.K * layer.N
    codes = np.zeros((n + 7) // 8, np.uint32)
    scales = np.zeros((n + 127) // 128, np.uint16)
    zeros = np.zeros((n + 127) // 128, np.uint16)
    d = layer.desc()
    _check(_lib.accel_int4_repack_host(ctypes.byref(d), _ptr(codes), _ptr(scales), _ptr(zeros)))
    return codes, scales, zeros


def int4_dequantize(packed, scales, zeros, n: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint32)
    scales = np.ascontiguousarray(scales, np.uint16)
    zeros = np.ascontiguousarray(zeros, np.uint16)
    out = np.zeros(n, np.float32)
    if n:
        _check(_lib.accel_int4_dequantize(_ptr(packed), _ptr(scales), _ptr(zeros), n,
                                          _ptr(out)))
    return out


# ---- device objects ---------------------------------------------------------

@dataclass
class Buffer:
    """One device allocation with a dtype code and a shape (row-major)."""
    device: "Device"
    ptr: int
    nbytes: int
    dtype: int
    shape: tuple

    def tensor(self, shape=None, dtype=None) -> Tensor:
        shape = tuple(self.shape if shape is None else shape)
        t = Tensor()
        t.data = self.ptr
        t.dtype = self.dtype if dtype is None else dtype
        t.rank = len(shape)
        for i, s in enumerate(shape):
            t.shape[i] = int(s)
        return t

    def numpy(self) -> np.ndarray:
        host = np.empty(self.shape, _NP_DTYPE[self.dtype])
        if self.nbytes:
            _check(_lib.accel_hip_read(self.device.index, self.ptr, 0, _ptr(host),
                                       host.nbytes))
        return host

    def write(self, host: np.ndarray) -> None:
        host = np.ascontiguousarray(host)
        if host.nbytes > self.nbytes:
            raise ValueError("host array is larger than the buffer")
        if host.nbytes:
            _check(_lib.accel_hip_write(self.device.index, self.ptr, 0, _ptr(host),
                                        host.nbytes))

    def free(self) -> None:
        if self.ptr:
            _lib.accel_hip_free(self.device.index, self.ptr)
            self.ptr = 0


class PreparedInt4:
    """An Int4 weight bound for one-row products (accel_int4_prepare): the
    library's K-major panel copy of its planes, K x N."""

    def __init__(self, device: "Device", handle: int, K: int, N: int):
        self.device, self.handle, self.K, self.N = device, handle, K, N

    @property
    def nbytes(self) -> int:
        n = ctypes.c_uint64()
        _check(_lib.accel_int4_prepared_bytes(self.handle, ctypes.byref(n)))
        return n.value

    def free(self) -> None:
        if self.handle:
            _check(_lib.accel_int4_prepared_free(self.device.index, self.handle))
            self.handle = None


@dataclass
class Int4Weights:
    """tensor.Int4 on the device: codes, scales, zeros and the weight count."""
    codes: Buffer
    scales: Buffer
    zeros: Buffer
    weights: int

    def desc(self) -> Int4Desc:
        d = Int4Desc()
        d.codes = self.codes.ptr if self.codes else None
        d.codes_len = self.codes.shape[0] if self.codes else 0
        d.scales = self.scales.ptr if self.scales else None
        d.scales_len = self.scales.shape[0] if self.scales else 0
        d.zeros = self.zeros.ptr if self.zeros else None
        d.zeros_len = self.zeros.shape[0] if self.zeros else 0
        d.weights = self.weights
        return d

    def free(self) -> None:
        for b in (self.codes, self.scales, self.zeros):
            if b:
                b.free()


class Device:
    """An opened HIP device (accel_hip_open)."""

    def __init__(self, index: int = 0):
        self.index = index
        _check(_lib.accel_hip_open(index))

    def info(self) -> HipInfo:
        info = HipInfo()
        _check(_lib.accel_hip_info(self.index, ctypes.byref(info)))
        return info

    def close(self) -> None:
        _check(_lib.accel_hip_close(self.index))

    @property
    def lost(self) -> bool:
        return bool(_lib.accel_hip_lost(self.index))

    def inject_loss(self, at_submission: int) -> None:
        _check(_lib.accel_hip_inject_loss(self.index, at_submission))

    def set_wait_limit(self, spins: int) -> None:
        """Spins a split-K hand-off's bounded wait may take before it gives up
        and reports the fault (a test hook)."""
        _check(_lib.accel_hip_set_wait_limit(self.index, spins))

    def floor(self, kind: int, src, nbytes: int, sink, stream=None) -> None:
        """A launch-floor probe: kind 0 an empty kernel, kind 1 a pure read of
        nbytes from src, both with the M = 1 decode kernel's launch shape."""
        _check(_lib.accel_hip_floor(self.index, stream, kind, src.ptr if src else None, nbytes,
                                    sink.ptr))

    def last_selection(self) -> Selection:
        """What the last int4 product on this device became
        (accel_hip_last_selection)."""
        desc = SelectionDesc()
        _check(_lib.accel_hip_last_selection(self.index, ctypes.byref(desc)))
        return Selection(desc)

    def workspace_generation(self):
        """(allocations of the workspace so far, replaced workspaces still held
        by live executables)."""
        g, r = ctypes.c_uint64(), ctypes.c_int32()
        _check(_lib.accel_hip_workspace_generation(self.index, ctypes.byref(g), ctypes.byref(r)))
        return g.value, r.value

    # memory
    def alloc(self, shape, dtype: int) -> Buffer:
        shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) \
            else tuple(int(s) for s in shape)
        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(_NP_DTYPE[dtype]).itemsize
        p = ctypes.c_void_p()
        _check(_lib.accel_hip_alloc(self.index, max(nbytes, 1), ctypes.byref(p)))
        return Buffer(self, p.value, nbytes, dtype, shape)

    def upload(self, host: np.ndarray, dtype: int = None) -> Buffer:
        host = np.ascontiguousarray(host)
        if dtype is None:
            dtype = {np.dtype(np.float32): F32, np.dtype(np.uint32): U32,
                     np.dtype(np.uint16): F16, np.dtype(np.int8): I8}[host.dtype]
        buf = self.alloc(host.shape if host.shape else (1,), dtype)
        buf.write(host)
        return buf

    def upload_int4(self, packed, scales, zeros, weights: int) -> Int4Weights:
        return Int4Weights(self.upload(np.asarray(packed, np.uint32), U32),
                           self.upload(np.asarray(scales, np.uint16), F16),
                           self.upload(np.asarray(zeros, np.uint16), F16), int(weights))

    # streams and events
    def stream(self) -> int:
        s = ctypes.c_void_p()
        _check(_lib.accel_hip_stream_create(self.index, ctypes.byref(s)))
        return s.value

    def destroy_stream(self, s) -> None:
        _check(_lib.accel_hip_stream_destroy(self.index, s))

    def sync(self, stream=None) -> None:
        _check(_lib.accel_hip_stream_sync(self.index, stream))

    def event(self) -> int:
        e = ctypes.c_void_p()
        _check(_lib.accel_hip_event_create(self.index, ctypes.byref(e)))
        return e.value

    def record(self, event, stream=None) -> None:
        _check(_lib.accel_hip_event_record(self.index, event, stream))

    def event_done(self, event) -> bool:
        return _check(_lib.accel_hip_event_query(self.index, event)) == 1

    def wait(self, event) -> None:
        _check(_lib.accel_hip_event_sync(self.index, event))

    def elapsed_ms(self, start, end) -> float:
        ms = ctypes.c_float()
        _check(_lib.accel_hip_event_elapsed(self.index, start, end, ctypes.byref(ms)))
        return ms.value

    def destroy_event(self, e) -> None:
        _check(_lib.accel_hip_event_destroy(self.index, e))

    # graphs: the resubmittable executable
    def capture_begin(self, stream) -> None:
        _check(_lib.accel_hip_capture_begin(self.index, stream))

    def capture_end(self, stream) -> int:
        e = ctypes.c_void_p()
        _check(_lib.accel_hip_capture_end(self.index, stream, ctypes.byref(e)))
        return e.value

    def launch(self, exec_, stream=None) -> None:
        _check(_lib.accel_hip_exec_launch(self.index, exec_, stream))

    def destroy_exec(self, exec_) -> None:
        _check(_lib.accel_hip_exec_destroy(self.index, exec_))

    # ---- operators ----------------------------------------------------------
    def Int4MatVec(self, a: Buffer, w: Int4Weights, out: Buffer, stream=None) -> None:
        ta, tw, to = a.tensor(), w.desc(), out.tensor()
        _check(_lib.accel_int4_matvec(self.index, stream, ctypes.byref(ta), ctypes.byref(tw),
                                      ctypes.byref(to)))

    def prepare_int4(self, w: "Int4Weights", K: int, N: int, stream=None,
                     tiles: bool = False) -> PreparedInt4:
        """Binds w once, on the device, waited for: a panel copy of its planes
        for one- and few-row products (accel_int4_prepare), or with tiles=True
        the codes and a side copy of the scales and zeros for the matrix-core
        decode (accel_int4_prepare_tiles)."""
        h = ctypes.c_void_p()
        tw = w.desc()
        fn = _lib.accel_int4_prepare_tiles if tiles else _lib.accel_int4_prepare
        _check(fn(self.index, stream, ctypes.byref(tw), int(K), int(N), ctypes.byref(h)))
        return PreparedInt4(self, h.value, int(K), int(N))

    def prepare_int4_grouped(self, w: "Int4Weights", experts: int, K: int, N: int,
                             stream=None, panels: bool = False) -> PreparedInt4:
        """Binds `experts` stacked [K, N] int4 matrices once, on the device,
        waited for: the planes and each expert's side copy of its scales and
        zeros for the matrix-core decode (accel_int4_prepare_grouped), or with
        panels=True each expert's panel-layout copy for few routed rows
        (accel_int4_prepare_grouped_panels)."""
        h = ctypes.c_void_p()
        tw = w.desc()
        fn = (_lib.accel_int4_prepare_grouped_panels if panels
              else _lib.accel_int4_prepare_grouped)
        _check(fn(self.index, stream, ctypes.byref(tw), int(experts), int(K), int(N),
                  ctypes.byref(h)))
        return PreparedInt4(self, h.value, int(K), int(N))

    def Int4MatVecPrepared(self, a: Buffer, w: PreparedInt4, out: Buffer, stream=None) -> None:
        ta, to = a.tensor(), out.tensor()
        _check(_lib.accel_int4_matvec_prepared(self.index, stream, ctypes.byref(ta), w.handle,
                                               ctypes.byref(to)))

    def Int4MatVecPreparedSet(self, a: Buffer, ws, outs, stream=None) -> None:
        """Int4MatVecPrepared of each of ws (1..4 prepared weights sharing the
        input vector a) into outs, in one launch."""
        n = len(ws)
        hs = (ctypes.c_void_p * max(n, 1))(*[w.handle for w in ws])
        outt = (Tensor * max(n, 1))(*[o.tensor() for o in outs])
        ta = a.tensor()
        _check(_lib.accel_int4_matvec_prepared_set(self.index, stream, ctypes.byref(ta), hs,
                                                   outt, n))

    def Int4MatVecPreparedSwiGLU(self, a: Buffer, gate: PreparedInt4, up: PreparedInt4,
                                 out: Buffer, stream=None) -> None:
        """out = SwiGLU(a . gate, a . up) for two panel-prepared weights, one
        launch (Int4MatVecPreparedSet of {gate, up} then SwiGLU, bit for bit)."""
        ta, to = a.tensor(), out.tensor()
        _check(_lib.accel_int4_matvec_prepared_swiglu(self.index, stream, ctypes.byref(ta),
                                                      gate.handle, up.handle, ctypes.byref(to)))

    def Int4MatMulPrepared(self, a: Buffer, w: PreparedInt4, out: Buffer, stream=None) -> None:
        """Int4MatMul of a ([M, K] f32) and a prepared weight into out ([M, N])."""
        ta, to = a.tensor(), out.tensor()
        _check(_lib.accel_int4_matmul_prepared(self.index, stream, ctypes.byref(ta), w.handle,
                                               ctypes.byref(to)))

    def Int4MatMulPreparedSet(self, a: Buffer, ws, outs, stream=None) -> None:
        """Int4MatMulPrepared of each of ws (1..4 prepared weights sharing the
        input rows a) into outs, in one launch a pass of eight rows."""
        n = len(ws)
        hs = (ctypes.c_void_p * max(n, 1))(*[w.handle for w in ws])
        outt = (Tensor * max(n, 1))(*[o.tensor() for o in outs])
        ta = a.tensor()
        _check(_lib.accel_int4_matmul_prepared_set(self.index, stream, ctypes.byref(ta), hs,
                                                   outt, n))

    def Int4MatVecNoAlloc(self, a: Buffer, w: Int4Weights, out: Buffer, stream=None) -> None:
        """Int4MatVec with its split-K buffers in the library's static scratch
        (allocates nothing; calls that overlap on one GPU race)."""
        ta, tw, to = a.tensor(), w.desc(), out.tensor()
        _check(_lib.accel_int4_matvec_noalloc(self.index, stream, ctypes.byref(ta),
                                              ctypes.byref(tw), ctypes.byref(to)))

    def Int4G32MatVec(self, a: Buffer, codes: Buffer, scales: Buffer, K: int, N: int,
                      out: Buffer, stream=None) -> None:
        """BASELINE config 1's literal format: out[N] = a[K] @ ((q - 8) * s),
        32-row groups along K with an f32 scale (no counterpart in the
        reference).  The C struct carries no plane lengths, so the buffers
        are checked against K and N here: undersized planes would be read
        past their end on the device."""
        K, N = int(K), int(N)
        if K <= 0 or N <= 0:
            raise ValueError(f"Int4G32MatVec: K={K} and N={N} must be positive")
        need = {"codes": (codes, K * N // 2), "scales": (scales, (K // 32) * N * 4)}
        for name, (buf, nbytes) in need.items():
            if buf.nbytes < nbytes:
                raise ValueError(f"Int4G32MatVec: the {name} buffer holds {buf.nbytes} bytes "
                                 f"and [{K}, {N}] needs {nbytes}")
        if a.nbytes < K * 4:
            raise ValueError(f"Int4G32MatVec: the activations hold {a.nbytes} bytes and "
                             f"K={K} needs {K * 4}")
        if out.nbytes < N * 4:
            raise ValueError(f"Int4G32MatVec: the output holds {out.nbytes} bytes and "
                             f"N={N} needs {N * 4}")
        ta, to = a.tensor(), out.tensor()
        tw = Int4G32Desc(codes.ptr, scales.ptr, K, N)
        _check(_lib.accel_int4_g32_matvec(self.index, stream, ctypes.byref(ta),
                                          ctypes.byref(tw), ctypes.byref(to)))

    def Int4MatMul(self, a: Buffer, w: Int4Weights, out: Buffer, stream=None) -> None:
        ta, tw, to = a.tensor(), w.desc(), out.tensor()
        _check(_lib.accel_int4_matmul(self.index, stream, ctypes.byref(ta), ctypes.byref(tw),
                                      ctypes.byref(to)))

    def Int4MatVecSet(self, a: Buffer, ws, outs, stream=None) -> None:
        """Int4MatVec of each of ws (1..4 matrices sharing the input vector a)
        into outs, in one launch where the decode kernel takes them all."""
        n = len(ws)
        descs = (Int4Desc * max(n, 1))(*[w.desc() for w in ws])
        outt = (Tensor * max(n, 1))(*[o.tensor() for o in outs])
        ta = a.tensor()
        _check(_lib.accel_int4_matvec_set(self.index, stream, ctypes.byref(ta), descs, outt, n))

    def Int4MatMulSet(self, a: Buffer, ws, outs, stream=None) -> None:
        """Int4MatMul of f32 rows a [M, K] against each of ws (1..4 matrices)
        into outs, one launch per tile width where the decode kernels take them."""
        n = len(ws)
        descs = (Int4Desc * max(n, 1))(*[w.desc() for w in ws])
        outt = (Tensor * max(n, 1))(*[o.tensor() for o in outs])
        ta = a.tensor()
        _check(_lib.accel_int4_matmul_set(self.index, stream, ctypes.byref(ta), descs, outt, n))

    def Int4Linear(self, x: Buffer, w: Int4Weights, bias, out: Buffer, stream=None) -> None:
        """The int4 analogue of tensor.Linear (tensor/matmul.go:184-225): the
        product plus a per-column f32 bias (or None) in one kernel; out is f32
        or bf16."""
        tx, tw, to = x.tensor(), w.desc(), out.tensor()
        tb = ctypes.byref(bias.tensor()) if bias is not None else None
        _check(_lib.accel_int4_linear(self.index, stream, ctypes.byref(tx), ctypes.byref(tw),
                                      tb, ctypes.byref(to)))

    def Int4Repack(self, layer: ForeignInt4, stream=None) -> Int4Weights:
        """A published AWQ / GPTQ layer, uploaded and repacked on the device into
        the reference int4 format; the published planes are freed after."""
        layer.check_lengths()
        n = layer.K * layer.N
        up = [self.upload(layer.qweight, U32), self.upload(layer.qzeros, U32),
              self.upload(layer.scales, F16)]
        gi = self.upload(layer.g_idx.view(np.uint32), U32) if layer.g_idx is not None else None
        w = Int4Weights(self.alloc(((n + 7) // 8,), U32), self.alloc(((n + 127) // 128,), F16),
                        self.alloc(((n + 127) // 128,), F16), n)
        d = layer.desc(up[0].ptr, up[1].ptr, up[2].ptr, gi.ptr if gi is not None else None)
        tw = w.desc()
        try:
            _check(_lib.accel_int4_repack(self.index, stream, ctypes.byref(d), ctypes.byref(tw)))
        except Exception:
            w.free()
            raise
        finally:
            for b in up + ([gi] if gi is not None else []):
                b.free()
        return w

    def SegmentOffsets(self, counts: Buffer, offsets: Buffer, stream=None) -> None:
        tc, to = counts.tensor(), offsets.tensor()
        _check(_lib.accel_segment_offsets(self.index, stream, ctypes.byref(tc),
                                          ctypes.byref(to)))

    def GroupedMatVec(self, x: Buffer, w: Buffer, counts: Buffer, out: Buffer,
                      stream=None) -> None:
        tx, tw, tc, to = x.tensor(), w.tensor(), counts.tensor(), out.tensor()
        _check(_lib.accel_grouped_matvec(self.index, stream, ctypes.byref(tx), ctypes.byref(tw),
                                         ctypes.byref(tc), ctypes.byref(to)))

    def GroupedMatMul(self, x: Buffer, w: Buffer, counts: Buffer, out: Buffer,
                      stream=None) -> None:
        tx, tw, tc, to = x.tensor(), w.tensor(), counts.tensor(), out.tensor()
        _check(_lib.accel_grouped_matmul(self.index, stream, ctypes.byref(tx), ctypes.byref(tw),
                                         ctypes.byref(tc), ctypes.byref(to)))

    def Int4GroupedMatVec(self, x: Buffer, w: Int4Weights, experts: int, counts: Buffer,
                          out: Buffer, stream=None) -> None:
        tx, tw, tc, to = x.tensor(), w.desc(), counts.tensor(), out.tensor()
        _check(_lib.accel_int4_grouped_matvec(self.index, stream, ctypes.byref(tx),
                                              ctypes.byref(tw), experts, ctypes.byref(tc),
                                              ctypes.byref(to)))

    def Int4GroupedMatMul(self, x: Buffer, w: Int4Weights, experts: int, counts: Buffer,
                          out: Buffer, stream=None) -> None:
        tx, tw, tc, to = x.tensor(), w.desc(), counts.tensor(), out.tensor()
        _check(_lib.accel_int4_grouped_matmul(self.index, stream, ctypes.byref(tx),
                                              ctypes.byref(tw), experts, ctypes.byref(tc),
                                              ctypes.byref(to)))

    def Int4GroupedMatVecPrepared(self, x: Buffer, w: PreparedInt4, counts: Buffer, out: Buffer,
                                  stream=None) -> None:
        """Int4GroupedMatVec over experts bound by prepare_int4_grouped."""
        tx, tc, to = x.tensor(), counts.tensor(), out.tensor()
        _check(_lib.accel_int4_grouped_matvec_prepared(self.index, stream, ctypes.byref(tx),
                                                       w.handle, ctypes.byref(tc),
                                                       ctypes.byref(to)))

    def Int4GroupedMatMulPrepared(self, x: Buffer, w: PreparedInt4, counts: Buffer, out: Buffer,
                                  stream=None) -> None:
        """Int4GroupedMatMul over experts bound by prepare_int4_grouped."""
        tx, tc, to = x.tensor(), counts.tensor(), out.tensor()
        _check(_lib.accel_int4_grouped_matmul_prepared(self.index, stream, ctypes.byref(tx),
                                                       w.handle, ctypes.byref(tc),
                                                       ctypes.byref(to)))

    def SwiGLU(self, gate: Buffer, value: Buffer, out: Buffer, stream=None) -> None:
        """tensor.SwiGLU (tensor/elementwise.go:161-188)."""
        tg, tv, to = gate.tensor(), value.tensor(), out.tensor()
        _check(_lib.accel_swiglu(self.index, stream, ctypes.byref(tg), ctypes.byref(tv),
                                 ctypes.byref(to)))

    def RMSNorm(self, x: Buffer, gain: Buffer, eps: float, out: Buffer, stream=None) -> None:
        """tensor.RMSNorm (tensor/ops.go:105-135)."""
        tx, tg, to = x.tensor(), gain.tensor(), out.tensor()
        _check(_lib.accel_rmsnorm(self.index, stream, ctypes.byref(tx), ctypes.byref(tg),
                                  ctypes.c_float(eps), ctypes.byref(to)))

    def QuantMatMul(self, x: Buffer, quants: Buffer, scales: Buffer, out: Buffer,
                    stream=None) -> None:
        """tensor.QuantMatMul (tensor/quantized.go:72-163): int8 weights."""
        tx, tq, ts, to = x.tensor(), quants.tensor(), scales.tensor(), out.tensor()
        _check(_lib.accel_quant_matmul(self.index, stream, ctypes.byref(tx), ctypes.byref(tq),
                                       ctypes.byref(ts), ctypes.byref(to)))

    def MatVecF32F16(self, x: Buffer, w: Buffer, out: Buffer, stream=None) -> None:
        """tensor.MatMul's M = 1 selection for f32 x and f16 w (MatVecF32F16,
        tensor/matmul.go:113-121)."""
        tx, tw, to = x.tensor(), w.tensor(), out.tensor()
        _check(_lib.accel_matvec_f32_f16(self.index, stream, ctypes.byref(tx), ctypes.byref(tw),
                                         ctypes.byref(to)))

    def int4_quantize(self, w: Buffer, n: int, packed: Buffer, scales: Buffer, zeros: Buffer,
                      stream=None) -> None:
        _check(_lib.accel_int4_quantize_device(self.index, stream, w.ptr, n, packed.ptr,
                                               scales.ptr, zeros.ptr))

    def dispatch(self, kernel: str, bindings, lens, uniform: bytes, count=(1, 1, 1),
                 stream=None) -> None:
        """One kernel-record dispatch through the backend seam."""
        n = len(bindings)
        b = (ctypes.c_void_p * n)(*[x.ptr if isinstance(x, Buffer) else x for x in bindings])
        ln = (ctypes.c_uint64 * n)(*lens)
        u = ctypes.create_string_buffer(uniform, len(uniform))
        c = (ctypes.c_uint32 * 3)(*count)
        _check(_lib.accel_hip_dispatch(self.index, stream, kernel.encode(), b, ln, n,
                                       ctypes.cast(u, ctypes.c_void_p), len(uniform), c))


def supports_kernel(name: str) -> bool:
    return bool(_lib.accel_hip_supports_kernel(name.encode()))
