"""The C ABI on the CPU: the library loads, exports every symbol the header
declares, its host packer is bit-exact with the oracle, and the operator
layer refuses what the reference refuses (tensor/int4_test.go:121-273,
357-420; tensor/grouped_test.go:92-202,295-330) -- validation runs before
any device is touched, so none of this needs a GPU.
"""
import ctypes
import struct
import os
import re

import numpy as np
import pytest

import accel_amd
import oracle
from accel_amd import F16, F32, U32, BF16

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "accel_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(accel_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    syms = declared_symbols()
    assert len(syms) >= 30
    lib = ctypes.CDLL(accel_amd.LIB_PATH)
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(accel_amd.SIGNATURES), \
        set(syms) ^ set(accel_amd.SIGNATURES)


def test_abi_version():
    assert accel_amd.lib().accel_hip_abi_version() == 1


def test_probe_reports_a_count_without_failing():
    assert accel_amd.device_count() >= 0


@pytest.mark.parametrize("n", [1, 5, 128, 129, 1000, 4096 * 2 + 77])
@pytest.mark.parametrize("kind", ["normal", "far", "denorm", "huge", "nan_inf", "zeros"])
def test_host_packer_is_bit_exact_with_the_oracle(n, kind):
    rng = np.random.default_rng(n * 7 + len(kind))
    if kind == "normal":
        w = rng.standard_normal(n) * 0.02
    elif kind == "far":
        w = 1000 + rng.random(n)
    elif kind == "denorm":
        w = rng.standard_normal(n) * 1e-40
    elif kind == "huge":
        w = rng.standard_normal(n) * 3e38
    elif kind == "nan_inf":
        w = np.where(rng.random(n) < 0.05, np.nan,
                     np.where(rng.random(n) < 0.05, -np.inf, rng.standard_normal(n)))
    else:
        w = np.where(rng.random(n) < 0.5, -0.0, 0.0)
    w = np.asarray(w, np.float32)
    got = accel_amd.int4_quantize(w)
    want = oracle.int4_quantize(w)
    for g, x, what in zip(got, want, ("codes", "scales", "zeros")):
        assert np.array_equal(g, x), what
    back = accel_amd.int4_dequantize(*got, n)
    ref = oracle.int4_dequantize(*want, n)
    assert np.array_equal(back.view(np.uint32), ref.view(np.uint32))


def test_host_packer_at_a_baseline_shape():
    rng = np.random.Generator(np.random.PCG64(0))
    w = (rng.standard_normal((1024, 4096)) * 0.02).astype(np.float32)
    got = accel_amd.int4_quantize(w)
    want = oracle.int4_quantize(w)
    for g, x in zip(got, want):
        assert np.array_equal(g, x)


def test_kernel_support_names_the_records():
    for k in ["QuantMatVecInt4", "QuantMatMulInt4", "GroupedMatVec", "GroupedMatMul",
              "SegmentOffsets", "SwiGLU", "RMSNorm", "MatVecF32F16", "QuantMatVecF32",
              "QuantMatVec", "QuantMatMulTiledF32", "QuantMatMulTiled"]:
        assert accel_amd.supports_kernel(k)
    assert not accel_amd.supports_kernel("MatMulTiledF32")
    assert not accel_amd.supports_kernel("")


# ---- refusals ---------------------------------------------------------------
# Fake device pointers: validation never dereferences them.
FAKE = 0x1000


def t(shape, dtype, data=FAKE):
    x = accel_amd.Tensor()
    x.data = data
    x.dtype = dtype
    x.rank = len(shape)
    for i, s in enumerate(shape):
        x.shape[i] = s
    return x


def w4(weights, codes=None, scales=None, zeros=None, c=FAKE, s=FAKE, z=FAKE):
    d = accel_amd.Int4Desc()
    d.codes, d.scales, d.zeros = c, s, z
    d.codes_len = (weights + 7) // 8 if codes is None else codes
    d.scales_len = (weights + 127) // 128 if scales is None else scales
    d.zeros_len = (weights + 127) // 128 if zeros is None else zeros
    d.weights = weights
    return d


def call(fn, *args):
    lib = accel_amd.lib()
    rc = getattr(lib, fn)(0, None, *[ctypes.byref(a) if not isinstance(a, int) else a
                                     for a in args])
    return rc, accel_amd.last_error()


K, N = 128, 2


@pytest.mark.parametrize("mut,want", [
    (dict(z=None), "the zero point is what makes four bits usable"),
    (dict(s=None), "needs a code plane, a scale plane and a zero plane"),
    (dict(codes=31), "which is 32 words, and the code plane holds 31"),
    (dict(scales=3), "which is 2 groups of 128, and 3 scales"),
    (dict(zeros=1), "which is 2 groups of 128, and 1 zeros"),
])
def test_a_mismatched_triple_is_refused(mut, want):   # tensor/int4_test.go:121-172
    kw = {k: v for k, v in mut.items() if k in ("codes", "scales", "zeros")}
    ptrs = {k: v for k, v in mut.items() if k in ("c", "s", "z")}
    w = w4(K * N, **kw, **ptrs)
    rc, msg = call("accel_int4_matvec", t([K], F32), w, t([N], F32))
    assert rc == accel_amd.E_INVALID and want in msg and "Int4MatVec" in msg, msg


def test_zero_weights_are_refused():
    rc, msg = call("accel_int4_matvec", t([K], F32), w4(0, codes=0, scales=0, zeros=0),
                   t([N], F32))
    assert rc == accel_amd.E_INVALID and "declares 0 weights" in msg


@pytest.mark.parametrize("a,want", [
    (t([K], BF16), "activations are bf16 and this kernel reads f32"),
    (t([2, K], F32), "a matvec takes a vector"),
    (t([100], F32), "activations are 100 long and the matrix holds 256 weights"),
])
def test_int4_matvec_refuses_wrong_activations(a, want):   # tensor/int4_test.go:224-273
    rc, msg = call("accel_int4_matvec", a, w4(K * N), t([N], F32))
    assert rc == accel_amd.E_INVALID and want in msg, msg


def test_int4_matmul_refuses_a_vector_and_names_matvec():   # :357-385
    rc, msg = call("accel_int4_matmul", t([64], F32), w4(64 * 4), t([1, 4], F32))
    assert rc == accel_amd.E_INVALID and "Int4MatVec" in msg


@pytest.mark.parametrize("a,out,want", [
    (t([2, K], U32), t([2, N], F32), "activations are u32"),
    (t([2, 100], F32), t([2, N], F32), "100 wide and the matrix holds 256"),
    (t([2, K], F32), t([2, N + 1], F32), "the output is [2 3] and the product is [2 2]"),
    (t([2, K], F32), t([2, N], BF16), "the output is bf16 and this product writes f32"),
])
def test_int4_matmul_refusals(a, out, want):   # :387-420
    rc, msg = call("accel_int4_matmul", a, w4(K * N), out)
    assert rc == accel_amd.E_INVALID and want in msg, msg


def test_grouped_refusals():   # tensor/grouped_test.go:92-202,295-330
    x = t([6, 32], F32)
    w = t([3, 32, 4], F32)
    c = t([3], U32)
    o = t([6, 4], F32)
    rc, msg = call("accel_grouped_matvec", x, w, t([2], U32), o)
    assert rc == accel_amd.E_INVALID and "counts holds 2 entries and w has 3 experts" in msg
    rc, msg = call("accel_grouped_matvec", x, t([3, 31, 4], F32), c, o)
    assert rc == accel_amd.E_INVALID and "every expert contracts against the same width" in msg
    rc, msg = call("accel_grouped_matmul", t([6, 32], BF16), w, c, o)
    assert rc == accel_amd.E_INVALID and "x is bf16 and this kernel reads f32" in msg
    rc, msg = call("accel_grouped_matmul", x, t([32, 4], F32), c, o)
    assert rc == accel_amd.E_INVALID and "one matrix per expert" in msg
    rc, msg = call("accel_grouped_matmul", x, t([0, 32, 4], F32), t([0], U32), o)
    assert rc == accel_amd.E_INVALID and "w declares no experts" in msg
    rc, msg = call("accel_grouped_matvec", x, w, t([3], U32, data=0), o)
    assert rc == accel_amd.E_INVALID and "counts is nil" in msg


def test_int4_grouped_refuses_straddling_groups():
    lib = accel_amd.lib()
    x = t([4, 8], F32)
    w = w4(3 * 8 * 4)  # 96 weights per... K*N = 32, not a multiple of 128
    rc = lib.accel_int4_grouped_matmul(0, None, ctypes.byref(x), ctypes.byref(w), 3,
                                       ctypes.byref(t([3], U32)), ctypes.byref(t([4, 4], F32)))
    assert rc == accel_amd.E_INVALID and "straddles" in accel_amd.last_error()


def test_swiglu_refusals():   # tensor/elementwise.go:161-188; ops_test.go:563-569
    rc, msg = call("accel_swiglu", t([8], F32), t([8], F16), t([8], F32))
    assert rc == accel_amd.E_INVALID and "operands are f32 and f16" in msg, msg
    rc, msg = call("accel_swiglu", t([8], F32), t([4, 2], F32), t([8], F32))
    assert rc == accel_amd.E_INVALID and "the fused kernel indexes both operands" in msg, msg
    rc, msg = call("accel_swiglu", t([8], BF16), t([8], BF16), t([8], BF16))
    assert rc == accel_amd.E_INVALID and "reads f32" in msg, msg


def test_rmsnorm_refusals():   # tensor/ops.go:105-135; ops_test.go:448-456
    lib = accel_amd.lib()

    def rms(x, g, eps, o):
        rc = lib.accel_rmsnorm(0, None, ctypes.byref(x), ctypes.byref(g), ctypes.c_float(eps),
                               ctypes.byref(o))
        return rc, accel_amd.last_error()

    rc, msg = rms(t([4, 8], F32), t([4], F32), 1e-5, t([4, 8], F32))
    assert rc == accel_amd.E_INVALID and "the gain is one value per feature" in msg, msg
    rc, msg = rms(t([4, 8], F32), t([8], F32), 0.0, t([4, 8], F32))
    assert rc == accel_amd.E_INVALID and "must be positive and finite" in msg, msg
    rc, msg = rms(t([4, 8], F16), t([8], F16), 1e-5, t([4, 8], F16))
    assert rc == accel_amd.E_INVALID and "x is f16 and gain is f16" in msg, msg
    rc, msg = rms(t([], F32), t([1], F32), 1e-5, t([], F32))
    assert rc == accel_amd.E_INVALID and "x has no shape" in msg, msg


def test_matvec_f32_f16_refusals():   # tensor/matmul.go:45-121
    rc, msg = call("accel_matvec_f32_f16", t([16], F32), t([16, 4], F32), t([4], F32))
    assert rc == accel_amd.E_INVALID and "operands are f32 and f32" in msg, msg
    rc, msg = call("accel_matvec_f32_f16", t([15], F32), t([16, 4], F16), t([4], F32))
    assert rc == accel_amd.E_INVALID and "the inner dimensions must agree" in msg, msg
    rc, msg = call("accel_matvec_f32_f16", t([2, 16], F32), t([16, 4], F16), t([2, 4], F32))
    assert rc == accel_amd.E_UNSUPPORTED and "M = 1" in msg, msg


def test_int4_linear_refusals():   # tensor/matmul.go:189-225's checks on an int4 product
    lib = accel_amd.lib()

    def lin(x, w, b, o):
        rc = lib.accel_int4_linear(0, None, ctypes.byref(x), ctypes.byref(w),
                                   ctypes.byref(b) if b is not None else None, ctypes.byref(o))
        return rc, accel_amd.last_error()

    K, N = 256, 128
    w = w4(K * N)
    x, b, o = t([2, K], F32), t([N], F32), t([2, N], F32)
    rc, msg = lin(x, w, t([N], F16), o)
    assert rc == accel_amd.E_INVALID and "the bias is f16 and the epilogue adds in f32" in msg
    rc, msg = lin(x, w, t([N + 1], F32), o)
    assert rc == accel_amd.E_INVALID and "the bias is [129] and the output is 128 wide" in msg
    rc, msg = lin(x, w, t([1, N], F32), o)
    assert rc == accel_amd.E_INVALID and "a bias is one value per output column" in msg
    rc, msg = lin(x, w, t([N], F32, data=0), o)
    assert rc == accel_amd.E_INVALID and "passes no bias tensor" in msg
    rc, msg = lin(x, w, b, t([2, N], F16))
    assert rc == accel_amd.E_INVALID and "the epilogue writes f32 or bf16" in msg
    rc, msg = lin(t([2, K], BF16), w, b, o)
    assert rc == accel_amd.E_INVALID and "bf16 activations give a bf16 result" in msg
    rc, msg = lin(t([2, K], F16), w, b, o)
    assert rc == accel_amd.E_INVALID and "activations are f16" in msg
    rc, msg = lin(t([1, 2, K], F32), w, b, o)
    assert rc == accel_amd.E_INVALID and "one vector [K] or rows [M, K]" in msg
    rc, msg = lin(t([2, K + 1], F32), w, b, o)
    assert rc == accel_amd.E_INVALID and "a multiple of the first" in msg
    rc, msg = lin(t([K], F32), w, b, o)
    assert rc == accel_amd.E_INVALID and "the output is [2 128] and the product is [128]" in msg
    rc, msg = lin(x, w4(K * N, zeros=0), b, o)
    assert rc == accel_amd.E_INVALID and "256 groups of 128, and 0 zeros" in msg, msg
    # valid: f32 -> bf16 with a bias, vector form, and no bias at all
    assert lin(x, w, b, t([2, N], BF16))[0] == accel_amd.E_NO_DEVICE
    assert lin(t([K], F32), w, b, t([N], F32))[0] == accel_amd.E_NO_DEVICE
    assert lin(x, w, None, t([2, N], BF16))[0] == accel_amd.E_NO_DEVICE
    assert lin(t([2, K], BF16), w, b, t([2, N], BF16))[0] == accel_amd.E_NO_DEVICE


def test_int4_matvec_set_refusals():
    lib = accel_amd.lib()
    K, N = 256, 128

    def call(a, ws, outs, count):
        wd = (accel_amd.Int4Desc * max(len(ws), 1))(*ws)
        od = (accel_amd.Tensor * max(len(outs), 1))(*outs)
        rc = lib.accel_int4_matvec_set(0, None, ctypes.byref(a), wd, od, count)
        return rc, accel_amd.last_error()

    a = t([K], F32)
    rc, msg = call(a, [w4(K * N)], [t([N], F32)], 0)
    assert rc == accel_amd.E_INVALID and "a set holds one to four" in msg
    rc, msg = call(a, [w4(K * N)] * 5, [t([N], F32)] * 5, 5)
    assert rc == accel_amd.E_INVALID and "a set holds one to four" in msg
    rc, msg = call(a, [w4(K * N), w4(K * N + 8)], [t([N], F32)] * 2, 2)
    assert rc == accel_amd.E_INVALID and "Int4MatVecSet" in msg and "multiple of the first" in msg
    rc, msg = call(a, [w4(K * N), w4(K * 64)], [t([N], F32), t([N], F32)], 2)
    assert rc == accel_amd.E_INVALID and "the output is [128] and the product is [64]" in msg
    rc, msg = call(a, [w4(K * N), w4(K * 64)], [t([N], F32), t([64], F32)], 2)
    assert rc == accel_amd.E_NO_DEVICE


def test_int4_matmul_set_refusals():
    lib = accel_amd.lib()
    K, N = 256, 128

    def call(a, ws, outs, count):
        wd = (accel_amd.Int4Desc * max(len(ws), 1))(*ws)
        od = (accel_amd.Tensor * max(len(outs), 1))(*outs)
        rc = lib.accel_int4_matmul_set(0, None, ctypes.byref(a), wd, od, count)
        return rc, accel_amd.last_error()

    a = t([8, K], F32)
    rc, msg = call(a, [w4(K * N)], [t([8, N], F32)], 5)
    assert rc == accel_amd.E_INVALID and "a set holds one to four" in msg
    rc, msg = call(t([8, K], BF16), [w4(K * N)], [t([8, N], F32)], 1)
    assert rc == accel_amd.E_INVALID and "a set takes f32 rows [M, K]" in msg
    rc, msg = call(t([K], F32), [w4(K * N)], [t([N], F32)], 1)
    assert rc == accel_amd.E_INVALID and "a set takes f32 rows [M, K]" in msg
    rc, msg = call(a, [w4(K * N), w4(K * N + 8)], [t([8, N], F32)] * 2, 2)
    assert rc == accel_amd.E_INVALID and "matrix 1 holds" in msg
    rc, msg = call(a, [w4(K * N)], [t([8, N + 1], F32)], 1)
    assert rc == accel_amd.E_INVALID and "the product is [8 128]" in msg
    rc, msg = call(a, [w4(K * N), w4(K * 64)], [t([8, N], F32), t([8, 64], F32)], 2)
    assert rc == accel_amd.E_NO_DEVICE


def test_quant_matmul_refusals():   # tensor/quantized.go:32-110
    I8 = accel_amd.I8
    lib = accel_amd.lib()

    def qmm(x, q, sc, o):
        rc = lib.accel_quant_matmul(0, None, ctypes.byref(x), ctypes.byref(q), ctypes.byref(sc),
                                    ctypes.byref(o))
        return rc, accel_amd.last_error()

    x, q, sc, o = t([2, 64], F32), t([64, 8], I8), t([16], F16), t([2, 8], F32)
    rc, msg = qmm(x, t([64, 8], I8, data=0), sc, o)
    assert rc == accel_amd.E_INVALID and "needs both a quant plane and a scale plane" in msg
    rc, msg = qmm(x, t([64, 8], U32), sc, o)
    assert rc == accel_amd.E_INVALID and "quants are u32 and must be i8" in msg, msg
    rc, msg = qmm(x, q, t([15], F16), o)
    assert rc == accel_amd.E_INVALID and "512 quants, which is 16 blocks of 32, and 15" in msg
    rc, msg = qmm(t([2, 64], BF16), q, sc, o)
    assert rc == accel_amd.E_INVALID and "registers f16 and f32 activations" in msg, msg
    rc, msg = qmm(t([64], F32), q, sc, o)
    assert rc == accel_amd.E_INVALID and "v0 multiplies two matrices" in msg, msg
    rc, msg = qmm(t([2, 63], F32), t([63, 8], I8), t([17], F16), o)
    assert rc == accel_amd.E_INVALID and "504 quants, which is 16 blocks of 32, and 17" in msg, msg
    rc, msg = qmm(t([2, 32], F32), q, sc, o)
    assert rc == accel_amd.E_INVALID and "the contracted axes are 32 and 64" in msg, msg


def test_dispatch_refuses_an_unknown_record():
    lib = accel_amd.lib()
    u = (ctypes.c_char * 16)()
    rc = lib.accel_hip_dispatch(0, None, b"MatMulTiledF32", None, None, 0,
                                ctypes.cast(u, ctypes.c_void_p), 16, None)
    assert rc == accel_amd.E_UNSUPPORTED
    assert "no gfx950 implementation" in accel_amd.last_error()


def _record_cases():
    M, K, N, E, T, rows, width = 2, 256, 256, 4, 6, 3, 64
    g = struct.pack("<IIII", M, N, K, 0)
    v = struct.pack("<IIII", 0, N, K, 0)
    W = K * N
    return {
        "QuantMatVecInt4": ([K, W // 8, W // 128, W // 128, N], v),
        "QuantMatMulInt4": ([M * K, W // 8, W // 128, W // 128, M * N], g),
        "GroupedMatVec": ([T * K, E * K * N, E + 1, T * N], struct.pack("<IIII", E, K, N, 0)),
        "GroupedMatMul": ([T * K, E * K * N, E + 1, T * N], struct.pack("<IIII", E, T, K, N)),
        "SegmentOffsets": ([rows, rows + 1], struct.pack("<IIII", rows, 0, 0, 0)),
        "SwiGLU": ([77, 77, 77], b""),
        "RMSNorm": ([rows * width, width, rows * width], struct.pack("<IIfI", rows, width, 1e-5, 0)),
        "MatVecF32F16": ([K, W, N], struct.pack("<IIII", 1, N, K, 0)),
        "QuantMatVecF32": ([K, W, W // 32, N], v),
        "QuantMatVec": ([K, W, W // 32, N], v),
        "QuantMatMulTiledF32": ([M * K, W, W // 32, M * N], g),
        "QuantMatMulTiled": ([M * K, W, W // 32, M * N], g),
    }


@pytest.mark.parametrize("kernel", sorted(_record_cases()))
def test_every_record_with_full_bindings_reaches_the_device(kernel):
    # each record routes to its own operator: bindings long enough for its
    # dims pass validation and stop only at the unopened device
    lens, uniform = _record_cases()[kernel]
    lib = accel_amd.lib()
    host = (ctypes.c_uint8 * 256)()
    n = len(lens)
    b = (ctypes.c_void_p * n)(*[ctypes.addressof(host)] * n)
    ln = (ctypes.c_uint64 * n)(*lens)
    u = ctypes.create_string_buffer(uniform, max(len(uniform), 1))
    rc = lib.accel_hip_dispatch(63, None, kernel.encode(), b, ln, n,
                                ctypes.cast(u, ctypes.c_void_p) if uniform else None,
                                len(uniform), None)
    assert rc == accel_amd.E_NO_DEVICE, (kernel, rc, accel_amd.last_error())


def test_a_closed_device_is_refused():
    lib = accel_amd.lib()
    p = ctypes.c_void_p()
    assert lib.accel_hip_alloc(63, 16, ctypes.byref(p)) == accel_amd.E_NO_DEVICE
    assert lib.accel_hip_lost(63) == 0


# ---- prepared weights: refusals made before any device is touched ----------

def _fake_int4(K, N):
    n = K * N
    return accel_amd.Int4Desc(1 << 20, (n + 7) // 8, 1 << 21, (n + 127) // 128, 1 << 22,
                              (n + 127) // 128, n)


@pytest.mark.parametrize("K,N,why", [
    (256, 100, "N a multiple of 128"),
    (256, 200, "N a multiple of 128"),
])
def test_prepare_refuses_shapes_the_panels_cannot_hold(K, N, why):
    h = ctypes.c_void_p()
    d = _fake_int4(K, N)
    rc = accel_amd.lib().accel_int4_prepare(0, None, ctypes.byref(d), K, N, ctypes.byref(h))
    assert rc == accel_amd.E_INVALID
    assert why in accel_amd.last_error()
    assert h.value is None


def test_prepare_refuses_a_count_that_is_not_k_times_n():
    h = ctypes.c_void_p()
    d = _fake_int4(256, 128)
    rc = accel_amd.lib().accel_int4_prepare(0, None, ctypes.byref(d), 256, 256, ctypes.byref(h))
    assert rc == accel_amd.E_INVALID
    assert "is 65536 weights and the matrix holds 32768" in accel_amd.last_error()


def test_prepared_matvec_refuses_a_missing_weight():
    t = accel_amd.Tensor()
    rc = accel_amd.lib().accel_int4_matvec_prepared(0, None, ctypes.byref(t), None,
                                                   ctypes.byref(t))
    assert rc == accel_amd.E_INVALID
    assert "prepared weight is missing" in accel_amd.last_error()


@pytest.mark.parametrize("E,K,N,why", [
    (2, 16, 4096, "K a multiple of 32"),
    (1, 2048, 64, "N a multiple of 128"),
    (3, 256, 256, "3 experts of [256, 256] are 196608 weights and the matrix holds 131072"),
])
def test_prepare_grouped_refuses_what_the_side_copies_cannot_hold(E, K, N, why):
    h = ctypes.c_void_p()
    d = _fake_int4(256, 512)
    rc = accel_amd.lib().accel_int4_prepare_grouped(0, None, ctypes.byref(d), E, K, N,
                                                    ctypes.byref(h))
    assert rc == accel_amd.E_INVALID
    assert why in accel_amd.last_error()
    assert h.value is None


@pytest.mark.parametrize("fn", ["accel_int4_grouped_matvec_prepared",
                                "accel_int4_grouped_matmul_prepared"])
def test_grouped_prepared_refuses_a_missing_weight(fn):
    t = accel_amd.Tensor()
    rc = getattr(accel_amd.lib(), fn)(0, None, ctypes.byref(t), None, ctypes.byref(t),
                                      ctypes.byref(t))
    assert rc == accel_amd.E_INVALID
    assert "prepared weight is missing" in accel_amd.last_error()


def test_prepared_swiglu_refuses_a_missing_weight():
    t = accel_amd.Tensor()
    rc = accel_amd.lib().accel_int4_matvec_prepared_swiglu(0, None, ctypes.byref(t), None, None,
                                                          ctypes.byref(t))
    assert rc == accel_amd.E_INVALID
    assert "prepared gate weight is missing" in accel_amd.last_error()


@pytest.mark.parametrize("E,K,N,why", [
    (1, 2048, 64, "N a multiple of 128"),
    (3, 256, 256, "3 experts of [256, 256] are 196608 weights and the matrix holds 131072"),
])
def test_prepare_grouped_panels_refuses_what_the_panels_cannot_hold(E, K, N, why):
    h = ctypes.c_void_p()
    d = _fake_int4(256, 512)
    rc = accel_amd.lib().accel_int4_prepare_grouped_panels(0, None, ctypes.byref(d), E, K, N,
                                                           ctypes.byref(h))
    assert rc == accel_amd.E_INVALID
    assert why in accel_amd.last_error()
    assert h.value is None
