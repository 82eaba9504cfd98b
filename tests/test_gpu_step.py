"""Decode-step neighbours on the GPU through the C ABI: SwiGLU, RMSNorm and
MatVecF32F16 against the oracle.

SwiGLU and RMSNorm keep the reference's evaluation order (f64 exponential and
reciprocal square root rounded to f32; the 128-lane strided fold and halving
tree), so they are compared bit for bit; the one allowance is that SwiGLU's
f64 exponential may differ from the host's by an ulp of f64, which can move
an f32 rounding in a vanishing fraction of elements (at most 1e-5 of them,
by one f32 ulp).  MatVecF32F16 sums in its own order: rel-L2 <= 1e-5.
"""
import struct

import numpy as np
import pytest

import oracle
from accel_amd import F16, F32
from conftest import rel_l2

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


def _ulps(got, want):
    g = got.view(np.int32).astype(np.int64)
    w = want.view(np.int32).astype(np.int64)
    return np.abs(g - w)


@pytest.mark.parametrize("n", [1, 7, 64, 4099, 14336 * 8, 1 << 20])
def test_swiglu_matches_the_oracle(dev, n):
    rng = np.random.default_rng(n)
    a = (rng.standard_normal(n) * 5).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    a[: min(n, 4)] = np.array([0.0, 100.0, -100.0, -0.0], np.float32)[: min(n, 4)]
    want = oracle.swiglu(a, b)
    ab, bb = dev.upload(a), dev.upload(b)
    ob = dev.alloc((n,), F32)
    dev.SwiGLU(ab, bb, ob)
    got = ob.numpy()
    d = _ulps(got, want)
    assert d.max() <= 1 and np.count_nonzero(d) <= max(1, n // 100000), (d.max(), np.count_nonzero(d))
    for x in (ab, bb, ob):
        x.free()


def test_swiglu_unaligned_buffers(dev):
    # a sub-buffer one element in: the four-wide path is off
    n = 1001
    rng = np.random.default_rng(3)
    a = rng.standard_normal(n + 1).astype(np.float32)
    b = rng.standard_normal(n + 1).astype(np.float32)
    ab, bb = dev.upload(a), dev.upload(b)
    ob = dev.alloc((n + 1,), F32)
    import accel_amd
    import ctypes
    ta, tb, to = ab.tensor(), bb.tensor(), ob.tensor()
    for tt in (ta, tb, to):
        tt.data += 4
        tt.shape[0] = n
    rc = accel_amd.lib().accel_swiglu(0, None, ctypes.byref(ta), ctypes.byref(tb),
                                      ctypes.byref(to))
    assert rc == 0, accel_amd.last_error()
    got = ob.numpy()[1:]
    want = oracle.swiglu(a[1:], b[1:])
    assert _ulps(got, want).max() <= 1
    for x in (ab, bb, ob):
        x.free()


@pytest.mark.parametrize("rows,width", [(3, 1), (3, 63), (3, 128), (3, 129), (3, 500),
                                        (3, 1024), (1, 4096), (8, 4096), (2, 14336),
                                        (33, 300)])
def test_rmsnorm_is_bit_exact(dev, rows, width):
    rng = np.random.default_rng(rows * 7 + width)
    x = (rng.standard_normal((rows, width)) * np.exp2(rng.integers(-6, 6, (rows, width)))
         ).astype(np.float32)
    w = (rng.standard_normal(width) + 1.5).astype(np.float32)
    want = oracle.rmsnorm(x, w, 1e-5)
    xb, wb = dev.upload(x), dev.upload(w)
    ob = dev.alloc((rows, width), F32)
    dev.RMSNorm(xb, wb, 1e-5, ob)
    got = ob.numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for t in (xb, wb, ob):
        t.free()


def test_rmsnorm_zero_row(dev):
    x = np.zeros((2, 64), np.float32)
    x[1] = 1.0
    w = np.ones(64, np.float32)
    xb, wb = dev.upload(x), dev.upload(w)
    ob = dev.alloc((2, 64), F32)
    dev.RMSNorm(xb, wb, 1e-5, ob)
    got = ob.numpy()
    assert np.all(got[0] == 0)
    assert np.array_equal(got, oracle.rmsnorm(x, w, 1e-5))
    for t in (xb, wb, ob):
        t.free()


@pytest.mark.parametrize("K,N", [(40, 12), (17, 33), (1000, 384), (4096, 4096),
                                 (4096, 14336), (14336, 4096), (300, 256), (96, 128)])
def test_matvec_f32_f16_matches_the_oracle(dev, K, N):
    rng = np.random.default_rng(K + 3 * N)
    a = rng.standard_normal(K).astype(np.float32)
    w = oracle.to_f16((rng.standard_normal(K * N) * 0.02).astype(np.float32)).reshape(K, N)
    want = oracle.matvec_f32_f16(a, w, K, N)
    ab, wb = dev.upload(a), dev.upload(w, F16)
    ob = dev.alloc((N,), F32)
    dev.MatVecF32F16(ab, wb, ob)
    assert rel_l2(ob.numpy(), want) <= F32_TOL
    # twice: the split-K hand-off leaves its tickets ready and is deterministic
    first = ob.numpy().copy()
    dev.MatVecF32F16(ab, wb, ob)
    assert np.array_equal(ob.numpy(), first)
    for t in (ab, wb, ob):
        t.free()


def test_records_dispatch(dev):
    rng = np.random.default_rng(9)
    # SwiGLU record: a, b, out; no uniform
    n = 777
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    ab, bb, ob = dev.upload(a), dev.upload(b), dev.alloc((n,), F32)
    dev.dispatch("SwiGLU", [ab, bb, ob], [n, n, n], b"")
    assert _ulps(ob.numpy(), oracle.swiglu(a, b)).max() <= 1
    # RMSNorm record: RowDims {Rows, Width, Eps}
    rows, width = 4, 200
    x = rng.standard_normal((rows, width)).astype(np.float32)
    g = rng.standard_normal(width).astype(np.float32)
    xb, gb, rb = dev.upload(x), dev.upload(g), dev.alloc((rows, width), F32)
    dev.dispatch("RMSNorm", [xb, gb, rb], [rows * width, width, rows * width],
                 struct.pack("<IIfI", rows, width, 1e-5, 0))
    assert np.array_equal(rb.numpy(), oracle.rmsnorm(x, g, 1e-5))
    # MatVecF32F16 record: GEMMDims {M, N, K}
    K, N = 512, 256
    av = rng.standard_normal(K).astype(np.float32)
    wv = oracle.to_f16(rng.standard_normal(K * N).astype(np.float32) * 0.05).reshape(K, N)
    avb, wvb, mvb = dev.upload(av), dev.upload(wv, F16), dev.alloc((N,), F32)
    dev.dispatch("MatVecF32F16", [avb, wvb, mvb], [K, K * N, N], struct.pack("<IIII", 1, N, K, 0))
    assert rel_l2(mvb.numpy(), oracle.matvec_f32_f16(av, wv, K, N)) <= F32_TOL
    for t in (ab, bb, ob, xb, gb, rb, avb, wvb, mvb):
        t.free()
