"""GPU parity of the int8 weight products (tensor.QuantMatMul,
tensor/quantized.go:72-163) against the oracle, through the C ABI.

The library sums in its own order, so random inputs are held to rel-L2 <=
1e-5 against the oracle's QuantMatVecF32 (internal/kernels/matvec.go:204-235)
and QuantMatMulTiledF32 (internal/kernels/quant.go:195-238); inputs whose
every product and partial sum is exact in f32 (the reference's
prefill_test.go:934-960 style) are compared exactly.  Both kernels run: the
decode kernel (M <= 8, N a multiple of 256, 16-byte aligned quants) and the
tiled kernel (everything else).
"""
import ctypes
import struct

import numpy as np
import pytest

import accel_amd
import oracle
from accel_amd import F16, F32, I8
from conftest import rel_l2

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5


def _weights(rng, K, N):
    return oracle.int8_quantize((rng.standard_normal(K * N) * 0.05).astype(np.float32))


def _want(a, q, s, M, K, N):
    if M == 1:
        return oracle.quant_matvec_i8(a, q, s, K, N).reshape(1, N)
    return oracle.quant_matmul_i8(a, q, s, M, K, N)


def run(dev, a, q, s, M, K, N, f16=False, twice=False):
    if f16:
        ab = dev.upload(a.reshape(M, K), F16)
    else:
        ab = dev.upload(np.ascontiguousarray(a.reshape(M, K), np.float32))
    qb = dev.upload(q.reshape(K, N))
    sb = dev.upload(s)
    ob = dev.alloc((M, N), F32)
    dev.QuantMatMul(ab, qb, sb, ob)
    got = ob.numpy().copy()
    if twice:
        # the split-K hand-off leaves its tickets ready and sums in a fixed order
        dev.QuantMatMul(ab, qb, sb, ob)
        assert np.array_equal(ob.numpy(), got)
    for b in (ab, qb, sb, ob):
        b.free()
    return got


def _exact_inputs(M, K, N):
    a = (np.arange(M * K) % 7 - 3).astype(np.float32)
    q = (np.arange(K * N) % 201 - 100).astype(np.int8)
    s = oracle.to_f16((0.25 + (np.arange((K * N + 31) // 32) % 3) / 8).astype(np.float32))
    return a, q, s


@pytest.mark.parametrize("M,K,N", [(1, 32, 8), (1, 40, 21), (11, 40, 21), (1, 256, 256),
                                   (4, 1000, 512), (8, 64, 768), (9, 96, 256)])
def test_exact_inputs_are_exact(dev, M, K, N):
    a, q, s = _exact_inputs(M, K, N)
    want = _want(a, q, s, M, K, N)
    got = run(dev, a, q, s, M, K, N)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("M,K,N", [
    (1, 4096, 4096), (2, 4096, 4096), (3, 4096, 4096), (4, 4096, 4096), (5, 4096, 4096),
    (6, 4096, 4096), (7, 4096, 4096), (8, 4096, 4096),
    (1, 4096, 14336), (8, 4096, 14336), (1, 14336, 4096), (4, 14336, 4096),
    (3, 1000, 512), (2, 1, 256), (1, 17, 768), (5, 33, 256)])
def test_decode_shapes_match_the_oracle(dev, M, K, N):
    rng = np.random.default_rng(M * 7919 + K + 3 * N)
    a = rng.standard_normal(M * K).astype(np.float32)
    q, s = _weights(rng, K, N)
    got = run(dev, a, q, s, M, K, N, twice=True)
    assert rel_l2(got, _want(a, q, s, M, K, N)) <= F32_TOL


@pytest.mark.parametrize("M,K,N", [(9, 300, 96), (64, 512, 300), (17, 33, 7), (1, 4096, 1000),
                                   (2, 2048, 4000), (130, 256, 256), (3, 1, 1), (65, 96, 65)])
def test_tiled_shapes_match_the_oracle(dev, M, K, N):
    rng = np.random.default_rng(M * 31 + K * 17 + N)
    a = rng.standard_normal(M * K).astype(np.float32)
    q, s = _weights(rng, K, N)
    got = run(dev, a, q, s, M, K, N)
    assert rel_l2(got, _want(a, q, s, M, K, N)) <= F32_TOL


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (6, 1024, 512), (20, 256, 100)])
def test_f16_activations(dev, M, K, N):
    # QuantMatVec / QuantMatMulTiled: f16 activations widen exactly to f32
    rng = np.random.default_rng(M + K + N)
    a16 = oracle.to_f16(rng.standard_normal(M * K).astype(np.float32))
    q, s = _weights(rng, K, N)
    got = run(dev, a16, q, s, M, K, N, f16=True)
    want = _want(oracle.f16_to_f32(a16), q, s, M, K, N)
    assert rel_l2(got, want) <= F32_TOL


def test_empty_and_zero_depth(dev):
    # K = 0: every output is the empty sum
    M, K, N = 3, 0, 40
    ab = dev.alloc((M, 1), F32)
    lib = accel_amd.lib()
    x = ab.tensor(); x.shape[1] = 0
    qb = dev.alloc((1, N), I8); tq = qb.tensor(); tq.shape[0] = 0
    sb = dev.alloc((1,), F16); ts = sb.tensor(); ts.shape[0] = 0
    ob = dev.alloc((M, N), F32)
    ob.write(np.full((M, N), 7.0, np.float32))
    to = ob.tensor()
    rc = lib.accel_quant_matmul(0, None, ctypes.byref(x), ctypes.byref(tq), ctypes.byref(ts),
                                ctypes.byref(to))
    assert rc == 0, accel_amd.last_error()
    assert np.all(ob.numpy() == 0)
    for b in (ab, qb, sb, ob):
        b.free()


def test_unaligned_quants_take_the_tiled_kernel(dev):
    # quants one byte into their allocation: the decode kernel's 16-byte loads
    # are off, the tiled kernel reads any address
    M, K, N = 2, 300, 512
    rng = np.random.default_rng(77)
    a = rng.standard_normal(M * K).astype(np.float32)
    q, s = _weights(rng, K, N)
    ab = dev.upload(a.reshape(M, K))
    qb = dev.upload(np.concatenate([np.zeros(1, np.int8), q]))
    sb = dev.upload(s)
    ob = dev.alloc((M, N), F32)
    tq = qb.tensor()
    tq.data += 1
    tq.rank = 2
    tq.shape[0], tq.shape[1] = K, N
    ta, ts, to = ab.tensor(), sb.tensor(), ob.tensor()
    rc = accel_amd.lib().accel_quant_matmul(0, None, ctypes.byref(ta), ctypes.byref(tq),
                                            ctypes.byref(ts), ctypes.byref(to))
    assert rc == 0, accel_amd.last_error()
    assert rel_l2(ob.numpy(), _want(a, q, s, M, K, N)) <= F32_TOL
    for b in (ab, qb, sb, ob):
        b.free()


def test_records_dispatch(dev):
    # the four int8 records, GEMMDims {M, N, K} (tensor/quantized.go:95-160)
    rng = np.random.default_rng(5)
    for name, M, f16 in [("QuantMatVecF32", 1, False), ("QuantMatVec", 1, True),
                         ("QuantMatMulTiledF32", 5, False), ("QuantMatMulTiled", 12, True)]:
        K, N = 200, 256
        a = rng.standard_normal(M * K).astype(np.float32)
        if f16:
            a = oracle.to_f16(a)
        q, s = _weights(rng, K, N)
        ab = dev.upload(a, F16 if f16 else F32)
        qb, sb = dev.upload(q), dev.upload(s)
        ob = dev.alloc((M * N,), F32)
        dev.dispatch(name, [ab, qb, sb, ob], [M * K, K * N, s.size, M * N],
                     struct.pack("<IIII", 0 if M == 1 else M, N, K, 0))
        want = _want(oracle.f16_to_f32(a) if f16 else a, q, s, M, K, N)
        assert rel_l2(ob.numpy().reshape(M, N), want) <= F32_TOL, name
        for b in (ab, qb, sb, ob):
            b.free()
