"""The int8 weight path on the CPU: the library's host packer against the
oracle, the reference's quantizer tests (quant/quant_test.go:22-237), and the
oracle's int8 kernels (QuantMatVecF32, internal/kernels/matvec.go:204-235;
QuantMatMulTiledF32, internal/kernels/quant.go:195-238) pinned by the
reference's exact-input cases, f64 brute force within the reduction bound,
and independent numpy restatements of their evaluation orders."""
import numpy as np
import pytest

import accel_amd
import oracle


def _cases():
    return {
        "smooth": (np.sin(np.arange(200) * 0.31) * 3).astype(np.float32),
        "outliers": np.where(np.arange(128) % 32 == 0, 100.0, 0.01).astype(np.float32),
        "ragged": np.array([1, -2, 3, -4, 5], np.float32),
        "zeros": np.zeros(64, np.float32),
        "zero_block_then_values": np.concatenate([np.zeros(32), np.arange(32, 64)]).astype(np.float32),
        "negatives": (-np.arange(40) - 1).astype(np.float32),
        "underflow": np.full(32, 1e-12, np.float32),
        "clamp": np.array([np.frombuffer(np.uint32(0x3F800000 - i).tobytes(), np.float32)[0]
                           for i in range(32)], np.float32),
        "random": (np.random.default_rng(3).standard_normal(4099) * 0.05).astype(np.float32),
    }


@pytest.mark.parametrize("name", sorted(_cases()))
def test_host_packer_is_the_oracle_bit_for_bit(name):
    w = _cases()[name]
    q0, s0 = oracle.int8_quantize(w)
    q1, s1 = accel_amd.int8_quantize(w)
    assert np.array_equal(q0, q1) and np.array_equal(s0, s1)
    assert np.array_equal(oracle.int8_dequantize(q0, s0), accel_amd.int8_dequantize(q1, s1))


@pytest.mark.parametrize("name", ["smooth", "outliers", "ragged", "zeros",
                                  "zero_block_then_values", "negatives"])
def test_every_weight_is_within_half_a_step(name):   # quant_test.go:22-108
    w = _cases()[name]
    q, s = oracle.int8_quantize(w)
    assert s.size == (w.size + 31) // 32
    back = oracle.int8_dequantize(q, s)
    step = oracle.f16_to_f32(s)[np.arange(w.size) // 32].astype(np.float64)
    assert np.all(np.abs(back.astype(np.float64) - w) <= step / 2 * (1 + 1e-3))
    assert np.all(np.abs(q.astype(np.int32)) <= 127)


def test_the_clamp_catches_the_wrap_around():   # quant_test.go:110-133
    w = _cases()["clamp"]
    q, s = oracle.int8_quantize(w)
    assert np.all(q >= 0) and np.all(oracle.int8_dequantize(q, s) >= 0)


def test_scales_that_underflow_f16():   # quant_test.go:203-225
    q, s = oracle.int8_quantize(_cases()["underflow"])
    assert oracle.f16_to_f32(s)[0] == 0 and np.all(q == 0)
    assert np.all(oracle.int8_dequantize(q, s) == 0)


def test_dequantize_is_the_reference():   # quant_test.go:227-237
    q = np.array([1, -2, 127, -127], np.int8)
    s = oracle.to_f16(np.array([0.5], np.float32))
    assert np.array_equal(oracle.int8_dequantize(q, s), np.array([0.5, -1, 63.5, -63.5], np.float32))


def _exact_inputs(M, K, N):
    # prefill_test.go:934-960, differential_cases_test.go:950-1010: few
    # significant bits, so every product and sum is exact in f32
    a = (np.arange(M * K) % 7 - 3).astype(np.float32)
    q = (np.arange(K * N) % 201 - 100).astype(np.int8)
    s = oracle.to_f16((0.25 + (np.arange((K * N + 31) // 32) % 3) / 8).astype(np.float32))
    return a, q, s


def _f64(a, q, s, M, K, N):
    w = q.astype(np.float64) * oracle.f16_to_f32(s).astype(np.float64)[np.arange(K * N) // 32]
    return a.reshape(M, K).astype(np.float64) @ w.reshape(K, N)


@pytest.mark.parametrize("K,N", [(32, 8), (40, 21), (256, 64)])
def test_matvec_exact_inputs(K, N):
    a, q, s = _exact_inputs(1, K, N)
    got = oracle.quant_matvec_i8(a, q, s, K, N)
    assert np.array_equal(got.astype(np.float64), _f64(a, q, s, 1, K, N)[0])


@pytest.mark.parametrize("M,K,N", [(11, 40, 21), (3, 64, 32), (1, 17, 5)])
def test_matmul_exact_inputs(M, K, N):
    a, q, s = _exact_inputs(M, K, N)
    got = oracle.quant_matmul_i8(a, q, s, M, K, N)
    assert np.array_equal(got.astype(np.float64), _f64(a, q, s, M, K, N))


def _phase_order_np(a, q, s, K, N):
    w = (q.astype(np.float32) * oracle.f16_to_f32(s)[np.arange(K * N) // 32]).reshape(K, N)
    ph = np.zeros((16, N), np.float32)
    for k in range(K):
        ph[k % 16] = (ph[k % 16] + (a[k] * w[k]).astype(np.float32)).astype(np.float32)
    out = np.zeros(N, np.float32)
    for p in range(16):
        out = (out + ph[p]).astype(np.float32)
    return out


def _sequential_np(a, q, s, M, K, N):
    w = (q.astype(np.float32) * oracle.f16_to_f32(s)[np.arange(K * N) // 32]).reshape(K, N)
    a = a.reshape(M, K)
    out = np.zeros((M, N), np.float32)
    for k in range(K):
        out = (out + (a[:, k:k + 1] * w[k]).astype(np.float32)).astype(np.float32)
    return out


@pytest.mark.parametrize("M,K,N", [(1, 300, 40), (1, 1024, 96), (5, 200, 33), (16, 96, 64)])
def test_kernels_order_and_f64_bound(M, K, N):
    rng = np.random.default_rng(M * 1000 + K + N)
    a = rng.standard_normal(M * K).astype(np.float32)
    q, s = oracle.int8_quantize((rng.standard_normal(K * N) * 0.05).astype(np.float32))
    want64 = _f64(a, q, s, M, K, N)
    mag = np.abs(a.reshape(M, K).astype(np.float64)) @ np.abs(
        (q.astype(np.float64) * oracle.f16_to_f32(s)[np.arange(K * N) // 32]).reshape(K, N))
    if M == 1:
        got = oracle.quant_matvec_i8(a, q, s, K, N)
        assert np.array_equal(got.view(np.uint32), _phase_order_np(a, q, s, K, N).view(np.uint32))
        nu = (K // 16 + 18) * 2.0 ** -24
        assert np.all(np.abs(got - want64[0]) <= nu * mag[0] + 1e-30)
    got = oracle.quant_matmul_i8(a, q, s, M, K, N)
    assert np.array_equal(got.view(np.uint32), _sequential_np(a, q, s, M, K, N).view(np.uint32))
    nu = (K + 2) * 2.0 ** -24
    assert np.all(np.abs(got - want64) <= nu * mag + 1e-30)
