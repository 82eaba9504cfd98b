"""The oracle's int4 Linear (CPU only): the composed form the reference keeps
as the fused kernel's reference (tensor/matmul.go:184-188), the int4 product
followed by ElemAdd (internal/kernels/elementwise.go:19-27) of the bias
broadcast over rows and, for a bf16 result, one narrowing.

ElemAdd is pinned against numpy's IEEE f32 addition, including signed zeros,
infinities and NaN; the composition by its two special cases (a bias of -0.0
returns the product bit for bit, all-zero weights return the bias on every
row) and by the narrowing being the oracle's pinned ToBFloat16.
"""
import numpy as np
import pytest

import oracle


def test_add_rows_is_ieee_f32_addition():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((7, 33)) * np.exp2(rng.integers(-30, 30, (7, 33)))).astype(np.float32)
    v = (rng.standard_normal(33) * np.exp2(rng.integers(-30, 30, 33))).astype(np.float32)
    got = oracle.add_rows(x, v)
    assert np.array_equal(got.view(np.uint32), (x + v[None, :]).view(np.uint32))


def test_add_rows_special_values():
    x = np.array([[-0.0, -0.0, 0.0, np.inf, np.inf, np.nan, 1.0, 3.4e38]], np.float32)
    v = np.array([-0.0, 0.0, -0.0, -np.inf, 1.0, 1.0, -1.0, 3.4e38], np.float32)
    got = oracle.add_rows(x, v)[0]
    assert got[0] == 0 and np.signbit(got[0])           # -0 + -0 = -0
    assert got[1] == 0 and not np.signbit(got[1])       # -0 + +0 = +0
    assert got[2] == 0 and not np.signbit(got[2])
    assert np.isnan(got[3]) and got[4] == np.inf and np.isnan(got[5])
    assert got[6] == 0 and not np.signbit(got[6])       # 1 + -1 = +0
    assert got[7] == np.inf                              # overflow rounds to inf


def test_negative_zero_vector_is_the_identity():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((4, 50)).astype(np.float32)
    x[0, :5] = -0.0
    got = oracle.add_rows(x, np.full(50, -0.0, np.float32))
    assert np.array_equal(got.view(np.uint32), x.view(np.uint32))


def _weights(rng, K, N):
    w = (rng.standard_normal(K * N) * 0.02).astype(np.float32)
    return oracle.int4_quantize(w)


@pytest.mark.parametrize("M,K,N", [(1, 256, 128), (3, 128, 256), (5, 40, 7)])
def test_linear_with_negative_zero_bias_is_the_product(M, K, N):
    rng = np.random.default_rng(M + K + N)
    x = rng.standard_normal(M * K).astype(np.float32)
    p, s, z = _weights(rng, K, N)
    got = oracle.int4_linear(x, p, s, z, np.full(N, -0.0, np.float32), M, K, N)
    want = (oracle.quant_matvec_int4(x, p, s, z, K, N).reshape(1, N) if M == 1
            else oracle.quant_matmul_int4(x, p, s, z, M, K, N))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(oracle.int4_linear(x, p, s, z, None, M, K, N).view(np.uint32),
                          want.view(np.uint32))


def test_linear_with_zero_weights_is_the_bias_on_every_row():
    M, K, N = 6, 256, 128
    rng = np.random.default_rng(4)
    x = rng.standard_normal(M * K).astype(np.float32)
    p, s, z = oracle.int4_quantize(np.zeros(K * N, np.float32))
    bias = rng.standard_normal(N).astype(np.float32)
    got = oracle.int4_linear(x, p, s, z, bias, M, K, N)
    assert np.array_equal(got, np.broadcast_to(bias, (M, N)))


def test_linear_bf16_result_is_one_narrowing_of_the_f32_one():
    M, K, N = 4, 128, 256
    rng = np.random.default_rng(6)
    x = rng.standard_normal(M * K).astype(np.float32)
    p, s, z = _weights(rng, K, N)
    bias = rng.standard_normal(N).astype(np.float32)
    f32 = oracle.int4_linear(x, p, s, z, bias, M, K, N)
    b16 = oracle.int4_linear(x, p, s, z, bias, M, K, N, bf16_out=True)
    assert b16.dtype == np.uint16
    assert np.array_equal(b16.reshape(-1), oracle.to_bf16(f32))
    # one rounding: within half a bf16 ulp of the f32 result
    back = oracle.bf16_to_f32(b16)
    assert np.all(np.abs(back - f32) <= np.abs(f32) * 2.0 ** -8 + 1e-38)
