"""GPU parity of the fused int4 Linear (the int4 analogue of tensor.Linear,
tensor/matmul.go:184-225) through the C ABI.

The reference keeps the composed form (the product, then ElemAdd of the bias,
then a cast) as the fused kernel's reference.  For f32 activations the fused
epilogue adds the bias to the very f32 sum the plain product stores, so the
fused result equals the device's own Int4MatMul plus the bias bit for bit,
and its bf16 form is that f32 value rounded once (RNE), also bit for bit;
against the oracle's composed form it is held to rel-L2 <= 1e-5.  bf16
activations round once after the bias, where the composed form rounds
twice: rel-L2 <= 2e-2 against the oracle's composed form on bf16-rounded
inputs, and within one bf16 rounding of it elementwise.

Shapes cover every kernel the product routes to: the VALU decode kernel
(M = 1, 2, and 9..16 rows as eight plus the rest), the matrix-core decode
kernel (M = 3..16), the f32 tiled kernel (M > 16), the per-element kernels
(ragged N) and the bf16 matrix-core tiles.
"""
import numpy as np
import pytest

import oracle
from accel_amd import BF16, F32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 2e-2


def _problem(M, K, N, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal(K * N) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    bias = rng.standard_normal(N).astype(np.float32)
    return x, p, s, z, bias


def _free(*bufs):
    for b in bufs:
        b.free()


@pytest.mark.parametrize("M,K,N,vector", [
    (1, 4096, 4096, True),     # VALU decode, one row, split K
    (1, 300, 256, False),
    (2, 1024, 384, False),     # matrix-core decode, two rows, one-group tiles
    (2, 1000, 384, False),     # K % 32 != 0: VALU decode, 128-column tiles
    (5, 4096, 4096, False),    # matrix-core decode
    (16, 1024, 768, False),
    (12, 200, 256, False),     # K % 32 != 0: VALU decode, eight rows then four
    (40, 256, 384, False),     # f32 tiled
    (20, 2048, 4096, False),   # the f32 tiles, one m-tile of rows, K split
    (3, 40, 21, False),        # per-element kernel
])
def test_f32_activations_equal_the_product_plus_bias(dev, M, K, N, vector):
    x, p, s, z, bias = _problem(M, K, N, M * 131 + K + N)
    w = dev.upload_int4(p, s, z, K * N)
    shape = (N,) if vector else (M, N)
    xb = dev.upload(x[0] if vector else x)
    bb = dev.upload(bias)
    prod = dev.alloc(shape, F32)
    if vector:
        dev.Int4MatVec(xb, w, prod)
    else:
        dev.Int4MatMul(xb, w, prod)
    plain = prod.numpy().reshape(M, N)
    composed = (plain + bias[None, :]).astype(np.float32)

    of = dev.alloc(shape, F32)
    dev.Int4Linear(xb, w, bb, of)
    got = of.numpy().reshape(M, N)
    assert np.array_equal(got.view(np.uint32), composed.view(np.uint32))
    assert rel_l2(got, oracle.int4_linear(x, p, s, z, bias, M, K, N)) <= F32_TOL
    # again: the split-K hand-off is ready for the next call and deterministic
    dev.Int4Linear(xb, w, bb, of)
    assert np.array_equal(of.numpy().reshape(M, N).view(np.uint32), got.view(np.uint32))

    ob = dev.alloc(shape, BF16)
    dev.Int4Linear(xb, w, bb, ob)
    assert np.array_equal(ob.numpy().reshape(-1), oracle.to_bf16(composed))
    # no bias: the epilogue only narrows
    dev.Int4Linear(xb, w, None, ob)
    assert np.array_equal(ob.numpy().reshape(-1), oracle.to_bf16(plain))
    dev.Int4Linear(xb, w, None, of)
    assert np.array_equal(of.numpy().reshape(M, N).view(np.uint32), plain.view(np.uint32))
    _free(xb, bb, prod, of, ob)
    w.free()


@pytest.mark.parametrize("M,K,N", [(256, 512, 512), (300, 128, 256), (7, 100, 50)])
def test_bf16_activations(dev, M, K, N):
    x, p, s, z, bias = _problem(M, K, N, M + 7 * K + N)
    xbits = workloads.bf16_bits(x)
    xr = workloads.bf16_to_f32(xbits)
    w = dev.upload_int4(p, s, z, K * N)
    xb, bb = dev.upload(xbits, BF16), dev.upload(bias)
    ob = dev.alloc((M, N), BF16)
    dev.Int4Linear(xb, w, bb, ob)
    got = workloads.bf16_to_f32(ob.numpy())
    want = oracle.bf16_to_f32(oracle.int4_linear(xr, p, s, z, bias, M, K, N, bf16_out=True))
    want = want.reshape(M, N)
    assert rel_l2(got, want) <= BF16_TOL
    f32 = oracle.int4_linear(xr, p, s, z, bias, M, K, N)
    # one rounding of a sum within f32 reduction error of the oracle's
    assert np.all(np.abs(got - f32) <= np.abs(f32) * 2.0 ** -8 + 1e-3 * np.abs(f32).max())
    # without a bias the fused kernel is the plain bf16 product
    pb = dev.alloc((M, N), BF16)
    dev.Int4MatMul(xb, w, pb)
    dev.Int4Linear(xb, w, None, ob)
    assert np.array_equal(ob.numpy(), pb.numpy())
    _free(xb, bb, ob, pb)
    w.free()
