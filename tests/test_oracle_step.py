"""The oracle's decode-step neighbours of the int4 products (CPU only).

SwiGLU (internal/kernels/elementwise.go:85-91), RMSNorm
(internal/kernels/norm.go:47-80) and MatVecF32F16
(internal/kernels/matvec.go:79-105) are pinned by:

* the reference's own tests for RMSNorm (internal/kernels/norm_test.go:34-191):
  the widths, inputs and f64 comparison of TestRMSNormMatchesItsReference and
  the zero row of TestRMSNormHandlesAZeroRow;
* f64 closed forms within the f32 rounding budget (a dropped term, a wrong
  sign, a wrong divisor or a missing gain fails them);
* for the evaluation order, which an f64 comparison cannot see, independent
  numpy restatements of the reference's reduction shapes (the 128-invocation
  strided fold and halving tree; the 16-phase column sum), bit for bit, on
  inputs where a different order gives a different f32 result;
* exact answers where every partial is an exact integer.
"""
import numpy as np
import pytest

import oracle


# ---- SwiGLU -----------------------------------------------------------------

def test_swiglu_matches_the_f64_closed_form():
    rng = np.random.default_rng(11)
    a = (rng.standard_normal(4096) * 6).astype(np.float32)
    b = rng.standard_normal(4096).astype(np.float32)
    got = oracle.swiglu(a, b).astype(np.float64)
    x = a.astype(np.float64)
    want = x / (1.0 + np.exp(-x)) * b.astype(np.float64)
    # four roundings (exp, add, divide, multiply), each at most half an ulp
    assert np.all(np.abs(got - want) <= 4 * 2.0 ** -24 * np.abs(want) + 1e-45)


def test_swiglu_special_values():
    a = np.array([0.0, -0.0, 100.0, -100.0, 1.0, -1.0, np.inf, -np.inf], np.float32)
    b = np.array([3.0, 3.0, 2.0, 2.0, 1.0, 1.0, 1.0, 1.0], np.float32)
    got = oracle.swiglu(a, b)
    assert got[0] == 0.0 and got[1] == 0.0
    # e^-100 is a positive f32 subnormal: 1 + e rounds to 1
    assert got[2] == np.float32(200.0)
    # e^100 overflows to +inf in f32: -100 / inf = -0
    assert got[3] == 0.0 and np.signbit(got[3])
    assert got[4] == np.float32(np.float32(1.0) / np.float32(1.0 + np.float32(np.exp(-1.0))))
    assert got[6] == np.inf  # inf / (1 + 0) * 1
    assert np.isnan(got[7])  # -inf / inf
    assert np.isnan(oracle.swiglu(np.array([np.nan], np.float32), np.array([1.0], np.float32)))[0]


# ---- RMSNorm ------------------------------------------------------------------

def _rmsnorm_tree_np(x, w, eps):
    """An independent numpy statement of the reference's reduction shape."""
    rows, width = x.shape
    out = np.empty_like(x)
    for r in range(rows):
        sq = x[r] * x[r]                                  # f32 products
        pad = np.zeros(((width + 127) // 128) * 128, np.float32)
        pad[:width] = sq
        lanes = pad.reshape(-1, 128)                     # row j: elements 128 j .. 128 j + 127
        part = np.zeros(128, np.float32)
        for j in range(lanes.shape[0]):                  # increasing i within each lane
            valid = np.arange(128) + 128 * j < width
            part = np.where(valid, part + lanes[j], part).astype(np.float32)
        stride = 64
        while stride:
            part[:stride] = part[:stride] + part[stride:2 * stride]
            stride //= 2
        mean = np.float32(part[0] / np.float32(width))
        scale = np.float32(1.0 / np.sqrt(np.float64(np.float32(mean + np.float32(eps)))))
        out[r] = (x[r] * scale) * w
    return out


@pytest.mark.parametrize("width", [1, 63, 128, 129, 500, 1024])
def test_rmsnorm_matches_its_reference(width):
    # TestRMSNormMatchesItsReference (norm_test.go:34-83): x = sin(i) * 3,
    # w = cos(i) + 1.5, three rows, eps 1e-5
    rows = 3
    x = (np.sin(np.arange(rows * width, dtype=np.float64)) * 3).astype(np.float32)
    x = x.reshape(rows, width)
    w = (np.cos(np.arange(width, dtype=np.float64)) + 1.5).astype(np.float32)
    got = oracle.rmsnorm(x, w, 1e-5)
    xd = x.astype(np.float64)
    scale = 1.0 / np.sqrt((xd * xd).sum(axis=1) / width + np.float64(np.float32(1e-5)))
    want = xd * scale[:, None] * w.astype(np.float64)
    # the tree's rounding of the sum of squares, halved by the square root,
    # plus the final products
    depth = int(np.ceil(np.log2(min(width, 128)))) + (width + 127) // 128
    rel = depth * 2.0 ** -24 + 4 * 2.0 ** -24
    assert np.all(np.abs(got - want) <= np.abs(want) * rel + 1e-6)


def test_rmsnorm_zero_row_reads_zero():
    # TestRMSNormHandlesAZeroRow (norm_test.go:166-191)
    x = np.zeros((1, 64), np.float32)
    w = np.ones(64, np.float32)
    got = oracle.rmsnorm(x, w, 1e-5)
    assert np.all(got == 0) and np.all(np.isfinite(got))


def test_rmsnorm_order_is_the_references_tree():
    # values spanning 2^20: a sequential sum and the strided tree round
    # differently, so this fixes the order, not just the value
    rng = np.random.default_rng(5)
    for width in (100, 128, 300, 4096):
        x = (rng.standard_normal((4, width)) * np.exp2(rng.integers(-10, 10, (4, width)))
             ).astype(np.float32)
        w = rng.standard_normal(width).astype(np.float32)
        got = oracle.rmsnorm(x, w, 1e-6)
        want = _rmsnorm_tree_np(x, w, 1e-6)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), width
        seq = np.zeros(4, np.float32)
        for i in range(width):
            seq = (seq + x[:, i] * x[:, i]).astype(np.float32)
        # the reference order is observable on these inputs
        if width > 128:
            tree = np.array([_tree_total(x[r]) for r in range(4)], np.float32)
            assert np.any(tree != seq)


def _tree_total(row):
    width = row.size
    part = np.zeros(128, np.float32)
    for i in range(width):
        part[i % 128] = np.float32(part[i % 128] + np.float32(row[i] * row[i]))
    stride = 64
    while stride:
        part[:stride] = part[:stride] + part[stride:2 * stride]
        stride //= 2
    return part[0]


def test_rmsnorm_ones_row():
    # mean of squares of ones is exactly 1: out = w * RSqrt(1 + eps), the
    # value the f64 definition gives after one rounding of the scale
    w = np.linspace(-2, 2, 256, dtype=np.float32)
    got = oracle.rmsnorm(np.ones((2, 256), np.float32), w, 1e-5)
    scale = np.float32(1.0 / np.sqrt(np.float64(np.float32(1.0) + np.float32(1e-5))))
    assert np.array_equal(got, np.stack([w * scale, w * scale]))


# ---- MatVecF32F16 -------------------------------------------------------------

def _matvec_phases_np(a, b, K, N):
    """An independent numpy statement of the 16-phase column sum."""
    bf = oracle.f16_to_f32(b.reshape(-1)).reshape(K, N)
    ph = np.zeros((16, N), np.float32)
    for k in range(K):
        ph[k % 16] = (ph[k % 16] + (a[k] * bf[k]).astype(np.float32)).astype(np.float32)
    out = np.zeros(N, np.float32)
    for p in range(16):
        out = (out + ph[p]).astype(np.float32)
    return out


@pytest.mark.parametrize("K,N", [(40, 12), (1, 5), (17, 33), (256, 64), (1000, 7)])
def test_matvec_f32_f16_order_and_f64(K, N):
    rng = np.random.default_rng(K * 131 + N)
    a = rng.standard_normal(K).astype(np.float32)
    w = (rng.standard_normal((K, N)) * 0.05).astype(np.float32)
    b = oracle.to_f16(w.reshape(-1)).reshape(K, N)
    got = oracle.matvec_f32_f16(a, b, K, N)
    assert np.array_equal(got.view(np.uint32), _matvec_phases_np(a, b, K, N).view(np.uint32))
    bf = oracle.f16_to_f32(b.reshape(-1)).reshape(K, N).astype(np.float64)
    want = a.astype(np.float64) @ bf
    mag = np.abs(a.astype(np.float64)) @ np.abs(bf)
    nu = (K // 16 + 16 + 1) * 2.0 ** -24
    assert np.all(np.abs(got - want) <= nu * mag + 1e-30)


def test_matvec_f32_f16_exact_integers():
    K, N = 96, 20
    a = np.arange(K, dtype=np.float32) % 7 - 3
    w = (np.arange(K * N, dtype=np.float32) % 11 - 5).reshape(K, N)
    b = oracle.to_f16(w.reshape(-1)).reshape(K, N)
    got = oracle.matvec_f32_f16(a, b, K, N)
    assert np.array_equal(got, (a.astype(np.float64) @ w.astype(np.float64)).astype(np.float32))
