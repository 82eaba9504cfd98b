"""Pins the oracle's kernels (reference evaluation order) against closed
forms, the reference's kernel tests and f64 brute force.

Sources: internal/kernels/int4_test.go, internal/kernels/grouped_test.go,
internal/kernels/differential_cases_test.go:1347-1460, tensor/int4_test.go,
tensor/grouped_test.go.
"""
import math

import numpy as np
import pytest

import oracle

GROUP = 128


def default_seed(b, i):
    """differential_cases_test.go:78-80"""
    return np.float32(((i + b * 7) % 13 - 6) / 4)


def gamma(n):
    nu = n * 2.0 ** -24
    return nu / (1 - nu)


# ---- differential cases with closed forms ---------------------------------

def _closed_form_matvec(a, words, scales, zeros, K, N):
    """sum_k a[k] * w(k,n) in f64 with w = s==0 ? z : (code-z)*s."""
    out = np.zeros(N)
    for n in range(N):
        for k in range(K):
            i = k * N + n
            code = (int(words[i // 8]) >> (4 * (i % 8))) & 0xF
            s = float(scales[i // GROUP])
            z = float(zeros[i // GROUP])
            wv = z if s == 0 else (code - z) * s
            out[n] += float(a[k]) * wv
    return out


@pytest.mark.parametrize("case", ["plain", "constant_group"])
def test_differential_matvec_cases_match_their_closed_form(case):
    if case == "plain":   # differential_cases_test.go:1347-1368
        K, N = 128, 2
        sc = [0.25] * 2
        zc = [4.0] * 2
    else:                 # :1370-1398
        K, N = 256, 2
        sc = [0.0, 0.25, 0.25, 0.25]
        zc = [0.75, 4.0, 4.0, 4.0]
    a = np.array([default_seed(0, i) for i in range(K)], np.float32)
    words = np.array([abs(i % 251 + 1) for i in range(K * N // 8)], np.uint32)
    s16 = oracle.to_f16(np.array(sc, np.float32))
    z16 = oracle.to_f16(np.array(zc, np.float32))
    got = oracle.quant_matvec_int4(a, words, s16, z16, K, N)
    want = _closed_form_matvec(a, words, oracle.f16_to_f32(s16), oracle.f16_to_f32(z16), K, N)
    mag = _closed_form_mag(a, words, oracle.f16_to_f32(s16), oracle.f16_to_f32(z16), K, N)
    for n in range(N):
        assert abs(got[n] - want[n]) <= gamma(K) * mag[n], (n, got[n], want[n])


def _closed_form_mag(a, words, scales, zeros, K, N):
    out = np.zeros(N)
    for n in range(N):
        for k in range(K):
            i = k * N + n
            code = (int(words[i // 8]) >> (4 * (i % 8))) & 0xF
            s = float(scales[i // GROUP]); z = float(zeros[i // GROUP])
            wv = z if s == 0 else (code - z) * s
            out[n] += abs(float(a[k]) * wv)
    return out


def test_differential_tiled_case_matches_its_closed_form():
    # differential_cases_test.go:1400-1424: M=3, K=40, N=16
    M, K, N = 3, 40, 16
    a = np.array([default_seed(0, i) for i in range(M * K)], np.float32)
    words = np.array([i % 251 + 1 for i in range(K * N // 8)], np.uint32)
    s16 = oracle.to_f16(np.full(8, 0.25, np.float32))
    z16 = oracle.to_f16(np.full(8, 4.0, np.float32))
    got = oracle.quant_matmul_int4(a, words, s16, z16, M, K, N)
    for m in range(M):
        want = _closed_form_matvec(a[m * K:(m + 1) * K], words, oracle.f16_to_f32(s16),
                                   oracle.f16_to_f32(z16), K, N)
        mag = _closed_form_mag(a[m * K:(m + 1) * K], words, oracle.f16_to_f32(s16),
                               oracle.f16_to_f32(z16), K, N)
        assert np.all(np.abs(got[m] - want) <= gamma(K) * mag + 1e-30)


# ---- internal/kernels/int4_test.go ------------------------------------------

def test_the_kernel_reads_what_the_quantizer_wrote():   # :31-85
    K, N = 256, 4
    rng = np.random.default_rng(1923)
    w = (0.75 + rng.random(K * N, np.float32) * np.float32(0.5)).astype(np.float32)
    a = np.sin(np.arange(K) * 0.37).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    out = oracle.quant_matvec_int4(a, p, s, z, K, N)
    for n in range(N):
        idx = np.arange(K) * N + n
        exact = float(np.dot(a.astype(np.float64), w[idx].astype(np.float64)))
        bound = oracle.int4_error_bound(a, s[idx // GROUP], z[idx // GROUP])
        bound += float(np.sum(np.abs(a.astype(np.float64) * w[idx]))) * 1e-6
        assert abs(float(out[n]) - exact) <= bound


def test_both_kernels_read_a_constant_group_as_the_quantizer_wrote_it():   # :99-182
    K, N, M = 2 * GROUP, 2, 3
    c = 0.75
    rng = np.random.default_rng(5359)
    w = np.where(np.arange(K * N) < GROUP, np.float32(c),
                 rng.random(K * N, np.float32) * 2 - 1).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    assert s[0] == 0 and oracle.f16_to_f32(z)[0] == np.float32(c)
    back = oracle.int4_dequantize(p, s, z, K * N).astype(np.float64).reshape(K, N)
    a = np.ones(M * K, np.float32)
    want = a.reshape(M, K).astype(np.float64) @ back
    mag = np.abs(a.reshape(M, K)).astype(np.float64) @ np.abs(back)
    row = oracle.quant_matvec_int4(a[:K], p, s, z, K, N)
    tiled = oracle.quant_matmul_int4(a, p, s, z, M, K, N)
    g = gamma(K - 1)
    assert np.all(np.abs(row - want[0]) <= g * mag[0])
    assert np.all(np.abs(tiled - want) <= g * mag)


def test_the_kernel_agrees_about_which_nibble_is_which():   # :189-228
    K, N = 8, 1
    w = np.ones(K, np.float32)
    w[0], w[1] = 0, 4
    a = np.zeros(K, np.float32)
    a[0], a[1] = 1, 10
    p, s, z = oracle.int4_quantize(w)
    got = float(oracle.quant_matvec_int4(a, p, s, z, K, N)[0])
    assert abs(got - 40) < abs(got - 4)
    assert abs(got - 40) <= 1


def test_the_tiled_kernel_matches_the_row_kernel():   # :291-350
    K, N, M = 200, 20, 13
    rng = np.random.default_rng(4143)
    w = (0.75 + rng.random(K * N, np.float32) * np.float32(0.5)).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    a = np.sin(np.arange(M * K) * 0.29).astype(np.float32)
    tiled = oracle.quant_matmul_int4(a, p, s, z, M, K, N)
    for m in range(M):
        row = oracle.quant_matvec_int4(a[m * K:(m + 1) * K], p, s, z, K, N)
        mag = np.abs(a[m * K:(m + 1) * K].astype(np.float64)) @ \
            np.abs(w.reshape(K, N).astype(np.float64))
        assert np.all(np.abs(tiled[m] - row) <= mag * 1e-6)


def _py_matvec_reference_order(a, p, s, z, K, N):
    """The lowering's order (accel_kernels.go:6748-6796) as scalar numpy f32."""
    f32 = np.float32
    sf = oracle.f16_to_f32(s)
    zf = oracle.f16_to_f32(z)
    out = np.zeros(N, f32)
    for col in range(N):
        phases = []
        for ly in range(16):
            acc = f32(0)
            for k in range(ly, K, 16):
                i = k * N + col
                code = f32((int(p[i // 8]) >> (4 * (i % 8))) & 0xF)
                g = i // 128
                wv = f32(f32(code - zf[g]) * sf[g])
                if sf[g] == 0:
                    wv = zf[g]
                acc = f32(acc + f32(a[k] * wv))
            phases.append(acc)
        tot = f32(0)
        for v in phases:
            tot = f32(tot + v)
        out[col] = tot
    return out


def test_matvec_is_bitwise_the_reference_order():
    K, N = 160, 40
    rng = np.random.default_rng(99)
    w = rng.standard_normal(K * N).astype(np.float32) * np.float32(0.02)
    p, s, z = oracle.int4_quantize(w)
    a = rng.standard_normal(K).astype(np.float32)
    got = oracle.quant_matvec_int4(a, p, s, z, K, N)
    want = _py_matvec_reference_order(a, p, s, z, K, N)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # and the threaded pool changes nothing
    got8 = oracle.quant_matvec_int4(a, p, s, z, K, N, threads=8)
    assert np.array_equal(got.view(np.uint32), got8.view(np.uint32))


def test_matmul_tile_order_is_bitwise_stable_across_threads():
    M, K, N = 19, 72, 48
    rng = np.random.default_rng(7)
    w = rng.standard_normal(K * N).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    a = rng.standard_normal(M * K).astype(np.float32)
    one = oracle.quant_matmul_int4(a, p, s, z, M, K, N, threads=1)
    many = oracle.quant_matmul_int4(a, p, s, z, M, K, N, threads=8)
    assert np.array_equal(one, many)
    # sequential within each 16-k tile, tiles in order: a numpy restatement
    f32 = np.float32
    wd = oracle.int4_dequantize(p, s, z, K * N).reshape(K, N)
    m, n = 5, 17
    acc = f32(0)
    for k in range(0, ((K + 15) // 16) * 16):
        av = a[m * K + k] if k < K else f32(0)
        bv = wd[k, n] if k < K else f32(0)
        acc = f32(acc + f32(av * bv))
    assert one[m, n] == acc


# ---- segment offsets ---------------------------------------------------------

def test_segment_offsets_is_the_exclusive_prefix_sum():
    counts = np.array([3, 0, 5, 2, 0, 7], np.uint32)
    off = oracle.segment_offsets(counts)
    assert list(off) == [0, 3, 3, 8, 10, 10, 17]
    big = np.array([0xFFFFFFFF, 2], np.uint32)  # wraps like Go's uint32
    assert list(oracle.segment_offsets(big)) == [0, 0xFFFFFFFF, 1]


# ---- internal/kernels/grouped_test.go ---------------------------------------

def grouped_fixture(E, K, N, counts):
    """grouped_test.go:26-50"""
    off = oracle.segment_offsets(np.array(counts, np.uint32))
    total = int(off[E])
    x = np.sin(np.arange(total * K) * 0.23).astype(np.float32)
    w = np.zeros(E * K * N, np.float32)
    base = np.cos(np.arange(K * N) * 0.17).astype(np.float32)
    for e in range(E):
        w[e * K * N:(e + 1) * K * N] = base * np.float32(e + 1)
    return x, w, off


def _expert_ref(x, w, tok, e, K, N):
    return x[tok * K:(tok + 1) * K].astype(np.float64) @ \
        w[e * K * N:(e + 1) * K * N].reshape(K, N).astype(np.float64)


def test_a_grouped_product_matches_each_expert_alone():   # :65-92
    E, K, N = 3, 64, 5
    x, w, off = grouped_fixture(E, K, N, [2, 1, 3])
    T = int(off[E])
    got = oracle.grouped_matvec(x, w, off, E, T, K, N)
    for e in range(E):
        for tok in range(off[e], off[e + 1]):
            assert np.all(np.abs(got[tok] - _expert_ref(x, w, tok, e, K, N)) <= 1e-4)


def test_a_grouped_product_accepts_an_empty_expert():   # :94-122
    E, K, N = 4, 64, 3
    x, w, off = grouped_fixture(E, K, N, [2, 0, 2, 0])
    got = oracle.grouped_matvec(x, w, off, E, int(off[E]), K, N)
    assert got.shape == (4, N)
    assert np.all(np.abs(got[2] - _expert_ref(x, w, 2, 2, K, N)) <= 1e-4)


def test_a_grouped_product_uses_the_expert_it_looked_up():   # :124-155
    E, K, N = 2, 64, 2
    x, w, off = grouped_fixture(E, K, N, [1, 1])
    got = oracle.grouped_matvec(x, w, off, E, 2, K, N)
    for tok, e in enumerate([0, 1]):
        mine = _expert_ref(x, w, tok, e, K, N)
        theirs = _expert_ref(x, w, tok, 1 - e, K, N)
        assert np.all(np.abs(got[tok] - mine) <= 1e-4)
        assert np.all(np.abs(mine - theirs) >= 1e-3)


def test_a_grouped_token_past_the_last_expert_is_padding():   # :188-267
    E, K, N = 3, 64, 4
    x, w, _ = grouped_fixture(E, K, N, [2, 1, 2])
    short = np.array([0, 2, 2, 4], np.uint32)
    rows = 5
    got = oracle.grouped_matvec(x, w, short, E, rows, K, N,
                                out=np.full(rows * N, 7.0, np.float32))
    for e in range(E):
        for tok in range(short[e], short[e + 1]):
            assert np.all(np.abs(got[tok] - _expert_ref(x, w, tok, e, K, N)) <= 1e-4)
    assert np.all(got[4] == 0)


def test_the_tiled_grouped_product_matches_the_row_kernel():   # :269-302
    E, K, N = 4, 40, 20
    x, w, off = grouped_fixture(E, K, N, [11, 0, 3, 20])
    T = int(off[E])
    want = oracle.grouped_matvec(x, w, off, E, T, K, N)
    got = oracle.grouped_matmul(x, w, off, E, T, K, N)
    assert np.all(np.abs(got - want) <= 1e-4)


def test_a_tiled_grouped_product_clamps_counts_past_the_rows():   # :304-336
    E, K, N = 2, 40, 20
    x, w, off = grouped_fixture(E, K, N, [4, 4])
    T = int(off[E])
    over = np.array([0, 4, 16], np.uint32)
    got = oracle.grouped_matmul(x, w, over, E, T, K, N)
    for tok in range(4, T):
        assert np.all(np.abs(got[tok] - _expert_ref(x, w, tok, 1, K, N)) <= 1e-4)


def test_the_matmul_form_leaves_uncovered_rows_alone():
    E, K, N = 2, 16, 16
    x, w, _ = grouped_fixture(E, K, N, [3, 3])
    off = np.array([0, 2, 4], np.uint32)
    got = oracle.grouped_matmul(x, w, off, E, 6, K, N, out=np.full(6 * N, 7.0, np.float32))
    assert np.all(got[4:] == 7.0)


# ---- the int4 composition ---------------------------------------------------

@pytest.mark.parametrize("form", ["matvec", "matmul"])
def test_int4_grouped_is_grouped_over_the_dequantized_weights(form):
    E, K, N = 3, 64, 32
    rng = np.random.default_rng(31)
    counts = [5, 0, 9]
    off = oracle.segment_offsets(np.array(counts, np.uint32))
    T = int(off[E]) + 2  # two padding rows
    x = rng.standard_normal(T * K).astype(np.float32)
    w = (rng.standard_normal(E * K * N) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    wd = oracle.int4_dequantize(p, s, z, E * K * N)
    init = np.full(T * N, 3.0, np.float32)
    if form == "matvec":
        got = oracle.int4_grouped_matvec(x, p, s, z, off, E, T, K, N, out=init)
        want = oracle.grouped_matvec(x, wd, off, E, T, K, N, out=init)
    else:
        got = oracle.int4_grouped_matmul(x, p, s, z, off, E, T, K, N, out=init)
        want = oracle.grouped_matmul(x, wd, off, E, T, K, N, out=init)
    assert np.array_equal(got, want)  # same weights, same order: bitwise
