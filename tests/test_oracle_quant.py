"""Pins the oracle's packer against the reference's own tests
(quant/int4_test.go) and against the independent numpy restatement.

The reference draws its inputs from Go's PCG; these tests use numpy's with
the same spans and structure, since every assertion is a property or a bound
that holds for any draw.  Where a test has a known answer (nibble order,
constant groups, odd length) the answer is asserted exactly.
"""
import numpy as np
import pytest

import oracle
from oracle import oracle_np

GROUP = 128


def q(w):
    return oracle.int4_quantize(np.asarray(w, np.float32))


# quant/int4_test.go:22-36
@pytest.mark.parametrize("c", [0.0, 1.0, -2.5, 0.125])
def test_a_constant_group_reconstructs_exactly(c):
    w = np.full(GROUP, c, np.float32)
    p, s, z = q(w)
    assert s[0] == 0 and oracle.f16_to_f32(z)[0] == np.float32(c)
    assert np.array_equal(oracle.int4_dequantize(p, s, z, GROUP), w)


# quant/int4_test.go:46-88
@pytest.mark.parametrize("lo,hi", [(-1, 1), (0.9, 1.0), (-3, -2.75), (-0.25, 4),
                                   (1000, 1001), (-2000, -1999)])
def test_reconstruction_is_inside_its_derived_bound(lo, hi):
    rng = np.random.default_rng(711)
    n = 3 * GROUP + 17
    w = (np.float32(lo) + rng.random(n, np.float32) * np.float32(hi - lo)).astype(np.float32)
    for g in range(0, n, GROUP):
        w[g] = lo
        w[min(g + 1, n - 1)] = hi
    p, s, z = q(w)
    back = oracle.int4_dequantize(p, s, z, n)
    for i in range(n):
        g = i // GROUP
        bound = oracle.int4_error_bound([1.0], s[g:g + 1], z[g:g + 1])
        assert abs(float(w[i]) - float(back[i])) <= bound, (i, w[i], back[i], bound)


# quant/int4_test.go:102-158
@pytest.mark.parametrize("lo,hi,exceeds_old", [(1000, 1001, True), (0.9, 1.0, False)])
def test_error_bound_holds_where_the_zero_point_rounds(lo, hi, exceeds_old):
    rng = np.random.default_rng(1317)
    n = 2 * GROUP + 17
    w = (np.float32(lo) + rng.random(n, np.float32) * np.float32(hi - lo)).astype(np.float32)
    x = np.zeros(n, np.float32)
    for g in range(0, n, GROUP):
        a, b = g, min(g + 1, n - 1)
        w[a], w[b] = lo, hi
        x[a], x[b] = 1, 1
    p, s, z = q(w)
    back = oracle.int4_dequantize(p, s, z, n)
    exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
    quantized = float(np.dot(back.astype(np.float64), x.astype(np.float64)))
    old = float(np.sum(np.abs(x.astype(np.float64)) * (np.float64(np.float32(hi - lo)) / 30)))
    ts = s[np.arange(n) // GROUP]
    tz = z[np.arange(n) // GROUP]
    bound = oracle.int4_error_bound(x, ts, tz)
    err = abs(quantized - exact)
    assert err <= bound
    if exceeds_old:
        assert err > old, "the fixture no longer reaches the zero point's rounding"
    ceiling = float(np.sum(np.abs(x.astype(np.float64)) * np.float64(np.float32(hi - lo))))
    assert bound <= ceiling


# quant/int4_test.go:166-219
def test_int4_beats_int8_clustered_and_loses_centred():
    rng = np.random.default_rng(35)
    w = (0.9 + rng.random(GROUP, np.float32) * np.float32(0.1)).astype(np.float32)
    p, s, z = q(w)
    worst4 = np.max(np.abs(w - oracle.int4_dequantize(p, s, z, GROUP)))
    q8, s8 = oracle.int8_quantize(w)
    worst8 = np.max(np.abs(w - oracle.int8_dequantize(q8, s8)))
    assert worst4 < worst8

    w = (-1 + rng.random(GROUP, np.float32) * np.float32(2)).astype(np.float32)
    p, s, z = q(w)
    worst4 = np.max(np.abs(w - oracle.int4_dequantize(p, s, z, GROUP)))
    q8, s8 = oracle.int8_quantize(w)
    worst8 = np.max(np.abs(w - oracle.int8_dequantize(q8, s8)))
    assert worst4 > worst8


# quant/int4_test.go:225-253
def test_packing_round_trips_at_an_odd_length():
    n = GROUP + 1
    w = (np.arange(n) % 16).astype(np.float32) / 4
    p, s, z = q(w)
    assert p.size == (n + 7) // 8
    back = oracle.int4_dequantize(p, s, z, n)
    assert back.size == n
    assert back[-1] == w[-1]  # alone in its group, so exact


# quant/int4_test.go:261-286
def test_packs_low_nibble_first():
    w = np.full(GROUP, 0.5, np.float32)
    w[0], w[1] = 0, 10
    p, _, _ = q(w)
    assert oracle.int4_nibble(p, 0) == 0
    assert oracle.int4_nibble(p, 1) == 15
    assert p[0] & 0xFF == 0xF0


# quant/int4_test.go:291-310
def test_error_bound_needs_one_scale_and_zero_per_term():
    three = oracle.to_f16(np.ones(3, np.float32))
    with pytest.raises(ValueError):
        oracle.int4_error_bound([1, 2, 3], three[:2], three)
    with pytest.raises(ValueError):
        oracle.int4_error_bound([1, 2, 3], three, three[:2])


# specs/048-int4.md:45-47 -- q=0 reconstructs the minimum, q=15 the maximum
def test_endpoints_reconstruct_near_min_and_max():
    rng = np.random.default_rng(5)
    w = rng.standard_normal(GROUP).astype(np.float32)
    p, s, z = q(w)
    lo_i, hi_i = int(np.argmin(w)), int(np.argmax(w))
    assert oracle.int4_nibble(p, lo_i) == 0
    assert oracle.int4_nibble(p, hi_i) == 15
    back = oracle.int4_dequantize(p, s, z, GROUP)
    step = float(oracle.f16_to_f32(s)[0])
    assert abs(back[lo_i] - w[lo_i]) <= step and abs(back[hi_i] - w[hi_i]) <= step


def test_scale_underflow_takes_the_constant_path():
    # range 2^-30: s = range/15 underflows f16 to zero, so z carries the min
    w = np.full(GROUP, 1e-3, np.float32)
    w[5] = np.float32(1e-3) + np.float32(2.0 ** -30)
    p, s, z = q(w)
    assert s[0] == 0 and np.all(p == 0)
    assert oracle.f16_to_f32(z)[0] == oracle.f16_to_f32(oracle.to_f16(np.float32(1e-3)))[0]


ADVERSARIAL = [
    ("normal", lambda r, n: r.standard_normal(n) * 0.02),
    ("far", lambda r, n: 1000 + r.random(n)),
    ("tiny", lambda r, n: r.standard_normal(n) * 1e-7),
    ("denorm", lambda r, n: r.standard_normal(n) * 1e-40),
    ("huge", lambda r, n: r.standard_normal(n) * 1e30),
    ("ties", lambda r, n: np.round(r.standard_normal(n) * 8) / 8),
    ("signed_zero", lambda r, n: np.where(r.random(n) < 0.5, -0.0, 0.0)),
    ("nan_inf", lambda r, n: np.where(r.random(n) < 0.02, np.nan,
                                      np.where(r.random(n) < 0.02, np.inf, r.standard_normal(n)))),
]


@pytest.mark.parametrize("name,gen", ADVERSARIAL)
@pytest.mark.parametrize("n", [1, 7, 128, 129, 1000, 4096 + 3])
def test_c_and_numpy_restatements_agree_bit_for_bit(name, gen, n):
    rng = np.random.default_rng(hash((name, n)) & 0xFFFF)
    w = np.asarray(gen(rng, n), np.float32)
    a = oracle.int4_quantize(w)
    b = oracle_np.int4_quantize(w)
    for x, y, what in zip(a, b, ("codes", "scales", "zeros")):
        assert x.dtype == y.dtype and np.array_equal(x, y), what


def test_nibbles_past_the_count_are_zero():
    w = np.linspace(-1, 1, 13).astype(np.float32)
    p, _, _ = q(w)
    assert p.size == 2 and (p[1] >> (4 * 5)) == 0
