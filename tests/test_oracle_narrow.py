"""Pins the oracle's f16/bf16 conversions (internal/kernel/narrow.go:67-176).

ToFloat16 is checked over every one of the 2^32 f32 bit patterns against the
host's hardware RNE conversion (F16C), which would catch a dropped carry, a
wrong subnormal shift or a wrong overflow threshold.  The one range where
the reference is not IEEE RNE -- magnitudes in (2^-25, 2^-24), which its
``exp < -24`` branch returns as a signed zero -- is counted separately and
asserted to be exactly that range.
"""
import concurrent.futures as cf
import ctypes

import numpy as np
import pytest

import oracle
from oracle import oracle_np


def _check_chunk(lo, hi):
    L = oracle.lib()
    fl = ctypes.c_int64(0)
    fb = ctypes.c_uint64(0)
    bad = L.orc_check_f16_range(lo, hi, ctypes.byref(fl), ctypes.byref(fb))
    return bad, fl.value, fb.value


@pytest.mark.slow
def test_to_f16_is_rne_over_every_f32_pattern():
    if not hasattr(oracle.lib(), "orc_check_f16_range"):
        pytest.skip("exhaustive check needs an x86-64 host with F16C")
    step = 1 << 27
    chunks = [(i, min(i + step, 1 << 32)) for i in range(0, 1 << 32, step)]
    with cf.ThreadPoolExecutor(8) as ex:
        results = list(ex.map(lambda c: _check_chunk(*c), chunks))
    bad = sum(r[0] for r in results)
    flushed = sum(r[1] for r in results)
    assert bad == 0, f"{bad} patterns differ from RNE, first {[r[2] for r in results if r[0]]}"
    # (2^-25, 2^-24) exclusive, both signs: mantissas 1..2^23-1 at exponent -25
    assert flushed == 2 * ((1 << 23) - 1)


def test_the_flush_range_is_the_reference_branch():
    tiny = np.array([2.0**-25 * 1.5, -(2.0**-25) * 1.0000001, 2.0**-24, 2.0**-25],
                    np.float32)
    h = oracle.to_f16(tiny)
    assert h[0] == 0x0000 and h[1] == 0x8000  # flushed, sign kept
    assert h[2] == 0x0001                       # 2^-24 is representable
    assert h[3] == 0x0000                       # the tie goes to even (zero)


def test_to_f16_specials():
    cases = [
        (0.0, 0x0000), (-0.0, 0x8000), (1.0, 0x3C00), (-2.0, 0xC000), (65504.0, 0x7BFF),
        (65520.0, 0x7C00),           # rounds up out of range -> inf
        (65519.996, 0x7BFF),
        (float("inf"), 0x7C00), (float("-inf"), 0xFC00),
        (1.9997, 0x4000),            # the mantissa carry moves into the exponent
        (2.0**-14, 0x0400), (2.0**-24, 0x0001), (1e30, 0x7C00), (-1e30, 0xFC00),
    ]
    for x, want in cases:
        assert oracle.to_f16(np.float32(x))[0] == want, (x, hex(oracle.to_f16(x)[0]))
    nan = np.array([np.nan, -np.nan], np.float32)
    nan[1] = np.frombuffer(np.uint32(0xFFC00001).tobytes(), np.float32)[0]
    assert list(oracle.to_f16(nan)) == [0x7E00, 0x7E00]


def test_f16_widening_is_exact_for_every_pattern():
    h = np.arange(1 << 16, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = oracle.f16_to_f32(h)
    finite = np.isfinite(want) | np.isinf(want)
    assert np.array_equal(got.view(np.uint32)[finite], want.view(np.uint32)[finite])
    # NaNs widen with their payload (narrow.go:133-135)
    nanmask = ~finite
    assert np.all(np.isnan(got[nanmask]))
    assert np.array_equal(got.view(np.uint32)[nanmask] & 0x7FFFE000,
                          ((h[nanmask].astype(np.uint32) & 0x7FFF) << 13) | 0x7F800000)


def test_to_bf16_is_rne_against_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 1 << 32, size=1 << 22, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000, 0xFF800000,
                        0x00000001, 0x3F808000, 0x3F818000, 0x3F80FFFF, 0x7F7F8000],
                       np.uint32)
    bits = np.concatenate([bits, special])
    x = bits.view(np.float32)
    got = oracle.to_bf16(x)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)
    isnan = np.isnan(x)
    assert np.array_equal(got[~isnan], want[~isnan])
    assert np.all(got[isnan] == 0x7FC0)


def test_numpy_restatement_agrees_on_narrowing(rng):
    x = rng.standard_normal(1 << 16).astype(np.float32) * np.float32(2.0) ** \
        rng.integers(-30, 20, 1 << 16).astype(np.float32)
    assert np.array_equal(oracle.to_f16(x), oracle_np.to_f16(x))
