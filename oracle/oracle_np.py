"""Independent numpy restatement of quant.Int4Quantize -- TEST INFRASTRUCTURE ONLY.

Written separately from oracle.c so the two can check each other bit for bit.
Vectorised over groups; the f16 narrowing uses numpy's own float16 cast and
then applies the reference's one departure from IEEE RNE (see ``to_f16``).

Follows quant/int4.go:71-138 and internal/kernel/narrow.go:67-106.
"""
from __future__ import annotations

import numpy as np

GROUP = 128


def to_f16(x) -> np.ndarray:
    """f32 -> f16 bits as the reference narrows (narrow.go:67-106).

    numpy rounds to nearest-even like the reference, except where the
    reference's ``exp < -24`` branch returns a signed zero: magnitudes in
    (2^-25, 2^-24), which IEEE rounds up to the smallest subnormal.  NaN
    becomes the canonical 0x7e00.
    """
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        h = x.astype(np.float16).view(np.uint16)
    b = x.view(np.uint32)
    mag = b & np.uint32(0x7FFFFFFF)
    h = np.where(mag < np.uint32(0x33800000), (b >> np.uint32(16)) & np.uint32(0x8000),
                 h).astype(np.uint16)
    h = np.where(mag > np.uint32(0x7F800000), np.uint16(0x7E00), h).astype(np.uint16)
    return h


def f16_to_f32(h) -> np.ndarray:
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float32)


def int4_quantize(w):
    """Returns (packed u32, scales f16 bits, zeros f16 bits)."""
    w = np.ascontiguousarray(w, np.float32).ravel()
    n = w.size
    groups = (n + GROUP - 1) // GROUP
    padded = np.full(groups * GROUP, np.nan, np.float32)
    padded[:n] = w
    blk = padded.reshape(groups, GROUP)
    valid = np.arange(groups * GROUP).reshape(groups, GROUP) < n
    # min/max over the valid part of each group.  A NaN weight makes the
    # reference's comparisons false, so it never becomes the min or max unless
    # it is the group's first weight; replicate that with explicit masking.
    first = blk[:, 0]
    lo = first.copy()
    hi = first.copy()
    for j in range(GROUP):
        v = blk[:, j]
        ok = valid[:, j]
        lo = np.where(ok & (v < lo), v, lo)
        hi = np.where(ok & (v > hi), v, hi)
    const = hi == lo
    with np.errstate(over="ignore", invalid="ignore"):
        s = ((hi - lo) / np.float32(15)).astype(np.float32)
    s_bits = to_f16(s)
    s_bits = np.where(const, to_f16(np.float32(0.0)), s_bits).astype(np.uint16)
    s16 = f16_to_f32(s_bits)
    flat = (~const) & (s16 == 0)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        z = (-lo / s16).astype(np.float32)
    z_bits = to_f16(z)
    z_bits = np.where(const | flat, to_f16(lo), z_bits).astype(np.uint16)
    z16 = f16_to_f32(z_bits)
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        q = np.rint(blk.astype(np.float64) / s16.astype(np.float64)[:, None]
                    + z16.astype(np.float64)[:, None])
    q = np.where(q > 15, 15.0, q)
    q = np.where(q < 0, 0.0, q)
    q = np.where(np.isnan(q), 0.0, q)
    codes = q.astype(np.uint32)
    codes = np.where((const | flat)[:, None] | ~valid, np.uint32(0), codes)
    # groups*128 is a multiple of 8 and at least n, so it covers every word
    nib = codes.ravel()[: ((n + 7) // 8) * 8].reshape(-1, 8)
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))[None, :]
    packed = np.bitwise_or.reduce(nib << shifts, axis=1).astype(np.uint32)
    return packed, s_bits, z_bits
