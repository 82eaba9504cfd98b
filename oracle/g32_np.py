"""Config 1's literal weight format -- TEST INFRASTRUCTURE ONLY.

BASELINE config 1 describes its weights as "int4 with group size 32 along K,
per-group f32 scale, packed by quant/int4".  The reference has no such
format (its groups are 128 consecutive flat weights with an f16 scale and an
f16 zero, quant/int4.go:29,71-138), so this is the definition the build's
additive variant is checked against, not a restatement of reference code
(parity unpinned against the reference: there is nothing to pin it to).

Definition, for a weight [K, N] (element (k, n) at flat index k*N + n) with
K % 32 == 0:
  * group (g, n) is rows 32g .. 32g+31 of column n;
  * s = f32(amax / 7) with amax = max |w| over the group (f32); a group of
    zeros has s = 0;
  * q = clamp(rne(f32(w / s)), -8, 7) + 8 (codes 0..15; a zero group codes 8);
  * codes packed as quant/int4 packs them: nibble (k*N + n) % 8 of u32 word
    (k*N + n) / 8, low nibble first (quant/int4.go:141-153);
  * w' = (q - 8) * s.
Finite weights only (a NaN orders differently in numpy's max and C's fmaxf).
"""
from __future__ import annotations

import numpy as np

GROUP = 32


def quantize_g32(w: np.ndarray):
    """w f32 [K, N] -> (packed u32 [K*N/8], scales f32 [K/32, N])."""
    w = np.ascontiguousarray(w, np.float32)
    K, N = w.shape
    assert K % GROUP == 0 and (K * N) % 8 == 0
    g = w.reshape(K // GROUP, GROUP, N)
    amax = np.abs(g).max(axis=1)                                  # [K/32, N] f32
    s = (amax / np.float32(7.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint((g / s[:, None, :]).astype(np.float32))
    r = np.where(s[:, None, :] == 0, 0.0, r)
    q = (np.clip(r, -8, 7) + 8).astype(np.uint32).reshape(K * N)
    packed = np.zeros(K * N // 8, np.uint32)
    for j in range(8):
        packed |= q[j::8] << np.uint32(4 * j)
    return packed, s


def dequantize_g32(packed: np.ndarray, scales: np.ndarray, K: int, N: int) -> np.ndarray:
    """(packed, scales) -> w' f32 [K, N] = (q - 8) * s."""
    q = np.empty(K * N, np.uint32)
    for j in range(8):
        q[j::8] = (packed >> np.uint32(4 * j)) & np.uint32(0xF)
    q = q.reshape(K // GROUP, GROUP, N).astype(np.float32) - np.float32(8.0)
    return (q * scales[:, None, :]).reshape(K, N).astype(np.float32)


def matvec_g32(x: np.ndarray, packed: np.ndarray, scales: np.ndarray, K: int, N: int):
    """x [K] @ w' in f64: the product the variant's GEMV is held to."""
    w = dequantize_g32(packed, scales, K, N).astype(np.float64)
    return np.asarray(x, np.float64) @ w
