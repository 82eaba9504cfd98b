"""Numpy restatements of the published 4-bit packers -- TEST INFRASTRUCTURE ONLY.

They build AWQ and GPTQ layers from integer codes, integer zeros and f16
scales, the way the published tools write them, so that the oracle's unpack
(``orc_foreign_dequant``) and the library's repack can be checked against a
packing written separately from either.  The tools themselves are not part of
the reference (which names reading their files as unbuilt,
specs/048-int4.md:126-131,167), so the loops below restate them:

* AutoAWQ 0.2, "gemm" version (its WQLinear_GEMM packer): intweight [K, N];
  for each word column j and each i in 0..7, word (k, j) |= intweight[k,
  8j + order[i]] << 4i with order = [0, 2, 4, 6, 1, 3, 5, 7]; zeros [groups,
  N] are packed the same way; scales are [groups, N].
* AutoGPTQ 0.7 (its QuantLinear packer, checkpoint format "gptq"): qweight
  [K/8, N] with row (i, n) |= intweight[8i + j, n] << 4j; zeros are decreased
  by one and packed along N, word (g, j) |= (zeros[g, 8j + c] - 1) << 4c, in
  32-bit unsigned arithmetic (a zero of 0 becomes 0xffffffff and fills the
  word's higher nibbles, as the published packer does); "gptq_v2" (GPTQModel)
  stores the zeros themselves.
"""
from __future__ import annotations

import numpy as np

AWQ_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]


def pack_awq(q: np.ndarray, z: np.ndarray):
    """q [K, N] and z [groups, N] integer codes -> (qweight [K, N/8],
    qzeros [groups, N/8]) as u32."""
    q = np.asarray(q, np.int64)
    z = np.asarray(z, np.int64)
    K, N = q.shape
    qweight = np.zeros((K, N // 8), np.uint32)
    for col in range(N // 8):
        for i in range(8):
            qweight[:, col] |= (q[:, col * 8 + AWQ_ORDER[i]].astype(np.uint32) << np.uint32(4 * i))
    qzeros = np.zeros((z.shape[0], N // 8), np.uint32)
    for col in range(N // 8):
        for i in range(8):
            qzeros[:, col] |= (z[:, col * 8 + AWQ_ORDER[i]].astype(np.uint32) << np.uint32(4 * i))
    return qweight, qzeros


def pack_gptq(q: np.ndarray, z: np.ndarray, v2: bool = False):
    """q [K, N] and z [groups, N] integer codes -> (qweight [K/8, N],
    qzeros [groups, N/8]) as u32, zeros stored z - 1 unless v2."""
    q = np.asarray(q, np.int64)
    K, N = q.shape
    intweight = q.astype(np.uint32)
    qweight = np.zeros((K // 8, N), np.uint32)
    i = 0
    row = 0
    while row < qweight.shape[0]:
        for j in range(i, i + 8):
            qweight[row] |= intweight[j] << np.uint32(4 * (j - i))
        i += 8
        row += 1
    zeros = np.asarray(z, np.int64)
    if not v2:
        zeros = zeros - 1
    zeros = (zeros & 0xFFFFFFFF).astype(np.uint32)
    qzeros = np.zeros((zeros.shape[0], N // 8), np.uint32)
    i = 0
    col = 0
    while col < qzeros.shape[1]:
        for j in range(i, i + 8):
            qzeros[:, col] |= zeros[:, j] << np.uint32(4 * (j - i))
        i += 8
        col += 1
    return qweight, qzeros
