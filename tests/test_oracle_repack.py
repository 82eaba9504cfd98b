"""Published 4-bit layers (AWQ, GPTQ) into the reference int4 format, on the CPU.

The reference names reading these files as unbuilt (specs/048-int4.md:126-131,
167), so there is no reference code or fixture to match; the repack is pinned
by:

* round trips through independent numpy restatements of the published packers
  (``oracle/foreign_np.py``): the oracle's unpack must give back exactly
  (q - z) * s for every weight, in every format, with and without act-order;
* a closed form: where each reference group (128 consecutive weights of a row)
  shares one published (scale, zero) and spans all sixteen codes, the
  reference quantizer must return those codes, that scale and that zero
  exactly -- a wrong nibble order, column permutation or zero offset fails it;
* the reference's own error bound (Int4ErrorBound, quant/int4.go:177-250) for
  the second rounding everywhere else;
* the library's host repack against the oracle's, bit for bit, and its
  refusals.
"""
import ctypes

import numpy as np
import pytest

import accel_amd
import oracle
from oracle import foreign_np

AWQ, GPTQ, GPTQ2 = 1, 2, 3


def _random_layer(rng, fmt, K, N, G, act_order=False, zmin=0):
    groups = -(-K // G)
    q = rng.integers(0, 16, (K, N))
    z = rng.integers(zmin, 16, (groups, N))
    s = oracle.to_f16((rng.random((groups, N)) * 0.02 + 1e-3).astype(np.float32)).reshape(groups, N)
    g_idx = None
    if act_order:
        g_idx = (np.arange(K) // G).astype(np.int32)
        rng.shuffle(g_idx)
    if fmt == AWQ:
        qw, qz = foreign_np.pack_awq(q, z)
    else:
        qw, qz = foreign_np.pack_gptq(q, z, v2=fmt == GPTQ2)
    return q, z, s, g_idx, qw, qz


def _expected_weights(q, z, s, g_idx, G):
    K = q.shape[0]
    g = g_idx if g_idx is not None else np.arange(K) // G
    sf = oracle.f16_to_f32(s.reshape(-1)).reshape(s.shape)
    return ((q - z[g]).astype(np.float32) * sf[g]).astype(np.float32)


@pytest.mark.parametrize("fmt,K,N,G,act", [
    (AWQ, 256, 64, 128, False), (AWQ, 96, 40, 32, False),
    (GPTQ, 256, 64, 128, False), (GPTQ, 200, 24, 64, False), (GPTQ, 256, 64, 32, True),
    (GPTQ2, 256, 64, 128, False), (GPTQ2, 128, 16, 128, True),
])
def test_unpack_round_trips_the_published_packers(fmt, K, N, G, act):
    rng = np.random.default_rng(fmt * 100 + K + N + G)
    # the first GPTQ format stores z - 1, and a zero of 0 corrupts the word
    # (tested below); round trips use zeros from 1 there
    q, z, s, g_idx, qw, qz = _random_layer(rng, fmt, K, N, G, act, zmin=1 if fmt == GPTQ else 0)
    got = oracle.foreign_dequant(fmt, K, N, G, qw, qz, s, g_idx)
    want = _expected_weights(q, z, s, g_idx, G)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_awq_column_order_is_not_the_identity():
    # one column set: the packer puts column 1 in nibble 4, not nibble 1
    q = np.zeros((8, 8), np.int64)
    q[:, 1] = 9
    qw, _ = foreign_np.pack_awq(q, np.zeros((1, 8), np.int64))
    assert np.all(qw[:, 0] == np.uint32(9 << 16))
    got = oracle.foreign_dequant(AWQ, 8, 8, 8, qw, np.zeros((1, 1), np.uint32),
                                 oracle.to_f16(np.ones(8, np.float32)))
    assert np.all(got[:, 1] == 9) and np.all(got[:, [0, 2, 3, 4, 5, 6, 7]] == 0)


def test_gptq_zero_of_zero_corrupts_the_higher_nibbles():
    # the published packer stores z - 1 in unsigned 32-bit arithmetic: a zero
    # of 0 becomes 0xffffffff and fills its own and the higher nibbles, so
    # readers see 16 there; the unpack reads what the file holds
    K, N = 8, 8
    z = np.full((1, N), 5)
    z[0, 3] = 0
    qw, qz = foreign_np.pack_gptq(np.zeros((K, N), np.int64), z)
    assert qz[0, 0] == np.uint32(0xFFFFF444)
    got = oracle.foreign_dequant(GPTQ, K, N, K, qw, qz, oracle.to_f16(np.ones(N, np.float32)))
    assert np.all(got[:, :3] == -5) and np.all(got[:, 3:] == -16)


def _aligned_layer(rng, fmt, K, N, G):
    """Reference groups (128 columns of a row) that share one published
    (scale, zero) and use codes 0 and 15."""
    groups = K // G
    blocks = N // 128
    sb = oracle.to_f16((np.exp2(rng.integers(-9, 0, (groups, blocks)))
                        * (1 + rng.integers(0, 64, (groups, blocks)) / 64)).astype(np.float32))
    sb = sb.reshape(groups, blocks)
    zb = rng.integers(0, 16, (groups, blocks))
    s = np.repeat(sb, 128, axis=1)
    z = np.repeat(zb, 128, axis=1)
    q = rng.integers(0, 16, (K, N))
    q[:, 0::128] = 0
    q[:, 1::128] = 15
    if fmt == AWQ:
        qw, qz = foreign_np.pack_awq(q, z)
    else:
        qw, qz = foreign_np.pack_gptq(q, z, v2=fmt == GPTQ2)
    return q, z, s, qw, qz


def _reference_codes(q):
    flat = q.reshape(-1).astype(np.uint32)
    codes = np.zeros((flat.size + 7) // 8, np.uint32)
    for j in range(8):
        codes |= flat[j::8] << np.uint32(4 * j)
    return codes


@pytest.mark.parametrize("fmt", [AWQ, GPTQ2])
def test_the_repack_is_lossless_where_the_grids_agree(fmt):
    K, N, G = 256, 384, 128
    rng = np.random.default_rng(fmt)
    q, z, s, qw, qz = _aligned_layer(rng, fmt, K, N, G)
    codes, scales, zeros = oracle.int4_repack(fmt, K, N, G, qw, qz, s)
    assert np.array_equal(codes, _reference_codes(q))
    g = np.arange(K) // G
    want_s = s[g][:, ::128].reshape(-1)          # one per (row, 128-column block)
    want_z = z[g][:, ::128].reshape(-1).astype(np.float32)
    assert np.array_equal(scales, want_s)
    assert np.array_equal(oracle.f16_to_f32(zeros), want_z)


def test_the_repack_is_lossless_for_first_format_gptq_too():
    # z from 1 (the first format's z - 1 cannot hold a zero of 0)
    K, N, G = 128, 256, 64
    rng = np.random.default_rng(11)
    q, z, s, _, _ = _aligned_layer(rng, GPTQ, K, N, G)
    z = np.maximum(z, 1)
    qw, qz = foreign_np.pack_gptq(q, z)
    codes, scales, zeros = oracle.int4_repack(GPTQ, K, N, G, qw, qz, s)
    assert np.array_equal(codes, _reference_codes(q))
    g = np.arange(K) // G
    assert np.array_equal(oracle.f16_to_f32(zeros), z[g][:, ::128].reshape(-1).astype(np.float32))


@pytest.mark.parametrize("fmt,act", [(AWQ, False), (GPTQ, False), (GPTQ2, True)])
def test_the_second_rounding_is_within_the_reference_bound(fmt, act):
    K, N, G = 128, 256, 32
    rng = np.random.default_rng(fmt + 40)
    q, z, s, g_idx, qw, qz = _random_layer(rng, fmt, K, N, G, act, zmin=1 if fmt == GPTQ else 0)
    w = oracle.foreign_dequant(fmt, K, N, G, qw, qz, s, g_idx).reshape(-1)
    codes, scales, zeros = oracle.int4_repack(fmt, K, N, G, qw, qz, s, g_idx)
    back = oracle.int4_dequantize(codes, scales, zeros, K * N)
    for grp in range(K * N // 128):
        sl = slice(128 * grp, 128 * grp + 128)
        bound = oracle.int4_error_bound([1.0], scales[grp:grp + 1], zeros[grp:grp + 1])
        assert np.abs(back[sl].astype(np.float64) - w[sl]).max() <= bound


@pytest.mark.parametrize("fmt,K,N,G,act", [
    (AWQ, 256, 128, 128, False), (AWQ, 64, 40, 16, False),       # 40 columns: groups straddle rows
    (GPTQ, 256, 136, 128, False), (GPTQ, 200, 64, 64, False),    # K not a multiple of G
    (GPTQ, 128, 256, 32, True), (GPTQ2, 256, 128, 128, True), (GPTQ2, 64, 8, 64, False),
])
def test_host_repack_is_the_oracle_bit_for_bit(fmt, K, N, G, act):
    rng = np.random.default_rng(fmt * 7 + K + N + G)
    _, _, s, g_idx, qw, qz = _random_layer(rng, fmt, K, N, G, act)
    want = oracle.int4_repack(fmt, K, N, G, qw, qz, s, g_idx)
    layer = accel_amd.ForeignInt4(fmt, G, K, N, qw, qz, s, g_idx)
    got = accel_amd.int4_repack_host(layer)
    for a, b in zip(got, want):
        assert np.array_equal(a, b)


def _refusal(layer):
    n = layer.K * layer.N
    c = np.zeros(max(1, (n + 7) // 8), np.uint32)
    s = np.zeros(max(1, (n + 127) // 128), np.uint16)
    z = np.zeros_like(s)
    d = layer.desc()
    rc = accel_amd.lib().accel_int4_repack_host(ctypes.byref(d), c.ctypes.data, s.ctypes.data,
                                                z.ctypes.data)
    return rc, accel_amd.last_error()


def test_host_repack_refusals():
    rng = np.random.default_rng(3)
    _, _, s, _, qw, qz = _random_layer(rng, GPTQ, 64, 16, 32)
    ok = accel_amd.ForeignInt4(GPTQ, 32, 64, 16, qw, qz, s)
    assert _refusal(ok)[0] == 0
    cases = [
        (accel_amd.ForeignInt4(7, 32, 64, 16, qw, qz, s), "none of AWQ (1), GPTQ (2)"),
        (accel_amd.ForeignInt4(GPTQ, 32, 60, 16, qw, qz, s), "multiple of 8"),
        (accel_amd.ForeignInt4(GPTQ, 32, 64, 12, qw, qz, s), "N = 12 is not a multiple of 8"),
        (accel_amd.ForeignInt4(GPTQ, 16, 64, 16, qw, qz, s), "need 4"),
        (accel_amd.ForeignInt4(AWQ, 24, 64, 16, qw, qz, s), "multiple of group_size"),
        (accel_amd.ForeignInt4(AWQ, 32, 64, 16, qw, qz, s, np.zeros(64, np.int32)),
         "AWQ has no g_idx"),
        (accel_amd.ForeignInt4(GPTQ, 32, 64, 16, qw, qz, s,
                               np.r_[np.zeros(63), [2]].astype(np.int32)),
         "g_idx[63] = 2 is outside the layer's 2 groups"),
        (accel_amd.ForeignInt4(GPTQ, 0, 64, 16, qw, qz, s), "group_size 0"),
    ]
    for layer, text in cases:
        rc, msg = _refusal(layer)
        assert rc == accel_amd.E_INVALID and text in msg, (text, msg)
