"""BASELINE config 1's literal weight format (32-row groups along K, f32
scale, no zero point): the library's host packer against the definition in
oracle/g32_np.py, and that definition against hand-worked and closed-form
cases.  The reference has no such format, so nothing here pins it to the
reference: it is an additive variant, reported separately."""
import numpy as np
import pytest

import accel_amd
from oracle import g32_np


def test_hand_worked_group():
    # one group: amax 7 gives s = 1; codes are rne(w) + 8
    K, N = 32, 8
    w = np.zeros((K, N), np.float32)
    w[:, 0] = 0.5                      # rne(0.5) = 0 (ties to even) -> code 8
    w[0, 0] = 7.0
    w[1, 0] = -7.0
    w[2, 0] = 3.5                      # rne(3.5) = 4 -> code 12
    w[3, 0] = -2.5                     # rne(-2.5) = -2 -> code 6
    p, s = g32_np.quantize_g32(w)
    assert s[0, 0] == np.float32(1.0)
    assert np.all(s[0, 1:] == 0)       # groups of zeros: s = 0, codes 8
    q = np.array([(p[i // 8] >> (4 * (i % 8))) & 15 for i in range(K * N)]).reshape(K, N)
    assert q[0, 0] == 15 and q[1, 0] == 1 and q[2, 0] == 12 and q[3, 0] == 6
    assert np.all(q[4:, 0] == 8) and np.all(q[:, 1:] == 8)
    back = g32_np.dequantize_g32(p, s, K, N)
    assert back[2, 0] == 4.0 and back[3, 0] == -2.0 and back[0, 0] == 7.0


@pytest.mark.parametrize("K,N,seed", [(32, 8, 1), (256, 384, 2), (4096, 256, 3)])
def test_host_packer_matches_the_definition_bit_for_bit(K, N, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    w[:32, 0] = 0.0                    # a group of zeros
    w[32:64, 1] = -3.0                 # a constant negative group (only -7 codes)
    got_p, got_s = accel_amd.int4_g32_quantize(w)
    want_p, want_s = g32_np.quantize_g32(w)
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))
    assert np.array_equal(got_p, want_p)


def test_rounding_error_is_at_most_half_a_step():
    rng = np.random.default_rng(7)
    K, N = 512, 128
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    p, s = accel_amd.int4_g32_quantize(w)
    back = g32_np.dequantize_g32(p, s, K, N).astype(np.float64)
    step = np.repeat(s.astype(np.float64), 32, axis=0)
    # |w - w'| <= s/2 up to the f32 rounding of w / s and of (q - 8) * s
    assert np.all(np.abs(w - back) <= step * (0.5 + 1e-6) + 1e-12)
    q = np.array([(p[i // 8] >> (4 * (i % 8))) & 15 for i in range(K * N)])
    assert q.min() >= 1 and q.max() <= 15   # symmetric: code 0 (-8) is never needed


def test_shapes_the_packer_refuses():
    with pytest.raises(accel_amd.AccelError):
        accel_amd.int4_g32_quantize(np.zeros((48, 8), np.float32))   # K % 32 != 0
