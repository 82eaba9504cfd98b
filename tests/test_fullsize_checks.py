"""The full-size checks of config 3 (tests/test_gpu_int4.py) see the mistakes
they are there for: planted on the CPU in a copy of the oracle's own result,
a row swapped with its neighbour, and a band whose rows are shifted by one,
each fail them, while the unchanged result passes."""
import numpy as np
import pytest

import oracle
from accel_amd import workloads
from test_gpu_int4 import BF16_TOL, SUM_TOL_BF16, _bf16_oracle, _full_size_rows


def _case():
    rng = np.random.Generator(np.random.PCG64(9))
    M, K, N = 512, 256, 256

    class L:
        pass
    L.M, L.K, L.N = M, K, N
    L.x = workloads.bf16_to_f32(workloads.bf16_bits(rng.standard_normal((M, K)).astype(np.float32)))
    L.packed, L.scales, L.zeros = oracle.int4_quantize(
        (rng.standard_normal((K, N)) * 0.02).astype(np.float32))
    return L, _bf16_oracle(L.x, L.packed, L.scales, L.zeros, M, K, N)


def test_the_oracle_result_passes():
    L, good = _case()
    _full_size_rows(good, L, BF16_TOL, SUM_TOL_BF16, bf16=True)


@pytest.mark.parametrize("pair", [(300, 301), (40, 41), (510, 511)])
def test_a_swapped_neighbour_fails(pair):
    L, good = _case()
    bad = good.copy()
    bad[list(pair)] = bad[list(pair[::-1])]
    with pytest.raises(AssertionError):
        _full_size_rows(bad, L, BF16_TOL, SUM_TOL_BF16, bf16=True)


def test_a_shifted_band_fails():
    L, good = _case()
    bad = good.copy()
    bad[256:511] = good[257:512]
    with pytest.raises(AssertionError):
        _full_size_rows(bad, L, BF16_TOL, SUM_TOL_BF16, bf16=True)
