"""BASELINE config 1's literal format on the GPU (an additive variant with no
counterpart in the reference): the GEMV against the f64 product of the
dequantized weights, rel-L2 <= 1e-5 (f32 activations)."""
import numpy as np
import pytest

import accel_amd
from accel_amd import F32, U32
from conftest import rel_l2
from oracle import g32_np

pytestmark = pytest.mark.gpu


def run_g32(dev, x, p, s, K, N):
    xb = dev.upload(x.astype(np.float32))
    cb = dev.upload(p, U32)
    sb = dev.upload(s.reshape(-1), F32)
    ob = dev.alloc((N,), F32)
    dev.Int4G32MatVec(xb, cb, sb, K, N, ob)
    got = ob.numpy()
    for b in (xb, cb, sb, ob):
        b.free()
    return got


@pytest.mark.parametrize("K,N", [(32, 256), (64, 512), (4096, 256), (288, 768), (16384, 256),
                                 (4096, 4096)])
def test_g32_matvec_matches_the_dequantized_product(dev, K, N):
    rng = np.random.Generator(np.random.PCG64(K + N))
    x = rng.standard_normal(K).astype(np.float32)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    p, s = accel_amd.int4_g32_quantize(w)
    got = run_g32(dev, x, p, s, K, N)
    want = g32_np.matvec_g32(x, p, s, K, N)
    assert rel_l2(got, want) <= 1e-5, rel_l2(got, want)


def test_config1_literal_full_size(dev):
    # BASELINE config 1 as it states the format: seed 0, x first, then W [out, in]
    rng = np.random.Generator(np.random.PCG64(0))
    x = rng.standard_normal((1, 4096)).astype(np.float32)
    w = np.ascontiguousarray((rng.standard_normal((4096, 4096)) * 0.02).astype(np.float32).T)
    p, s = accel_amd.int4_g32_quantize(w)
    got = run_g32(dev, x[0], p, s, 4096, 4096)
    want = g32_np.matvec_g32(x[0], p, s, 4096, 4096)
    assert rel_l2(got, want) <= 1e-5


def test_g32_refuses_a_width_off_the_tile(dev):
    p, s = accel_amd.int4_g32_quantize(np.zeros((64, 128), np.float32))
    with pytest.raises(accel_amd.Refused):
        run_g32(dev, np.zeros(64, np.float32), p, s, 64, 128)
