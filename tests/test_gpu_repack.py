"""GPU parity of the published-checkpoint repack (AWQ, GPTQ -> the reference
int4 format) through the C ABI: the device repack equals the host repack
(which equals the oracle's, tests/test_oracle_repack.py) bit for bit, the
repacked weights multiply like the oracle's repacked weights (rel-L2 <= 1e-5
in f32), a layer read from a safetensors file repacks on the device, and a
g_idx entry outside the layer's groups is reported."""
import ctypes

import numpy as np
import pytest
from safetensors.numpy import save_file

import accel_amd
import oracle
from accel_amd import F32, U32, F16, checkpoint
from conftest import rel_l2
from oracle import foreign_np

pytestmark = pytest.mark.gpu

AWQ, GPTQ, GPTQ2 = accel_amd.QFMT_AWQ, accel_amd.QFMT_GPTQ, accel_amd.QFMT_GPTQ_V2


def _layer(fmt, K, N, G, act=False, seed=0):
    rng = np.random.default_rng(seed)
    groups = -(-K // G)
    q = rng.integers(0, 16, (K, N), dtype=np.int64)
    z = rng.integers(1 if fmt == GPTQ else 0, 16, (groups, N), dtype=np.int64)
    s = oracle.to_f16((rng.random((groups, N)) * 0.02 + 1e-3).astype(np.float32)).reshape(groups, N)
    g_idx = None
    if act:
        g_idx = (np.arange(K) // G).astype(np.int32)
        rng.shuffle(g_idx)
    qw, qz = foreign_np.pack_awq(q, z) if fmt == AWQ else foreign_np.pack_gptq(q, z, fmt == GPTQ2)
    return accel_amd.ForeignInt4(fmt, G, K, N, qw, qz, s, g_idx)


@pytest.mark.parametrize("fmt,K,N,G,act", [
    (AWQ, 4096, 4096, 128, False),
    (GPTQ, 4096, 1024, 128, True),
    (GPTQ2, 1024, 4096, 64, False),
    (AWQ, 64, 40, 16, False),          # 40 columns: reference groups straddle rows
    (GPTQ, 200, 136, 64, False),       # K not a multiple of the group
    (GPTQ2, 256, 8, 256, True),
])
def test_device_repack_is_the_host_repack(dev, fmt, K, N, G, act):
    lay = _layer(fmt, K, N, G, act, seed=fmt * 1000 + K + N)
    want = accel_amd.int4_repack_host(lay)
    w = dev.Int4Repack(lay)
    got = (w.codes.numpy(), w.scales.numpy(), w.zeros.numpy())
    for a, b in zip(got, want):
        assert np.array_equal(a.reshape(-1), b)
    w.free()


@pytest.mark.parametrize("fmt", [AWQ, GPTQ2])
def test_device_repack_at_rounding_ties(dev, fmt):
    """Published scales alternating 1 and 1/2 by column with zero points 0 and
    every row of 128 columns spanning codes 0..15: each reference group comes
    out with scale 1 and zero 0, so its odd codes in the half-scale columns
    sit exactly on a tie of the round-half-to-even rule."""
    K, N, G = 256, 1024, 128
    rng = np.random.default_rng(fmt)
    q = rng.integers(0, 16, (K, N), dtype=np.int64)
    q[:, 0::128], q[:, 2::128] = 15, 0
    z = np.zeros((K // G, N), np.int64)
    s = oracle.to_f16(np.tile(np.float32([1.0, 0.5]), (K // G, N // 2))).reshape(K // G, N)
    qw, qz = foreign_np.pack_awq(q, z) if fmt == AWQ else foreign_np.pack_gptq(q, z, True)
    lay = accel_amd.ForeignInt4(fmt, G, K, N, qw, qz, s, None)
    want = accel_amd.int4_repack_host(lay)
    assert np.all(want[1] == 0x3C00)   # every reference scale is 1
    w = dev.Int4Repack(lay)
    for a, b in zip((w.codes.numpy(), w.scales.numpy(), w.zeros.numpy()), want):
        assert np.array_equal(a.reshape(-1), b)
    w.free()


@pytest.mark.parametrize("fmt,M,K,N,G", [(AWQ, 1, 4096, 4096, 128), (GPTQ, 4, 1024, 512, 32)])
def test_repacked_weights_multiply_like_the_oracles(dev, fmt, M, K, N, G):
    lay = _layer(fmt, K, N, G, seed=M + K)
    p, s, z = oracle.int4_repack(fmt, K, N, G, lay.qweight, lay.qzeros, lay.scales, lay.g_idx)
    rng = np.random.default_rng(M)
    x = rng.standard_normal((M, K)).astype(np.float32)
    want = oracle.quant_matmul_int4(x, p, s, z, M, K, N)
    w = dev.Int4Repack(lay)
    xb, ob = dev.upload(x), dev.alloc((M, N), F32)
    dev.Int4MatMul(xb, w, ob)
    assert rel_l2(ob.numpy(), want) <= 1e-5
    for b in (xb, ob):
        b.free()
    w.free()


def test_a_checkpoint_file_repacks_on_the_device(dev, tmp_path):
    K, N, G = 512, 256, 128
    lay = _layer(AWQ, K, N, G, seed=5)
    save_file({"layers.3.o_proj.qweight": lay.qweight.view(np.int32),
               "layers.3.o_proj.qzeros": lay.qzeros.view(np.int32),
               "layers.3.o_proj.scales": lay.scales.view(np.float16)},
              str(tmp_path / "model.safetensors"))
    cfg = checkpoint.QuantConfig(AWQ, G)
    w, k, n = checkpoint.load_linear(dev, str(tmp_path / "model.safetensors"),
                                     "layers.3.o_proj", cfg)
    assert (k, n) == (K, N)
    want = accel_amd.int4_repack_host(lay)
    for a, b in zip((w.codes.numpy(), w.scales.numpy(), w.zeros.numpy()), want):
        assert np.array_equal(a.reshape(-1), b)
    w.free()


def test_a_g_idx_outside_the_groups_is_reported(dev):
    lay = _layer(GPTQ, 64, 16, 32, act=True, seed=9)
    lay.g_idx[17] = 5   # the layer has two groups
    with pytest.raises(accel_amd.Refused, match="outside the layer's groups"):
        dev.Int4Repack(lay)
    # the device is still usable
    lay.g_idx[17] = 1
    w = dev.Int4Repack(lay)
    w.free()
