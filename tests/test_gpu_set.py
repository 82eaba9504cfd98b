"""Several Int4MatVec products that share one input vector in one launch
(accel_int4_matvec_set): every result equals its own Int4MatVec bit for bit,
on the decode kernel's 256- and 128-column tiles, its pipelined multi-batch
form (long K), and the per-matrix fallback for shapes the decode kernel does
not take."""
import numpy as np
import pytest

import oracle
from accel_amd import F32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _weights(dev, K, N, rng):
    p, s, z = workloads.fast_int4(K, N, rng)
    return dev.upload_int4(p, s, z, K * N), (p, s, z)


@pytest.mark.parametrize("K,Ns", [
    (4096, [4096, 1024, 1024]),       # q, k, v of a Llama-3-8B layer
    (4096, [14336, 14336]),           # gate, up
    (1024, [384, 256, 128, 512]),     # 128-column tiles (384 is not a multiple of 256)
    (20000, [256, 512]),              # more batches than slices: the pipelined kernel
    (300, [40, 256]),                 # 40 columns: one launch per matrix
    (512, [256]),
    (2048, [8192, 4096, 384]),        # 512-, 256- and 128-column tiles in one set
    (9000, [8704, 256]),              # the 512-column tile's pipelined kernel
])
def test_set_equals_separate_matvecs(dev, K, Ns):
    rng = np.random.Generator(np.random.PCG64(K + sum(Ns)))
    x = rng.standard_normal(K).astype(np.float32)
    xb = dev.upload(x)
    ws, planes = zip(*[_weights(dev, K, N, rng) for N in Ns])
    singles, outs = [], [dev.alloc((N,), F32) for N in Ns]
    for w, N in zip(ws, Ns):
        ob = dev.alloc((N,), F32)
        dev.Int4MatVec(xb, w, ob)
        singles.append(ob.numpy().copy())
        ob.free()
    for rep in range(2):   # the second call reuses the hand-off's tickets
        dev.Int4MatVecSet(xb, list(ws), outs)
        for o, want in zip(outs, singles):
            assert np.array_equal(o.numpy().view(np.uint32), want.view(np.uint32))
    # and every matrix against the oracle
    for o, (p, s, z), N in zip(outs, planes, Ns):
        assert rel_l2(o.numpy(), oracle.quant_matvec_int4(x, p, s, z, K, N)) <= 1e-5
    for b in list(outs) + [xb]:
        b.free()
    for w in ws:
        w.free()


@pytest.mark.parametrize("M,K,Ns", [
    (8, 4096, [4096, 1024, 1024]),    # q, k, v at batch 8: matrix-core decode
    (8, 4096, [14336, 14336]),        # gate, up
    (5, 1024, [384, 256, 512]),       # one- and two-group tiles: two launches
    (16, 2048, [1024, 2048]),
    (3, 512, [128]),
    (2, 1024, [256, 512]),            # two rows: matrix-core decode too
    (2, 100, [256, 128]),             # two rows, K % 32 != 0: one Int4MatMul each
    (1, 4096, [4096, 1024]),          # one row: the vector set
    (4, 100, [256, 128]),             # K % 32 != 0: one Int4MatMul each
])
def test_matmul_set_equals_separate_matmuls(dev, M, K, Ns):
    rng = np.random.Generator(np.random.PCG64(M * 1000 + K + sum(Ns)))
    x = rng.standard_normal((M, K)).astype(np.float32)
    xb = dev.upload(x)
    ws, planes = zip(*[_weights(dev, K, N, rng) for N in Ns])
    singles, outs = [], [dev.alloc((M, N), F32) for N in Ns]
    for w, N in zip(ws, Ns):
        ob = dev.alloc((M, N), F32)
        dev.Int4MatMul(xb, w, ob)
        singles.append(ob.numpy().copy())
        ob.free()
    for rep in range(2):
        dev.Int4MatMulSet(xb, list(ws), outs)
        for o, want in zip(outs, singles):
            assert np.array_equal(o.numpy().view(np.uint32), want.view(np.uint32))
    for o, (p, s, z), N in zip(outs, planes, Ns):
        assert rel_l2(o.numpy(), oracle.quant_matmul_int4(x, p, s, z, M, K, N, threads=8)) <= 1e-5
    for b in list(outs) + [xb]:
        b.free()
    for w in ws:
        w.free()
