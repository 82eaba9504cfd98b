"""The no-allocation Int4MatVec (accel_int4_matvec_noalloc), through the C ABI:
its results equal accel_int4_matvec's bit for bit (the same kernels and plan,
with the split-K buffers in the library's static scratch) on two calls in a
row, the second smaller, and against the oracle within the f32 tolerance; a
shape whose split-K sums exceed the scratch is refused before anything is
launched; and it runs under graph capture without allocating."""
import ctypes

import numpy as np
import pytest

import accel_amd
import oracle
from accel_amd import F32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _both(dev, K, N, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    p, s, z = workloads.fast_int4(K, N, rng)
    x = rng.standard_normal(K).astype(np.float32)
    w = dev.upload_int4(p, s, z, K * N)
    a = dev.upload(x)
    ref, got = dev.alloc((N,), F32), dev.alloc((N,), F32)
    lib = accel_amd.lib()
    ta, tw = a.tensor(), w.desc()
    tr, tg = ref.tensor(), got.tensor()
    accel_amd._check(lib.accel_int4_matvec(dev.index, None, ctypes.byref(ta), ctypes.byref(tw),
                                           ctypes.byref(tr)))
    accel_amd._check(lib.accel_int4_matvec_noalloc(dev.index, None, ctypes.byref(ta),
                                                   ctypes.byref(tw), ctypes.byref(tg)))
    dev.sync()
    r, g = ref.numpy(), got.numpy()
    want = oracle.quant_matvec_int4(x, p, s, z, K, N)
    for b in (a, ref, got):
        b.free()
    w.free()
    return r, g, want


@pytest.mark.parametrize("shapes", [
    [(4096, 4096), (1024, 2048)],        # split K; the second call is smaller
    [(14336, 4096), (4096, 384)],        # 256- then 128-column tiles
    [(4096, 14336), (300, 40)],          # the second takes the per-element kernel
])
def test_noalloc_equals_int4_matvec(dev, shapes):
    for i, (K, N) in enumerate(shapes):
        r, g, want = _both(dev, K, N, seed=K + N + i)
        assert np.array_equal(r.view(np.uint32), g.view(np.uint32)), (K, N)
        assert rel_l2(g, want) <= 1e-5


def test_noalloc_refuses_what_exceeds_the_scratch(dev):
    # K = 16384 takes 64 slices; 64 x 65536 columns x 4 bytes is 16 MiB of sums
    K, N = 16384, 65536
    n = K * N
    w = accel_amd.Int4Weights(dev.alloc((n // 8,), accel_amd.U32),
                              dev.alloc((n // 128,), accel_amd.F16),
                              dev.alloc((n // 128,), accel_amd.F16), n)
    a = dev.upload(np.zeros(K, np.float32))
    out = dev.alloc((N,), F32)
    with pytest.raises(accel_amd.Refused, match="static scratch holds"):
        dev.Int4MatVecNoAlloc(a, w, out)
    dev.sync()
    for b in (a, out):
        b.free()
    w.free()


def test_noalloc_under_graph_capture(dev):
    rng = np.random.Generator(np.random.PCG64(41))
    K, N = 4096, 4096
    p, s, z = workloads.fast_int4(K, N, rng)
    x = rng.standard_normal(K).astype(np.float32)
    w = dev.upload_int4(p, s, z, K * N)
    a = dev.upload(x)
    eager, replayed = dev.alloc((N,), F32), dev.alloc((N,), F32)
    dev.Int4MatVecNoAlloc(a, w, eager)
    dev.sync()
    stream = dev.stream()
    dev.capture_begin(stream)
    dev.Int4MatVecNoAlloc(a, w, replayed, stream)
    ex = dev.capture_end(stream)
    for _ in range(3):
        dev.launch(ex, stream)
        dev.sync(stream)
        assert np.array_equal(replayed.numpy().view(np.uint32), eager.numpy().view(np.uint32))
    dev.destroy_exec(ex)
    dev.destroy_stream(stream)
    assert rel_l2(eager.numpy(), oracle.quant_matvec_int4(x, p, s, z, K, N)) <= 1e-5
    for b in (a, eager, replayed):
        b.free()
    w.free()


def test_noalloc_never_asks_for_the_workspace(dev):
    """After a reopen the device has no workspace, and any call that asked
    for one would allocate it and bump the generation: the no-allocation
    entry point, eager and under capture, leaves the generation where it
    was."""
    dev.close()
    accel_amd.Device(dev.index)
    gen0, _ = dev.workspace_generation()
    rng = np.random.Generator(np.random.PCG64(43))
    K, N = 4096, 4096
    p, s, z = workloads.fast_int4(K, N, rng)
    x = rng.standard_normal(K).astype(np.float32)
    w = dev.upload_int4(p, s, z, K * N)
    a = dev.upload(x)
    eager, replayed = dev.alloc((N,), F32), dev.alloc((N,), F32)
    dev.Int4MatVecNoAlloc(a, w, eager)
    dev.sync()
    assert dev.workspace_generation()[0] == gen0
    stream = dev.stream()
    dev.capture_begin(stream)
    dev.Int4MatVecNoAlloc(a, w, replayed, stream)
    ex = dev.capture_end(stream)
    dev.launch(ex, stream)
    dev.sync(stream)
    assert dev.workspace_generation()[0] == gen0
    assert np.array_equal(replayed.numpy().view(np.uint32), eager.numpy().view(np.uint32))
    assert rel_l2(eager.numpy(), oracle.quant_matvec_int4(x, p, s, z, K, N)) <= 1e-5
    dev.destroy_exec(ex)
    dev.destroy_stream(stream)
    for b in (a, eager, replayed):
        b.free()
    w.free()
