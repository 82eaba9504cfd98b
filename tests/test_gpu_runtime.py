"""The runtime's own guarantees, on the GPU, through the C ABI.

* An executable stays valid when a later eager call grows the workspace: the
  workspace it was captured against is kept (retired) while it lives, and
  freed when it is destroyed.
* A call that would grow the workspace inside a graph capture is refused.
* A split-K hand-off whose bounded wait gives up reports it through the
  device's fault word at the next wait (forced from the host with a zero wait
  limit, so every kernel still exits normally), and products are correct
  again afterwards.
* A split-K prefill (slices, then a reduction pass) replays from a graph
  bit for bit like the eager call.
"""
import numpy as np
import pytest

import accel_amd
import oracle
from accel_amd import F32, U32, F16, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _reopen(dev):
    """A fresh workspace: close frees it, open starts without one."""
    dev.close()
    accel_amd.Device(dev.index)


def _big_matvec_args(dev):
    """An Int4MatVec whose split-K partial sums need 16 MiB (64 slices x 65536
    columns x 4 bytes), twice the workspace's first allocation.  Its weights
    are left uninitialised: only the workspace it asks for matters here."""
    K, N = 16384, 65536
    n = K * N
    w = accel_amd.Int4Weights(dev.alloc((n // 8,), U32), dev.alloc((n // 128,), F16),
                              dev.alloc((n // 128,), F16), n)
    a = dev.upload(np.zeros(K, np.float32))
    out = dev.alloc((N,), F32)
    return a, w, out


def test_executable_survives_workspace_growth(dev):
    _reopen(dev)
    rng = np.random.Generator(np.random.PCG64(31))
    K, N = 4096, 4096
    p, s, z = workloads.fast_int4(K, N, rng)
    x = rng.standard_normal(K).astype(np.float32)
    w = dev.upload_int4(p, s, z, K * N)
    a = dev.upload(x)
    eager = dev.alloc((N,), F32)
    dev.Int4MatVec(a, w, eager)           # allocates the first workspace
    dev.sync()
    gen0, retired0 = dev.workspace_generation()
    assert gen0 >= 1 and retired0 == 0

    stream = dev.stream()
    replayed = dev.alloc((N,), F32)
    dev.capture_begin(stream)
    dev.Int4MatVec(a, w, replayed, stream)
    ex = dev.capture_end(stream)

    ba, bw, bo = _big_matvec_args(dev)
    dev.Int4MatVec(ba, bw, bo, stream)     # grows the workspace
    dev.sync(stream)
    gen1, retired1 = dev.workspace_generation()
    assert gen1 == gen0 + 1 and retired1 == 1   # the executable's workspace is kept

    for _ in range(3):
        dev.launch(ex, stream)
        dev.sync(stream)
        assert np.array_equal(replayed.numpy().view(np.uint32), eager.numpy().view(np.uint32))
    assert rel_l2(replayed.numpy(), oracle.quant_matvec_int4(x, p, s, z, K, N)) <= 1e-5

    dev.destroy_exec(ex)
    assert dev.workspace_generation() == (gen1, 0)   # freed with its last executable
    # eager calls after the growth still agree
    dev.Int4MatVec(a, w, replayed, stream)
    dev.sync(stream)
    assert np.array_equal(replayed.numpy().view(np.uint32), eager.numpy().view(np.uint32))
    for b in (a, eager, replayed, ba, bo):
        b.free()
    w.free()
    bw.free()
    dev.destroy_stream(stream)


def test_growth_inside_a_capture_is_refused(dev):
    _reopen(dev)
    rng = np.random.Generator(np.random.PCG64(32))
    K, N = 1024, 1024
    p, s, z = workloads.fast_int4(K, N, rng)
    w = dev.upload_int4(p, s, z, K * N)
    a = dev.upload(rng.standard_normal(K).astype(np.float32))
    out = dev.alloc((N,), F32)
    dev.Int4MatVec(a, w, out)
    dev.sync()
    gen0, _ = dev.workspace_generation()
    ba, bw, bo = _big_matvec_args(dev)
    stream = dev.stream()
    dev.capture_begin(stream)
    with pytest.raises(accel_amd.Refused, match="cannot grow inside a graph capture"):
        dev.Int4MatVec(ba, bw, bo, stream)
    ex = dev.capture_end(stream)
    dev.destroy_exec(ex)
    assert dev.workspace_generation()[0] == gen0
    # outside the capture the same call grows the workspace and runs
    dev.Int4MatVec(ba, bw, bo, stream)
    dev.sync(stream)
    assert dev.workspace_generation()[0] == gen0 + 1
    for b in (a, out, ba, bo):
        b.free()
    w.free()
    bw.free()
    dev.destroy_stream(stream)


def test_bounded_wait_that_gives_up_is_reported(dev):
    # The matrix-core decode product (3..16 rows) hands its K slices to the
    # last arriver, which waits (bounded) for the others' stores.
    rng = np.random.Generator(np.random.PCG64(33))
    M, K, N = 8, 4096, 4096
    p, s, z = workloads.fast_int4(K, N, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = dev.upload_int4(p, s, z, K * N)
    a = dev.upload(x)
    out = dev.alloc((M, N), F32)
    want = oracle.quant_matmul_int4(x, p, s, z, M, K, N, threads=8)
    dev.Int4MatMul(a, w, out)
    dev.sync()
    assert rel_l2(out.numpy(), want) <= 1e-5
    try:
        dev.set_wait_limit(0)             # every such wait gives up at once
        dev.Int4MatMul(a, w, out)
        with pytest.raises(accel_amd.AccelError, match="bounded wait gave up") as ei:
            dev.sync()
        assert ei.value.code == accel_amd.E_HIP
        assert not dev.lost
    finally:
        dev.set_wait_limit(1 << 22)
    dev.sync()                            # reported once, then cleared
    for _ in range(2):
        dev.Int4MatMul(a, w, out)
        dev.sync()
        assert rel_l2(out.numpy(), want) <= 1e-5
    for b in (a, out):
        b.free()
    w.free()


@pytest.mark.parametrize("bf16", [True, False])
def test_split_k_prefill_replays_like_eager(dev, bf16):
    """A short prefill (M = 64: its 32 tiles split K, then a reduction pass)
    captured in a graph replays bit for bit like the eager call, three times
    with eager work between the replays."""
    M, K, N = 64, 2048, 1024
    rng = np.random.Generator(np.random.PCG64(77 + bf16))
    p, s, z = workloads.fast_int4(K, N, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = dev.upload_int4(p, s, z, K * N)
    if bf16:
        a = dev.upload(workloads.bf16_bits(x), accel_amd.BF16)
        eager, replayed = dev.alloc((M, N), accel_amd.BF16), dev.alloc((M, N), accel_amd.BF16)
    else:
        a = dev.upload(x)
        eager, replayed = dev.alloc((M, N), F32), dev.alloc((M, N), F32)
    stream = dev.stream()
    dev.Int4MatMul(a, w, eager, stream)        # sizes the workspace outside the capture
    dev.sync(stream)
    dev.capture_begin(stream)
    dev.Int4MatMul(a, w, replayed, stream)
    ex = dev.capture_end(stream)
    want = eager.numpy().copy()
    for _ in range(3):
        dev.Int4MatMul(a, w, eager, stream)    # eager work between the replays
        dev.sync(stream)
        dev.launch(ex, stream)
        dev.sync(stream)
        assert np.array_equal(replayed.numpy().view(np.uint16 if bf16 else np.uint32),
                              want.view(np.uint16 if bf16 else np.uint32))
    xf = workloads.bf16_to_f32(workloads.bf16_bits(x)) if bf16 else x
    ref = oracle.quant_matmul_int4(xf, p, s, z, M, K, N, threads=8)
    got = workloads.bf16_to_f32(want) if bf16 else want
    assert rel_l2(got, ref) <= (2e-2 if bf16 else 1e-5)
    dev.destroy_exec(ex)
    for b in (a, eager, replayed):
        b.free()
    w.free()
    dev.destroy_stream(stream)


def test_decode_moe_replays_like_eager(dev):
    """The decode MoE (f32 rows, two rows or more an expert: the padding-row
    launch, then each expert's rows as matrix-core blocks with split K)
    captured in a graph replays bit for bit like the eager call, three times
    with eager work between the replays; the matvec form's padding rows stay
    zero."""
    E, K, N, counts, pad = 4, 1024, 1024, [5, 0, 19, 3], 2
    rng = np.random.Generator(np.random.PCG64(78))
    off = oracle.segment_offsets(np.array(counts, np.uint32))
    T = int(off[E]) + pad
    x = rng.standard_normal((T, K)).astype(np.float32)
    w32 = (rng.standard_normal(E * K * N) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w32)
    w = dev.upload_int4(p, s, z, E * K * N)
    a = dev.upload(x)
    cb = dev.upload(np.array(counts, np.uint32), accel_amd.U32)
    eager, replayed = dev.alloc((T, N), F32), dev.alloc((T, N), F32)
    replayed.write(np.full((T, N), 7.0, np.float32))
    stream = dev.stream()
    dev.Int4GroupedMatVec(a, w, E, cb, eager, stream)   # sizes the workspace outside the capture
    dev.sync(stream)
    dev.capture_begin(stream)
    dev.Int4GroupedMatVec(a, w, E, cb, replayed, stream)
    ex = dev.capture_end(stream)
    want = eager.numpy().copy()
    for _ in range(3):
        dev.Int4GroupedMatVec(a, w, E, cb, eager, stream)   # eager work between the replays
        dev.sync(stream)
        dev.launch(ex, stream)
        dev.sync(stream)
        assert np.array_equal(replayed.numpy().view(np.uint32), want.view(np.uint32))
    ref = oracle.int4_grouped_matvec(x, p, s, z, off, E, T, K, N, threads=8,
                                     out=np.full(T * N, 7.0, np.float32))
    assert rel_l2(want.ravel(), np.asarray(ref).ravel()) <= 1e-5
    assert np.all(want[int(off[E]):] == 0)
    dev.destroy_exec(ex)
    for b in (a, cb, eager, replayed, w):
        b.free()
    dev.destroy_stream(stream)
