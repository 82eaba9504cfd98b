"""Weights prepared for the matrix-core decode (accel_int4_prepare_tiles):
the code plane as it is and a side copy of the scales and zeros, one block
per (group, 32-row step), through accel_int4_matmul_prepared[_set] and
accel_int4_matvec_prepared[_set], against the oracle and against the same
products on the reference planes.

Only where a step's scales and zeros are read from changes, not the plan or
the arithmetic, so past one row the results are Int4MatMul's on the planes
bit for bit (the planes' route for 2..16 aligned rows is this kernel): at
one- and two-group tiles (N a multiple of 128 and not of 256), one step and
many, several K slices, config 2 at full size.  One row (the planes take the
VALU kernel there) and more than 16 rows (passes of 16) are held to the f32
tolerance against the oracle (rel-L2 <= 1e-5, tensor/int4_test.go:275-354).
A set gives each matrix its own result bit for bit, a graph replay the
eager result; unaligned activations, K % 32 != 0 and sets that mix the two
prepared forms are refused."""
import numpy as np
import pytest

import accel_amd as A
import oracle
from accel_amd import F32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-5

SAME = [(2, 4096, 14336), (8, 4096, 4096), (16, 4096, 14336), (3, 14336, 4096),
        (5, 1024, 640), (16, 2048, 384), (12, 512, 256), (7, 32, 128), (9, 4096, 1024)]


def _case(M, K, N, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    return x, p, s, z


@pytest.mark.parametrize("M,K,N", SAME)
def test_tiles_equal_the_planes_bit_for_bit(dev, M, K, N):
    x, p, s, z = _case(M, K, N, M + K + N)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N, tiles=True)
    assert pw.nbytes >= K * N // 2 + K * N // 128 * 4
    a = dev.upload(x)
    got, ref = dev.alloc((M, N), F32), dev.alloc((M, N), F32)
    dev.Int4MatMulPrepared(a, pw, got)
    sel = dev.last_selection()
    assert sel.op == "Int4MatMulPrepared"
    assert sel.launches[0].startswith("int4_decode_mfma_side_kernel<"), sel
    assert sel.kernel == A.select(M, K, N, F32, a=a.ptr, op="Int4MatMulPreparedTiles",
                                  dev=dev.index).kernel
    dev.Int4MatMul(a, w, ref)
    assert dev.last_selection().launches[0].startswith("int4_decode_mfma_kernel<")
    g, r = got.numpy(), ref.numpy()
    assert np.array_equal(g.view(np.uint32), r.view(np.uint32))
    want = oracle.quant_matmul_int4(x, p, s, z, M, K, N, threads=8)
    assert rel_l2(g, want) <= TOL
    for b in (a, got, ref):
        b.free()
    pw.free()
    w.free()


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (1, 4096, 14336), (17, 4096, 1024),
                                   (33, 1024, 512), (40, 2048, 2048)])
def test_tiles_one_row_and_passes_match_the_oracle(dev, M, K, N):
    x, p, s, z = _case(M, K, N, 7 * M + K)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N, tiles=True)
    want = oracle.quant_matmul_int4(x, p, s, z, M, K, N, threads=8)
    if M == 1:
        a, o = dev.upload(x[0]), dev.alloc((N,), F32)
        dev.Int4MatVecPrepared(a, pw, o)
        got = o.numpy().reshape(1, N)
    else:
        a, o = dev.upload(x), dev.alloc((M, N), F32)
        dev.Int4MatMulPrepared(a, pw, o)
        got = o.numpy()
        assert len(dev.last_selection().launches) >= (M + 15) // 16
    assert rel_l2(got, want) <= TOL, rel_l2(got, want)
    for m in range(M):
        assert rel_l2(got[m], want[m]) <= TOL, m
    for b in (a, o):
        b.free()
    pw.free()
    w.free()


def test_a_tiles_set_gives_each_matrix_its_own_result(dev):
    """q/k/v-like and gate/up-like sets at batch 8: one- and two-group tiles
    in one call, each matrix's result its own product's, and the planes'
    set's, bit for bit."""
    M, K = 8, 4096
    for widths in ((4096, 1024, 1024), (14336, 14336)):
        rng = np.random.Generator(np.random.PCG64(sum(widths)))
        x = rng.standard_normal((M, K)).astype(np.float32)
        ws, pws = [], []
        for i, N in enumerate(widths):
            _, p, s, z = _case(1, K, N, 100 + i + N)
            w = dev.upload_int4(p, s, z, K * N)
            ws.append(w)
            pws.append(dev.prepare_int4(w, K, N, tiles=True))
        a = dev.upload(x)
        singles = []
        for pw, N in zip(pws, widths):
            o = dev.alloc((M, N), F32)
            dev.Int4MatMulPrepared(a, pw, o)
            singles.append(o.numpy())
            o.free()
        outs = [dev.alloc((M, N), F32) for N in widths]
        dev.Int4MatMulPreparedSet(a, pws, outs)
        assert dev.last_selection().op == "Int4MatMulPreparedSet"
        refs = [dev.alloc((M, N), F32) for N in widths]
        dev.Int4MatMulSet(a, ws, refs)
        for one, o, r in zip(singles, outs, refs):
            assert np.array_equal(one.view(np.uint32), o.numpy().view(np.uint32))
            assert np.array_equal(one.view(np.uint32), r.numpy().view(np.uint32))
        for b in outs + refs + [a]:
            b.free()
        for pw in pws:
            pw.free()
        for w in ws:
            w.free()


def test_graph_replay_equals_the_eager_call(dev):
    M, K, N = 16, 4096, 14336
    x, p, s, z = _case(M, K, N, 91)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N, tiles=True)
    a = dev.upload(x)
    eager, replayed = dev.alloc((M, N), F32), dev.alloc((M, N), F32)
    dev.Int4MatMulPrepared(a, pw, eager)
    dev.sync()
    st = dev.stream()
    dev.capture_begin(st)
    dev.Int4MatMulPrepared(a, pw, replayed, st)
    ex = dev.capture_end(st)
    for _ in range(3):
        dev.launch(ex, st)
        dev.sync(st)
        assert np.array_equal(replayed.numpy().view(np.uint32), eager.numpy().view(np.uint32))
    dev.destroy_exec(ex)
    dev.destroy_stream(st)
    for b in (a, eager, replayed):
        b.free()
    pw.free()
    w.free()


def test_config2_full_size(dev):
    L = workloads.linear(**workloads.CONFIGS["decode_m16"])
    w = dev.upload_int4(L.packed, L.scales, L.zeros, L.K * L.N)
    pw = dev.prepare_int4(w, L.K, L.N, tiles=True)
    a, got, ref = dev.upload(L.x), dev.alloc((L.M, L.N), F32), dev.alloc((L.M, L.N), F32)
    dev.Int4MatMulPrepared(a, pw, got)
    dev.Int4MatMul(a, w, ref)
    assert np.array_equal(got.numpy().view(np.uint32), ref.numpy().view(np.uint32))
    want = oracle.quant_matmul_int4(L.x, L.packed, L.scales, L.zeros, L.M, L.K, L.N, threads=8)
    assert rel_l2(got.numpy(), want) <= TOL
    for b in (a, got, ref):
        b.free()
    pw.free()
    w.free()


def test_tiles_refusals(dev):
    K, N = 96, 128
    _, p, s, z = _case(1, K, N, 5)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N, tiles=True)
    base = dev.upload(np.zeros(2 * K + 4, np.float32))
    un = A.Buffer(dev, base.ptr + 4, 2 * K * 4, F32, (2, K))   # 4-byte aligned rows
    out = dev.alloc((2, N), F32)
    with pytest.raises(A.Refused, match="16-byte aligned"):
        dev.Int4MatMulPrepared(un, pw, out)
    panel = dev.prepare_int4(w, K, N)
    a = dev.upload(np.zeros((2, K), np.float32))
    outs = [dev.alloc((2, N), F32) for _ in range(2)]
    with pytest.raises(A.Refused, match="prepared the same way"):
        dev.Int4MatMulPreparedSet(a, [pw, panel], outs)
    for b in [base, out, a] + outs:
        b.free()
    pw.free()
    panel.free()
    w.free()
    K2 = 100
    _, p2, s2, z2 = _case(1, K2, N, 6)
    w2 = dev.upload_int4(p2, s2, z2, K2 * N)
    with pytest.raises(A.Refused, match="K a multiple of 32"):
        dev.prepare_int4(w2, K2, N, tiles=True)
    w2.free()
