"""Int4MatMul over prepared weights (accel_int4_matmul_prepared[_set]): two
to eight rows a launch on the rows kernel, more in passes of eight, through
the C ABI, against the oracle.

As for one row, the panel layout only reorders the planes and each weight's
arithmetic is the decode kernels' fold; only the order of the f32 sums
differs, so the bar is the f32 tolerance (rel-L2 <= 1e-5) against the
oracle's QuantMatMulInt4 in reference order (internal/kernels/int4tiled.go:
66-137), on: every row count of one launch (2..8, each rounded up to the
kernel's 2, 4 or 8 rows), passes of eight (9, 16, 17 rows); K a whole chunk
and not (256, 1002 rows), past one chunk (the decoder layer's 14336); widths
whose panel count is a multiple of 64 and not; config 5's seven products at
batch 8 at full size.  One row is Int4MatVecPrepared bit for bit; a set
gives each matrix its own result bit for bit, and a graph replay the eager
result.  Odd K and rows that are not 8-byte aligned are refused."""
import numpy as np
import pytest

import accel_amd as A
import oracle
from accel_amd import F32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-5

CASES = [(M, K, N) for M in (2, 3, 5, 8) for K, N in ((4096, 4096), (256, 128))] + [
    (4, 1002, 384), (6, 2048, 1152), (7, 4096, 14336), (8, 14336, 4096),
    (9, 4096, 1024), (16, 4096, 1024), (17, 2048, 512), (2, 64, 8192)]


def _case(dev, M, K, N, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    return x, p, s, z


@pytest.mark.parametrize("M,K,N", CASES)
def test_prepared_rows_match_the_oracle(dev, M, K, N):
    x, p, s, z = _case(dev, M, K, N, M * 7 + K + N)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N)
    a, out = dev.upload(x), dev.alloc((M, N), F32)
    dev.Int4MatMulPrepared(a, pw, out)
    got = out.numpy()
    want = oracle.quant_matmul_int4(x, p, s, z, M, K, N, threads=8)
    assert rel_l2(got, want) <= TOL, rel_l2(got, want)
    for m in range(M):
        assert rel_l2(got[m], want[m]) <= TOL, m
    sel = dev.last_selection()
    assert sel.op == "Int4MatMulPrepared"
    assert len(sel.launches) == (M + 7) // 8
    assert all(k.startswith("int4_panel_rows_kernel<") for k in sel.launches), sel
    assert sel.kernel == A.select(M, K, N, F32, a=a.ptr, op="Int4MatMulPrepared",
                                  dev=dev.index).kernel
    for b in (a, out):
        b.free()
    pw.free()
    w.free()


def test_one_row_is_the_matvec(dev):
    K, N = 4096, 1024
    x, p, s, z = _case(dev, 1, K, N, 5)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N)
    a2, a1 = dev.upload(x), dev.upload(x[0])
    o2, o1 = dev.alloc((1, N), F32), dev.alloc((N,), F32)
    dev.Int4MatMulPrepared(a2, pw, o2)
    dev.Int4MatVecPrepared(a1, pw, o1)
    assert np.array_equal(o2.numpy()[0].view(np.uint32), o1.numpy().view(np.uint32))
    for b in (a2, a1, o2, o1):
        b.free()
    pw.free()
    w.free()


def test_a_rows_set_gives_each_matrix_its_own_result(dev):
    M, K = 8, 4096
    widths = (4096, 1024, 1024)
    rng = np.random.Generator(np.random.PCG64(70))
    x = rng.standard_normal((M, K)).astype(np.float32)
    ws, pws = [], []
    for i, N in enumerate(widths):
        _, p, s, z = _case(dev, 1, K, N, 71 + i)
        w = dev.upload_int4(p, s, z, K * N)
        ws.append(w)
        pws.append(dev.prepare_int4(w, K, N))
    a = dev.upload(x)
    singles = []
    for pw, N in zip(pws, widths):
        o = dev.alloc((M, N), F32)
        dev.Int4MatMulPrepared(a, pw, o)
        singles.append(o.numpy())
        o.free()
    outs = [dev.alloc((M, N), F32) for N in widths]
    dev.Int4MatMulPreparedSet(a, pws, outs)
    sel = dev.last_selection()
    assert sel.op == "Int4MatMulPreparedSet" and len(sel.launches) == 1
    assert sel.launches[0].startswith("int4_panel_rows_kernel<8, 2, true, true>"), sel
    for one, o in zip(singles, outs):
        assert np.array_equal(one.view(np.uint32), o.numpy().view(np.uint32))
    for b in outs + [a]:
        b.free()
    for pw in pws:
        pw.free()
    for w in ws:
        w.free()


def test_graph_replay_equals_the_eager_call(dev):
    M, K, N = 8, 14336, 4096
    x, p, s, z = _case(dev, M, K, N, 81)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N)
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


def test_config5_batch8_full_size(dev):
    """The decoder layer's seven products at batch 8 on prepared weights,
    q/k/v and gate/up as sets, each against the oracle."""
    rng = np.random.Generator(np.random.PCG64(90))
    x = rng.standard_normal((8, 4096)).astype(np.float32)
    got = {}
    planes = {}
    prepared = {}
    raw = []
    for name, (K, N) in workloads.LAYER_SHAPES.items():
        w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
        planes[name] = oracle.int4_quantize(w)
        wb = dev.upload_int4(*planes[name], K * N)
        raw.append(wb)
        prepared[name] = dev.prepare_int4(wb, K, N)
    a = dev.upload(x)
    bufs = {n: dev.alloc((8, N), F32) for n, (K, N) in workloads.LAYER_SHAPES.items()}
    dev.Int4MatMulPreparedSet(a, [prepared[n] for n in ("q", "k", "v")],
                              [bufs[n] for n in ("q", "k", "v")])
    dev.Int4MatMulPreparedSet(a, [prepared[n] for n in ("gate", "up")],
                              [bufs[n] for n in ("gate", "up")])
    for n in ("o", "down"):
        K, N = workloads.LAYER_SHAPES[n]
        xa = dev.upload(rng.standard_normal((8, K)).astype(np.float32))
        dev.Int4MatMulPrepared(xa, prepared[n], bufs[n])
        got[n] = (xa.numpy(), bufs[n].numpy())
        xa.free()
    for n, (K, N) in workloads.LAYER_SHAPES.items():
        xin, out = got[n] if n in got else (x, bufs[n].numpy())
        want = oracle.quant_matmul_int4(xin, *planes[n], 8, K, N, threads=8)
        assert rel_l2(out, want) <= TOL, (n, rel_l2(out, want))
    for b in list(bufs.values()) + [a] + raw:
        b.free()
    for pw in prepared.values():
        pw.free()


def test_rows_refusals(dev):
    K, N = 256, 128
    _, p, s, z = _case(dev, 1, K, N, 3)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N)
    a = dev.upload(np.zeros((2, K + 2), np.float32))
    out = dev.alloc((2, N), F32)
    with pytest.raises(A.Refused, match=r"activations are \[2, 258\] and matrix 0 is \[256, 128\]"):
        dev.Int4MatMulPrepared(a, pw, out)
    base = dev.upload(np.zeros(2 * K + 1, np.float32))
    un = A.Buffer(dev, base.ptr + 4, 2 * K * 4, F32, (2, K))   # 4-byte aligned rows
    with pytest.raises(A.Refused, match="8-byte aligned rows"):
        dev.Int4MatMulPrepared(un, pw, out)
    a2 = dev.upload(np.zeros((2, K), np.float32))
    out2 = dev.alloc((3, N), F32)
    with pytest.raises(A.Refused, match="the output is"):
        dev.Int4MatMulPrepared(a2, pw, out2)
    for b in (a, out, base, a2, out2):
        b.free()
    pw.free()
    w.free()
    # odd K: one row is the matvec's, more rows are refused
    K2 = 255 * 2 + 1
    _, p2, s2, z2 = _case(dev, 1, K2, 128, 4)
    w2 = dev.upload_int4(p2, s2, z2, K2 * 128)
    pw2 = dev.prepare_int4(w2, K2, 128)
    a3, o3 = dev.upload(np.zeros((2, K2), np.float32)), dev.alloc((2, 128), F32)
    with pytest.raises(A.Refused, match="K even"):
        dev.Int4MatMulPrepared(a3, pw2, o3)
    for b in (a3, o3):
        b.free()
    pw2.free()
    w2.free()
