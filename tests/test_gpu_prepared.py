"""Prepared (bind-time) weights for one-row products (accel_int4_prepare,
accel_int4_matvec_prepared[_set]), through the C ABI, against the oracle.

The panel layout only reorders the planes, and the product's arithmetic per
weight is the decode kernel's; only the order of the f32 sums differs, so the
bar is the f32 tolerance (rel-L2 <= 1e-5) against the oracle in reference
order, on: config 1 at full size; K odd (a padding row), K = 1, K past one
4096-row chunk (the pipelined kernel) and past it by one row; N = 128 (one
group) and widths whose panel count is or is not a multiple of 64 (the two
placements); unaligned activations (the scalar activation loads).  A set
gives each matrix's own result bit for bit, a graph replay the eager result
bit for bit, and the selection report names the panel kernel."""
import numpy as np
import pytest

import accel_amd as A
import oracle
from accel_amd import F32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu

TOL = 1e-5

SHAPES = [(4096, 4096), (1, 128), (7, 256), (1001, 384), (4096, 1024), (4097, 256),
          (8192, 128), (14336, 4096), (4096, 14336), (300, 640), (5000, 1152), (64, 8192)]


def _weights(dev, K, N, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    return x, p, s, z


@pytest.mark.parametrize("K,N", SHAPES)
def test_prepared_matvec_matches_the_oracle(dev, K, N):
    x, p, s, z = _weights(dev, K, N, K * 3 + N)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N)
    assert pw.nbytes >= K * N // 2 + K * N // 128 * 4
    a, out = dev.upload(x), dev.alloc((N,), F32)
    dev.Int4MatVecPrepared(a, pw, out)
    got = out.numpy()
    want = oracle.quant_matvec_int4(x, p, s, z, K, N, threads=8)
    assert rel_l2(got, want) <= TOL, rel_l2(got, want)
    sel = dev.last_selection()
    assert sel.op == "Int4MatVecPrepared"
    assert sel.launches[0].startswith("int4_panel_matvec_kernel<"), sel
    assert sel.kernel == A.select(1, K, N, F32, a=a.ptr, op="Int4MatVecPrepared",
                                  dev=dev.index).kernel
    for b in (a, out):
        b.free()
    pw.free()
    w.free()


def test_config1_prepared_full_size(dev):
    L = workloads.linear(**workloads.CONFIGS["gemv_m1"])
    w = dev.upload_int4(L.packed, L.scales, L.zeros, L.K * L.N)
    pw = dev.prepare_int4(w, L.K, L.N)
    a, out, ref = dev.upload(L.x[0]), dev.alloc((L.N,), F32), dev.alloc((L.N,), F32)
    dev.Int4MatVecPrepared(a, pw, out)
    dev.Int4MatVec(a, w, ref)
    got = out.numpy()
    want = oracle.quant_matvec_int4(L.x[0], L.packed, L.scales, L.zeros, L.K, L.N, threads=8)
    assert rel_l2(got, want) <= TOL
    # the reference-plane kernel agrees to the f32 rounding of the sums
    assert rel_l2(got, ref.numpy().astype(np.float64)) <= TOL
    for b in (a, out, ref):
        b.free()
    pw.free()
    w.free()


def test_unaligned_activations(dev):
    K, N = 4096, 512
    x, p, s, z = _weights(dev, K, N, 17)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N)
    base = dev.upload(np.concatenate([np.zeros(1, np.float32), x]))
    a = A.Buffer(dev, base.ptr + 4, K * 4, F32, (K,))   # 4-byte aligned only
    out = dev.alloc((N,), F32)
    dev.Int4MatVecPrepared(a, pw, out)
    assert dev.last_selection().launches[0].startswith(
        "int4_panel_matvec_kernel<4, false, false, false, false>")
    want = oracle.quant_matvec_int4(x, p, s, z, K, N, threads=8)
    assert rel_l2(out.numpy(), want) <= TOL
    base.free(); out.free(); pw.free(); w.free()


def test_a_set_gives_each_matrix_its_own_result(dev):
    K = 4096
    widths = (4096, 1024, 1024)
    xs = None
    pws, ws, singles = [], [], []
    for i, N in enumerate(widths):
        x, p, s, z = _weights(dev, K, N, 50 + i)
        xs = x if xs is None else xs
        w = dev.upload_int4(p, s, z, K * N)
        ws.append(w)
        pws.append(dev.prepare_int4(w, K, N))
    a = dev.upload(xs)
    outs = [dev.alloc((N,), F32) for N in widths]
    for pw, o in zip(pws, outs):
        dev.Int4MatVecPrepared(a, pw, o)
        singles.append(o.numpy())
    sets = [dev.alloc((N,), F32) for N in widths]
    dev.Int4MatVecPreparedSet(a, pws, sets)
    sel = dev.last_selection()
    assert sel.op == "Int4MatVecPreparedSet" and len(sel.launches) == 1
    for one, o in zip(singles, sets):
        assert np.array_equal(one.view(np.uint32), o.numpy().view(np.uint32))
    for b in outs + sets + [a]:
        b.free()
    for pw in pws:
        pw.free()
    for w in ws:
        w.free()


def test_graph_replay_equals_the_eager_call(dev):
    K, N = 14336, 4096
    x, p, s, z = _weights(dev, K, N, 61)
    w = dev.upload_int4(p, s, z, K * N)
    pw = dev.prepare_int4(w, K, N)
    a = dev.upload(x)
    eager, replayed = dev.alloc((N,), F32), dev.alloc((N,), F32)
    dev.Int4MatVecPrepared(a, pw, eager)
    dev.sync()
    st = dev.stream()
    dev.capture_begin(st)
    dev.Int4MatVecPrepared(a, pw, replayed, st)
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


def test_refusals(dev):
    K, N = 256, 128
    x, p, s, z = _weights(dev, K, N, 3)
    w = dev.upload_int4(p, s, z, K * N)
    with pytest.raises(A.Refused, match="is 65536 weights and the matrix holds 32768"):
        dev.prepare_int4(w, K, 2 * N)
    pw = dev.prepare_int4(w, K, N)
    a = dev.upload(np.zeros(K + 1, np.float32))
    out = dev.alloc((N,), F32)
    with pytest.raises(A.Refused, match="activations are 257 long"):
        dev.Int4MatVecPrepared(a, pw, out)
    a2 = dev.upload(np.zeros(K, np.float32))
    out2 = dev.alloc((N + 128,), F32)
    with pytest.raises(A.Refused, match="the output is"):
        dev.Int4MatVecPrepared(a2, pw, out2)
    for b in (a, out, a2, out2):
        b.free()
    pw.free()
    w.free()
