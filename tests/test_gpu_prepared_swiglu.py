"""SwiGLU of two one-row products on prepared weights in one launch
(accel_int4_matvec_prepared_swiglu): a decode step's gate and up
projections and the SwiGLU that joins them.

Each of the two products is computed with Int4MatVecPrepared's own loads,
sums and reduction, and SwiGLU with the SwiGLU kernel's function, so the
result equals Int4MatVecPreparedSet of {gate, up} followed by SwiGLU bit for
bit: config 5's gate/up shape (4096 x 14336), K past one 4096-row chunk
(the pipelined kernel, and K = 14336's seven pairs a lane), K odd (a padding
row), unaligned activations (the scalar loads), one group of columns, and a
graph replay.  Against the oracle in reference order the bar is the f32
tolerance of the two products (rel-L2 <= 1e-5) carried through SwiGLU.
Weights prepared for the matrix cores and matrices of two shapes are
refused."""
import numpy as np
import pytest

import accel_amd as A
import oracle
from accel_amd import F32
from conftest import rel_l2

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 14336), (4096, 4096), (8192, 1024), (14336, 2048), (1001, 384), (7, 128),
          (4097, 256)]


def _pair(K, N, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal(K).astype(np.float32)
    planes = []
    for _ in range(2):
        w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
        planes.append(oracle.int4_quantize(w))
    return x, planes


def _unfused(dev, a, pg, pu, N):
    g, u, o = dev.alloc((N,), F32), dev.alloc((N,), F32), dev.alloc((N,), F32)
    dev.Int4MatVecPreparedSet(a, [pg, pu], [g, u])
    dev.SwiGLU(g, u, o)
    r = o.numpy()
    for b in (g, u, o):
        b.free()
    return r


@pytest.mark.parametrize("K,N", SHAPES)
@pytest.mark.parametrize("aligned", [True, False])
def test_fused_equals_the_set_and_swiglu(dev, K, N, aligned):
    x, ((p0, s0, z0), (p1, s1, z1)) = _pair(K, N, 5 * K + N)
    wg = dev.upload_int4(p0, s0, z0, K * N)
    wu = dev.upload_int4(p1, s1, z1, K * N)
    pg, pu = dev.prepare_int4(wg, K, N), dev.prepare_int4(wu, K, N)
    if aligned:
        a = dev.upload(x)
        view = a
    else:
        # activations one float past an 8-byte boundary: the scalar loads
        a = dev.upload(np.concatenate([np.zeros(1, np.float32), x]))
        view = A.Buffer(dev, a.ptr + 4, K * 4, F32, (K,))
    out = dev.alloc((N,), F32)
    dev.Int4MatVecPreparedSwiGLU(view, pg, pu, out)
    sel = dev.last_selection()
    assert sel.op == "Int4MatVecPreparedSwiGLU"
    assert sel.launches == [k for k in sel.launches if k.startswith("int4_panel_swiglu_kernel<")]
    got = out.numpy()
    ref = _unfused(dev, view, pg, pu, N)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    gate = oracle.quant_matvec_int4(x, p0, s0, z0, K, N, threads=8)
    up = oracle.quant_matvec_int4(x, p1, s1, z1, K, N, threads=8)
    assert rel_l2(got, oracle.swiglu(gate, up)) <= 1e-5
    for b in (a, out):
        b.free()
    for w in (pg, pu, wg, wu):
        w.free()


def test_fused_graph_replay(dev):
    K, N = 4096, 14336
    x, ((p0, s0, z0), (p1, s1, z1)) = _pair(K, N, 77)
    wg = dev.upload_int4(p0, s0, z0, K * N)
    wu = dev.upload_int4(p1, s1, z1, K * N)
    pg, pu = dev.prepare_int4(wg, K, N), dev.prepare_int4(wu, K, N)
    a, out = dev.upload(x), dev.alloc((N,), F32)
    st = dev.stream()
    dev.Int4MatVecPreparedSwiGLU(a, pg, pu, out, st)
    dev.sync(st)
    eager = out.numpy()
    dev.capture_begin(st)
    dev.Int4MatVecPreparedSwiGLU(a, pg, pu, out, st)
    ex = dev.capture_end(st)
    for _ in range(3):
        out.write(np.zeros(N, np.float32))
        dev.launch(ex, st)
        dev.sync(st)
        assert np.array_equal(out.numpy().view(np.uint32), eager.view(np.uint32))
    dev.destroy_exec(ex)
    dev.destroy_stream(st)
    for b in (a, out):
        b.free()
    for w in (pg, pu, wg, wu):
        w.free()


def test_fused_refusals(dev):
    K, N = 256, 256
    x, ((p0, s0, z0), (p1, s1, z1)) = _pair(K, N, 3)
    wg = dev.upload_int4(p0, s0, z0, K * N)
    wu = dev.upload_int4(p1, s1, z1, K * N)
    pg, pu = dev.prepare_int4(wg, K, N), dev.prepare_int4(wu, K, N)
    pt = dev.prepare_int4(wu, K, N, tiles=True)
    wn = dev.upload_int4(p1[:K * 128 // 8], s1[:K * 128 // 128], z1[:K * 128 // 128], K * 128)
    pn = dev.prepare_int4(wn, K, 128)
    a, out = dev.upload(x), dev.alloc((N,), F32)
    with pytest.raises(A.AccelError, match="not prepared with accel_int4_prepare"):
        dev.Int4MatVecPreparedSwiGLU(a, pg, pt, out)
    with pytest.raises(A.AccelError, match="they share a shape"):
        dev.Int4MatVecPreparedSwiGLU(a, pg, pn, out)
    short = dev.alloc((N - 128,), F32)
    with pytest.raises(A.AccelError):
        dev.Int4MatVecPreparedSwiGLU(a, pg, pu, short)
    for b in (a, out, short):
        b.free()
    for w in (pg, pu, pt, pn, wg, wu, wn):
        w.free()
