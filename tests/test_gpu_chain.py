"""Config 5 as a chain: one Llama-3-8B-shaped decoder layer's decode step on
the GPU, at batch 1 and 8, against the oracle.

The step (as bench.py times it): h1 = RMSNorm(x); q, k, v <- h1 (one set
launch); o <- q; h2 = RMSNorm(o); gate, up <- h2 (one set launch);
act = SwiGLU(gate, up); down <- act.  Inputs come from seed 4 (x, the two
RMSNorm gains, then the seven weights in LAYER_SHAPES order).

Checked:
  * every product against the oracle fed the same device inputs (rel-L2
    <= 1e-5, the f32 tolerance);
  * each RMSNorm bit for bit and SwiGLU within one ulp against the oracle on
    the device's own inputs;
  * the chain's final output against the whole chain run in the oracle from
    x (rel-L2 <= 1e-5).
"""
import numpy as np
import pytest

import oracle
from accel_amd import F32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
EPS = 1e-5


def _inputs(batch):
    rng = np.random.Generator(np.random.PCG64(4))
    x = rng.standard_normal((batch, 4096)).astype(np.float32)
    g1 = (rng.standard_normal(4096) * 0.1 + 1).astype(np.float32)
    g2 = (rng.standard_normal(4096) * 0.1 + 1).astype(np.float32)
    planes = {name: workloads.fast_int4(K, N, rng)
              for name, (K, N) in workloads.LAYER_SHAPES.items()}
    return x, g1, g2, planes


def _product(a, planes, name):
    K, N = workloads.LAYER_SHAPES[name]
    p, s, z = planes[name]
    M = a.shape[0]
    if M == 1:
        return oracle.quant_matvec_int4(a[0], p, s, z, K, N, threads=16)[None]
    return oracle.quant_matmul_int4(a, p, s, z, M, K, N, threads=16)


@pytest.mark.parametrize("batch", [1, 8])
def test_decode_step_chain_matches_the_oracle(dev, batch):
    x, g1, g2, planes = _inputs(batch)
    shapes = workloads.LAYER_SHAPES
    shape = (lambda n: (batch, n)) if batch > 1 else (lambda n: (n,))
    ws = {n: dev.upload_int4(*planes[n], K * N) for n, (K, N) in shapes.items()}
    out = {n: dev.alloc(shape(N), F32) for n, (K, N) in shapes.items()}
    xin = dev.upload(x if batch > 1 else x[0])
    gb1, gb2 = dev.upload(g1), dev.upload(g2)
    h1, h2 = dev.alloc(shape(4096), F32), dev.alloc(shape(4096), F32)
    act = dev.alloc(shape(14336), F32)

    def op(a, n):
        (dev.Int4MatMul if batch > 1 else dev.Int4MatVec)(a, ws[n], out[n])

    def ops(a, names):
        (dev.Int4MatMulSet if batch > 1 else dev.Int4MatVecSet)(
            a, [ws[n] for n in names], [out[n] for n in names])

    dev.RMSNorm(xin, gb1, EPS, h1)
    ops(h1, ("q", "k", "v"))
    op(out["q"], "o")
    dev.RMSNorm(out["o"], gb2, EPS, h2)
    ops(h2, ("gate", "up"))
    dev.SwiGLU(out["gate"], out["up"], act)
    op(act, "down")
    dev.sync()

    rows = lambda b: b.numpy().reshape(batch, -1)
    d = {n: rows(b) for n, b in out.items()}
    dh1, dh2, dact = rows(h1), rows(h2), rows(act)

    # each stage against the oracle on the device's own inputs
    assert np.array_equal(dh1, oracle.rmsnorm(x, g1, EPS))
    for n in ("q", "k", "v"):
        assert rel_l2(d[n], _product(dh1, planes, n)) <= F32_TOL, n
    assert rel_l2(d["o"], _product(d["q"], planes, "o")) <= F32_TOL
    assert np.array_equal(dh2, oracle.rmsnorm(d["o"], g2, EPS))
    for n in ("gate", "up"):
        assert rel_l2(d[n], _product(dh2, planes, n)) <= F32_TOL, n
    want_act = oracle.swiglu(d["gate"].ravel(), d["up"].ravel()).reshape(batch, -1)
    ulps = np.abs(dact.view(np.int32).astype(np.int64) - want_act.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1
    assert rel_l2(d["down"], _product(dact, planes, "down")) <= F32_TOL

    # the whole chain in the oracle, from x
    o_h1 = oracle.rmsnorm(x, g1, EPS)
    o_q = _product(o_h1, planes, "q")
    o_o = _product(o_q, planes, "o")
    o_h2 = oracle.rmsnorm(o_o, g2, EPS)
    o_act = oracle.swiglu(_product(o_h2, planes, "gate").ravel(),
                          _product(o_h2, planes, "up").ravel()).reshape(batch, -1)
    o_down = _product(o_act, planes, "down")
    assert rel_l2(d["down"], o_down) <= F32_TOL, rel_l2(d["down"], o_down)
    assert rel_l2(d["k"], _product(o_h1, planes, "k")) <= F32_TOL
    assert rel_l2(d["v"], _product(o_h1, planes, "v")) <= F32_TOL

    for b in list(out.values()) + [xin, gb1, gb2, h1, h2, act]:
        b.free()
    for w in ws.values():
        w.free()


def test_prepared_fused_step_at_batch_1(dev):
    """The step as bench.py times config 5 at batch 1: every weight prepared
    into the panel layout, q/k/v as a prepared set, and gate, up and SwiGLU
    as one launch (Int4MatVecPreparedSwiGLU).  Each product against the
    oracle on the device's own inputs, SwiGLU's output against the oracle's
    SwiGLU of the oracle's gate and up products (the f32 tolerance carried
    through), and the step's output against the whole step in the oracle."""
    x, g1, g2, planes = _inputs(1)
    shapes = workloads.LAYER_SHAPES
    ws = {n: dev.upload_int4(*planes[n], K * N) for n, (K, N) in shapes.items()}
    pws = {n: dev.prepare_int4(ws[n], K, N) for n, (K, N) in shapes.items()}
    out = {n: dev.alloc((N,), F32) for n, (K, N) in shapes.items()}
    xin, gb1, gb2 = dev.upload(x[0]), dev.upload(g1), dev.upload(g2)
    h1, h2, act = dev.alloc((4096,), F32), dev.alloc((4096,), F32), dev.alloc((14336,), F32)
    dev.RMSNorm(xin, gb1, EPS, h1)
    dev.Int4MatVecPreparedSet(h1, [pws[n] for n in ("q", "k", "v")],
                              [out[n] for n in ("q", "k", "v")])
    dev.Int4MatVecPrepared(out["q"], pws["o"], out["o"])
    dev.RMSNorm(out["o"], gb2, EPS, h2)
    dev.Int4MatVecPreparedSwiGLU(h2, pws["gate"], pws["up"], act)
    dev.Int4MatVecPrepared(act, pws["down"], out["down"])
    dev.sync()
    d = {n: out[n].numpy()[None] for n in ("q", "k", "v", "o", "down")}
    dh1, dh2, dact = h1.numpy()[None], h2.numpy()[None], act.numpy()[None]
    for n in ("q", "k", "v"):
        assert rel_l2(d[n], _product(dh1, planes, n)) <= F32_TOL, n
    assert rel_l2(d["o"], _product(d["q"], planes, "o")) <= F32_TOL
    want_act = oracle.swiglu(_product(dh2, planes, "gate").ravel(),
                             _product(dh2, planes, "up").ravel())[None]
    assert rel_l2(dact, want_act) <= F32_TOL
    assert rel_l2(d["down"], _product(dact, planes, "down")) <= F32_TOL
    o_h1 = oracle.rmsnorm(x, g1, EPS)
    o_o = _product(_product(o_h1, planes, "q"), planes, "o")
    o_h2 = oracle.rmsnorm(o_o, g2, EPS)
    o_act = oracle.swiglu(_product(o_h2, planes, "gate").ravel(),
                          _product(o_h2, planes, "up").ravel())[None]
    o_down = _product(o_act, planes, "down")
    assert rel_l2(d["down"], o_down) <= F32_TOL, rel_l2(d["down"], o_down)
    for b in list(out.values()) + [xin, gb1, gb2, h1, h2, act]:
        b.free()
    for w in list(pws.values()) + list(ws.values()):
        w.free()
