"""Grouped experts prepared for the matrix-core decode
(accel_int4_prepare_grouped): the planes copied as they are and each
expert's side copy of its scales and zeros, through
accel_int4_grouped_matvec_prepared and accel_int4_grouped_matmul_prepared.

Only where a matrix-core step reads its scales and zeros from changes, not
the routes, the plans or the arithmetic, so the results are the grouped
products' on the planes bit for bit: f32 and bf16 rows, both forms, blocks
of up to 16 rows of an expert with the padding launch for the rest, split
K, one- and two-group tiles, every row on the VALU kernel (T < 2E), wrapped
offsets, the f32 and bf16 tiles past the decode route's rows, and the
decode MoE and config 4's f32 rows at full size.  The small cases are also
held to the oracle at the path's tolerance (f32 1e-5, bf16 2e-2, rel-L2;
tensor/int4_test.go:275-354).  A prepared set of experts is refused by the
single-matrix operators and a single prepared matrix by the grouped ones.

Experts prepared into the panel layout (accel_int4_prepare_grouped_panels)
take f32 rows with 3 <= T < 2E on the few-rows panel kernel, whose sums run
in another order: held to the oracle row for row at the f32 tolerance
(passes of two rows ending in one, padding rows, wrapped offsets, the 4-token
decode MoE at full size); their other rows, bf16 rows included, take the
planes' routes and equal the planes' products bit for bit."""
import numpy as np
import pytest

import accel_amd as A
import oracle
from accel_amd import BF16, F32, U32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _case(E, K, N, counts, pad, seed, bf16):
    rng = np.random.default_rng(seed)
    off = oracle.segment_offsets(np.array(counts, np.uint32))
    T = int(off[E]) + pad
    x = rng.standard_normal((T, K)).astype(np.float32)
    if bf16:
        x = workloads.bf16_to_f32(workloads.bf16_bits(x))
    w = (rng.standard_normal(E * K * N) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    return x, p, s, z, off, T


def _both(dev, form, x, w, pw, E, counts, T, N, bf16):
    """The product on the planes and on the prepared experts, into outputs
    that start as 7.0 (the matmul form leaves rows outside every segment)."""
    dt = BF16 if bf16 else F32
    xb = dev.upload(workloads.bf16_bits(x), BF16) if bf16 else dev.upload(x)
    cb = dev.upload(np.asarray(counts, np.uint32), U32)
    init = np.full((T, N), 7.0, np.float32)
    outs = []
    for prepared in (False, True):
        ob = dev.alloc((T, N), dt)
        ob.write(workloads.bf16_bits(init) if bf16 else init)
        if prepared:
            getattr(dev, form + "Prepared")(xb, pw, cb, ob)
        else:
            getattr(dev, form)(xb, w, E, cb, ob)
        outs.append((ob.numpy(), dev.last_selection()))
        ob.free()
    xb.free()
    cb.free()
    return outs


CASES = [
    # blocks of up to 16 rows with the padding launch: 16 + 1, 16 + 2, 16 + 3
    (3, 256, 512, [17, 18, 19], 1),
    # one-group tiles (N % 256 != 0) and 16 + 16 + 3 rows
    (2, 2048, 384, [16, 35], 2),
    # split K over 4096 rows, empty experts
    (8, 4096, 1024, [2, 0, 3, 1, 0, 4, 2, 4], 1),
    # padding rows past 512-column tiles
    (2, 1024, 2048, [9, 7], 3),
    (4, 512, 640, [3, 1, 0, 2], 2),
    # T < 2E: every row on the VALU kernel, the side copies unread
    (8, 256, 256, [3, 0, 0, 0, 0, 0, 0, 1], 1),
    # f32 past 64 rows (the decode route to 1024) and bf16 past 64 (the tiles)
    (4, 512, 1024, [300, 0, 41, 260], 2),
]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("form", ["Int4GroupedMatVec", "Int4GroupedMatMul"])
@pytest.mark.parametrize("E,K,N,counts,pad", CASES)
def test_prepared_experts_equal_the_planes(dev, bf16, form, E, K, N, counts, pad):
    x, p, s, z, off, T = _case(E, K, N, counts, pad, seed=3 * E + K, bf16=bf16)
    w = dev.upload_int4(p, s, z, E * K * N)
    pw = dev.prepare_int4_grouped(w, E, K, N)
    assert pw.nbytes >= E * K * N // 2 + E * K * N // 128 * 8
    (ref, rsel), (got, gsel) = _both(dev, form, x, w, pw, E, counts, T, N, bf16)
    assert gsel.op == form + "Prepared"
    side = [k for k in gsel.launches if k.startswith("int4_grouped_decode_mfma_side_kernel<")]
    plain = [k for k in rsel.launches if k.startswith("int4_grouped_decode_mfma_kernel<")]
    # the same routes, the matrix-core launch swapped for its side twin
    assert len(side) == len(plain)
    assert [k for k in gsel.launches if "mfma" not in k] == \
           [k for k in rsel.launches if "mfma" not in k]
    assert np.array_equal(got, ref)
    want = oracle.int4_grouped_matvec(x, p, s, z, off, E, T, K, N, threads=8,
                                      out=np.full(T * N, 7.0, np.float32)) \
        if form == "Int4GroupedMatVec" else \
        oracle.int4_grouped_matmul(x, p, s, z, off, E, T, K, N, threads=8,
                                   out=np.full(T * N, 7.0, np.float32))
    g = workloads.bf16_to_f32(got) if bf16 else got
    if bf16:
        want = oracle.round_bf16(want)
    assert rel_l2(g, want) <= (2e-2 if bf16 else 1e-5)
    pw.free()
    w.free()


def test_prepared_experts_wrapped_offsets(dev):
    """Counts whose running sum wraps u32: off = [0, 2^32 - 1, 2, 4], not
    sorted, so every row goes to the VALU launch on the planes the prepared
    copy keeps; rows 0-1, 2-3 and 4-5 on experts 0, 1 and 2
    (internal/kernels/grouped.go:66-77)."""
    E, K, N, counts, pad = 3, 512, 256, [0xFFFFFFFF, 3, 2], 2
    x, p, s, z, off, T = _case(E, K, N, counts, pad, seed=11, bf16=False)
    w = dev.upload_int4(p, s, z, E * K * N)
    pw = dev.prepare_int4_grouped(w, E, K, N)
    (ref, _), (got, _) = _both(dev, "Int4GroupedMatVec", x, w, pw, E, counts, T, N, False)
    assert np.array_equal(got, ref)
    want = oracle.int4_grouped_matvec(x, p, s, z, off, E, T, K, N, threads=8,
                                      out=np.full(T * N, 7.0, np.float32))
    assert rel_l2(got, want) <= 1e-5
    pw.free()
    w.free()


@pytest.mark.parametrize("tokens,form", [(8, "Int4GroupedMatVec"),
                                         (512, "Int4GroupedMatMul")])
def test_full_size_moe_equals_the_planes(dev, tokens, form):
    """The decode MoE (8 tokens top-2: 16 f32 rows) and config 4's 1024
    routed f32 rows, 8 experts of [4096, 14336], prepared against the planes
    bit for bit, and each expert's rows through an f64 checksum of the
    output columns weighted by the row's place in its segment (which a
    dropped, duplicated or misplaced row changes), at the f32 tolerance."""
    m = workloads.moe_fast(tokens=tokens)
    R = int(m.counts.sum())
    w = dev.upload_int4(m.packed, m.scales, m.zeros, m.E * m.K * m.N)
    pw = dev.prepare_int4_grouped(w, m.E, m.K, m.N)
    (ref, _), (got, gsel) = _both(dev, form, np.ascontiguousarray(m.x, np.float32), w, pw,
                                  m.E, m.counts, R, m.N, False)
    assert any(k.startswith("int4_grouped_decode_mfma_side_kernel<") for k in gsel.launches)
    assert np.array_equal(got, ref)
    off = oracle.segment_offsets(m.counts)
    for e in range(m.E):
        lo, hi = int(off[e]), int(off[e + 1])
        if lo == hi:
            continue
        base = e * m.K * m.N
        wdq = oracle.dequantized(m.packed[base // 8:(base + m.K * m.N) // 8],
                                 m.scales[base // 128:(base + m.K * m.N) // 128],
                                 m.zeros[base // 128:(base + m.K * m.N) // 128],
                                 m.K * m.N).reshape(m.K, m.N).astype(np.float64)
        pos = np.arange(1, hi - lo + 1, dtype=np.float64)[:, None]
        want = (pos * m.x[lo:hi].astype(np.float64)).sum(axis=0) @ wdq
        have = (pos * got[lo:hi].astype(np.float64)).sum(axis=0)
        assert rel_l2(have, want) <= 1e-5, e
        del wdq
    pw.free()
    w.free()


def test_prepared_forms_are_not_mixed(dev):
    E, K, N = 2, 256, 256
    x, p, s, z, off, T = _case(E, K, N, [3, 2], 0, seed=5, bf16=False)
    w = dev.upload_int4(p, s, z, E * K * N)
    pw = dev.prepare_int4_grouped(w, E, K, N)
    one = dev.upload_int4(p[:K * N // 8], s[:K * N // 128], z[:K * N // 128], K * N)
    pt = dev.prepare_int4(one, K, N, tiles=True)
    xb, cb = dev.upload(x), dev.upload(np.array([3, 2], np.uint32), U32)
    x0, o0 = dev.upload(x[0]), dev.alloc((N,), F32)
    ob = dev.alloc((T, N), F32)
    with pytest.raises(A.AccelError, match="prepared as grouped experts"):
        dev.Int4MatMulPrepared(xb, pw, ob)
    with pytest.raises(A.AccelError, match="prepared as grouped experts"):
        dev.Int4MatVecPreparedSet(x0, [pw], [o0])
    with pytest.raises(A.AccelError, match="prepared as one matrix"):
        dev.Int4GroupedMatVecPrepared(xb, pt, cb, ob)
    # two experts of [16, 4096]: the same weights, K not a multiple of 32
    with pytest.raises(A.AccelError, match="multiple of 32"):
        dev.prepare_int4_grouped(w, 2, 16, 4096)
    for b in (xb, cb, ob, x0, o0):
        b.free()
    pt.free()
    pw.free()
    one.free()
    w.free()


# ---- experts prepared into the panel layout -----------------------------------

PANEL_CASES = [
    # f32 rows, 3 <= T < 2E: the panel kernel
    (8, 4096, 1024, [2, 0, 3, 1, 0, 4, 2, 1], 1),
    (4, 512, 640, [3, 1, 0, 2], 1),
    (3, 256, 512, [5, 0, 0], 0),          # five rows: passes of two, two and one
    (2, 1024, 8192, [2, 1], 0),
    (4, 2048, 384, [1, 1, 1, 1], 0),      # 24 panels an expert
    (4, 4096, 256, [7, 0, 0, 0], 0),      # seven rows: three passes of two and one
]

def _run(dev, form, x, w, E, counts, T, N):
    xb = dev.upload(x)
    cb = dev.upload(np.asarray(counts, np.uint32), U32)
    ob = dev.alloc((T, N), F32)
    ob.write(np.full((T, N), 7.0, np.float32))
    if isinstance(w, A.PreparedInt4):
        getattr(dev, form + "Prepared")(xb, w, cb, ob)
    else:
        getattr(dev, form)(xb, w, E, cb, ob)
    got, sel = ob.numpy(), dev.last_selection()
    for b in (xb, cb, ob):
        b.free()
    return got, sel


def _want(form, x, p, s, z, off, E, T, K, N):
    init = np.full(T * N, 7.0, np.float32)
    if form == "Int4GroupedMatVec":
        return oracle.int4_grouped_matvec(x, p, s, z, off, E, T, K, N, threads=8, out=init)
    return oracle.int4_grouped_matmul(x, p, s, z, off, E, T, K, N, threads=8, out=init)


@pytest.mark.parametrize("form", ["Int4GroupedMatVec", "Int4GroupedMatMul"])
@pytest.mark.parametrize("E,K,N,counts,pad", PANEL_CASES)
def test_panel_experts_match_the_oracle(dev, form, E, K, N, counts, pad):
    x, p, s, z, off, T = _case(E, K, N, counts, pad, seed=7 * E + K, bf16=False)
    w = dev.upload_int4(p, s, z, E * K * N)
    pw = dev.prepare_int4_grouped(w, E, K, N, panels=True)
    assert pw.nbytes >= 2 * (E * K * N // 2)
    got, sel = _run(dev, form, x, pw, E, counts, T, N)
    assert sel.op == form + "Prepared"
    assert any(k.startswith("int4_grouped_panel_rows_kernel<") for k in sel.launches), sel
    assert not any("mfma" in k for k in sel.launches), sel
    want = _want(form, x, p, s, z, off, E, T, K, N)
    assert rel_l2(got, want) <= 1e-5, rel_l2(got, want)
    covered = int(off[E])
    assert np.all(got[covered:] == (0 if form == "Int4GroupedMatVec" else 7.0))
    # every covered row on its own, so no row is dropped, doubled or misplaced
    for t in range(covered):
        assert rel_l2(got[t], want[t]) <= 1e-5, t
    pw.free()
    w.free()


@pytest.mark.parametrize("E,K,N,counts,pad", [
    (2, 2048, 384, [16, 35], 2),            # two rows an expert or more: matrix cores
    (4, 512, 1024, [300, 0, 41, 260], 2),   # past 64 rows
    (3, 1001, 256, [2, 1, 1], 0),           # K odd: the VALU decode kernel
    (4, 512, 256, [1, 1, 0, 0], 0),         # two rows: the VALU decode kernel
])
def test_panel_experts_other_rows_take_the_planes_routes(dev, E, K, N, counts, pad):
    x, p, s, z, off, T = _case(E, K, N, counts, pad, seed=E + 3 * K, bf16=False)
    w = dev.upload_int4(p, s, z, E * K * N)
    pw = dev.prepare_int4_grouped(w, E, K, N, panels=True)
    got, gsel = _run(dev, "Int4GroupedMatMul", x, pw, E, counts, T, N)
    ref, rsel = _run(dev, "Int4GroupedMatMul", x, w, E, counts, T, N)
    assert not any(k.startswith("int4_grouped_panel_rows_kernel") for k in gsel.launches)
    assert gsel.launches == rsel.launches
    assert np.array_equal(got, ref)
    pw.free()
    w.free()


def test_panel_experts_wrapped_offsets(dev):
    """off = [0, 2^32 - 1, 2, 4, 4]: not sorted, so the panel launch's
    workgroups return and the VALU launch takes every row on the planes the
    prepared copy keeps; e(t) = #{r : off[r+1] <= t} puts rows 0-1, 2-3 and
    4-5 on experts 0, 1 and 3 (internal/kernels/grouped.go:66-77)."""
    E, K, N, counts, pad = 4, 512, 256, [0xFFFFFFFF, 3, 2, 0], 2
    x, p, s, z, off, T = _case(E, K, N, counts, pad, seed=11, bf16=False)
    w = dev.upload_int4(p, s, z, E * K * N)
    pw = dev.prepare_int4_grouped(w, E, K, N, panels=True)
    got, sel = _run(dev, "Int4GroupedMatVec", x, pw, E, counts, T, N)
    assert any(k.startswith("int4_grouped_panel_rows_kernel<") for k in sel.launches)
    want = _want("Int4GroupedMatVec", x, p, s, z, off, E, T, K, N)
    for t in range(T):
        assert rel_l2(got[t], want[t]) <= 1e-5, t
    pw.free()
    w.free()


def test_panel_experts_decode_moe_full_size(dev):
    """The decode MoE at full size (4 tokens top-2 over config 4's experts,
    8 f32 rows): every row against the oracle row for row, and the same
    rows on the planes within the f32 tolerance."""
    m = workloads.moe_fast(tokens=4)
    R = int(m.counts.sum())
    w = dev.upload_int4(m.packed, m.scales, m.zeros, m.E * m.K * m.N)
    pw = dev.prepare_int4_grouped(w, m.E, m.K, m.N, panels=True)
    x = np.ascontiguousarray(m.x, np.float32)
    got, sel = _run(dev, "Int4GroupedMatVec", x, pw, m.E, m.counts, R, m.N)
    assert any(k.startswith("int4_grouped_panel_rows_kernel<") for k in sel.launches)
    off = oracle.segment_offsets(m.counts)
    for e in range(m.E):
        lo, hi = int(off[e]), int(off[e + 1])
        if lo == hi:
            continue
        base = e * m.K * m.N
        want = oracle.quant_matmul_int4(np.ascontiguousarray(x[lo:hi]),
                                        m.packed[base // 8:(base + m.K * m.N) // 8],
                                        m.scales[base // 128:(base + m.K * m.N) // 128],
                                        m.zeros[base // 128:(base + m.K * m.N) // 128],
                                        hi - lo, m.K, m.N, threads=16)
        for r in range(hi - lo):
            assert rel_l2(got[lo + r], want[r]) <= 1e-5, (e, r)
    ref, _ = _run(dev, "Int4GroupedMatVec", x, w, m.E, m.counts, R, m.N)
    assert rel_l2(got, ref) <= 1e-5
    pw.free()
    w.free()


@pytest.mark.parametrize("form", ["Int4GroupedMatVec", "Int4GroupedMatMul"])
def test_panel_experts_with_bf16_rows_take_the_planes_route(dev, form):
    """bf16 rows on experts prepared into the panel layout, 3 <= T < 2E: the
    panel kernel takes f32 rows only, so these run the VALU decode kernel on
    the planes with K split, and the workspace area for its split-K sums is
    planned for that route (a plan for the panel route's one-slice padding
    launch left the sums no room).  Equal to the planes' product bit for bit
    and to the oracle at the bf16 tolerance."""
    E, K, N, counts, pad = 8, 1024, 128, [0, 1, 0, 1, 0, 0, 0, 0], 2
    x, p, s, z, off, T = _case(E, K, N, counts, pad, seed=9, bf16=True)
    assert 3 <= T < 2 * E
    w = dev.upload_int4(p, s, z, E * K * N)
    pw = dev.prepare_int4_grouped(w, E, K, N, panels=True)
    (ref, rsel), (got, gsel) = _both(dev, form, x, w, pw, E, counts, T, N, True)
    assert not any(k.startswith("int4_grouped_panel_rows_kernel") for k in gsel.launches)
    assert gsel.launches == rsel.launches
    assert np.array_equal(got, ref)
    want = oracle.round_bf16(_want(form, x, p, s, z, off, E, T, K, N))
    assert rel_l2(workloads.bf16_to_f32(got), want) <= 2e-2
    pw.free()
    w.free()
