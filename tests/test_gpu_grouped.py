"""GPU parity of the grouped (ragged, mixture-of-experts) products and the
segment offsets, through the C ABI.  Cases follow
internal/kernels/grouped_test.go and tensor/grouped_test.go; the f32 forms
carry the reference's 1e-4 element bound, the int4 forms the path's rel-L2
tolerances.
"""
import struct

import numpy as np
import pytest

import accel_amd
import oracle
from accel_amd import BF16, F32, U32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def grouped_fixture(E, K, N, counts):
    off = oracle.segment_offsets(np.array(counts, np.uint32))
    total = int(off[E])
    x = np.sin(np.arange(total * K) * 0.23).astype(np.float32)
    base = np.cos(np.arange(K * N) * 0.17).astype(np.float32)
    w = np.concatenate([base * np.float32(e + 1) for e in range(E)]).astype(np.float32)
    return x, w, off


def run_grouped(dev, form, x, w, counts, E, T, K, N, init=None):
    xb = dev.upload(np.ascontiguousarray(x, np.float32).reshape(T, K))
    wb = dev.upload(np.ascontiguousarray(w, np.float32).reshape(E, K, N))
    cb = dev.upload(np.asarray(counts, np.uint32), U32)
    ob = dev.alloc((T, N), F32)
    ob.write(np.full((T, N), 7.0, np.float32) if init is None else init)
    getattr(dev, form)(xb, wb, cb, ob)
    got = ob.numpy()
    for b in (xb, wb, cb, ob):
        b.free()
    return got


def test_segment_offsets_on_device(dev):
    for counts in ([3, 0, 5, 2, 0, 7], list(range(200)), [0xFFFFFFFF, 2], [9]):
        c = np.array(counts, np.uint32)
        cb = dev.upload(c, U32)
        ob = dev.alloc((c.size + 1,), U32)
        dev.SegmentOffsets(cb, ob)
        assert np.array_equal(ob.numpy(), oracle.segment_offsets(c))
        cb.free(); ob.free()


@pytest.mark.parametrize("form", ["GroupedMatVec", "GroupedMatMul"])
@pytest.mark.parametrize("E,K,N,counts", [(3, 64, 5, [2, 1, 3]), (4, 64, 3, [2, 0, 2, 0]),
                                          (2, 64, 2, [1, 1]), (4, 40, 20, [11, 0, 3, 20])])
def test_grouped_f32_matches_each_expert_alone(dev, form, E, K, N, counts):
    x, w, off = grouped_fixture(E, K, N, counts)
    T = int(off[E])
    got = run_grouped(dev, form, x, w, counts, E, T, K, N)
    ref = oracle.grouped_matvec if form == "GroupedMatVec" else oracle.grouped_matmul
    want = ref(x, w, off, E, T, K, N)
    assert np.all(np.abs(got - want) <= 1e-4)


def test_grouped_matvec_writes_zero_past_the_last_segment(dev):
    E, K, N = 3, 64, 4
    x, w, _ = grouped_fixture(E, K, N, [2, 1, 2])
    counts = [2, 0, 2]          # offsets 0,2,2,4; row 4 is padding
    T = 5
    xs = np.concatenate([x, np.zeros(K, np.float32)])[:T * K]
    got = run_grouped(dev, "GroupedMatVec", xs, w, counts, E, T, K, N)
    want = oracle.grouped_matvec(xs, w, oracle.segment_offsets(np.array(counts, np.uint32)),
                                 E, T, K, N)
    assert np.all(got[4] == 0)
    assert np.all(np.abs(got - want) <= 1e-4)


def test_grouped_matmul_clamps_and_leaves_other_rows(dev):
    E, K, N = 2, 40, 20
    x, w, _ = grouped_fixture(E, K, N, [4, 4])
    T = 8
    counts = [4, 12]            # offsets 0,4,16 clamp to the 8 rows
    got = run_grouped(dev, "GroupedMatMul", x, w, counts, E, T, K, N)
    want = oracle.grouped_matmul(x, w, oracle.segment_offsets(np.array(counts, np.uint32)),
                                 E, T, K, N)
    assert np.all(np.abs(got - want) <= 1e-4)
    # and rows no segment covers keep their contents
    counts = [2, 2]
    got = run_grouped(dev, "GroupedMatMul", x, w, counts, E, T, K, N)
    assert np.all(got[4:] == 7.0)


def test_dispatch_of_the_grouped_records(dev):
    E, K, N = 3, 32, 4
    counts = [2, 0, 4]
    x, w, off = grouped_fixture(E, K, N, counts)
    T = int(off[E])
    bufs = [dev.upload(x), dev.upload(w), dev.upload(off, U32), dev.alloc((T, N), F32)]
    dev.dispatch("GroupedMatVec", bufs, [T * K, E * K * N, E + 1, T * N],
                 struct.pack("<IIII", E, K, N, 0))
    assert np.all(np.abs(bufs[3].numpy() - oracle.grouped_matvec(x, w, off, E, T, K, N))
                  <= 1e-4)
    dev.dispatch("GroupedMatMul", bufs, [T * K, E * K * N, E + 1, T * N],
                 struct.pack("<IIII", E, T, K, N))
    assert np.all(np.abs(bufs[3].numpy() - oracle.grouped_matmul(x, w, off, E, T, K, N))
                  <= 1e-4)
    cb = dev.upload(np.array(counts, np.uint32), U32)
    ob = dev.alloc((E + 1,), U32)
    dev.dispatch("SegmentOffsets", [cb, ob], [E, E + 1], struct.pack("<IIII", E, 0, 0, 0))
    assert np.array_equal(ob.numpy(), off)
    for b in bufs + [cb, ob]:
        b.free()


# ---- int4 grouped -------------------------------------------------------------

def int4_case(E, K, N, counts, pad, seed, bf16):
    rng = np.random.default_rng(seed)
    off = oracle.segment_offsets(np.array(counts, np.uint32))
    T = int(off[E]) + pad
    x = rng.standard_normal((T, K)).astype(np.float32)
    if bf16:
        x = workloads.bf16_to_f32(workloads.bf16_bits(x))
    w = (rng.standard_normal(E * K * N) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    return x, p, s, z, off, T


def run_int4_grouped(dev, form, x, p, s, z, counts, E, T, K, N, bf16):
    w = dev.upload_int4(p, s, z, E * K * N)
    if bf16:
        xb = dev.upload(workloads.bf16_bits(x), BF16)
        ob = dev.alloc((T, N), BF16)
        ob.write(workloads.bf16_bits(np.full((T, N), 7.0, np.float32)))
    else:
        xb = dev.upload(x)
        ob = dev.alloc((T, N), F32)
        ob.write(np.full((T, N), 7.0, np.float32))
    cb = dev.upload(np.asarray(counts, np.uint32), U32)
    getattr(dev, form)(xb, w, E, cb, ob)
    got = ob.numpy()
    if bf16:
        got = workloads.bf16_to_f32(got)
    for b in (xb, ob, cb):
        b.free()
    w.free()
    return got


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("form", ["Int4GroupedMatVec", "Int4GroupedMatMul"])
@pytest.mark.parametrize("E,K,N,counts,pad", [(3, 128, 128, [5, 0, 9], 2),
                                              (8, 256, 384, [1, 130, 0, 7, 64, 0, 3, 260], 3),
                                              (2, 64, 256, [0, 0], 4),
                                              # decode MoE (f32: decode products, rows of
                                              # an expert two at a time):
                                              # split-K over 4096 rows, 128-column tiles,
                                              # the 64-row limit, one row
                                              (8, 4096, 1024, [2, 0, 3, 1, 0, 4, 2, 4], 1),
                                              (4, 512, 640, [3, 1, 0, 2], 2),
                                              (4, 1024, 256, [20, 10, 30, 4], 0),
                                              (5, 2048, 512, [0, 0, 1, 0, 0], 0),
                                              # few rows of a wide matrix: 512-column
                                              # tiles, a pair and single rows
                                              (3, 512, 8192, [1, 0, 1], 1),
                                              (2, 1024, 8192, [2, 1], 0),
                                              # blocks of up to 16 rows on the
                                              # matrix cores (T >= 2E):
                                              # 16 + 1, 16 + 2, 16 + 3 rows; 16 and
                                              # 16 + 16 + 3 with one-group tiles;
                                              # 5 and 3 rows over split K
                                              (3, 256, 512, [17, 18, 19], 1),
                                              (2, 2048, 384, [16, 35], 2),
                                              # padding rows past 512-column tiles
                                              (2, 1024, 2048, [9, 7], 3),
                                              (2, 4096, 2048, [5, 3], 0),
                                              # T < 2E: every row on the VALU kernel
                                              (8, 256, 256, [3, 0, 0, 0, 0, 0, 0, 1], 1),
                                              # f32 past 64 rows: the decode kernels up
                                              # to 1024 rows, the f32 matrix-core tiles
                                              # past (K % 64 == 0)
                                              (4, 512, 1024, [300, 0, 41, 260], 2),
                                              (2, 64, 128, [600, 500], 0)])
def test_int4_grouped_matches_the_oracle(dev, bf16, form, E, K, N, counts, pad):
    x, p, s, z, off, T = int4_case(E, K, N, counts, pad, seed=E + K, bf16=bf16)
    got = run_int4_grouped(dev, form, x, p, s, z, counts, E, T, K, N, bf16)
    init = np.full(T * N, 7.0, np.float32)
    if form == "Int4GroupedMatVec":
        want = oracle.int4_grouped_matvec(x, p, s, z, off, E, T, K, N, threads=8, out=init)
    else:
        want = oracle.int4_grouped_matmul(x, p, s, z, off, E, T, K, N, threads=8, out=init)
    if bf16:
        want = oracle.round_bf16(want)
    tol = 2e-2 if bf16 else 1e-5
    assert rel_l2(got, want) <= tol
    covered = int(off[E])
    if form == "Int4GroupedMatVec":
        assert np.all(got[covered:] == 0)
    else:
        assert np.all(got[covered:] == 7.0)


@pytest.mark.parametrize("N", [256, 2048])
def test_int4_grouped_matvec_wrapped_offsets(dev, N):
    """Counts whose running sum wraps u32 (segmentOffsets keeps the wrap,
    tensor/segment.go:40-50): off = [0, 2^32 - 1, 2, 4] is not sorted, and the
    row -> expert rule e(t) = #{r : off[r+1] <= t} (internal/kernels/
    grouped.go:66-77) puts rows 0-1, 2-3 and 4-5 on experts 0, 1 and 2.  The
    decode path pairs rows of one expert only under sorted offsets; here every
    row has to be computed on its own, by the VALU launch (the matrix-core
    launch takes sorted offsets only), whose workgroups each walk a row's
    column tiles: one tile at N = 256, four at N = 2048."""
    E, K, counts, pad = 3, 512, [0xFFFFFFFF, 3, 2], 2
    x, p, s, z, off, T = int4_case(E, K, N, counts, pad, seed=11, bf16=False)
    assert T == 6 and list(off) == [0, 0xFFFFFFFF, 2, 4]
    got = run_int4_grouped(dev, "Int4GroupedMatVec", x, p, s, z, counts, E, T, K, N, False)
    want = oracle.int4_grouped_matvec(x, p, s, z, off, E, T, K, N, threads=8,
                                      out=np.full(T * N, 7.0, np.float32))
    assert np.all(np.abs(want).sum(axis=1) > 0)   # every row belongs to an expert
    assert rel_l2(got, want) <= 1e-5
    for t in range(T):
        assert rel_l2(got[t], want[t]) <= 1e-5, t


@pytest.mark.parametrize("bf16", [True, False])
def test_config4_moe_full_size(dev, bf16):
    """Config 4 at full size (1024 routed rows, 8 experts of [4096, 14336]),
    with bf16 rows (the config's dtype) and with f32 rows (the reference
    API's grouped dtype, on the f32 matrix-core tiles): every row through two
    per-expert f64 checksums of the output columns, the plain column sum and
    one weighted by the row's position in its segment (which a dropped,
    duplicated or misplaced row changes), plus the first and last row of every
    expert and 64 seeded rows against the oracle row for row.  Tolerances:
    the path's, 2e-2 for bf16 and 1e-5 for f32."""
    m = workloads.moe()
    R = int(m.counts.sum())
    assert R == 1024
    tol = 2e-2 if bf16 else 1e-5
    w = dev.upload_int4(m.packed, m.scales, m.zeros, m.E * m.K * m.N)
    if bf16:
        xb = dev.upload(workloads.bf16_bits(m.x), BF16)
        ob = dev.alloc((R, m.N), BF16)
    else:
        xb = dev.upload(np.ascontiguousarray(m.x, np.float32))
        ob = dev.alloc((R, m.N), F32)
    cb = dev.upload(m.counts, U32)
    dev.Int4GroupedMatMul(xb, w, m.E, cb, ob)
    sel = dev.last_selection()
    assert sel.op == "Int4GroupedMatMul"
    assert any(k.startswith("int4_grouped_bf16_kernel" if bf16 else "int4_grouped_decode")
               for k in sel.launches), sel
    got = ob.numpy()
    got = (workloads.bf16_to_f32(got) if bf16 else got).astype(np.float64)
    off = oracle.segment_offsets(m.counts)
    rng = np.random.Generator(np.random.PCG64(44))
    sampled = set(rng.choice(R, 64, replace=False).tolist())
    for e in range(m.E):
        lo, hi = int(off[e]), int(off[e + 1])
        if lo == hi:
            continue
        base = e * m.K * m.N
        pe = m.packed[base // 8:(base + m.K * m.N) // 8]
        se = m.scales[base // 128:(base + m.K * m.N) // 128]
        ze = m.zeros[base // 128:(base + m.K * m.N) // 128]
        wdq = oracle.dequantized(pe, se, ze, m.K * m.N).reshape(m.K, m.N).astype(np.float64)
        xs = m.x[lo:hi].astype(np.float64)
        pos = np.arange(1, hi - lo + 1, dtype=np.float64)[:, None]
        for weights in (np.ones_like(pos), pos):
            want = (weights * xs).sum(axis=0) @ wdq
            have = (weights * got[lo:hi]).sum(axis=0)
            assert rel_l2(have, want) <= tol, (e, rel_l2(have, want))
        rows = sorted({lo, hi - 1} | {r for r in sampled if lo <= r < hi})
        want = oracle.quant_matmul_int4(np.ascontiguousarray(m.x[rows]), pe, se, ze,
                                        len(rows), m.K, m.N, threads=16)
        if bf16:
            want = oracle.round_bf16(want)
        assert rel_l2(got[rows], want) <= tol
        del wdq
    for b in (xb, cb, ob):
        b.free()
    w.free()


@pytest.mark.parametrize("bf16", [False, True])
def test_int4_grouped_matvec_wrapped_offsets_on_the_tiles(dev, bf16):
    """Wrapped offsets at the tiles' sizes (f32 past 1024 rows, bf16 past 64):
    counts [2^32 - 1, 700, 400] give off = [0, 2^32 - 1, 699, 1099], and
    e(t) = #{r : off[r+1] <= t} (internal/kernels/grouped.go:66-77) puts rows
    0-698 on expert 0, 699-1098 on expert 1 and every row from 1099 on
    expert 2 (no padding): the tiles walk the offsets sorted, not as given."""
    E, K, N, counts, pad = 3, 256, 256, [0xFFFFFFFF, 700, 400], 21
    x, p, s, z, off, T = int4_case(E, K, N, counts, pad, seed=12, bf16=bf16)
    assert T == 1120 and list(off) == [0, 0xFFFFFFFF, 699, 1099]
    got = run_int4_grouped(dev, "Int4GroupedMatVec", x, p, s, z, counts, E, T, K, N, bf16)
    want = oracle.int4_grouped_matvec(x, p, s, z, off, E, T, K, N, threads=8,
                                      out=np.full(T * N, 7.0, np.float32))
    if bf16:
        want = oracle.round_bf16(want)
    tol = 2e-2 if bf16 else 1e-5
    assert np.all(np.abs(want).sum(axis=1) > 0)   # every row belongs to an expert
    for lo, hi in ((0, 699), (699, 1099), (1099, T)):
        assert rel_l2(got[lo:hi], want[lo:hi]) <= tol, (lo, hi)


@pytest.mark.parametrize("form", ["Int4GroupedMatVec", "Int4GroupedMatMul"])
@pytest.mark.parametrize("E,K,N,counts", [(4, 512, 384, [100, 0, 900, 30]),
                                          (3, 1024, 256, [600, 500, 1]),
                                          # K % 64 != 0: one lane per element
                                          (2, 32, 128, [600, 500])])
def test_int4_grouped_f32_tiles_match_the_oracle(dev, form, E, K, N, counts):
    """f32 rows past 1024 on the matrix-core tiles: blocks of 128 rows with a
    short last block, an empty expert, a one-row expert, padding rows; and a
    K the tiles cannot take (one lane per element)."""
    x, p, s, z, off, T = int4_case(E, K, N, counts, 5, seed=K + N, bf16=False)
    assert T > 1024
    got = run_int4_grouped(dev, form, x, p, s, z, counts, E, T, K, N, False)
    init = np.full(T * N, 7.0, np.float32)
    ref = oracle.int4_grouped_matvec if form == "Int4GroupedMatVec" else \
        oracle.int4_grouped_matmul
    want = ref(x, p, s, z, off, E, T, K, N, threads=8, out=init)
    covered = int(off[E])
    assert rel_l2(got[:covered], want[:covered]) <= 1e-5
    for e in range(E):
        if off[e + 1] > off[e]:
            assert rel_l2(got[off[e]:off[e + 1]], want[off[e]:off[e + 1]]) <= 1e-5, e
    if form == "Int4GroupedMatVec":
        assert np.all(got[covered:] == 0)
    else:
        assert np.all(got[covered:] == 7.0)


@pytest.mark.parametrize("form", ["Int4GroupedMatVec", "Int4GroupedMatMul"])
def test_int4_grouped_decode_clamps_counts_past_the_rows(dev, form):
    """Counts that run past the T rows (`groupedtiled.go:87-91`: expert e's
    rows are [off[e], min(off[e+1], T))): with 10 + 30 routed rows over 24,
    expert 1 keeps 14, one matrix-core block; a third expert starting past T
    has none."""
    E, K, N, counts, T = 3, 1024, 512, [10, 30, 5], 24
    rng = np.random.Generator(np.random.PCG64(90))
    off = oracle.segment_offsets(np.array(counts, np.uint32))
    x = rng.standard_normal((T, K)).astype(np.float32)
    w = (rng.standard_normal(E * K * N) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    got = run_int4_grouped(dev, form, x, p, s, z, counts, E, T, K, N, False)
    ref = oracle.int4_grouped_matvec if form == "Int4GroupedMatVec" else \
        oracle.int4_grouped_matmul
    want = ref(x, p, s, z, off, E, T, K, N, threads=8, out=np.full(T * N, 7.0, np.float32))
    assert rel_l2(got, want) <= 1e-5
    for t in (0, 9, 10, 23):
        assert rel_l2(got[t], want[t]) <= 1e-5, t
