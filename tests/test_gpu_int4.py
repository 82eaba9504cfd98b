"""GPU parity of the int4 products against the oracle, through the C ABI.

Tolerances: rel-L2 <= 1e-5 for f32 activations, <= 2e-2
for bf16 activations, against the oracle in reference order (bf16 configs:
the f32 oracle on bf16-rounded inputs, output rounded to bf16).  Known-answer
cases carry the reference tests' own bounds.
"""
import struct

import numpy as np
import pytest

import accel_amd
import oracle
from accel_amd import BF16, F32, U32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 2e-2


def run_matmul(dev, x, packed, scales, zeros, M, K, N, bf16=False):
    w = dev.upload_int4(packed, scales, zeros, K * N)
    if bf16:
        xb = dev.upload(workloads.bf16_bits(x.reshape(M, K)), BF16)
        out = dev.alloc((M, N), BF16)
        dev.Int4MatMul(xb, w, out)
        got = workloads.bf16_to_f32(out.numpy())
    else:
        xb = dev.upload(np.ascontiguousarray(x.reshape(M, K), np.float32))
        out = dev.alloc((M, N), F32)
        dev.Int4MatMul(xb, w, out)
        got = out.numpy()
    for b in (xb, out):
        b.free()
    w.free()
    return got


def run_matvec(dev, a, packed, scales, zeros, K, N):
    w = dev.upload_int4(packed, scales, zeros, K * N)
    ab = dev.upload(np.ascontiguousarray(a, np.float32))
    out = dev.alloc((N,), F32)
    dev.Int4MatVec(ab, w, out)
    got = out.numpy()
    ab.free(); out.free(); w.free()
    return got


# ---- known answers (internal/kernels/int4_test.go) --------------------------

def test_nibble_order_gives_forty_not_four(dev):
    K, N = 8, 1
    w = np.ones(K, np.float32); w[0], w[1] = 0, 4
    a = np.zeros(K, np.float32); a[0], a[1] = 1, 10
    p, s, z = oracle.int4_quantize(w)
    got = float(run_matvec(dev, a, p, s, z, K, N)[0])
    assert abs(got - 40) <= 1 and abs(got - 40) < abs(got - 4)


@pytest.mark.parametrize("M", [1, 3, 16, 64])
def test_a_constant_group_reads_as_its_zero_point(dev, M):
    K, N = 2 * 128, 128
    rng = np.random.default_rng(5359)
    w = np.where(np.arange(K * N) < 128, np.float32(0.75),
                 rng.random(K * N, np.float32) * 2 - 1).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    assert s[0] == 0
    back = oracle.int4_dequantize(p, s, z, K * N).astype(np.float64).reshape(K, N)
    a = np.ones((M, K), np.float32)
    want = a.astype(np.float64) @ back
    got = run_matmul(dev, a, p, s, z, M, K, N) if M > 1 else \
        run_matvec(dev, a[0], p, s, z, K, N)[None]
    mag = np.abs(a.astype(np.float64)) @ np.abs(back)
    nu = (K - 1) * 2.0 ** -24
    assert np.all(np.abs(got - want) <= nu / (1 - nu) * mag)


def test_differential_closed_form_case(dev):
    # differential_cases_test.go:1370-1398, padded to a 128-column matrix so the
    # decode kernel (not the per-element one) runs it
    K, N = 256, 128
    a = np.array([((i % 13) - 6) / 4 for i in range(K)], np.float32)
    words = np.array([i % 251 + 1 for i in range(K * N // 8)], np.uint32)
    groups = K * N // 128
    s16 = oracle.to_f16(np.where(np.arange(groups) == 0, 0.0, 0.25).astype(np.float32))
    z16 = oracle.to_f16(np.where(np.arange(groups) == 0, 0.75, 4.0).astype(np.float32))
    got = run_matvec(dev, a, words, s16, z16, K, N)
    want = oracle.quant_matvec_int4(a, words, s16, z16, K, N)
    assert rel_l2(got, want) <= F32_TOL


# ---- f32 decode shapes ------------------------------------------------------

SHAPES_F32 = [
    # (M, K, N): decode kernel paths, the per-element path, the fp32 tiles
    (1, 4096, 4096), (1, 128, 128), (1, 200, 20), (1, 256, 4), (1, 4096, 14336),
    (1, 1000, 384), (2, 512, 1024), (3, 256, 640), (5, 200, 20), (7, 384, 256),
    (8, 4096, 1024), (13, 200, 20), (16, 4096, 14336), (17, 256, 512),
    (64, 512, 256), (65, 320, 384),
    # the VALU decode kernel at its other widths: K % 32 != 0 keeps M >= 2 off
    # the matrix cores; 128-column tiles; two passes of eight rows
    (3, 200, 640), (6, 100, 1024), (12, 72, 512), (2, 4100, 1024), (1, 4096, 640),
    # two rows on the matrix-core decode kernel: one- and two-group tiles
    (2, 4096, 14336), (2, 1024, 640),
    # 17..48 rows: the f32 matrix-core tiles running only the m-tiles a short
    # band has rows for (one, one and two of four), K split
    (17, 1024, 8192), (18, 2048, 4096), (40, 8192, 4096),
    # K long enough that a workgroup loops over several batches of rows (256-
    # and 128-column tiles), and the layer chain's down projection
    (1, 16640, 256), (2, 33000, 128), (1, 14336, 4096),
    # 512-column tiles of wide one-row products: one batch a slice, and
    # several (pipelined) with a short last slice
    (1, 2048, 8192), (1, 9000, 8704),
    # the matrix-core decode kernel: one- and two-group tiles, one step, a few
    # steps, several slices, the layer chain's down projection
    (4, 4096, 4096), (9, 1024, 384), (11, 2048, 768), (15, 14336, 4096), (16, 96, 256),
    (6, 32, 128), (10, 4096, 1024),
    # config 5 at batch 8: q/o [4096,4096] and down [14336,4096] at their own size
    (8, 4096, 4096), (8, 14336, 4096),
    # M > 16 on the matrix cores (three-term split): one stage and three row
    # bands, a full band, a ragged band and several column tiles; K % 64 != 0
    # takes the fp32 VALU tiles
    (257, 64, 128), (128, 1024, 512), (300, 2048, 1024), (40, 96, 256),
    # split K on the matrix cores (too few tiles to fill the chip): eight
    # slices at M = 64, a last slice longer than the others (17 stages over 4)
    (64, 4096, 4096), (33, 1088, 256),
]


@pytest.mark.parametrize("M,K,N", SHAPES_F32)
def test_f32_products_match_the_oracle(dev, M, K, N):
    rng = np.random.Generator(np.random.PCG64(M * 7919 + K * 31 + N))
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    if M == 1:
        got = run_matvec(dev, x[0], p, s, z, K, N)[None]
        want = oracle.quant_matvec_int4(x[0], p, s, z, K, N, threads=8)[None]
    else:
        got = run_matmul(dev, x, p, s, z, M, K, N)
        want = oracle.quant_matmul_int4(x, p, s, z, M, K, N, threads=8)
    assert rel_l2(got, want) <= F32_TOL, rel_l2(got, want)


def test_config1_gemv_full_size(dev):
    L = workloads.linear(**workloads.CONFIGS["gemv_m1"])
    got = run_matvec(dev, L.x[0], L.packed, L.scales, L.zeros, L.K, L.N)
    want = oracle.quant_matvec_int4(L.x[0], L.packed, L.scales, L.zeros, L.K, L.N, threads=8)
    assert rel_l2(got, want) <= F32_TOL


def test_config2_decode_m16_full_size(dev):
    L = workloads.linear(**workloads.CONFIGS["decode_m16"])
    got = run_matmul(dev, L.x, L.packed, L.scales, L.zeros, L.M, L.K, L.N)
    want = oracle.quant_matmul_int4(L.x, L.packed, L.scales, L.zeros, L.M, L.K, L.N,
                                    threads=8)
    assert rel_l2(got, want) <= F32_TOL


@pytest.mark.parametrize("M", [1, 64])
def test_weights_far_from_zero_keep_f32_accuracy(dev, M):
    # groups clustered at 1000 +- 0.5: the zero point is large (quant/int4_test.go:93-101)
    K, N = 512, 256
    rng = np.random.default_rng(77)
    w = (1000 + rng.random((K, N))).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    if M == 1:
        got = run_matvec(dev, x[0], p, s, z, K, N)[None]
        want = oracle.quant_matvec_int4(x[0], p, s, z, K, N)[None]
    else:
        got = run_matmul(dev, x, p, s, z, M, K, N)
        want = oracle.quant_matmul_int4(x, p, s, z, M, K, N, threads=8)
    assert rel_l2(got, want) <= F32_TOL


def test_decode_is_deterministic(dev):
    L = workloads.linear(1, 4096, 4096, seed=9)
    a = run_matvec(dev, L.x[0], L.packed, L.scales, L.zeros, L.K, L.N)
    b = run_matvec(dev, L.x[0], L.packed, L.scales, L.zeros, L.K, L.N)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- bf16 prefill -------------------------------------------------------------

SHAPES_BF16 = [(1, 64, 128), (64, 256, 256), (100, 512, 384), (128, 128, 128),
               # decode sizes: one row on the VALU decode kernel, 2..16 rows on
               # the matrix-core decode kernel (bf16 staged), one- and two-group
               # tiles, and K % 32 != 0 (the tiles)
               (1, 4096, 14336), (2, 4096, 14336), (8, 1024, 640), (16, 2048, 4096),
               (5, 96, 256),
               (257, 1024, 640), (512, 2048, 1024),
               # the 256-row tiles with one stage, an odd stage count and a
               # ragged last row band
               (300, 64, 128), (256, 192, 384), (511, 320, 256),
               # last bands of 2, 4, 7 and 8 active 32-row m-tiles
               (832, 128, 256), (97, 64, 256), (200, 256, 128), (480, 128, 128),
               # split K (too few tiles to fill the chip): eight slices of a
               # prefill at M = 64, a ragged one-m-tile band, a last slice
               # longer than the others (17 stages over 4)
               (64, 4096, 4096), (17, 4096, 1024), (96, 1088, 256)]


def _bf16_oracle(x, p, s, z, M, K, N, rows=None):
    rows = np.arange(M) if rows is None else rows
    out = oracle.quant_matmul_int4(np.ascontiguousarray(x[rows]), p, s, z, len(rows), K, N,
                                   threads=8)
    return oracle.round_bf16(out)


@pytest.mark.parametrize("M,K,N", SHAPES_BF16)
def test_bf16_products_match_the_oracle(dev, M, K, N):
    rng = np.random.Generator(np.random.PCG64(M + K + N))
    x = workloads.bf16_to_f32(workloads.bf16_bits(rng.standard_normal((M, K)).astype(np.float32)))
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    got = run_matmul(dev, x, p, s, z, M, K, N, bf16=True)
    want = _bf16_oracle(x, p, s, z, M, K, N)
    assert rel_l2(got, want) <= BF16_TOL


# Config 3's full-size checks (both dtypes): 64 seeded rows and the first and
# last row of every 256-row band against the oracle row for row, and every
# row through f64 checksums per band of the output columns: the plain column
# sum, one weighted by the row's position in its band (which a row moved far
# or a wrong band changes) and two with seeded Gaussian weights per row
# (which a dropped, duplicated or swapped row changes, neighbours included).
# A checksum's tolerance: bf16 rounding of the outputs is ~0.11% rms per
# element and, the outputs having random signs, about as much relative to a
# band's sum, so 5e-3 holds it with room while one wrong row of a 256-row band
# moves the sum by ~1/16; f32 sums keep the f32 tolerance.
SUM_TOL_BF16 = 5e-3


def _full_size_rows(got, L, row_tol, sum_tol, bf16):
    M = L.M
    rng = np.random.Generator(np.random.PCG64(2048))
    rows = set(rng.choice(M, 64, replace=False).tolist())
    for b0 in range(0, M, 256):
        rows |= {b0, min(M, b0 + 256) - 1}
    rows = np.array(sorted(rows))
    if bf16:
        want = _bf16_oracle(L.x, L.packed, L.scales, L.zeros, M, L.K, L.N, rows=rows)
    else:
        want = oracle.quant_matmul_int4(np.ascontiguousarray(L.x[rows]), L.packed, L.scales,
                                        L.zeros, len(rows), L.K, L.N, threads=8)
    assert rel_l2(got[rows], want) <= row_tol, rel_l2(got[rows], want)
    for r in rows:   # row for row, so one wrong row is seen on its own
        assert rel_l2(got[r], want[list(rows).index(r)]) <= row_tol, r
    wd = oracle.int4_dequantize(L.packed, L.scales, L.zeros, L.K * L.N).reshape(L.K, L.N)
    wd = wd.astype(np.float64)
    g = got.astype(np.float64)
    for b0 in range(0, M, 256):
        b1 = min(M, b0 + 256)
        xs = L.x[b0:b1].astype(np.float64)
        pos = np.arange(1, b1 - b0 + 1, dtype=np.float64)[:, None]
        gauss = np.random.Generator(np.random.PCG64(b0)).standard_normal((2, b1 - b0, 1))
        for weights in (np.ones_like(pos), pos, gauss[0], gauss[1]):
            have = (weights * g[b0:b1]).sum(axis=0)
            expect = (weights * xs).sum(axis=0) @ wd
            assert rel_l2(have, expect) <= sum_tol, (b0, rel_l2(have, expect))


def test_config3_shape_in_f32_full_size(dev):
    # config 3's product in the reference API's dtype: f32 activations and
    # result on the matrix cores
    L = workloads.linear(2048, 4096, 4096, seed=2)
    got = run_matmul(dev, L.x, L.packed, L.scales, L.zeros, L.M, L.K, L.N)
    _full_size_rows(got, L, F32_TOL, F32_TOL, bf16=False)


def test_config3_prefill_full_size(dev):
    L = workloads.linear(**workloads.CONFIGS["prefill_m2048"])
    got = run_matmul(dev, L.x, L.packed, L.scales, L.zeros, L.M, L.K, L.N, bf16=True)
    _full_size_rows(got, L, BF16_TOL, SUM_TOL_BF16, bf16=True)


# ---- the backend seam -----------------------------------------------------------

def test_dispatch_of_the_matvec_record_equals_the_operator(dev):
    K, N = 1024, 512
    rng = np.random.default_rng(4)
    x = rng.standard_normal(K).astype(np.float32)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    want = run_matvec(dev, x, p, s, z, K, N)
    bufs = [dev.upload(x), dev.upload(p, U32), dev.upload(s), dev.upload(z),
            dev.alloc((N,), F32)]
    dims = struct.pack("<IIII", 0, N, K, 0)  # GEMMDims std140: M@0, N@4, K@8
    dev.dispatch("QuantMatVecInt4", bufs, [K, p.size, s.size, z.size, N], dims,
                 count=((N + 31) // 32, 1, 1))
    got = bufs[4].numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for b in bufs:
        b.free()


def test_dispatch_of_the_matmul_record(dev):
    M, K, N = 5, 256, 256
    rng = np.random.default_rng(6)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    bufs = [dev.upload(x), dev.upload(p, U32), dev.upload(s), dev.upload(z),
            dev.alloc((M, N), F32)]
    dims = struct.pack("<IIII", M, N, K, 0)
    dev.dispatch("QuantMatMulInt4", bufs, [M * K, p.size, s.size, z.size, M * N], dims)
    got = bufs[4].numpy()
    want = oracle.quant_matmul_int4(x, p, s, z, M, K, N)
    assert rel_l2(got, want) <= F32_TOL
    for b in bufs:
        b.free()


def test_streams_events_and_timing(dev):
    L = workloads.linear(1, 1024, 1024, seed=3)
    w = dev.upload_int4(L.packed, L.scales, L.zeros, L.K * L.N)
    a = dev.upload(L.x[0])
    out = dev.alloc((L.N,), F32)
    st = dev.stream()
    e0, e1 = dev.event(), dev.event()
    dev.record(e0, st)
    for _ in range(10):
        dev.Int4MatVec(a, w, out, stream=st)
    dev.record(e1, st)
    dev.wait(e1)
    assert dev.event_done(e1)
    assert dev.elapsed_ms(e0, e1) > 0
    want = oracle.quant_matvec_int4(L.x[0], L.packed, L.scales, L.zeros, L.K, L.N)
    assert rel_l2(out.numpy(), want) <= F32_TOL
    dev.destroy_event(e0); dev.destroy_event(e1); dev.destroy_stream(st)
    a.free(); out.free(); w.free()


def test_info_reports_gfx950(dev):
    info = dev.info()
    assert info.arch.decode().startswith("gfx950")
    assert info.compute_units >= 200 and info.wavefront == 64


@pytest.mark.parametrize("M,K,N", [(5, 200, 20), (5, 4096, 4096), (12, 1024, 384)])
def test_matmul_equals_matvec_row_for_row(dev, M, K, N):
    # TestAnInt4MatMulEqualsTheMatVecRowForRow (tensor/int4_test.go:275-354):
    # w uniform in [-1, 1), a[i] = sin(0.23 i); the batched product and the
    # row product sum in different orders (here on different kernels at the
    # larger shapes), so the bound is the reduction budget mag * 1e-6
    rng = np.random.default_rng(53)
    w = (rng.random(K * N) * 2 - 1).astype(np.float32)
    a = np.sin(np.arange(M * K, dtype=np.float64) * 0.23).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    batched = run_matmul(dev, a, p, s, z, M, K, N)
    wabs = np.abs(w.astype(np.float64)).reshape(K, N)
    for m in range(M):
        row = run_matvec(dev, a[m * K:(m + 1) * K], p, s, z, K, N)
        mag = np.abs(a[m * K:(m + 1) * K].astype(np.float64)) @ wabs
        assert np.all(np.abs(batched[m].astype(np.float64) - row) <= mag * 1e-6), m
