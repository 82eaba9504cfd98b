"""Seeded random-shape parity sweeps of the int4 products through the C ABI.

The shape tables of the other GPU tests pin the routes one by one; these
sweeps draw (rows, K, N, dtype, form) at random from pools that cross every
route boundary the launchers have: one and two rows (VALU decode), 3..16 rows
(matrix-core decode), 17+ rows (prefill tiles, split K when the tiles are
few), K and N that are and are not multiples of the tiles' 64 and 128 (the
generic kernels, groups that span rows), and 256 / 512-column decode tiles.
Every case is checked against the oracle at the path's tolerance (rel-L2 1e-5
for f32, 2e-2 for bf16, as `tensor/int4_test.go:275-354` and
`tensor/grouped_test.go:20-283` check their products).  Each case prints its
seed and shape before it runs, so a failure names it.
"""
import numpy as np
import pytest

import accel_amd
import oracle
from accel_amd import BF16, F32, U32, workloads
from conftest import rel_l2

pytestmark = pytest.mark.gpu

DENSE_M = [1, 1, 2, 3, 5, 8, 16, 17, 33, 64, 100, 128, 256, 513]
DENSE_K = [1, 7, 64, 100, 192, 320, 1024, 1088, 2048, 4096]
DENSE_N = [8, 20, 128, 136, 256, 384, 640, 1024, 2048, 8192]
MAX_MACS = 1 << 26


def tolerance(bf16: bool) -> float:
    return 2e-2 if bf16 else 1e-5


def upload_x(dev, x, bf16):
    """The activations as the product takes them, and their f32 values."""
    if bf16:
        bits = workloads.bf16_bits(x)
        return dev.upload(bits, BF16), workloads.bf16_to_f32(bits)
    return dev.upload(x), x


def read_out(ob, bf16):
    got = ob.numpy()
    return workloads.bf16_to_f32(got) if bf16 else got


@pytest.mark.parametrize("seed", range(16))
def test_random_dense_shapes_match_the_oracle(dev, seed):
    rng = np.random.Generator(np.random.PCG64(1000 + seed))
    done = 0
    while done < 16:
        M = int(rng.choice(DENSE_M))
        K = int(rng.choice(DENSE_K))
        N = int(rng.choice(DENSE_N))
        bf16 = bool(rng.integers(2))
        if M * K * N > MAX_MACS:
            continue
        matvec = M == 1 and not bf16 and bool(rng.integers(2))
        form = "Int4MatVec" if matvec else "Int4MatMul"
        print(f"sweep seed={seed} case={done}: {form} M={M} K={K} N={N} bf16={bf16}",
              flush=True)
        x = rng.standard_normal((M, K)).astype(np.float32)
        p, s, z = workloads.fast_int4(K, N, rng)
        wd = dev.upload_int4(p, s, z, K * N)
        # a matvec takes a vector (rank 1) and writes one
        xb, xf = upload_x(dev, x.reshape(K) if matvec else x, bf16)
        ob = dev.alloc((N,) if matvec else (M, N), BF16 if bf16 else F32)
        try:
            getattr(dev, form)(xb, wd, ob)
            got = read_out(ob, bf16)
        finally:
            for b in (xb, ob, wd):
                b.free()
        want = oracle.quant_matmul_int4(xf.reshape(M, K), p, s, z, M, K, N, threads=8)
        got = got.reshape(want.shape)
        if bf16:
            want = oracle.round_bf16(want)
        err = rel_l2(got, want)
        assert err <= tolerance(bf16), (seed, done, form, M, K, N, bf16, err)
        if not bf16:
            assert np.all(np.isfinite(got))
        done += 1


GROUPED_K = [64, 128, 256, 512, 1024, 2048]
GROUPED_N = [128, 256, 384, 512, 1024, 8192]


@pytest.mark.parametrize("seed", range(10))
def test_random_grouped_shapes_match_the_oracle(dev, seed):
    """Ragged expert counts (empty experts, padding rows past the last
    segment), both forms, both activation dtypes of the int4 grouped products:
    the decode-MoE kernel (f32, up to 64 rows), the lane-per-element form (f32,
    more rows) and the matrix-core grouped tiles (bf16)."""
    rng = np.random.Generator(np.random.PCG64(2000 + seed))
    done = 0
    while done < 10:
        bf16 = bool(rng.integers(2))
        E = int(rng.integers(1, 9))
        K = int(rng.choice(GROUPED_K))
        N = int(rng.choice(GROUPED_N))
        cap = int(rng.choice([3, 8, 40, 300]))
        counts = [int(c) if rng.random() > 0.2 else 0 for c in rng.integers(0, cap + 1, E)]
        off = oracle.segment_offsets(np.array(counts, np.uint32))
        T = int(off[E]) + int(rng.integers(0, 4))
        if T == 0 or T * K * N > MAX_MACS or E * K * N > MAX_MACS:
            continue
        form = "Int4GroupedMatVec" if rng.integers(2) else "Int4GroupedMatMul"
        print(f"sweep seed={seed} case={done}: {form} E={E} K={K} N={N} counts={counts} "
              f"T={T} bf16={bf16}", flush=True)
        x = rng.standard_normal((T, K)).astype(np.float32)
        w = (rng.standard_normal(E * K * N) * 0.02).astype(np.float32)
        p, s, z = oracle.int4_quantize(w)
        init = np.full((T, N), 7.0, np.float32)
        wd = dev.upload_int4(p, s, z, E * K * N)
        xb, xf = upload_x(dev, x, bf16)
        ob = dev.alloc((T, N), BF16 if bf16 else F32)
        ob.write(workloads.bf16_bits(init) if bf16 else init)
        cb = dev.upload(np.array(counts, np.uint32), U32)
        try:
            getattr(dev, form)(xb, wd, E, cb, ob)
            got = read_out(ob, bf16)
        finally:
            for b in (xb, ob, cb, wd):
                b.free()
        ref = oracle.int4_grouped_matvec if form == "Int4GroupedMatVec" else \
            oracle.int4_grouped_matmul
        want = ref(xf, p, s, z, off, E, T, K, N, threads=8, out=init.ravel().copy())
        if bf16:
            want = oracle.round_bf16(want)
        err = rel_l2(got.ravel(), np.asarray(want).ravel())
        assert err <= tolerance(bf16), (seed, done, form, E, K, N, counts, T, bf16, err)
        done += 1


PREP_M = [1, 1, 2, 3, 4, 5, 7, 8, 9, 16]
PREP_K = [1, 2, 7, 64, 130, 1000, 2048, 2050, 4096, 6144]
PREP_N = [128, 256, 384, 1024, 1152, 2048, 8192]


@pytest.mark.parametrize("seed", range(4))
def test_random_prepared_shapes_match_the_oracle(dev, seed):
    """Prepared weights (accel_int4_prepare) at random shapes: one row through
    Int4MatVecPrepared at any K, rows through Int4MatMulPrepared (K even),
    across the chunk boundaries (K a whole chunk or not, past one chunk) and
    the two panel placements (panel counts that are and are not multiples of
    64), against the oracle at the f32 tolerance."""
    rng = np.random.Generator(np.random.PCG64(3000 + seed))
    done = 0
    while done < 12:
        M = int(rng.choice(PREP_M))
        K = int(rng.choice(PREP_K))
        N = int(rng.choice(PREP_N))
        if M > 1 and K % 2:
            continue
        if M * K * N > MAX_MACS:
            continue
        form = "Int4MatVecPrepared" if M == 1 and bool(rng.integers(2)) else "Int4MatMulPrepared"
        print(f"prepared sweep seed={seed} case={done}: {form} M={M} K={K} N={N}", flush=True)
        x = rng.standard_normal((M, K)).astype(np.float32)
        p, s, z = workloads.fast_int4(K, N, rng)
        wd = dev.upload_int4(p, s, z, K * N)
        pw = dev.prepare_int4(wd, K, N)
        vec = form == "Int4MatVecPrepared"
        xb = dev.upload(x.reshape(K) if vec else x)
        ob = dev.alloc((N,) if vec else (M, N), F32)
        try:
            getattr(dev, form)(xb, pw, ob)
            got = ob.numpy()
        finally:
            for b in (xb, ob, wd):
                b.free()
            pw.free()
        want = oracle.quant_matmul_int4(x, p, s, z, M, K, N, threads=8)
        err = rel_l2(got.reshape(want.shape), want)
        assert err <= 1e-5, (seed, done, form, M, K, N, err)
        done += 1


@pytest.mark.parametrize("seed", range(6))
def test_random_grouped_prepared_shapes_match_the_oracle(dev, seed):
    """Experts bound once, in either prepared form, at random shapes and
    routings: side copies (accel_int4_prepare_grouped; the planes' grouped
    product bit for bit) and panel copies (accel_int4_prepare_grouped_panels;
    the panel kernel where 3 <= T < 2E), few rows an expert so that the panel
    route, the matrix-core blocks and the VALU decode kernel all come up,
    both forms, against the oracle at the path's tolerance."""
    rng = np.random.Generator(np.random.PCG64(4000 + seed))
    done = 0
    while done < 8:
        bf16 = rng.random() < 0.25
        E = int(rng.integers(2, 13))
        K = int(rng.choice([64, 256, 1024, 2048, 4096]))
        N = int(rng.choice([128, 256, 384, 1024, 8192]))
        cap = int(rng.choice([1, 2, 3, 8]))
        counts = [int(c) if rng.random() > 0.25 else 0 for c in rng.integers(0, cap + 1, E)]
        off = oracle.segment_offsets(np.array(counts, np.uint32))
        T = int(off[E]) + int(rng.integers(0, 3))
        if T == 0 or T * K * N > MAX_MACS or E * K * N > 4 * MAX_MACS:
            continue
        panels = bool(rng.integers(2))
        form = "Int4GroupedMatVec" if rng.integers(2) else "Int4GroupedMatMul"
        print(f"grouped prepared sweep seed={seed} case={done}: {form} E={E} K={K} N={N} "
              f"counts={counts} T={T} bf16={bf16} panels={panels}", flush=True)
        x = rng.standard_normal((T, K)).astype(np.float32)
        p, s, z = workloads.fast_int4(E * K, N, rng)
        init = np.full((T, N), 7.0, np.float32)
        wd = dev.upload_int4(p, s, z, E * K * N)
        pw = dev.prepare_int4_grouped(wd, E, K, N, panels=panels)
        xb, xf = upload_x(dev, x, bf16)
        cb = dev.upload(np.array(counts, np.uint32), U32)
        outs = []
        try:
            for prepared in (True, False):
                ob = dev.alloc((T, N), BF16 if bf16 else F32)
                ob.write(workloads.bf16_bits(init) if bf16 else init)
                if prepared:
                    getattr(dev, form + "Prepared")(xb, pw, cb, ob)
                else:
                    getattr(dev, form)(xb, wd, E, cb, ob)
                outs.append(read_out(ob, bf16))
                ob.free()
        finally:
            for b in (xb, cb, wd):
                b.free()
            pw.free()
        got, planes = outs
        ref = oracle.int4_grouped_matvec if form == "Int4GroupedMatVec" else \
            oracle.int4_grouped_matmul
        want = ref(xf, p, s, z, off, E, T, K, N, threads=8, out=init.ravel().copy())
        if bf16:
            want = oracle.round_bf16(want)
        err = rel_l2(got.ravel(), np.asarray(want).ravel())
        assert err <= tolerance(bf16), (seed, done, form, E, K, N, counts, T, bf16, panels, err)
        if not panels:
            assert np.array_equal(got, planes), (seed, done)
        done += 1
