"""The committed golden fixtures (tests/golden/, written by make_golden.py).

On the CPU: the files are the ones the manifest names, the oracle and the
library's host packer reproduce every fixture bit for bit, and the fixtures
carry the facts the reference's tests assert about the same inputs
(quant/int4_test.go:22-36,261-286).  On the GPU: the device packer
reproduces the packed planes bit for bit, the segment offsets exactly, and
the products stay within the path's tolerances of the fixtures' outputs,
with the matvec form's padding rows exactly zero (grouped.go:66-77).
"""
import hashlib
import json
import os

import numpy as np
import pytest

import accel_amd
import oracle
import oracle.oracle_np as oracle_np
from accel_amd import F16, F32, U32
from conftest import rel_l2

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
F32_TOL = 1e-5


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def quantize_cases():
    d = load("quantize.npz")
    names = sorted({k.split(".")[0] for k in d})
    return [(n, d[f"{n}.w"], d[f"{n}.codes"], d[f"{n}.scales"], d[f"{n}.zeros"]) for n in names]


def test_fixture_files_match_the_manifest():
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        manifest = json.load(f)
    assert set(manifest) == {"quantize.npz", "matvec.npz", "matmul.npz", "grouped.npz",
                             "segment.npz"}
    for name, digest in manifest.items():
        with open(os.path.join(GOLDEN, name), "rb") as f:
            assert hashlib.sha256(f.read()).hexdigest() == digest, name


@pytest.mark.parametrize("case", [c[0] for c in quantize_cases()])
def test_packers_reproduce_the_packed_planes(case):
    _, w, p, s, z = next(c for c in quantize_cases() if c[0] == case)
    for packer in (oracle.int4_quantize, oracle_np.int4_quantize, accel_amd.int4_quantize):
        got = packer(w)
        for g, want, what in zip(got, (p, s, z), ("codes", "scales", "zeros")):
            assert g.dtype == want.dtype and np.array_equal(g, want), (packer, what)


def test_fixtures_carry_the_reference_tests_known_answers():
    cases = {c[0]: c[1:] for c in quantize_cases()}
    # TestInt4PacksLowNibbleFirst: code 0 then code 15 in the low byte
    _, p, _, _ = cases["low_nibble_first"]
    assert p[0] & 0xFF == 0xF0
    # constant groups: zero scale, the constant as the zero point, exact readback
    w, p, s, z = cases["constant_groups"]
    assert np.all(s == 0)
    assert np.array_equal(oracle.f16_to_f32(z), np.array([0.0, 1.0, -2.5, 0.125], np.float32))
    back = oracle.int4_dequantize(p, s, z, w.size)
    assert np.array_equal(back, w)
    # odd length: the last weight is a group of its own and reads back exactly
    w, p, s, z = cases["odd_129"]
    assert s.size == 2 and s[1] == 0
    assert oracle.int4_dequantize(p, s, z, 129)[128] == w[128]


def test_the_oracle_reproduces_the_products():
    mv = load("matvec.npz")
    for c in ("seeded", "differential"):
        K, N = (int(v) for v in mv[f"{c}.shape"])
        got = oracle.quant_matvec_int4(mv[f"{c}.x"], mv[f"{c}.codes"], mv[f"{c}.scales"],
                                       mv[f"{c}.zeros"], K, N)
        assert np.array_equal(got.view(np.uint32), mv[f"{c}.out"].view(np.uint32)), c
    mm = load("matmul.npz")
    for c in ("seeded", "differential"):
        M, K, N = (int(v) for v in mm[f"{c}.shape"])
        got = oracle.quant_matmul_int4(mm[f"{c}.x"], mm[f"{c}.codes"], mm[f"{c}.scales"],
                                       mm[f"{c}.zeros"], M, K, N, threads=4)
        assert np.array_equal(got.view(np.uint32), mm[f"{c}.out"].view(np.uint32)), c


def test_the_oracle_reproduces_the_grouped_products_and_offsets():
    g = load("grouped.npz")
    E, T, K, N = (int(v) for v in g["shape"])
    off = oracle.segment_offsets(g["counts"])
    assert np.array_equal(off, g["offsets"])
    for name, fn, args in (
            ("grouped_matvec", oracle.grouped_matvec, (g["x"], g["w"])),
            ("grouped_matmul", oracle.grouped_matmul, (g["x"], g["w"])),
            ("int4_grouped_matvec", oracle.int4_grouped_matvec,
             (g["x"], g["codes"], g["scales"], g["zeros"])),
            ("int4_grouped_matmul", oracle.int4_grouped_matmul,
             (g["x"], g["codes"], g["scales"], g["zeros"]))):
        got = fn(*args, off, E, T, K, N)
        assert np.array_equal(got.view(np.uint32), g[name].view(np.uint32)), name
    seg = load("segment.npz")
    for c in ("ragged", "single", "wrap"):
        assert np.array_equal(oracle.segment_offsets(seg[f"{c}.counts"]), seg[f"{c}.offsets"])


# ---- the HIP path against the fixtures -----------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("case", [c[0] for c in quantize_cases()])
def test_device_packer_reproduces_the_packed_planes(dev, case):
    _, w, p, s, z = next(c for c in quantize_cases() if c[0] == case)
    n = w.size
    wb = dev.upload(np.ascontiguousarray(w, np.float32))
    pb = dev.alloc((p.size,), U32)
    sb = dev.alloc((s.size,), F16)
    zb = dev.alloc((z.size,), F16)
    pb.write(np.full(p.size, 0xDEADBEEF, np.uint32))
    dev.int4_quantize(wb, n, pb, sb, zb)
    for b, want, what in ((pb, p, "codes"), (sb, s, "scales"), (zb, z, "zeros")):
        assert np.array_equal(b.numpy(), want), what
    for b in (wb, pb, sb, zb):
        b.free()


@pytest.mark.gpu
def test_device_products_match_the_fixtures(dev):
    mv = load("matvec.npz")
    for c in ("seeded", "differential"):
        K, N = (int(v) for v in mv[f"{c}.shape"])
        w = dev.upload_int4(mv[f"{c}.codes"], mv[f"{c}.scales"], mv[f"{c}.zeros"], K * N)
        ab = dev.upload(mv[f"{c}.x"])
        ob = dev.alloc((N,), F32)
        dev.Int4MatVec(ab, w, ob)
        assert rel_l2(ob.numpy(), mv[f"{c}.out"]) <= F32_TOL, c
        ab.free(); ob.free(); w.free()
    mm = load("matmul.npz")
    for c in ("seeded", "differential"):
        M, K, N = (int(v) for v in mm[f"{c}.shape"])
        # the differential case's raw buffers carry more scales than its 640
        # weights own (the reference's kernel test binds buffers, not a
        # checked Int4); the operator takes exactly ceil(K*N/128)
        g = -(-K * N // 128)
        w = dev.upload_int4(mm[f"{c}.codes"], mm[f"{c}.scales"][:g], mm[f"{c}.zeros"][:g], K * N)
        ab = dev.upload(np.ascontiguousarray(mm[f"{c}.x"].reshape(M, K)))
        ob = dev.alloc((M, N), F32)
        dev.Int4MatMul(ab, w, ob)
        assert rel_l2(ob.numpy(), mm[f"{c}.out"]) <= F32_TOL, c
        ab.free(); ob.free(); w.free()


@pytest.mark.gpu
def test_device_grouped_products_and_offsets_match_the_fixtures(dev):
    g = load("grouped.npz")
    E, T, K, N = (int(v) for v in g["shape"])
    cb = dev.upload(g["counts"], U32)
    offb = dev.alloc((E + 1,), U32)
    dev.SegmentOffsets(cb, offb)
    assert np.array_equal(offb.numpy(), g["offsets"])
    offb.free()
    xb = dev.upload(g["x"])
    wb = dev.upload(g["w"])
    w4 = dev.upload_int4(g["codes"], g["scales"], g["zeros"], E * K * N)
    covered = int(g["offsets"][E])
    for name, call in (("grouped_matvec", lambda o: dev.GroupedMatVec(xb, wb, cb, o)),
                       ("grouped_matmul", lambda o: dev.GroupedMatMul(xb, wb, cb, o)),
                       ("int4_grouped_matvec", lambda o: dev.Int4GroupedMatVec(xb, w4, E, cb, o)),
                       ("int4_grouped_matmul", lambda o: dev.Int4GroupedMatMul(xb, w4, E, cb, o))):
        ob = dev.alloc((T, N), F32)
        ob.write(np.zeros((T, N), np.float32))
        call(ob)
        got, want = ob.numpy(), g[name]
        assert rel_l2(got[:covered], want[:covered]) <= F32_TOL, name
        if name.endswith("matvec"):
            assert np.all(got[covered:] == 0), name
        ob.free()
    for b in (xb, wb, cb):
        b.free()
    w4.free()
