#!/usr/bin/env python3
"""Writes the golden fixtures of the int4 path under tests/golden/.

    python tests/golden/make_golden.py

The reference (golang-design/accel) commits no data files for this path:
its int4 tests build their inputs in code.  These fixtures freeze small
inputs -- the reference tests' own constructions where they exist
(quant/int4_test.go, internal/kernels/differential_cases_test.go,
internal/kernels/grouped_test.go), seeded draws otherwise -- together with
the CPU oracle's outputs for them, which the oracle's tests pin against the
reference's known answers, closed forms and f64 brute force.  They are data
(numpy .npz, no pickles) plus a SHA-256 manifest; tests/test_golden.py
checks the oracle and the host packer against them on the CPU and the HIP
path against them on the GPU.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import oracle  # noqa: E402


def default_seed(b, i):
    """internal/kernels/differential_cases_test.go:78-80"""
    return np.float32(((i + b * 7) % 13 - 6) / 4)


def quantize_cases():
    rng = np.random.Generator(np.random.PCG64(20260))
    cases = {}
    # quant/int4_test.go:261-286: w[0]=0, w[1]=10, the rest 0.5
    w = np.full(128, 0.5, np.float32)
    w[0], w[1] = 0.0, 10.0
    cases["low_nibble_first"] = w
    # :22-36: constant groups reconstruct exactly
    cases["constant_groups"] = np.repeat(np.array([0.0, 1.0, -2.5, 0.125], np.float32), 128)
    # :225-253: an odd length, the last weight its own group (the test's
    # values, (i % 16) / 4)
    cases["odd_129"] = (np.arange(129) % 16).astype(np.float32) / 4
    # :93-158: clustered far from zero (the zero point rounds)
    cases["clustered_1000"] = (1000 + rng.random(256)).astype(np.float32)
    # seeded N(0, 0.02), the benchmark's distribution
    cases["normal"] = (rng.standard_normal(2048) * 0.02).astype(np.float32)
    # the f16 narrowing's edges: subnormal scales, the flush range, overflow
    cases["tiny"] = (rng.standard_normal(384) * 1e-7).astype(np.float32)
    cases["huge"] = (rng.standard_normal(256) * 1e30).astype(np.float32)
    w = rng.standard_normal(300).astype(np.float32)
    w[::37] = np.nan
    w[5::41] = np.inf
    cases["nan_inf"] = w
    return cases


def main():
    files = {}

    # packer
    out = {}
    for name, w in quantize_cases().items():
        p, s, z = oracle.int4_quantize(w)
        out[f"{name}.w"] = w
        out[f"{name}.codes"] = p
        out[f"{name}.scales"] = s
        out[f"{name}.zeros"] = z
    files["quantize.npz"] = out

    # QuantMatVecInt4: a seeded product and the differential raw-buffer case
    rng = np.random.Generator(np.random.PCG64(20261))
    K, N = 256, 384
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    mv = {"seeded.x": x, "seeded.codes": p, "seeded.scales": s, "seeded.zeros": z,
          "seeded.out": oracle.quant_matvec_int4(x, p, s, z, K, N),
          "seeded.shape": np.array([K, N], np.int64)}
    # differential_cases_test.go:1347-1368
    K2, N2 = 128, 2
    a2 = np.array([default_seed(0, i) for i in range(K2)], np.float32)
    words = np.array([i % 251 + 1 for i in range(K2 * N2 // 8)], np.uint32)
    s2 = oracle.to_f16(np.array([0.25, 0.25], np.float32))
    z2 = oracle.to_f16(np.array([4.0, 4.0], np.float32))
    mv.update({"differential.x": a2, "differential.codes": words, "differential.scales": s2,
               "differential.zeros": z2,
               "differential.out": oracle.quant_matvec_int4(a2, words, s2, z2, K2, N2),
               "differential.shape": np.array([K2, N2], np.int64)})
    files["matvec.npz"] = mv

    # QuantMatMulInt4: a seeded product and the differential tiled case
    M, K, N = 5, 256, 384
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    p, s, z = oracle.int4_quantize(w)
    mm = {"seeded.x": x, "seeded.codes": p, "seeded.scales": s, "seeded.zeros": z,
          "seeded.out": oracle.quant_matmul_int4(x, p, s, z, M, K, N),
          "seeded.shape": np.array([M, K, N], np.int64)}
    # differential_cases_test.go:1400-1424
    M3, K3, N3 = 3, 40, 16
    a3 = np.array([default_seed(0, i) for i in range(M3 * K3)], np.float32).reshape(M3, K3)
    words3 = np.array([i % 251 + 1 for i in range(K3 * N3 // 8)], np.uint32)
    s3 = oracle.to_f16(np.full(8, 0.25, np.float32))
    z3 = oracle.to_f16(np.full(8, 4.0, np.float32))
    mm.update({"differential.x": a3, "differential.codes": words3, "differential.scales": s3,
               "differential.zeros": z3,
               "differential.out": oracle.quant_matmul_int4(a3, words3, s3, z3, M3, K3, N3),
               "differential.shape": np.array([M3, K3, N3], np.int64)})
    files["matmul.npz"] = mm

    # grouped products: an empty expert and a padding row (grouped_test.go:94-267)
    E, T, K, N = 3, 10, 64, 128
    counts = np.array([4, 0, 5], np.uint32)
    off = oracle.segment_offsets(counts)
    x = rng.standard_normal((T, K)).astype(np.float32)
    wf = (rng.standard_normal((E, K, N)) * 0.05).astype(np.float32)
    p, s, z = oracle.int4_quantize(wf.ravel())
    gr = {"x": x, "w": wf, "counts": counts, "offsets": off, "codes": p, "scales": s, "zeros": z,
          "shape": np.array([E, T, K, N], np.int64),
          "grouped_matvec": oracle.grouped_matvec(x, wf, off, E, T, K, N),
          "grouped_matmul": oracle.grouped_matmul(x, wf, off, E, T, K, N),
          "int4_grouped_matvec": oracle.int4_grouped_matvec(x, p, s, z, off, E, T, K, N),
          "int4_grouped_matmul": oracle.int4_grouped_matmul(x, p, s, z, off, E, T, K, N)}
    files["grouped.npz"] = gr

    # SegmentOffsets, including the u32 wrap the reference's sum has
    seg = {}
    for name, c in {"ragged": [3, 0, 7, 1, 0, 12], "single": [5], "wrap": [0xFFFFFFF0, 0x20]}.items():
        c = np.array(c, np.uint32)
        seg[f"{name}.counts"] = c
        seg[f"{name}.offsets"] = oracle.segment_offsets(c)
    files["segment.npz"] = seg

    manifest = {}
    for name, arrays in files.items():
        path = os.path.join(HERE, name)
        # fixed member order and no timestamps: the file bytes are reproducible
        np.savez(path, **dict(sorted(arrays.items())))
        with open(path, "rb") as f:
            manifest[name] = hashlib.sha256(f.read()).hexdigest()
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
        f.write("\n")
    print(json.dumps(manifest, indent=1))


if __name__ == "__main__":
    main()
