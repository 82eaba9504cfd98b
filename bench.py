#!/usr/bin/env python3
"""Benchmark of the int4 weight-only linear path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-extra]

Headline (BASELINE.json's metric, M=1 leg): the decode product
Int4MatVec at M=1, K=N=4096, in the reference's int4 format (128-weight
groups, f16 scale and zero), f32 activations and output.  One step is one
product.  The weights rotate over enough device copies (> 512 MB in all) that
the 256 MB Infinity Cache cannot hold them, so each step reads its weights
from HBM.  K steps are captured into one HIP graph and replayed, bracketed
by events on the stream they run on; ``value`` is algorithmic bytes per step
over the per-step time.

The M=2048 leg (bf16 prefill product, TFLOP/s against the dense bf16 MFMA
peak) and the M=16 decode are reported under ``extra``.  ``cpu_baseline`` is
the oracle's restatement of the reference CPU backend's algorithm
(``oracle/``), timed on this host's cores on a bounded sample.

Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, vendor figure
METRIC = ("int4 linear: HBM GB/s (% peak) at M=1; TFLOP/s (% MFMA peak) at M=2048")
ROTATE_BYTES = 544 << 20       # weight copies in rotation, > 2x the Infinity Cache


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    return ap.parse_args()


def cpu_threads() -> int:
    # the GPU box grants 16 CPUs per GPU whatever os.cpu_count() reports
    n = os.cpu_count() or 1
    return max(1, min(n, 16))


class Timed:
    """Captures `count` calls of `issue(i)` into a graph and times replays."""

    def __init__(self, dev, stream, issue, count):
        self.dev, self.stream = dev, stream
        dev.capture_begin(stream)
        for i in range(count):
            issue(i)
        self.exec = dev.capture_end(stream)
        self.e0, self.e1 = dev.event(), dev.event()

    def run(self, replays: int) -> float:
        d = self.dev
        d.sync(self.stream)
        d.record(self.e0, self.stream)
        for _ in range(replays):
            d.launch(self.exec, self.stream)
        d.record(self.e1, self.stream)
        d.wait(self.e1)
        d.sync(self.stream)
        return d.elapsed_ms(self.e0, self.e1)

    def close(self):
        self.dev.destroy_exec(self.exec)
        self.dev.destroy_event(self.e0)
        self.dev.destroy_event(self.e1)


def bench_gemv(dev, stream, steps, warmup):
    import accel_amd
    from accel_amd import F32, workloads
    cfg = workloads.CONFIGS["gemv_m1"]
    L = workloads.linear(**cfg)
    K, N = L.K, L.N
    per_copy = L.packed.nbytes + L.scales.nbytes + L.zeros.nbytes
    copies = max(1, -(-ROTATE_BYTES // per_copy))
    w0 = dev.upload_int4(L.packed, L.scales, L.zeros, K * N)
    ws = [w0]
    for _ in range(copies - 1):
        w = accel_amd.Int4Weights(dev.alloc(w0.codes.shape, accel_amd.U32),
                                  dev.alloc(w0.scales.shape, accel_amd.F16),
                                  dev.alloc(w0.zeros.shape, accel_amd.F16), K * N)
        for src, dst in ((w0.codes, w.codes), (w0.scales, w.scales), (w0.zeros, w.zeros)):
            accel_amd._check(accel_amd.lib().accel_hip_copy(dev.index, stream, dst.ptr,
                                                            src.ptr, src.nbytes))
        ws.append(w)
    dev.sync(stream)
    a = dev.upload(L.x[0])
    out = dev.alloc((N,), F32)
    # eager once per copy: sizes the workspace and checks the result
    for w in ws:
        dev.Int4MatVec(a, w, out, stream=stream)
    dev.sync(stream)
    t = Timed(dev, stream, lambda i: dev.Int4MatVec(a, ws[i % copies], out, stream=stream),
              steps)
    if warmup:
        wt = Timed(dev, stream, lambda i: dev.Int4MatVec(a, ws[i % copies], out,
                                                         stream=stream), warmup)
        wt.run(1)
        wt.close()
    ms = t.run(1)
    t.close()
    got = out.numpy()
    bytes_per = workloads.algorithmic_bytes(1, K, N)
    ms_per = ms / steps
    for w in ws:
        w.free()
    a.free()
    out.free()
    return dict(ms_per_step=ms_per, bytes=bytes_per, gbs=bytes_per / (ms_per * 1e-3) / 1e9,
                copies=copies, L=L, out=got)


def bench_gemm(dev, stream, name, reps=20):
    from accel_amd import BF16, F32, workloads
    cfg = workloads.CONFIGS[name]
    L = workloads.linear(**cfg)
    M, K, N = L.M, L.K, L.N
    w = dev.upload_int4(L.packed, L.scales, L.zeros, K * N)
    if L.bf16:
        a = dev.upload(workloads.bf16_bits(L.x), BF16)
        out = dev.alloc((M, N), BF16)
    else:
        a = dev.upload(L.x)
        out = dev.alloc((M, N), F32)
    dev.Int4MatMul(a, w, out, stream=stream)
    dev.sync(stream)
    t = Timed(dev, stream, lambda i: dev.Int4MatMul(a, w, out, stream=stream), reps)
    t.run(1)
    ms = t.run(1) / reps
    t.close()
    flops = 2.0 * M * N * K
    act = 2 if L.bf16 else 4
    bytes_per = workloads.algorithmic_bytes(M, K, N, act, act)
    w.free(); a.free(); out.free()
    return dict(ms=ms, us=ms * 1e3, tflops=flops / (ms * 1e-3) / 1e12,
                gbs=bytes_per / (ms * 1e-3) / 1e9)


def cpu_baseline(L, seconds):
    import oracle
    threads = cpu_threads()
    x = L.x[0]
    oracle.quant_matvec_int4(x, L.packed, L.scales, L.zeros, L.K, L.N, threads=threads)
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.quant_matvec_int4(x, L.packed, L.scales, L.zeros, L.K, L.N, threads=threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    from accel_amd import workloads
    bytes_per = workloads.algorithmic_bytes(1, L.K, L.N)
    return dict(value=round(bytes_per * n / el / 1e9, 3), unit="GB/s", cores=threads,
                kind="port",
                sample=f"{n} calls of QuantMatVecInt4 at M=1 K=N=4096 in {el:.1f} s "
                       f"(oracle/oracle.c, reference order, {threads} threads)")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported "
              "(this build runs on a single MI355X; see DESIGN.md for how the path "
              "would shard)", file=sys.stderr)
        sys.exit(2)
    import accel_amd
    from accel_amd import workloads
    if accel_amd.device_count() < 1:
        print("no HIP device", file=sys.stderr)
        sys.exit(1)
    dev = accel_amd.Device(0)
    stream = dev.stream()
    steps = max(1, args.steps)
    r = bench_gemv(dev, stream, steps, args.warmup)
    L = r["L"]
    line = {
        "metric": METRIC,
        "value": round(r["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Int4MatVec M=1 K=4096 N=4096, int4 G=128 f16 scale+zero "
                        "(BASELINE config 1 shape in the reference format), f32 x/out, "
                        f"weights rotated over {r['copies']} device copies (HBM, not MALL)",
            "seed": 0,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(r["gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "int4_decode_f32_kernel<1, 32>",
            "bytes_per_launch": r["bytes"],
            "us_per_launch": round(r["ms_per_step"] * 1e3, 4),
        },
    }
    if not args.no_extra:
        extra = {}
        p = bench_gemm(dev, stream, "prefill_m2048")
        extra["prefill_m2048_bf16"] = {
            "tflops": round(p["tflops"], 2), "us": round(p["us"], 2),
            "frac_of_bf16_peak": round(p["tflops"] / BF16_PEAK_TFLOPS, 4)}
        d = bench_gemm(dev, stream, "decode_m16")
        extra["decode_m16_f32"] = {"us": round(d["us"], 2), "gbs": round(d["gbs"], 1),
                                   "frac_of_hbm": round(d["gbs"] / HBM_PEAK_GBS, 4)}
        line["extra"] = extra
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(L, args.cpu_seconds)
    dev.destroy_stream(stream)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
