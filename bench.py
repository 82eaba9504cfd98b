#!/usr/bin/env python3
"""Benchmark of the int4 weight-only linear path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-extra]
                    [--configs] [--eager]

Headline (the M=1 leg of BASELINE.json's metric): the decode product
Int4MatVec at M=1, K=N=4096, in the reference's int4 format (128-weight
groups, f16 scale and zero), f32 activations and output.  One step is one
product.  The weights rotate over device copies totalling more than 512 MB,
and the device's 256 MB Infinity Cache is flushed (a 512 MiB device copy,
untimed) before every timed replay, so each step reads its weights from HBM
at any --steps.  K steps are captured into one HIP graph and replayed,
bracketed by HIP events on the stream they run on; ``value`` is algorithmic
bytes per step over the per-step time, and ``roofline`` prices the same
kernel against the HBM peak.  ``roofline.traffic`` is the HBM bytes a launch
of that kernel moves, from the rocprofv3 FETCH_SIZE / WRITE_SIZE summary
committed under profiles/ (null when absent).

``extra`` holds every other BASELINE config, each with a roofline object of
its own and CPU baselines beside it: the M=2048 leg of the metric (config 3,
bf16 prefill on the matrix cores, TFLOP/s against the dense bf16 peak),
config 2 (M=16 decode), config 4 (the ragged MoE product), config 5 (the
seven-product layer chain at batch 1 and 8, weights rotated over five sets),
and the reference's own published workload (Int4MatVec 2048 x 2048, one
submission waited for per step), which ``vs_baseline`` compares with the
published 0.76 ms.  ``--configs`` adds the widened rows (int8, the f16
matvec, the fused Linear, the repack, whole decode steps).  ``--eager``
times plain stream launches instead of graph replays (for profiler runs).

``cpu_baseline`` is the oracle's restatement of the reference CPU backend's
algorithm (``oracle/``), timed on this host's cores on a bounded sample of
the headline workload; ``extra.cpu_baselines`` does the same for configs 2-5
at 16 threads and at one thread.

Prints one JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, vendor figure
METRIC = ("int4 linear: HBM GB/s (% peak) at M=1; TFLOP/s (% MFMA peak) at M=2048")
ROTATE_BYTES = 544 << 20       # weight copies in rotation, > 2x the Infinity Cache
TRAFFIC_FILE = os.path.join(HERE, "profiles", "traffic.json")
GEMV_KERNEL = "int4_panel_matvec_kernel<4, false, true, true, false>"
GEMV_REF_KERNEL = "int4_decode_f32_kernel<1, 256, 32, false, float>"
GEMM_KERNEL = "int4_gemm_bf16_kernel<8, false>"
GEMM_F32_KERNEL = "int4_gemm_f32x3_kernel"
DECODE_MFMA_KERNEL = "int4_decode_mfma_kernel<2, 8, float>"
DECODE_SIDE_KERNEL = "int4_decode_mfma_side_kernel<2, 8>"
SPLITK_BF16_KERNEL = "int4_gemm_bf16_splitk_kernel<2>"
SPLITK_F32_KERNEL = "int4_gemm_f32x3_kernel (split K, M=64)"
GROUPED_KERNEL = "int4_grouped_bf16_kernel"
G32_KERNEL = "int4_g32_matvec_kernel"
REDUCE_KERNEL = "int4_gemm_reduce_kernel"
# Keys of the PMC summary (profiles/traffic.json) for products of several
# launches: a key is the kernel's name, with the launch's role where one
# kernel serves two.  The short prefills are the split-K kernel and the
# reduction pass.
SPLITK_BF16_LAUNCHES = (SPLITK_BF16_KERNEL, f"{REDUCE_KERNEL} (after {SPLITK_BF16_KERNEL})")
SPLITK_F32_LAUNCHES = (SPLITK_F32_KERNEL, f"{REDUCE_KERNEL} (after int4_gemm_f32x3_kernel, M=64)")
# The grouped decode products are two launches: the VALU decode kernel (the
# padding rows, and every row should the offsets have wrapped), then each
# expert's rows in blocks of up to 16 on the matrix cores.
_GD = "int4_grouped_decode_kernel<512, 32, true, float>"
_GDM = "int4_grouped_decode_mfma_kernel<2, 8, float>"
_GDS = "int4_grouped_decode_mfma_side_kernel<2, 8, float>"
GROUPED_F32_LAUNCHES = (f"{_GD} (1024 rows)", f"{_GDS} (1024 rows)")
GROUPED_DECODE_LAUNCHES = (f"{_GD} (16 rows)", f"{_GDS} (16 rows)")
# the same products on the reference planes
GROUPED_F32_PLANES_LAUNCHES = (f"{_GD} (1024 rows)", f"{_GDM} (1024 rows)")
GROUPED_DECODE_PLANES_LAUNCHES = (f"{_GD} (16 rows)", f"{_GDM} (16 rows)")
# the decode MoE's rows on experts bound into the panel layout
GROUPED_DECODE_PANEL_LAUNCHES = (f"{_GD} (8 rows)",
                                 "int4_grouped_panel_rows_kernel<2, true> (8 rows)")
# config 5's five launches a step, by variant
_PS = "int4_panel_matvec_kernel<4, false, true, true, true>"
_MF1 = "int4_decode_mfma_kernel<1, 8, float>"
CHAIN_LAUNCHES = {
    "prepared_b1": (f"{_PS} (q/k/v set, batch 1)", GEMV_KERNEL,
                    "int4_panel_swiglu_kernel<4, false, true, true> (gate/up, batch 1)",
                    "int4_panel_matvec_kernel<7, true, true, true, false> (down, batch 1)"),
    "planes_b1": ("int4_decode_set_kernel<1, 256, 32, false> (q/k/v set, batch 1)",
                  GEMV_REF_KERNEL,
                  "int4_decode_set_kernel<1, 512, 32, false> (gate/up set, batch 1)",
                  "swiglu_kernel (batch 1)", f"{GEMV_REF_KERNEL} (down, batch 1)"),
    "prepared_b8": ("int4_decode_mfma_side_set_kernel<1, 8> (q/k/v set, batch 8)",
                    "int4_decode_mfma_side_kernel<1, 8> (o, batch 8)",
                    "int4_decode_mfma_side_set_kernel<2, 8> (gate/up set, batch 8)",
                    "swiglu_kernel (batch 8)",
                    "int4_decode_mfma_side_kernel<1, 8> (down, batch 8)"),
    "planes_b8": ("int4_decode_mfma_set_kernel<1, 8> (q/k/v set, batch 8)",
                  f"{_MF1} (o, batch 8)",
                  "int4_decode_mfma_set_kernel<2, 8> (gate/up set, batch 8)",
                  "swiglu_kernel (batch 8)", f"{_MF1} (down, batch 8)"),
}
FLUSH_BYTES = 1 << 30          # device read that evicts the Infinity Cache
EAGER_MAX = 64                 # timed regions of at most this many calls run as plain launches
PUBLISHED_US = 760.0           # Int4MatVec [2048] x [2048,2048] on an M2, one plan a step
PUBLISHED_SRC = "specs/010-kernel-corpus.md:593-602 (tensor/decodebench_darwin_test.go:148-189)"


def progress(msg: str) -> None:
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=640)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--configs", action="store_true",
                    help="also time BASELINE configs 2, 4 and 5 (slower)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default="",
                    help="comma-separated extra lines to time (e.g. prefill_m2048_bf16); "
                         "the headline always runs")
    ap.add_argument("--eager", action="store_true",
                    help="time plain stream launches, not graph replays (profiler runs)")
    return ap.parse_args()


def cpu_threads() -> int:
    # the GPU box grants 16 CPUs per GPU whatever os.cpu_count() reports
    n = os.cpu_count() or 1
    return max(1, min(n, 16))


def traffic_of(kernel: str):
    """HBM bytes per launch of `kernel` from the committed PMC summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)["kernels"][kernel]
        return int(t["hbm_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


def traffic_sum(kernels):
    """HBM bytes of a call made of one launch of each of `kernels`, or None
    when the summary lacks any of them."""
    parts = [traffic_of(k) for k in kernels]
    return None if any(p is None for p in parts) else sum(parts)


class Flusher:
    """Evicts the Infinity Cache with an untimed read of 1 GiB of device memory
    (accel_hip_floor kind 2), so that the calls timed after it read their
    weights from HBM.  A read, not a copy: a copy leaves up to the cache's
    256 MB of dirty lines whose writeback would land in the timed region."""

    def __init__(self, dev):
        import accel_amd
        self.dev = dev
        self.src = dev.alloc((FLUSH_BYTES // 4,), accel_amd.U32)
        self.sink = dev.alloc((1024,), accel_amd.U32)

    def __call__(self, stream):
        import accel_amd
        accel_amd._check(accel_amd.lib().accel_hip_floor(self.dev.index, stream, 2,
                                                         self.src.ptr, FLUSH_BYTES,
                                                         self.sink.ptr))

    def free(self):
        self.src.free()
        self.sink.free()


_FLUSH = None
EAGER = False


def flush(dev, stream):
    global _FLUSH
    if _FLUSH is None:
        _FLUSH = Flusher(dev)
    _FLUSH(stream)


class Timed:
    """Captures `count` calls of `issue(i)` into a graph and times replays
    with HIP events on the stream the graph runs on (or, with EAGER or a
    region of at most EAGER_MAX calls, issues the calls as plain launches
    between the events).  The Infinity Cache is evicted before every timed
    run, by a read that the calls and the events are queued behind, so the
    host has queued the whole region before the device reaches it.  A short
    region is timed as plain launches because a graph launch carries a fixed
    start-up on the device (measured at config 1: 4.69 us a call at 20 steps
    in a graph, 4.46 as plain launches, 4.35 either way at 640)."""

    def __init__(self, dev, stream, issue, count):
        self.dev, self.stream, self.issue, self.count = dev, stream, issue, count
        self.exec = None
        self.e0, self.e1 = dev.event(), dev.event()
        if not (EAGER or count <= EAGER_MAX):
            dev.capture_begin(stream)
            for i in range(count):
                issue(i)
            self.exec = dev.capture_end(stream)
        self.warm = False

    def _once(self):
        if self.exec is not None:
            self.dev.launch(self.exec, self.stream)
        else:
            for i in range(self.count):
                self.issue(i)

    def run(self) -> float:
        """Milliseconds for the K calls, timed after one untimed run (the
        first launch of a graph also uploads it)."""
        d = self.dev
        if not self.warm:
            self._once()
            d.sync(self.stream)
            self.warm = True
        flush(d, self.stream)
        d.record(self.e0, self.stream)
        self._once()
        d.record(self.e1, self.stream)
        d.sync(self.stream)
        return d.elapsed_ms(self.e0, self.e1)

    def close(self):
        if self.exec is not None:
            self.dev.destroy_exec(self.exec)
        self.dev.destroy_event(self.e0)
        self.dev.destroy_event(self.e1)


def median_replay(t, replays: int = 3) -> float:
    """Median over `replays` warm replays of a captured graph, in ms."""
    return float(np.median([t.run() for _ in range(replays)]))


def rotated_weights(dev, stream, L, total_bytes=ROTATE_BYTES):
    """Device copies of L's int4 planes, enough that they exceed the cache."""
    import accel_amd
    per_copy = L.packed.nbytes + L.scales.nbytes + L.zeros.nbytes
    copies = max(1, -(-total_bytes // per_copy))
    w0 = dev.upload_int4(L.packed, L.scales, L.zeros, L.K * L.N)
    ws = [w0]
    for _ in range(copies - 1):
        w = accel_amd.Int4Weights(dev.alloc(w0.codes.shape, accel_amd.U32),
                                  dev.alloc(w0.scales.shape, accel_amd.F16),
                                  dev.alloc(w0.zeros.shape, accel_amd.F16), L.K * L.N)
        for src, dst in ((w0.codes, w.codes), (w0.scales, w.scales), (w0.zeros, w.zeros)):
            accel_amd._check(accel_amd.lib().accel_hip_copy(dev.index, stream, dst.ptr,
                                                            src.ptr, src.nbytes))
        ws.append(w)
    dev.sync(stream)
    return ws


def time_product(dev, stream, L, call, steps, warmup, bf16=False, prepare=None):
    """Per-call time of `call(a, w, out)` over rotated weights, in ms.  With
    `prepare`, every copy is bound first (prepare(w), outside the timed
    region, its reference planes then freed) and `call` takes the bound
    weight."""
    from accel_amd import BF16, F32, workloads
    ws = rotated_weights(dev, stream, L)
    bind_ms = None
    if prepare is not None:
        bound = []
        for i, w in enumerate(ws):
            t0 = time.perf_counter()
            bound.append(prepare(w))
            if i == 0:
                bind_ms = (time.perf_counter() - t0) * 1e3
            w.free()
        ws = bound
    if bf16:
        a = dev.upload(workloads.bf16_bits(L.x), BF16)
        out = dev.alloc((L.M, L.N), BF16)
    else:
        a = dev.upload(L.x if L.M > 1 else L.x[0])
        out = dev.alloc((L.M, L.N) if L.M > 1 else (L.N,), F32)
    for w in ws:  # eager once per copy: sizes the workspace
        call(a, w, out, stream)
    dev.sync(stream)
    if warmup:
        wt = Timed(dev, stream, lambda i: call(a, ws[i % len(ws)], out, stream), warmup)
        wt.run()
        wt.close()
    t = Timed(dev, stream, lambda i: call(a, ws[i % len(ws)], out, stream), steps)
    ms = median_replay(t) / steps
    t.close()
    got = out.numpy()
    for w in ws:
        w.free()
    a.free()
    out.free()
    if prepare is not None:
        return ms, got, len(ws), bind_ms
    return ms, got, len(ws)


def bench_gemv(dev, stream, steps, warmup):
    """Config 1 on a bound weight: each rotated copy is prepared once
    (accel_int4_prepare, outside the timed region, as a backend does when it
    compiles a plan) and the step is Int4MatVecPrepared.  The same product on
    the reference planes (accel_int4_matvec) is timed beside it."""
    from accel_amd import workloads
    L = workloads.linear(**workloads.CONFIGS["gemv_m1"])
    ms, got, copies, bind_ms = time_product(
        dev, stream, L, lambda a, w, o, s: dev.Int4MatVecPrepared(a, w, o, s), steps, warmup,
        prepare=lambda w: dev.prepare_int4(w, L.K, L.N, stream))
    ms_ref, got_ref, _ = time_product(
        dev, stream, L, lambda a, w, o, s: dev.Int4MatVec(a, w, o, s), steps, warmup)
    bytes_per = workloads.algorithmic_bytes(1, L.K, L.N)
    return dict(ms=ms, bytes=bytes_per, gbs=bytes_per / (ms * 1e-3) / 1e9, copies=copies,
                L=L, out=got, bind_ms=bind_ms, ms_ref=ms_ref,
                gbs_ref=bytes_per / (ms_ref * 1e-3) / 1e9)


def bench_gemv_g32(dev, stream, steps=640, warmup=64):
    """Config 1 in BASELINE's literal format (32-row groups along K, f32 scale,
    no zero: no counterpart in the reference), the additive variant reported
    beside the reference-format headline.  Weights rotated over copies
    totalling more than 512 MB; cache flushed before the timed replay."""
    import accel_amd
    from accel_amd import F32, U32
    rng = np.random.Generator(np.random.PCG64(0))
    x = rng.standard_normal((1, 4096)).astype(np.float32)
    w = np.ascontiguousarray((rng.standard_normal((4096, 4096)) * 0.02).astype(np.float32).T)
    p, sc = accel_amd.int4_g32_quantize(w)
    K = N = 4096
    per = p.nbytes + sc.nbytes
    copies = max(1, -(-ROTATE_BYTES // per))
    cs = [dev.upload(p, U32) for _ in range(copies)]
    ss = [dev.upload(sc.reshape(-1), F32) for _ in range(copies)]
    a = dev.upload(x[0])
    out = dev.alloc((N,), F32)
    for i in range(copies):
        dev.Int4G32MatVec(a, cs[i], ss[i], K, N, out, stream)
    dev.sync(stream)
    if warmup:
        wt = Timed(dev, stream, lambda i: dev.Int4G32MatVec(a, cs[i % copies], ss[i % copies],
                                                             K, N, out, stream), warmup)
        wt.run()
        wt.close()
    t = Timed(dev, stream, lambda i: dev.Int4G32MatVec(a, cs[i % copies], ss[i % copies], K, N,
                                                        out, stream), steps)
    ms = median_replay(t) / steps
    t.close()
    for b in cs + ss + [a, out]:
        b.free()
    nbytes = K * N // 2 + 4 * (K // 32) * N + 4 * K + 4 * N
    gbs = nbytes / (ms * 1e-3) / 1e9
    return dict(workload="config 1 in BASELINE's literal format -- int4, 32-row groups along K, "
                         "f32 scale, no zero point (an additive variant: the reference format "
                         "has 128-weight groups with f16 scale and zero); Int4G32MatVec M=1 "
                         f"K=N=4096, f32 x/out, seed 0; weights rotated over {copies} copies",
                us=round(ms * 1e3, 3),
                roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                          "traffic": traffic_of(G32_KERNEL), "kernel": G32_KERNEL,
                          "bytes_per_launch": int(nbytes)})


def bench_gemm(dev, stream, name, steps=40, warmup=4, tiles=False):
    """Int4MatMul of a named config over rotated weights; with tiles, each
    weight bound once for the matrix-core decode (accel_int4_prepare_tiles,
    outside the timed region) and the calls Int4MatMulPrepared."""
    from accel_amd import workloads
    L = workloads.linear(**workloads.CONFIGS[name])
    bind_ms = None
    if tiles:
        ms, _, copies, bind_ms = time_product(
            dev, stream, L, lambda a, w, o, s: dev.Int4MatMulPrepared(a, w, o, s), steps,
            warmup, prepare=lambda w: dev.prepare_int4(w, L.K, L.N, stream, tiles=True))
    else:
        ms, _, copies = time_product(dev, stream, L,
                                     lambda a, w, o, s: dev.Int4MatMul(a, w, o, s), steps,
                                     warmup, bf16=L.bf16)
    flops = 2.0 * L.M * L.N * L.K
    act = 2 if L.bf16 else 4
    bytes_per = workloads.algorithmic_bytes(L.M, L.K, L.N, act, act)
    return dict(ms=ms, us=ms * 1e3, tflops=flops / (ms * 1e-3) / 1e12,
                gbs=bytes_per / (ms * 1e-3) / 1e9, copies=copies, bytes=bytes_per,
                bind_ms=bind_ms)


def _grouped_timings(dev, stream, steps, call, forms):
    """Median time of a grouped call over the rotating copies of each form
    of the experts (forms: key -> copies; call(copy, key))."""
    out = {}
    for key, copies in forms.items():
        for i in range(len(copies)):
            call(copies[i], key)
        dev.sync(stream)
        t = Timed(dev, stream, lambda i: call(copies[i % len(copies)], key), steps)
        out[key] = median_replay(t) / steps
        t.close()
    return out


def _prepare_grouped(dev, ws, m, panels=False):
    """Each copy of the experts bound once (accel_int4_prepare_grouped, or
    with panels accel_int4_prepare_grouped_panels); returns the copies and
    the host time of one bind in ms."""
    pws, bind_ms = [], None
    for w in ws:
        t0 = time.perf_counter()
        pws.append(dev.prepare_int4_grouped(w, m.E, m.K, m.N, panels=panels))
        bind_ms = bind_ms or (time.perf_counter() - t0) * 1e3
    return pws, bind_ms


def bench_moe(dev, stream, steps=20, bf16=True, prepared=False):
    """Config 4: Int4GroupedMatMul over 1024 routed bf16 rows, 8 experts (with
    bf16=False, the same rows in f32, the reference API's grouped dtype).  The
    experts' weights (250 MB) rotate over three copies (750 MB), so with the
    cache flushed before the timed replay every call reads them from HBM.
    With f32 rows the same call on experts bound once (outside the timed
    region, scales and zeros side-copied for the matrix-core decode) is timed
    beside it, as us_prepared; prepared=True makes that the line's figure."""
    both = prepared or not bf16
    from accel_amd import BF16, F32, U32, workloads
    progress("config 4: routing and quantizing eight experts")
    m = workloads.moe_fast()
    R = int(m.counts.sum())
    copies = 3
    ws = [dev.upload_int4(m.packed, m.scales, m.zeros, m.E * m.K * m.N) for _ in range(copies)]
    if bf16:
        xb = dev.upload(workloads.bf16_bits(m.x), BF16)
        ob = dev.alloc((R, m.N), BF16)
    else:
        xb = dev.upload(np.ascontiguousarray(m.x, np.float32))
        ob = dev.alloc((R, m.N), F32)
    cb = dev.upload(m.counts, U32)
    pws, bind_ms = _prepare_grouped(dev, ws, m) if both else (None, None)

    def call(w, prep):
        if prep:
            dev.Int4GroupedMatMulPrepared(xb, w, cb, ob, stream=stream)
        else:
            dev.Int4GroupedMatMul(xb, w, m.E, cb, ob, stream=stream)

    times = _grouped_timings(dev, stream, steps, call,
                             {True: pws, False: ws} if both else {False: ws})
    ms = times[prepared]
    for w in pws or ():
        w.free()
    flops = 2.0 * R * m.K * m.N
    wbytes = m.packed.nbytes + m.scales.nbytes + m.zeros.nbytes
    esz = 2 if bf16 else 4
    nbytes = wbytes + R * m.K * esz + R * m.N * esz
    for b in (xb, cb, ob):
        b.free()
    for w in ws:
        w.free()
    tflops = flops / (ms * 1e-3) / 1e12
    dt = "bf16" if bf16 else "f32"
    launches = (GROUPED_F32_LAUNCHES if prepared else GROUPED_F32_PLANES_LAUNCHES)
    kernel = GROUPED_KERNEL if bf16 else " + ".join(launches)
    extra = {}
    if prepared:
        extra = dict(us_reference_planes=round(times[False] * 1e3, 2), bind_ms=round(bind_ms, 1))
    elif both:
        extra = dict(us_prepared=round(times[True] * 1e3, 2), bind_ms=round(bind_ms, 1))
    op = "Int4GroupedMatMulPrepared" if prepared else "Int4GroupedMatMul"
    return dict(workload=f"{op}: {R} routed {dt} rows (512 tokens, top-2 of 8 "
                         f"experts, seed 3), K={m.K}, N={m.N}, {dt} out; expert weights "
                         f"rotated over {copies} copies"
                         + ("" if bf16 else "; each expert's rows in blocks of up to 16 on "
                            "the matrix-core decode kernel (x*512s in three bf16 terms)")
                         + ("; experts bound once (accel_int4_prepare_grouped: the planes and "
                            "a side copy of each expert's scales and zeros), the same call on "
                            "the planes in us_reference_planes" if prepared else "")
                         + ("; the same call on experts bound once (accel_int4_prepare_grouped) "
                            "in us_prepared" if both and not prepared else ""),
                us=round(ms * 1e3, 2), rows=R, experts=m.E, **extra,
                counts=[int(c) for c in m.counts],
                roofline={"bound": "mfma", "achieved": round(tflops, 1),
                          "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                          "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                          "traffic": traffic_sum((kernel,) if bf16 else launches),
                          "kernel": kernel,
                          "flops_per_launch": int(flops), "bytes_per_launch": int(nbytes),
                          "hbm_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1)})


def bench_moe_decode(dev, stream, tokens=8, steps=40, form="side"):
    """Decode MoE: `tokens` tokens routed top-2 over config 4's eight experts
    (K=4096, N=14336) as f32 rows, Int4GroupedMatVec -- decode products of
    each expert's routed rows against its matrix (blocks of up to 16 rows on
    the matrix cores).  Three copies of the experts
    (750 MB) rotate and the cache is flushed before the timed replay.
    The experts are bound once (outside the timed region) in both prepared
    forms, and the call is timed on each and on the planes: `form` ("panels":
    accel_int4_prepare_grouped_panels, the few-rows panel kernel; "side":
    accel_int4_prepare_grouped, the matrix-core blocks on side copies;
    "planes") is the line's figure, the others are reported beside it."""
    from accel_amd import F32, U32, workloads
    progress(f"decode MoE: {tokens} tokens, top-2 of 8 experts")
    m = workloads.moe_fast(tokens=tokens)
    R = int(m.counts.sum())
    copies = 3
    ws = [dev.upload_int4(m.packed, m.scales, m.zeros, m.E * m.K * m.N) for _ in range(copies)]
    xb = dev.upload(m.x)
    cb = dev.upload(m.counts, U32)
    ob = dev.alloc((R, m.N), F32)
    forms = {"planes": ws}
    bind = {}
    for f in ("panels", "side"):
        forms[f], bind[f] = _prepare_grouped(dev, ws, m, panels=f == "panels")

    def call(w, f):
        if f == "planes":
            dev.Int4GroupedMatVec(xb, w, m.E, cb, ob, stream=stream)
        else:
            dev.Int4GroupedMatVecPrepared(xb, w, cb, ob, stream=stream)

    times = _grouped_timings(dev, stream, steps, call, forms)
    ms = times[form]
    for f in ("panels", "side"):
        for w in forms[f]:
            w.free()
    active = int((m.counts > 0).sum())
    per_expert = (m.packed.nbytes + m.scales.nbytes + m.zeros.nbytes) // m.E
    nbytes = active * per_expert + R * m.K * 4 + R * m.N * 4
    for b in (xb, cb, ob):
        b.free()
    for w in ws:
        w.free()
    gbs = nbytes / (ms * 1e-3) / 1e9
    launches = {"panels": GROUPED_DECODE_PANEL_LAUNCHES, "side": GROUPED_DECODE_LAUNCHES,
                "planes": GROUPED_DECODE_PLANES_LAUNCHES}[form]
    extra = {f"us_{k}": round(v * 1e3, 2) for k, v in
             (("panels", times["panels"]), ("side_copies", times["side"]),
              ("reference_planes", times["planes"]))}
    extra.update({f"bind_ms_{k}": round(v, 1) for k, v in bind.items()})
    op = "Int4GroupedMatVec" if form == "planes" else "Int4GroupedMatVecPrepared"
    return dict(workload=f"{op}, decode MoE: {tokens} tokens routed top-2 over 8 "
                         f"experts ({R} f32 rows, seed 3's routing), K={m.K}, N={m.N}, f32 out; "
                         f"the {active} active experts' weights read once; experts rotated over "
                         f"{copies} copies"
                         + {"panels": "; experts bound once into the panel layout "
                                      "(accel_int4_prepare_grouped_panels): the few-rows panel "
                                      "kernel",
                            "side": "; experts bound once with side copies of their scales and "
                                    "zeros (accel_int4_prepare_grouped): the matrix-core blocks",
                            "planes": ""}[form]
                         + "; the same call on each form of the experts in us_panels, "
                           "us_side_copies and us_reference_planes",
                us=round(ms * 1e3, 2), rows=R, active_experts=active, **extra,
                counts=[int(c) for c in m.counts],
                roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                          "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                          "traffic": traffic_sum(launches),
                          "kernel": " + ".join(launches),
                          "bytes_per_launch": int(nbytes)})


_LAYER_PLANES = {}


def layer_planes(rng):
    """Config 5's seven weights (seed 4's stream, after x and the gains)."""
    from accel_amd import workloads
    if not _LAYER_PLANES:
        for name, (K, N) in workloads.LAYER_SHAPES.items():
            _LAYER_PLANES[name] = workloads.fast_int4(K, N, rng)
    return _LAYER_PLANES


def bench_layer_chain(dev, stream, batch, steps=100, merged=True, sets=5, prepared=None,
                      fused=None):
    """Config 5: one Llama-3-8B-shaped decoder layer's seven int4 products
    as a decode step: q,k,v <- x; o <- q; gate,up <- o; down <- SwiGLU(gate,
    up), the gate/up pair through tensor.SwiGLU (silu(gate) * up) on the
    device, so the step is seven products and the one elementwise operation
    that joins them.  merged: q, k, v and gate, up each as one set (the same
    results bit for bit).  prepared (the default): every matrix bound once
    (outside the timed region) -- at batch 1 into the panel layout, at batch 8
    as codes plus side copies of the scales and zeros for the matrix-core
    decode -- and the products run as Int4MatVecPrepared[Set] or
    Int4MatMulPrepared[Set].  fused (the default on prepared weights at batch
    1): gate, up and SwiGLU as one launch, Int4MatVecPreparedSwiGLU (the same
    result bit for bit), with the step's time unfused reported beside it.
    The layer's 115.9 MB of weights rotate over `sets` copies (580 MB), so
    with the cache flushed before the timed replay each step reads its
    weights from HBM."""
    from accel_amd import F32, workloads
    if prepared is None:
        prepared = batch in (1, 8)
    if fused is None:
        fused = prepared and merged and batch == 1
    shapes = workloads.LAYER_SHAPES  # name -> (K, N)
    rng = np.random.Generator(np.random.PCG64(4))
    x = rng.standard_normal((batch, 4096)).astype(np.float32)
    rng.standard_normal(4096)   # the two RMSNorm gains of the decode step
    rng.standard_normal(4096)
    planes = layer_planes(rng)
    wsets, bufs = [], {}
    total_bytes = 0
    for name, (K, N) in shapes.items():
        packed, scales, zeros = planes[name]
        total_bytes += packed.nbytes + scales.nbytes + zeros.nbytes
        bufs[name] = dev.alloc((batch, N) if batch > 1 else (N,), F32)
    bind_ms = None
    for _ in range(sets):
        ws = {name: dev.upload_int4(*planes[name], K * N) for name, (K, N) in shapes.items()}
        if prepared:
            t0 = time.perf_counter()
            # one row: the panel layout; eight: codes and side copies for
            # the matrix-core decode
            pws = {name: dev.prepare_int4(ws[name], K, N, stream, tiles=batch > 1)
                   for name, (K, N) in shapes.items()}
            bind_ms = bind_ms or (time.perf_counter() - t0) * 1e3
            for w in ws.values():
                w.free()
            ws = pws
        wsets.append(ws)
    xin = dev.upload(x if batch > 1 else x[0])
    act = dev.alloc((batch, 14336) if batch > 1 else (14336,), F32)   # SwiGLU(gate, up)

    def op(a, w, o):
        if prepared:
            if batch > 1:
                dev.Int4MatMulPrepared(a, w, o, stream)
            else:
                dev.Int4MatVecPrepared(a, w, o, stream)
        elif batch > 1:
            dev.Int4MatMul(a, w, o, stream)
        else:
            dev.Int4MatVec(a, w, o, stream)

    def ops(a, ws, names):
        if merged:
            fn = ((dev.Int4MatMulPreparedSet if batch > 1 else dev.Int4MatVecPreparedSet)
                  if prepared else
                  dev.Int4MatVecSet if batch == 1 else dev.Int4MatMulSet)
            fn(a, [ws[n] for n in names], [bufs[n] for n in names], stream)
        else:
            for n in names:
                op(a, ws[n], bufs[n])

    def step_with(i, fuse):
        ws = wsets[i % sets]
        ops(xin, ws, ("q", "k", "v"))
        op(bufs["q"], ws["o"], bufs["o"])
        if fuse:
            dev.Int4MatVecPreparedSwiGLU(bufs["o"], ws["gate"], ws["up"], act, stream)
        else:
            ops(bufs["o"], ws, ("gate", "up"))
            dev.SwiGLU(bufs["gate"], bufs["up"], act, stream)
        op(act, ws["down"], bufs["down"])

    def timed(fuse):
        for i in range(sets):
            step_with(i, fuse)
        dev.sync(stream)
        t = Timed(dev, stream, lambda i: step_with(i, fuse), steps)
        r = median_replay(t) / steps
        t.close()
        return r

    ms = timed(fused)
    ms_unfused = timed(False) if fused else None
    for ws in wsets:
        for w in ws.values():
            w.free()
    for b in list(bufs.values()) + [xin, act]:
        b.free()
    # activations read and results written by the products, and SwiGLU's
    # two reads and one write of the 14336-wide rows
    act_bytes = 4 * batch * (4096 + 4096 + 4096 + 14336) + 4 * batch * (
        4096 + 1024 + 1024 + 4096 + 14336 + 14336 + 4096) + 12 * batch * 14336
    if fused:
        # gate and up stay in the workgroup: only SwiGLU's result is written
        act_bytes = 4 * batch * (4096 + 4096 + 4096 + 14336) + 4 * batch * (
            4096 + 1024 + 1024 + 4096 + 14336 + 4096)
    gbs = (total_bytes + act_bytes) / (ms * 1e-3) / 1e9
    if prepared and fused:
        kernels = ("int4_panel_matvec_kernel (prepared weights) + int4_panel_swiglu_kernel "
                   "(gate, up and SwiGLU)")
    elif prepared:
        kernels = ("int4_decode_mfma_side_set_kernel + int4_decode_mfma_side_kernel "
                   "(matrix-core decode, scales and zeros from the side copies)"
                   if batch > 1 else "int4_panel_matvec_kernel (prepared weights)") + \
            " + swiglu_kernel"
    elif batch == 1:
        kernels = "int4_decode_set_kernel + int4_decode_f32_kernel (VALU decode) + swiglu_kernel"
    else:
        kernels = ("int4_decode_mfma_set_kernel + int4_decode_mfma_kernel (matrix-core decode) "
                   "+ swiglu_kernel")
    launches = (4 if merged else 7) + (0 if fused else 1)
    variant = ("prepared_b1" if batch == 1 else "prepared_b8") if prepared else (
        "planes_b1" if batch == 1 else "planes_b8")
    traffic = (traffic_sum(CHAIN_LAUNCHES[variant])
               if merged and batch in (1, 8) and variant else None)
    res = dict(workload=f"config 5: seven Llama-3-8B layer products as one decode step at "
                        f"batch {batch}, down fed SwiGLU(gate, up) computed on the device "
                        + (f"(q/k/v as a set, gate/up and SwiGLU as one launch: {launches} "
                           f"launches), f32 x, " if fused else
                           f"(q/k/v and gate/up as sets: {launches} launches), f32 x, ")
                        + (("weights bound once into the panel layout, " if batch == 1 else
                            "weights bound once as codes plus side copies of the scales and "
                            "zeros (matrix-core decode), ") if prepared else
                           "reference planes, ")
                        + f"rotated over {sets} sets",
               us_per_step=round(ms * 1e3, 2), batch=batch, launches=launches,
               weight_bytes=total_bytes,
               roofline={"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": traffic, "kernel": kernels,
                         "bytes_per_step": int(total_bytes + act_bytes)})
    if bind_ms is not None:
        res["bind_ms_per_layer"] = round(bind_ms, 3)
    if ms_unfused is not None:
        res["us_per_step_unfused"] = round(ms_unfused * 1e3, 2)
    return res


def bench_published(dev, stream, steps=200):
    """The reference's published decode benchmark, BenchmarkDecodeInt4MatMulOnMetal
    (tensor/decodebench_darwin_test.go:148-189): Int4MatVec of x[i] = (i%7)*0.25
    against a [2048, 2048] weight w[i] = (i%13)*0.125 - 0.75 packed by
    Int4Quantize, one submission waited for per step, so the host's part is
    in the figure (0.76 ms on an M2, specs/010-kernel-corpus.md:593-602).
    Timed the same way here: one Int4MatVec call and one stream wait per step,
    by the host's clock; the device time of the same calls beside it.  The
    reference's plan binds the weight once (its compile step), as the headline
    does: the weight is prepared once, outside the timed steps, and each step
    is Int4MatVecPrepared; the same steps on the planes as handed over are
    reported beside them."""
    import accel_amd
    from accel_amd import F32
    K = N = 2048
    wv = (np.arange(K * N) % 13).astype(np.float32) * np.float32(0.125) - np.float32(0.75)
    packed, scales, zeros = accel_amd.int4_quantize(wv)
    xs = (np.arange(K) % 7).astype(np.float32) * np.float32(0.25)
    w = dev.upload_int4(packed, scales, zeros, K * N)
    pw = dev.prepare_int4(w, K, N, stream)
    a = dev.upload(xs)
    out = dev.alloc((N,), F32)
    e0, e1 = dev.event(), dev.event()

    def steps_of(call):
        for _ in range(20):
            call()
            dev.sync(stream)
        walls, gpu = [], []
        for _ in range(steps):
            t0 = time.perf_counter()
            dev.record(e0, stream)
            call()
            dev.record(e1, stream)
            dev.sync(stream)
            walls.append(time.perf_counter() - t0)
            gpu.append(dev.elapsed_ms(e0, e1))
        return float(np.median(walls)) * 1e6, float(np.median(gpu)) * 1e3

    us, dev_us = steps_of(lambda: dev.Int4MatVecPrepared(a, pw, out, stream))
    us_planes, dev_us_planes = steps_of(lambda: dev.Int4MatVec(a, w, out, stream))
    dev.destroy_event(e0)
    dev.destroy_event(e1)
    for b in (a, out):
        b.free()
    pw.free()
    w.free()
    nbytes = K * N // 2 + 4 * (K * N // 128) + 4 * K + 4 * N
    return dict(workload="the reference's published decode benchmark: Int4MatVec [2048] x "
                         "[2048,2048], w[i] = (i%13)*0.125-0.75, x[i] = (i%7)*0.25, one "
                         "submission waited for per step (host time included); the weight "
                         "bound once (Int4MatVecPrepared), as the reference's plan binds it",
                us_per_step=round(us, 2), device_us=round(dev_us, 2),
                us_per_step_reference_planes=round(us_planes, 2),
                device_us_reference_planes=round(dev_us_planes, 2),
                gbs_effective=round(nbytes / (us * 1e-6) / 1e9, 2),
                published_us=PUBLISHED_US, published_hw="Apple M2 (Metal backend)",
                published_src=PUBLISHED_SRC, speedup_vs_published=round(PUBLISHED_US / us, 1))


def bench_matvec_f16(dev, stream, K=4096, N=4096, steps=200):
    """MatVecF32F16 (f32 x [K], f16 w [K,N]) over f16 weight copies totalling
    more than 512 MB, so every call reads HBM."""
    from accel_amd import F16, F32
    rng = np.random.Generator(np.random.PCG64(5))
    wbits = (rng.standard_normal(K * N, dtype=np.float32) * 0.02).astype(np.float16)
    wbits = wbits.view(np.uint16).reshape(K, N)
    copies = max(1, -(-ROTATE_BYTES // wbits.nbytes))
    ws = [dev.upload(wbits, F16) for _ in range(copies)]
    a = dev.upload(rng.standard_normal(K).astype(np.float32))
    out = dev.alloc((N,), F32)
    for w in ws:
        dev.MatVecF32F16(a, w, out, stream)
    dev.sync(stream)
    t = Timed(dev, stream, lambda i: dev.MatVecF32F16(a, ws[i % copies], out, stream), steps)
    ms = median_replay(t) / steps
    t.close()
    for b in ws + [a, out]:
        b.free()
    nbytes = K * N * 2 + 4 * K + 4 * N
    return dict(us=round(ms * 1e3, 3), gbs=round(nbytes / (ms * 1e-3) / 1e9, 1),
                frac_of_hbm=round(nbytes / (ms * 1e-3) / 8e12, 4), K=K, N=N, copies=copies)


def bench_int8(dev, stream, M=1, K=4096, N=4096, steps=200):
    """QuantMatMul on int8 weights (f32 x [M,K], i8 [K,N] with one f16 scale
    per 32 weights) over weight copies totalling more than 512 MB, so every
    call reads HBM.  Algorithmic bytes: K N (quants) + K N / 16 (scales) +
    4 M K + 4 M N."""
    from accel_amd import F32
    rng = np.random.Generator(np.random.PCG64(6))
    q = rng.integers(-127, 128, K * N, dtype=np.int8).reshape(K, N)
    s = np.full((K * N) // 32, 0x1c00, np.uint16)   # f16 2^-8
    per = q.nbytes + s.nbytes
    copies = max(1, -(-ROTATE_BYTES // per))
    ws = [(dev.upload(q), dev.upload(s)) for _ in range(copies)]
    a = dev.upload(rng.standard_normal((M, K)).astype(np.float32))
    out = dev.alloc((M, N), F32)
    for qb, sb in ws:
        dev.QuantMatMul(a, qb, sb, out, stream)
    dev.sync(stream)
    t = Timed(dev, stream, lambda i: dev.QuantMatMul(a, *ws[i % copies], out, stream), steps)
    ms = median_replay(t) / steps
    t.close()
    for qb, sb in ws:
        qb.free()
        sb.free()
    a.free()
    out.free()
    nbytes = per + 4 * M * K + 4 * M * N
    return dict(us=round(ms * 1e3, 3), gbs=round(nbytes / (ms * 1e-3) / 1e9, 1),
                frac_of_hbm=round(nbytes / (ms * 1e-3) / 8e12, 4), M=M, K=K, N=N,
                copies=copies)


def bench_linear(dev, stream, name, out_bf16, steps=200):
    """The fused int4 Linear on a config's shape (an f32 [N] bias added in the
    product's epilogue; f32 or bf16 result) over rotated weights, beside the
    plain product timed the same way on the same inputs."""
    from accel_amd import BF16, F32, workloads
    L = workloads.linear(**workloads.CONFIGS[name])
    ws = rotated_weights(dev, stream, L)
    rng = np.random.Generator(np.random.PCG64(9))
    bias = dev.upload(rng.standard_normal(L.N).astype(np.float32))
    shape = (L.M, L.N) if L.M > 1 else (L.N,)
    if L.bf16:
        a = dev.upload(workloads.bf16_bits(L.x), BF16)
    else:
        a = dev.upload(L.x if L.M > 1 else L.x[0])
    out = dev.alloc(shape, BF16 if (out_bf16 or L.bf16) else F32)
    plain = dev.alloc(shape, BF16 if L.bf16 else F32)

    def prod(w, o):
        if L.M == 1:
            dev.Int4MatVec(a, w, o, stream)
        else:
            dev.Int4MatMul(a, w, o, stream)

    for w in ws:
        dev.Int4Linear(a, w, bias, out, stream)
        prod(w, plain)
    dev.sync(stream)
    res = {}
    # each timed twice, alternating, the second kept: the first graphs of a
    # run also pay the clock ramp
    for _ in range(2):
        for key, fn in (("product_us", lambda i: prod(ws[i % len(ws)], plain)),
                        ("fused_us",
                         lambda i: dev.Int4Linear(a, ws[i % len(ws)], bias, out, stream))):
            t = Timed(dev, stream, fn, steps)
            res[key] = round(median_replay(t) / steps * 1e3, 3)
            t.close()
    for b in (bias, a, out, plain):
        b.free()
    for w in ws:
        w.free()
    res.update(M=L.M, K=L.K, N=L.N, x="bf16" if L.bf16 else "f32",
               out="bf16" if (out_bf16 or L.bf16) else "f32")
    return res


def bench_repack(dev, stream, fmt=1, K=4096, N=14336, G=128, calls=20):
    """Repacking one published 4-bit layer (AWQ by default) into the reference
    int4 format on the device, planes already resident: per call, the HIP-event
    time of the whole call on its stream (flag clear, repack kernel, flag
    read-back) and the wall time including the call's own synchronization;
    the host repack of the same layer beside it."""
    import ctypes
    import time
    import accel_amd
    from accel_amd import F16, U32
    rng = np.random.Generator(np.random.PCG64(12))
    groups = K // G
    qweight = rng.integers(0, 2**32, (K, N // 8) if fmt == 1 else (K // 8, N), dtype=np.uint32)
    qzeros = rng.integers(0, 2**32, (groups, N // 8), dtype=np.uint32)
    scales = (rng.random((groups, N), dtype=np.float32) * 0.02 + 1e-3).astype(np.float16)
    lay = accel_amd.ForeignInt4(fmt, G, K, N, qweight, qzeros, scales.view(np.uint16))
    up = [dev.upload(lay.qweight, U32), dev.upload(lay.qzeros, U32), dev.upload(lay.scales, F16)]
    n = K * N
    w = accel_amd.Int4Weights(dev.alloc(((n + 7) // 8,), U32), dev.alloc(((n + 127) // 128,), F16),
                              dev.alloc(((n + 127) // 128,), F16), n)
    d = lay.desc(up[0].ptr, up[1].ptr, up[2].ptr)
    tw = w.desc()
    lib = accel_amd.lib()

    def call():
        accel_amd._check(lib.accel_int4_repack(dev.index, stream, ctypes.byref(d),
                                               ctypes.byref(tw)))

    for _ in range(3):
        call()
    e0, e1 = dev.event(), dev.event()
    gpu_ms = []
    t0 = time.perf_counter()
    for _ in range(calls):
        dev.record(e0, stream)
        call()
        dev.record(e1, stream)
        dev.wait(e1)
        gpu_ms.append(dev.elapsed_ms(e0, e1))
    wall_us = (time.perf_counter() - t0) / calls * 1e6
    dev.destroy_event(e0)
    dev.destroy_event(e1)
    t0 = time.perf_counter()
    accel_amd.int4_repack_host(lay)
    host_ms = (time.perf_counter() - t0) * 1e3
    for b in up:
        b.free()
    w.free()
    read = qweight.nbytes + qzeros.nbytes + scales.nbytes
    written = n // 2 + (n // 128) * 4
    us = float(np.median(gpu_ms)) * 1e3
    return dict(format={1: "awq", 2: "gptq", 3: "gptq_v2"}[fmt], K=K, N=N, group=G,
                us=round(us, 2), wall_us=round(wall_us, 2),
                gbs=round((read + written) / (us * 1e-6) / 1e9, 1), host_ms=round(host_ms, 1),
                bytes=read + written)


def bench_decode_step(dev, stream, batch, steps=100, merged=True):
    """Config 5's layer as a whole decode step with its on-device neighbours:
    h = RMSNorm(x); q,k,v <- h; o <- q; h2 = RMSNorm(o); gate,up <- h2;
    a = SwiGLU(gate, up); down <- a.  Seven launches a step (q, k, v and
    gate, up each run as one set; ten with merged=False), captured in one
    HIP graph and replayed (attention itself is outside the int4 path)."""
    from accel_amd import F32, workloads
    shapes = workloads.LAYER_SHAPES
    rng = np.random.Generator(np.random.PCG64(4))
    x = rng.standard_normal((batch, 4096)).astype(np.float32)
    g1 = (rng.standard_normal(4096) * 0.1 + 1).astype(np.float32)
    g2 = (rng.standard_normal(4096) * 0.1 + 1).astype(np.float32)
    layer_planes(rng)
    ws, bufs = {}, {}
    total_bytes = 0
    shape = (lambda n: (batch, n)) if batch > 1 else (lambda n: (n,))
    for name, (K, N) in shapes.items():
        packed, scales, zeros = _LAYER_PLANES[name]
        ws[name] = dev.upload_int4(packed, scales, zeros, K * N)
        total_bytes += packed.nbytes + scales.nbytes + zeros.nbytes
        bufs[name] = dev.alloc(shape(N), F32)
    xin = dev.upload(x if batch > 1 else x[0])
    gb1, gb2 = dev.upload(g1), dev.upload(g2)
    h1, h2 = dev.alloc(shape(4096), F32), dev.alloc(shape(4096), F32)
    act = dev.alloc(shape(14336), F32)

    def op(a, w, o):
        if batch > 1:
            dev.Int4MatMul(a, w, o, stream)
        else:
            dev.Int4MatVec(a, w, o, stream)

    def ops(a, names):
        # products that share an input run as one launch per tile width
        if merged and batch == 1:
            dev.Int4MatVecSet(a, [ws[n] for n in names], [bufs[n] for n in names], stream)
        elif merged:
            dev.Int4MatMulSet(a, [ws[n] for n in names], [bufs[n] for n in names], stream)
        else:
            for n in names:
                op(a, ws[n], bufs[n])

    def step(i):
        dev.RMSNorm(xin, gb1, 1e-5, h1, stream)
        ops(h1, ("q", "k", "v"))
        op(bufs["q"], ws["o"], bufs["o"])
        dev.RMSNorm(bufs["o"], gb2, 1e-5, h2, stream)
        ops(h2, ("gate", "up"))
        dev.SwiGLU(bufs["gate"], bufs["up"], act, stream)
        op(act, ws["down"], bufs["down"])

    step(0)
    dev.sync(stream)
    t = Timed(dev, stream, step, steps)
    ms = median_replay(t) / steps
    t.close()
    for w in ws.values():
        w.free()
    for b in list(bufs.values()) + [xin, gb1, gb2, h1, h2, act]:
        b.free()
    return dict(us_per_step=round(ms * 1e3, 2),
                gbs=round(total_bytes / (ms * 1e-3) / 1e9, 1),
                weight_bytes=total_bytes, batch=batch,
                launches=7 if merged else 10)


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
                       f"(oracle/oracle.c: the reference CPU algorithm restated in C, "
                       f"reference evaluation order, {threads} threads)")


def _timed_once(fn, min_seconds):
    """Seconds per call of fn, repeated until min_seconds have passed (at least once)."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= min_seconds:
            return el / n, n


def cpu_baselines_configs(min_seconds=0.3):
    """The reference CPU algorithm restated in C (oracle/oracle.c, reference
    evaluation order: QuantMatVecInt4's 32 x 16 workgroups, QuantMatMulInt4's
    16 x 8 tiles, the grouped tiles) on bounded samples of configs 2-5, at the
    host's thread count and at one thread, reported in each config's unit."""
    import oracle
    from accel_amd import workloads
    out = {}
    hi = cpu_threads()
    rng = np.random.Generator(np.random.PCG64(21))
    K, N = 4096, 14336
    p2, s2, z2 = workloads.fast_int4(K, N, rng)
    x16 = rng.standard_normal((16, K)).astype(np.float32)
    rows = []
    for th, M in ((hi, 16), (1, 8)):
        per, n = _timed_once(lambda: oracle.quant_matmul_int4(x16[:M], p2, s2, z2, M, K, N,
                                                              threads=th), min_seconds)
        nbytes = workloads.algorithmic_bytes(M, K, N)
        rows.append(dict(cores=th, value=round(nbytes / per / 1e9, 3), unit="GB/s",
                         us_per_call=round(per * 1e6, 1),
                         sample=f"{n} calls of QuantMatMulInt4 on {M} of config 2's 16 rows"))
    out["decode_m16_f32"] = rows
    # config 3: bf16-rounded rows through the f32 oracle, a row sample
    K3 = N3 = 4096
    p3, s3, z3 = workloads.fast_int4(K3, N3, rng)
    x3 = workloads.bf16_to_f32(workloads.bf16_bits(
        rng.standard_normal((256, K3)).astype(np.float32)))
    rows = []
    for th, M in ((hi, 256), (1, 32)):
        per, n = _timed_once(lambda: oracle.quant_matmul_int4(x3[:M], p3, s3, z3, M, K3, N3,
                                                              threads=th), min_seconds)
        rows.append(dict(cores=th, value=round(2.0 * M * K3 * N3 / per / 1e12, 5),
                         unit="TFLOP/s", sample=f"{n} calls of QuantMatMulInt4 on {M} of "
                                                f"config 3's 2048 rows"))
    out["prefill_m2048_bf16"] = rows
    # config 4: one expert's segment through the grouped oracle
    E = 2
    pe = np.concatenate([p2, p2])
    se = np.concatenate([s2, s2])
    ze = np.concatenate([z2, z2])
    rows = []
    for th, R in ((hi, 128), (1, 16)):
        xr = workloads.bf16_to_f32(workloads.bf16_bits(
            rng.standard_normal((R, K)).astype(np.float32)))
        off = np.array([0, R, R], np.uint32)
        per, n = _timed_once(lambda: oracle.int4_grouped_matmul(xr, pe, se, ze, off, E, R, K, N,
                                                                threads=th), min_seconds)
        rows.append(dict(cores=th, value=round(2.0 * R * K * N / per / 1e12, 5),
                         unit="TFLOP/s", sample=f"{n} calls of GroupedMatMul (int4) over one "
                                                f"expert's {R} routed rows"))
    out["moe_grouped_bf16"] = rows
    # config 5: the seven products of a step in the oracle
    planes = layer_planes(np.random.Generator(np.random.PCG64(4)))
    wbytes = sum(p.nbytes + s.nbytes + z.nbytes for p, s, z in planes.values())
    for batch in (1, 8):
        xs = rng.standard_normal((batch, 14336)).astype(np.float32)
        rows = []
        for th in (hi, 1):
            def step():
                for name, (Kc, Nc) in workloads.LAYER_SHAPES.items():
                    p, s, z = planes[name]
                    if batch == 1:
                        oracle.quant_matvec_int4(xs[0, :Kc], p, s, z, Kc, Nc, threads=th)
                    else:
                        oracle.quant_matmul_int4(np.ascontiguousarray(xs[:, :Kc]), p, s, z,
                                                 batch, Kc, Nc, threads=th)
            per, n = _timed_once(step, min_seconds)
            rows.append(dict(cores=th, us_per_step=round(per * 1e6, 1),
                             value=round(wbytes / per / 1e9, 3), unit="GB/s",
                             sample=f"{n} steps of the seven products at batch {batch}"))
        out[f"layer_chain_b{batch}"] = rows
    return dict(kind="port", what="the reference CPU algorithm restated in C "
                                  "(oracle/oracle.c), not the Go backend (no Go toolchain)",
                rows=out)


def _time_calls(fn, seconds):
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return el / n, n


def cpu_baseline_extras(seconds=1.5):
    """The oracle's single-threaded C ports of the widened rows (the reference
    CPU algorithms in reference order), each timed on a bounded sample on the
    host cores, to sit beside the `extra` GPU figures."""
    import oracle
    rng = np.random.Generator(np.random.PCG64(21))
    K = N = 4096
    out = {}
    x = rng.standard_normal(K).astype(np.float32)
    q = rng.integers(-127, 128, K * N, dtype=np.int8)
    sc = np.full((K * N) // 32, 0x1c00, np.uint16)
    per, n = _time_calls(lambda: oracle.quant_matvec_i8(x, q, sc, K, N), seconds)
    nbytes = K * N + K * N // 16 + 4 * K + 4 * N
    out["int8_gemv_4096"] = dict(us=round(per * 1e6, 1), gbs=round(nbytes / per / 1e9, 3),
                                 calls=n, what="QuantMatVecF32, M=1 K=N=4096")
    wb = (rng.standard_normal(K * N, dtype=np.float32) * 0.02).astype(np.float16).view(np.uint16)
    per, n = _time_calls(lambda: oracle.matvec_f32_f16(x, wb, K, N), seconds)
    nbytes = 2 * K * N + 4 * K + 4 * N
    out["matvec_f32_f16"] = dict(us=round(per * 1e6, 1), gbs=round(nbytes / per / 1e9, 3),
                                 calls=n, what="MatVecF32F16, K=N=4096")
    from accel_amd import workloads
    L = workloads.linear(**workloads.CONFIGS["gemv_m1"])
    bias = rng.standard_normal(N).astype(np.float32)
    per, n = _time_calls(lambda: oracle.int4_linear(L.x[0], L.packed, L.scales, L.zeros, bias,
                                                    1, K, N), seconds)
    out["linear_gemv_f32"] = dict(us=round(per * 1e6, 1), calls=n,
                                  what="composed int4 Linear (QuantMatVecInt4 + ElemAdd), M=1 "
                                       "K=N=4096")
    a = rng.standard_normal(14336).astype(np.float32)
    b = rng.standard_normal(14336).astype(np.float32)
    per, n = _time_calls(lambda: oracle.swiglu(a, b), seconds / 3)
    out["swiglu_14336"] = dict(us=round(per * 1e6, 1), calls=n, what="SwiGLU over 14336")
    xr = rng.standard_normal((1, 4096)).astype(np.float32)
    g = rng.standard_normal(4096).astype(np.float32)
    per, n = _time_calls(lambda: oracle.rmsnorm(xr, g, 1e-5), seconds / 3)
    out["rmsnorm_4096"] = dict(us=round(per * 1e6, 1), calls=n, what="RMSNorm, one 4096 row")
    Kr, Nr, G = 4096, 14336, 128
    qw = rng.integers(0, 2**32, (Kr, Nr // 8), dtype=np.uint32)
    qz = rng.integers(0, 2**32, (Kr // G, Nr // 8), dtype=np.uint32)
    ss = (rng.random((Kr // G, Nr), dtype=np.float32) * 0.02 + 1e-3).astype(np.float16)
    per, n = _time_calls(lambda: oracle.int4_repack(1, Kr, Nr, G, qw, qz, ss.view(np.uint16)),
                         seconds)
    out["repack_awq_4096x14336"] = dict(ms=round(per * 1e3, 1), calls=n,
                                        what="AWQ unpack + Int4Quantize, one 4096x14336 layer")
    return dict(kind="port", cores=1, rows=out)


def bench_floors(dev, stream, steps=640):
    """What a decode product's launch shape costs before its arithmetic: an
    empty kernel of 256 x 512 lanes, and a pure read of config 1's 8 945 664
    algorithmic bytes with that shape (16-byte loads, all issued before any is
    used), over 64 device copies with the cache flushed, timed like the
    headline (graph replay, HIP events)."""
    from accel_amd import U32
    nbytes = 8945664
    copies = max(1, -(-ROTATE_BYTES // nbytes))
    bufs = [dev.alloc((nbytes // 4,), U32) for _ in range(copies)]
    sink = dev.alloc((256,), U32)
    res = {}
    for kind, key in ((0, "empty_kernel"), (1, "read_8945664_bytes")):
        t = Timed(dev, stream,
                  lambda i: dev.floor(kind, bufs[i % copies], nbytes, sink, stream), steps)
        t.run()
        ms = median_replay(t) / steps
        t.close()
        res[key] = {"us_per_launch": round(ms * 1e3, 3)}
        if kind == 1:
            res[key]["gbs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
            res[key]["frac_of_hbm_peak"] = round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
    for b in bufs + [sink]:
        b.free()
    res["what"] = ("launch floors of the M=1 decode kernel's shape (256 workgroups of 512 "
                   "lanes): an empty kernel, and a pure read of config 1's algorithmic bytes "
                   "over rotated copies with the cache flushed; graph replay, HIP events")
    return res


def gemm_line(p, workload, kernel, bound, flops, bytes_per, launches=None):
    """A product's bench line; `launches` names its launches in the PMC
    summary when it is more than the one kernel."""
    traffic = traffic_sum(launches or (kernel,))
    if bound == "mfma":
        rl = {"bound": "mfma", "achieved": round(p["tflops"], 1), "peak": BF16_PEAK_TFLOPS,
              "unit": "TFLOP/s", "frac": round(p["tflops"] / BF16_PEAK_TFLOPS, 4),
              "traffic": traffic, "kernel": kernel, "flops_per_launch": int(flops)}
    else:
        rl = {"bound": "hbm", "achieved": round(p["gbs"], 1), "peak": HBM_PEAK_GBS,
              "unit": "GB/s", "frac": round(p["gbs"] / HBM_PEAK_GBS, 4),
              "traffic": traffic, "kernel": kernel, "bytes_per_launch": int(bytes_per)}
    return {"workload": workload, "us": round(p["us"], 2), "roofline": rl}


def main():
    global EAGER
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this build "
              "runs on a single MI355X)",
              file=sys.stderr)
        sys.exit(2)
    EAGER = args.eager
    import accel_amd
    if accel_amd.device_count() < 1:
        print("no HIP device", file=sys.stderr)
        sys.exit(1)
    dev = accel_amd.Device(0)
    stream = dev.stream()
    steps = max(1, args.steps)
    progress("config 1 (headline): Int4MatVec M=1 K=N=4096")
    r = bench_gemv(dev, stream, steps, args.warmup)
    L = r["L"]
    pub = None
    line = {
        "metric": METRIC,
        "value": round(r["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "Int4MatVec M=1 K=4096 N=4096 (BASELINE config 1's shape and the "
                        "metric's M=1 leg) in the reference int4 format (128-weight groups, "
                        "f16 scale+zero), the weight bound once into the backend's K-major "
                        "panel layout (accel_int4_prepare, outside the timed region; "
                        f"{r['bind_ms']:.2f} ms a matrix), then Int4MatVecPrepared; f32 "
                        "activations and output; weights rotated over "
                        f"{r['copies']} device copies and the Infinity Cache flushed before "
                        "the timed replay, so every step reads HBM",
            "seed": 0,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(r["gbs"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(r["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": traffic_of(GEMV_KERNEL),
            "kernel": GEMV_KERNEL,
            "bytes_per_launch": r["bytes"],
            "us_per_launch": round(r["ms"] * 1e3, 4),
        },
    }
    only = {k for k in args.only.split(",") if k}

    def want(*keys):
        return not only or any(k in only for k in keys)

    if not args.no_extra:
        extra = {}
        gref = r["gbs_ref"]
        extra["gemv_m1_reference_planes"] = {
            "workload": "config 1 on the reference planes as given (accel_int4_matvec: the "
                        "decode kernel, K split across workgroups and a split-K hand-off), "
                        "the same inputs, rotation and protocol as the headline",
            "us": round(r["ms_ref"] * 1e3, 3),
            "roofline": {"bound": "hbm", "achieved": round(gref, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gref / HBM_PEAK_GBS, 4),
                         "traffic": traffic_of(GEMV_REF_KERNEL), "kernel": GEMV_REF_KERNEL,
                         "bytes_per_launch": r["bytes"]}}
        extra["gemv_m1_bind_ms"] = round(r["bind_ms"], 3)
        if want("gemv_m1_g32_literal"):
            progress("config 1 in BASELINE's literal format (G=32 along K, f32 scale)")
            extra["gemv_m1_g32_literal"] = bench_gemv_g32(dev, stream)
        if want("prefill_m2048_bf16"):
            progress("config 3: prefill M=2048 bf16")
            p = bench_gemm(dev, stream, "prefill_m2048")
            extra["prefill_m2048_bf16"] = gemm_line(
                p, "Int4MatMul M=2048 K=4096 N=4096, bf16 x/out, fp32 accumulate (BASELINE "
                   "config 3, the metric's M=2048 leg)", GEMM_KERNEL, "mfma",
                2 * 2048 * 4096 * 4096, p["bytes"])
    if not args.no_extra and want("prefill_m2048_f32"):
        progress("config 3 in f32: prefill M=2048 in the reference API's dtype")
        pf = bench_gemm(dev, stream, "prefill_m2048_f32", steps=20, warmup=2)
        lf = gemm_line(
            pf, "Int4MatMul M=2048 K=4096 N=4096, f32 x/out: config 3's shape in the reference "
                "API's own dtype (tensor/int4.go:176-179), on the bf16 matrix cores to f32 "
                "accuracy (x*512s in three bf16 terms against the exact codes)",
            GEMM_F32_KERNEL, "mfma", 2 * 2048 * 4096 * 4096, pf["bytes"])
        lf["roofline"]["mfma_issued_flops_per_launch"] = 3 * 2 * 2048 * 4096 * 4096
        lf["roofline"]["note"] = ("achieved counts the product's own flops; the three-term "
                                  "split issues three times as many on the matrix cores")
        extra["prefill_m2048_f32"] = lf
    if not args.no_extra:
        for key, name, launches in (("prefill_m64_bf16", "prefill_m64", SPLITK_BF16_LAUNCHES),
                                    ("prefill_m64_f32", "prefill_m64_f32", SPLITK_F32_LAUNCHES)):
            if not want(key):
                continue
            progress(f"short prefill: {key} (split K)")
            q = bench_gemm(dev, stream, name, steps=100, warmup=10)
            dt = "bf16" if name == "prefill_m64" else "f32"
            extra[key] = gemm_line(
                q, f"Int4MatMul M=64 K=4096 N=4096, {dt} x/out: a short prefill, whose 32 "
                   "tiles split K across the CUs (f32 sums per slice, one reduction pass)",
                " + ".join(launches), "hbm", 2 * 64 * 4096 * 4096, q["bytes"], launches)
            extra[key]["tflops"] = round(q["tflops"], 1)
        if want("decode_m16_f32"):
            progress("config 2: decode M=16 K=4096 N=14336")
            d = bench_gemm(dev, stream, "decode_m16", steps=200, warmup=10, tiles=True)
            extra["decode_m16_f32"] = gemm_line(
                d, "Int4MatMul M=16 K=4096 N=14336, f32 x/out (BASELINE config 2, Llama-3-8B "
                   "MLP up-projection at decode batch 16), the weight bound once for the "
                   "matrix-core decode (accel_int4_prepare_tiles: the codes as they are and a "
                   "side copy of the scales and zeros, outside the timed region), then "
                   "Int4MatMulPrepared", DECODE_SIDE_KERNEL, "hbm",
                2 * 16 * 4096 * 14336, d["bytes"])
            extra["decode_m16_f32"]["bind_ms"] = round(d["bind_ms"], 3)
        if want("decode_m16_f32_reference_planes"):
            d = bench_gemm(dev, stream, "decode_m16", steps=200, warmup=10)
            extra["decode_m16_f32_reference_planes"] = gemm_line(
                d, "config 2 on the reference planes as handed over (Int4MatMul, no bind "
                   "step)", DECODE_MFMA_KERNEL, "hbm", 2 * 16 * 4096 * 14336, d["bytes"])
        if want("moe_grouped_bf16"):
            progress("config 4: MoE grouped product")
            extra["moe_grouped_bf16"] = bench_moe(dev, stream)
        if want("moe_grouped_f32"):
            progress("config 4's shape in f32 rows (the reference API's grouped dtype)")
            extra["moe_grouped_f32"] = bench_moe(dev, stream, steps=10, bf16=False)
        if want("moe_decode_f32"):
            extra["moe_decode_f32"] = bench_moe_decode(dev, stream)
        if want("moe_decode_f32_4tok"):
            extra["moe_decode_f32_4tok"] = bench_moe_decode(dev, stream, tokens=4,
                                                            form="panels")
        for b in (1, 8):
            if want(f"layer_chain_b{b}"):
                progress(f"config 5: layer chain at batch {b}")
                extra[f"layer_chain_b{b}"] = bench_layer_chain(dev, stream, b)
        for b in (1, 8):
            if want(f"layer_chain_b{b}_reference_planes"):
                progress(f"config 5 at batch {b} on the reference planes")
                extra[f"layer_chain_b{b}_reference_planes"] = bench_layer_chain(
                    dev, stream, b, prepared=False)
        if want("floors"):
            progress("launch floors of the decode shape")
            extra["floors"] = bench_floors(dev, stream)
    if not args.no_extra and want("published_decode_2048"):
        progress("the reference's published workload (2048 x 2048, one wait a step)")
        pub = bench_published(dev, stream)
        extra["published_decode_2048"] = pub
        line["vs_baseline"] = pub["speedup_vs_published"]
        extra["vs_baseline_basis"] = (
            "vs_baseline is the reference's published figure for its own decode benchmark "
            f"({PUBLISHED_US:.0f} us a step, {PUBLISHED_SRC}) over this build's time for the "
            "same workload and protocol (extra.published_decode_2048); no figure is published "
            "for config 1 itself")
    if not args.no_extra:
        if args.configs:
            progress("--configs: widened rows")
            extra["layer_chain_b1_unmerged"] = bench_layer_chain(dev, stream, 1, merged=False)
            extra["layer_chain_b8_unmerged"] = bench_layer_chain(dev, stream, 8, merged=False)
            extra["matvec_f32_f16"] = bench_matvec_f16(dev, stream)
            extra["int8_gemv_4096"] = bench_int8(dev, stream, 1)
            extra["int8_m8_4096"] = bench_int8(dev, stream, 8)
            extra["int8_m1_4096x14336"] = bench_int8(dev, stream, 1, 4096, 14336)
            extra["linear_gemv_f32"] = bench_linear(dev, stream, "gemv_m1", False)
            extra["linear_gemv_bf16out"] = bench_linear(dev, stream, "gemv_m1", True)
            extra["linear_m16_f32"] = bench_linear(dev, stream, "decode_m16", False)
            extra["linear_prefill_bf16"] = bench_linear(dev, stream, "prefill_m2048", True,
                                                        steps=40)
            extra["repack_awq_4096x14336"] = bench_repack(dev, stream, 1)
            extra["repack_gptq_4096x14336"] = bench_repack(dev, stream, 2)
            extra["decode_step_b1"] = bench_decode_step(dev, stream, 1)
            extra["decode_step_b1_unmerged"] = bench_decode_step(dev, stream, 1, merged=False)
            extra["decode_step_b8"] = bench_decode_step(dev, stream, 8)
            extra["decode_step_b8_unmerged"] = bench_decode_step(dev, stream, 8, merged=False)
        line["extra"] = extra
    if not args.no_cpu:
        progress("CPU baseline: config 1")
        line["cpu_baseline"] = cpu_baseline(L, args.cpu_seconds)
        if not args.no_extra:
            progress("CPU baselines: configs 2-5")
            line["extra"]["cpu_baselines"] = cpu_baselines_configs()
            if args.configs:
                line["extra"]["cpu_baselines_widened"] = cpu_baseline_extras()
    dev.destroy_stream(stream)
    print(json.dumps(line), flush=True)
    progress("done")


if __name__ == "__main__":
    main()
