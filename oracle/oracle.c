/*
 * oracle.c -- CPU restatement of golang-design/accel's int4 weight-only
 * linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py load it to
 * compute expected values and to time the reference algorithm on host cores.
 * Nothing under accel_amd/ links, loads or calls it, and no product result is
 * ever produced by it.
 *
 * Every floating-point operation follows the reference's evaluation order and
 * is rounded to f32 on its own (the build uses -ffp-contract=off and no
 * fast-math), which is what the reference's generated Go lowering does: it
 * writes float32(...) around every product and every sum
 * (internal/kernels/accel_kernels.go:6769,6787,7021) and its MSL is compiled
 * with fp contract(off) (:6813,7066).  The results are therefore those of the
 * reference CPU backend (accel.OpenCPU), bit for bit, on the same inputs.
 *
 * What pins each function (the checks live in tests/test_oracle_*.py):
 *   orc_to_f16          exhaustive over all 2^32 f32 patterns against the
 *                       host's F16C RNE conversion, except the one documented
 *                       range where the reference flushes to zero; NaN -> 0x7e00
 *   orc_f16_to_f32      exhaustive over all 2^16 patterns against numpy
 *   orc_to_bf16         sampled + all specials against torch's RNE; NaN -> 0x7fc0
 *   orc_int4_quantize   the reference's KATs (quant/int4_test.go) + bit-exact
 *                       agreement with the independent numpy restatement
 *                       (oracle/oracle_np.py) on random and adversarial inputs
 *   orc_int4_error_bound  the reference's bound tests, including the case that
 *                       exceeds range/30 (quant/int4_test.go:102-158)
 *   orc_int8_quantize   the int4-vs-int8 KATs (quant/int4_test.go:166-219)
 *                       and the int8 quantizer's tests (quant/quant_test.go:
 *                       22-240: half-step bound, the clamp, scales that
 *                       underflow f16, the dequantize KAT)
 *   orc_quant_matvec_int4 / _matmul_int4  closed-form differential cases
 *                       (differential_cases_test.go:1347-1425), nibble-order
 *                       KAT (=40, not 4), constant-group KAT, f64 brute force
 *                       within Int4ErrorBound + reduction term, tiled == row
 *   orc_grouped_*       per-expert f64 brute force, empty expert, wrong-expert,
 *                       padding row, clamp (internal/kernels/grouped_test.go)
 *   orc_segment_offsets exclusive prefix sum against numpy.cumsum
 *   orc_swiglu          f64 closed form x*b/(1+e^-x) within one f32 rounding
 *                       chain, exact special values (0, +-inf limits, NaN)
 *   orc_rmsnorm         the reference's tests (norm_test.go:34-191): widths
 *                       1, 63, 128, 129, 500, 1024 against a straight f64
 *                       loop within the reduction budget, a zero row reads 0;
 *                       a row of ones equals w / sqrt(1 + eps) exactly
 *   orc_matvec_f32_f16  f64 brute force within the f32 reduction bound, and
 *                       exact sums where every partial is an exact integer
 *   orc_foreign_dequant round trips with independent numpy restatements of
 *                       the published packers (AutoAWQ's column order, GPTQ's
 *                       row packing and its z - 1 zeros, act-order g_idx);
 *                       the repack it feeds (with orc_int4_quantize) returns
 *                       codes, scales and zeros exactly where a reference
 *                       group shares one published (scale, zero) and spans
 *                       the full code range, a closed form a wrong nibble
 *                       order or column permutation fails
 *   orc_add_rows        IEEE f32 addition against numpy's, signed zeros,
 *                       infinities and NaN; a -0.0 vector returns x bit for
 *                       bit (the int4 Linear's composed form is this after
 *                       the int4 product; its tests check the composition's
 *                       special cases: a -0.0 bias gives the product, zero
 *                       weights give the bias on every row)
 *   orc_quant_matvec_i8 / orc_quant_matmul_i8  the reference's exact-input
 *                       cases (prefill_test.go:934-978, differential_cases_
 *                       test.go:950-1010: a = i%7-3, q = i%201-100, dyadic
 *                       scales) against f64, f64 brute force within the
 *                       reduction bound, independent numpy restatements of
 *                       the phase and sequential orders, bit for bit
 */
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Narrowing and widening: internal/kernel/narrow.go:56-176                  */
/* ------------------------------------------------------------------------ */

static inline uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }
static inline float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }

/* Shift right by n with round-to-nearest-even (narrow.go:162-176). */
static uint32_t rne_shift(uint32_t v, uint32_t n) {
    if (n == 0) return v;
    if (n > 31) return 0;
    uint32_t kept = v >> n;
    uint32_t half = 1u << (n - 1);
    uint32_t dropped = v & ((1u << n) - 1u);
    if (dropped > half || (dropped == half && (kept & 1u))) kept++;
    return kept;
}

/* f32 -> f16 bits, RNE, overflow to signed inf, NaN to 0x7e00
 * (narrow.go:67-106).  Note the reference's bottom case: a magnitude below
 * 2^-24 (unbiased exponent < -24) returns a signed zero, so values in
 * (2^-25, 2^-24) flush to zero where IEEE RNE would give 2^-24. */
uint16_t orc_to_f16(float x) {
    uint32_t b = f32_bits(x);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t e = (int32_t)((b >> 23) & 0xffu) - 127;
    uint32_t m = b & 0x7fffffu;
    if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7e00;          /* NaN */
    if (e == 128) return (uint16_t)(sign | 0x7c00u);              /* inf */
    if (e > 15) return (uint16_t)(sign | 0x7c00u);                /* overflow */
    if (e < -24) return sign;                                     /* to zero */
    if (e < -14) {                                                /* subnormal */
        m |= 0x800000u;
        uint32_t sh = (uint32_t)(-e - 14);
        return (uint16_t)(sign | rne_shift(m, 13u + sh));
    }
    /* added, so a mantissa carry moves into the exponent (and to inf) */
    uint32_t h = ((uint32_t)(e + 15) << 10) + rne_shift(m, 13);
    return (uint16_t)(sign | h);
}

/* f16 bits -> f32, exact (narrow.go:110-139). */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bits_f32(sign);
        uint32_t sh = 0;
        while ((m & 0x400u) == 0) { m <<= 1; sh++; }
        m &= 0x3ffu;
        return bits_f32(sign | ((127u - 15u + 1u - sh) << 23) | (m << 13));
    }
    if (e == 0x1f) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 127u - 15u) << 23) | (m << 13));
}

/* f32 -> bf16 bits, RNE, NaN to 0x7fc0 (narrow.go:147-156). */
uint16_t orc_to_bf16(float x) {
    uint32_t b = f32_bits(x);
    if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    uint32_t r = b + 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(r >> 16);
}

float orc_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* Batch forms, for the exhaustive conversion checks. */
void orc_to_f16_batch(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_to_f16(x[i]);
}
void orc_f16_to_f32_batch(const uint16_t* h, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(h[i]);
}
void orc_to_bf16_batch(const float* x, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_to_bf16(x[i]);
}

/* Exhaustive ToFloat16 check over the f32 patterns [lo, hi) against the
 * host's F16C conversion (vcvtps2ph, RNE).  Returns the number of patterns
 * that disagree outside the documented flush range; *flushed counts the
 * patterns inside it where the reference gives a signed zero and IEEE RNE
 * does not.  The first unexpected mismatch is stored in *first_bad. */
#if defined(__x86_64__)
#include <immintrin.h>
__attribute__((target("f16c")))
static uint16_t hw_f16(float x) {
    return (uint16_t)_cvtss_sh(x, _MM_FROUND_TO_NEAREST_INT);
}
int64_t orc_check_f16_range(uint64_t lo, uint64_t hi, int64_t* flushed,
                            uint64_t* first_bad) {
    int64_t bad = 0, fl = 0;
    for (uint64_t p = lo; p < hi; p++) {
        float x = bits_f32((uint32_t)p);
        uint16_t ref = orc_to_f16(x);
        uint16_t hw = hw_f16(x);
        if ((p & 0x7fffffffu) > 0x7f800000u) hw = 0x7e00;   /* canonical NaN */
        if (ref == hw) continue;
        uint32_t mag = (uint32_t)p & 0x7fffffffu;
        /* (2^-25, 2^-24): the reference's e < -24 branch returns zero */
        if (mag > 0x33000000u && mag < 0x33800000u && (ref & 0x7fffu) == 0 &&
            (hw & 0x7fffu) == 1) { fl++; continue; }
        if (bad == 0 && first_bad) *first_bad = p;
        bad++;
    }
    if (flushed) *flushed = fl;
    return bad;
}
#endif

/* ------------------------------------------------------------------------ */
/* Quantization: quant/int4.go:29-253, quant/quant.go:60-127                 */
/* ------------------------------------------------------------------------ */

#define INT4_GROUP 128
#define INT4_MAX 15

static void put_nibble(uint32_t* packed, int64_t i, uint32_t q) {
    int sh = (int)(4 * (i % 8));
    packed[i / 8] = (packed[i / 8] & ~(0xfu << sh)) | (q << sh);
}

uint32_t orc_int4_nibble(const uint32_t* packed, int64_t i) {
    return (packed[i / 8] >> (4 * (i % 8))) & 0xfu;
}

/* Go's float64 -> uint32 of a NaN is 0 on amd64 and arm64; the reference's
 * clamp lets a NaN through (both comparisons are false), so this is the
 * value its setNibble receives there. */
static uint32_t code_of(double q) {
    if (q != q) return 0;
    return (uint32_t)q;
}

/* quant.Int4Quantize (quant/int4.go:71-138).  packed must hold ceil(n/8)
 * words and is zeroed here; scales and zeros hold ceil(n/128) f16 each. */
void orc_int4_quantize(const float* w, int64_t n, uint32_t* packed,
                       uint16_t* scales, uint16_t* zeros) {
    int64_t groups = (n + INT4_GROUP - 1) / INT4_GROUP;
    memset(packed, 0, sizeof(uint32_t) * (size_t)((n + 7) / 8));
    for (int64_t g = 0; g < groups; g++) {
        int64_t lo = g * INT4_GROUP;
        int64_t hi = lo + INT4_GROUP < n ? lo + INT4_GROUP : n;
        float least = w[lo], most = w[lo];
        for (int64_t i = lo; i < hi; i++) {
            float v = w[i];
            if (v < least) least = v;
            if (v > most) most = v;
        }
        if (most == least) {
            scales[g] = orc_to_f16(0.0f);
            zeros[g] = orc_to_f16(least);
            continue;
        }
        float s = (most - least) / (float)INT4_MAX;
        scales[g] = orc_to_f16(s);
        float s16 = orc_f16_to_f32(scales[g]);
        if (s16 == 0.0f) {
            zeros[g] = orc_to_f16(least);
            continue;
        }
        float z = -least / s16;
        zeros[g] = orc_to_f16(z);
        float z16 = orc_f16_to_f32(zeros[g]);
        for (int64_t i = lo; i < hi; i++) {
            double q = nearbyint((double)w[i] / (double)s16 + (double)z16);
            if (q > INT4_MAX) q = INT4_MAX;
            if (q < 0) q = 0;
            put_nibble(packed, i, code_of(q));
        }
    }
}

/* quant.Int4Dequantize (quant/int4.go:160-175). */
void orc_int4_dequantize(const uint32_t* packed, const uint16_t* scales,
                         const uint16_t* zeros, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) {
        int64_t g = i / INT4_GROUP;
        float s = orc_f16_to_f32(scales[g]);
        float z = orc_f16_to_f32(zeros[g]);
        if (s == 0.0f) { out[i] = z; continue; }
        out[i] = ((float)orc_int4_nibble(packed, i) - z) * s;
    }
}

/* ulp16 (quant/int4.go:244-253). */
double orc_ulp16(uint16_t f) {
    int e = (f >> 10) & 0x1f;
    if (e == 0x1f) return INFINITY;
    if (e == 0) return ldexp(1.0, -24);
    return ldexp(1.0, e - 25);
}

/* quant.Int4ErrorBound (quant/int4.go:213-239).  The reference panics when
 * the term counts differ; this returns -1 instead so the caller can refuse. */
double orc_int4_error_bound(const float* x, int64_t nx, const uint16_t* ts,
                            int64_t ns, const uint16_t* tz, int64_t nz) {
    if (ns != nx || nz != nx) return -1.0;
    const double u = 1.0 / (double)(1 << 24);
    double sum = 0.0;
    for (int64_t i = 0; i < nx; i++) {
        double s = (double)orc_f16_to_f32(ts[i]);
        double z = (double)orc_f16_to_f32(tz[i]);
        double e;
        if (s == 0) {
            e = orc_ulp16(tz[i]) / 2;
        } else {
            double ds = orc_ulp16(ts[i]) / 2 + 2 * u * s;
            double dz = orc_ulp16(tz[i]) / 2 + u * fabs(z);
            e = s / 2 + 15 * ds + dz * s;
        }
        sum += fabs((double)x[i]) * e;
    }
    return sum;
}

/* quant.Int8Quantize / Int8Dequantize (quant/quant.go:60-127), kept for the
 * int4-versus-int8 KATs only. */
void orc_int8_quantize(const float* w, int64_t n, int8_t* quants, uint16_t* scales) {
    const int64_t B = 32;
    int64_t blocks = (n + B - 1) / B;
    memset(quants, 0, (size_t)n);
    for (int64_t b = 0; b < blocks; b++) {
        int64_t lo = b * B, hi = lo + B < n ? lo + B : n;
        float peak = 0.0f;
        for (int64_t i = lo; i < hi; i++) {
            float a = (float)fabs((double)w[i]);
            if (a > peak) peak = a;
        }
        if (peak == 0.0f) { scales[b] = orc_to_f16(0.0f); continue; }
        float s = peak / 127.0f;
        scales[b] = orc_to_f16(s);
        float s16 = orc_f16_to_f32(scales[b]);
        if (s16 == 0.0f) continue;
        for (int64_t i = lo; i < hi; i++) {
            double q = nearbyint((double)w[i] / (double)s16);
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            /* int8(NaN) is implementation-defined in Go; amd64 gives 0 */
            quants[i] = q == q ? (int8_t)q : 0;
        }
    }
}
void orc_int8_dequantize(const int8_t* q, const uint16_t* scales, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) out[i] = (float)q[i] * orc_f16_to_f32(scales[i / 32]);
}

/* ------------------------------------------------------------------------ */
/* Workgroup pool: internal/kernel/parallel.go:53-75,111-214.                */
/* Workgroups are claimed in chunks of max(1, min(64, total/(workers*64))).  */
/* ------------------------------------------------------------------------ */

typedef void (*wg_fn)(void* ctx, int64_t wg, float* scratch);

typedef struct {
    wg_fn fn;
    void* ctx;
    int64_t total;
    int64_t chunk;
    size_t scratch_floats;
    atomic_llong next;
} pool_t;

static void* pool_worker(void* arg) {
    pool_t* p = (pool_t*)arg;
    float* scratch = (float*)malloc(sizeof(float) * (p->scratch_floats + 1));
    for (;;) {
        int64_t start = atomic_fetch_add(&p->next, p->chunk);
        if (start >= p->total) break;
        int64_t end = start + p->chunk < p->total ? start + p->chunk : p->total;
        for (int64_t wg = start; wg < end; wg++) p->fn(p->ctx, wg, scratch);
    }
    free(scratch);
    return NULL;
}

static void run_grid(wg_fn fn, void* ctx, int64_t total, int threads,
                     size_t scratch_floats) {
    if (threads > total) threads = (int)total;
    if (threads < 2) {
        float* scratch = (float*)malloc(sizeof(float) * (scratch_floats + 1));
        for (int64_t wg = 0; wg < total; wg++) fn(ctx, wg, scratch);
        free(scratch);
        return;
    }
    pool_t p;
    p.fn = fn; p.ctx = ctx; p.total = total; p.scratch_floats = scratch_floats;
    int64_t c = total / ((int64_t)threads * 64);
    p.chunk = c < 1 ? 1 : (c > 64 ? 64 : c);
    atomic_init(&p.next, 0);
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    for (int i = 0; i < threads; i++) pthread_create(&th[i], NULL, pool_worker, &p);
    for (int i = 0; i < threads; i++) pthread_join(th[i], NULL);
    free(th);
}

/* ------------------------------------------------------------------------ */
/* Kernels in reference order.                                               */
/* ------------------------------------------------------------------------ */

/* One 4-bit weight as the kernels decode it: internal/kernels/int4.go:74-87
 * and int4tiled.go:93-103.  w is the flat index k*N+n (uint32 in the
 * reference; every size here keeps it below 2^32). */
static inline float decode_weight(const uint32_t* bq, const uint16_t* bs,
                                  const uint16_t* bz, uint32_t w) {
    uint32_t code = (bq[w / 8] >> (4 * (w % 8))) & 0xfu;
    uint32_t g = w / INT4_GROUP;
    float s = orc_f16_to_f32(bs[g]);
    float z = orc_f16_to_f32(bz[g]);
    float wv = ((float)code - z) * s;
    if (s == 0.0f) wv = z;
    return wv;
}

typedef struct {
    uint32_t M, K, N;
    const float* a;
    const uint32_t* bq;
    const uint16_t* bs;
    const uint16_t* bz;
    float* out;
} gemm_ctx;

/* QuantMatVecInt4, one workgroup of 32 columns x 16 phases
 * (internal/kernels/int4.go:59-101; lowering accel_kernels.go:6748-6796).
 * Phase p accumulates k = p, p+16, ... in increasing k; the column sum then
 * adds the 16 phase partials in phase order. */
static void matvec_int4_wg(void* vctx, int64_t gx, float* sh) {
    gemm_ctx* c = (gemm_ctx*)vctx;
    const uint32_t K = c->K, N = c->N;
    for (int i = 0; i < 512; i++) sh[i] = 0.0f;
    for (uint32_t k = 0; k < K; k++) {
        uint32_t ly = k % 16;
        float av = c->a[k];
        for (uint32_t lx = 0; lx < 32; lx++) {
            uint32_t col = (uint32_t)gx * 32 + lx;
            if (col >= N) break;
            float wv = decode_weight(c->bq, c->bs, c->bz, k * N + col);
            float prod = av * wv;
            sh[ly * 32 + lx] = sh[ly * 32 + lx] + prod;
        }
    }
    for (uint32_t lx = 0; lx < 32; lx++) {
        uint32_t col = (uint32_t)gx * 32 + lx;
        if (col >= N) break;
        float sum = 0.0f;
        for (uint32_t p = 0; p < 16; p++) sum = sum + sh[p * 32 + lx];
        c->out[col] = sum;
    }
}

void orc_quant_matvec_int4(uint32_t K, uint32_t N, const float* a, const uint32_t* bq,
                           const uint16_t* bs, const uint16_t* bz, float* out,
                           int threads) {
    gemm_ctx c = {1, K, N, a, bq, bs, bz, out};
    run_grid(matvec_int4_wg, &c, (N + 31) / 32, threads, 512);
}

/* QuantMatMulInt4, one 16(N) x 8(M) workgroup (int4tiled.go:66-137;
 * lowering accel_kernels.go:6949-7049).  Each K tile of 16 is staged with
 * zero pads past the edges, then every output accumulates all 16 products of
 * the tile in k order. */
static void matmul_int4_wg(void* vctx, int64_t wg, float* scratch) {
    gemm_ctx* c = (gemm_ctx*)vctx;
    const uint32_t M = c->M, K = c->K, N = c->N;
    uint32_t gxn = (N + 15) / 16;
    uint32_t gx = (uint32_t)(wg % gxn), gy = (uint32_t)(wg / gxn);
    float* tileA = scratch;        /* [8][16] */
    float* tileB = scratch + 128;  /* [16][16] */
    float* acc = scratch + 384;    /* [8][16] */
    for (int i = 0; i < 128; i++) acc[i] = 0.0f;
    for (uint32_t k0 = 0; k0 < K; k0 += 16) {
        for (uint32_t ly = 0; ly < 8; ly++)
            for (uint32_t lx = 0; lx < 16; lx++) {
                uint32_t row = gy * 8 + ly;
                tileA[ly * 16 + lx] =
                    (row < M && k0 + lx < K) ? c->a[row * K + k0 + lx] : 0.0f;
            }
        for (uint32_t kk = 0; kk < 16; kk++)
            for (uint32_t nn = 0; nn < 16; nn++) {
                uint32_t n = gx * 16 + nn;
                tileB[kk * 16 + nn] = (k0 + kk < K && n < N)
                    ? decode_weight(c->bq, c->bs, c->bz, (k0 + kk) * N + n) : 0.0f;
            }
        for (uint32_t ly = 0; ly < 8; ly++)
            for (uint32_t lx = 0; lx < 16; lx++) {
                float s = acc[ly * 16 + lx];
                for (uint32_t k = 0; k < 16; k++) {
                    float p = tileA[ly * 16 + k] * tileB[k * 16 + lx];
                    s = s + p;
                }
                acc[ly * 16 + lx] = s;
            }
    }
    for (uint32_t ly = 0; ly < 8; ly++)
        for (uint32_t lx = 0; lx < 16; lx++) {
            uint32_t row = gy * 8 + ly, col = gx * 16 + lx;
            if (row < M && col < N) c->out[row * N + col] = acc[ly * 16 + lx];
        }
}

void orc_quant_matmul_int4(uint32_t M, uint32_t K, uint32_t N, const float* a,
                           const uint32_t* bq, const uint16_t* bs, const uint16_t* bz,
                           float* out, int threads) {
    gemm_ctx c = {M, K, N, a, bq, bs, bz, out};
    int64_t total = (int64_t)((N + 15) / 16) * (int64_t)((M + 7) / 8);
    run_grid(matmul_int4_wg, &c, total, threads, 512);
}

/* SegmentOffsets (internal/kernels/segment.go:40-50): exclusive prefix sum,
 * rows+1 entries, the last the total.  u32 arithmetic wraps as in Go. */
void orc_segment_offsets(uint32_t rows, const uint32_t* counts, uint32_t* offsets) {
    uint32_t sum = 0;
    for (uint32_t r = 0; r < rows; r++) { offsets[r] = sum; sum = sum + counts[r]; }
    offsets[rows] = sum;
}

/* Weight source for the grouped kernels: f32 [E,K,N] (the reference's
 * GroupedMatVec/GroupedMatMul) or stacked int4 planes over the flat
 * [E,K,N] index (the int4 composition). */
typedef struct {
    uint32_t E, T, K, N;
    const float* x;
    const float* w;        /* f32 weights, or NULL */
    const uint32_t* bq;    /* int4 planes when w == NULL */
    const uint16_t* bs;
    const uint16_t* bz;
    const uint32_t* off;
    float* out;
} grouped_ctx;

static inline float grouped_weight(const grouped_ctx* c, uint32_t idx) {
    if (c->w) return c->w[idx];
    return decode_weight(c->bq, c->bs, c->bz, idx);
}

/* GroupedMatVec, one workgroup per (token, column) of 128 lanes
 * (internal/kernels/grouped.go:47-97): expert lookup e = #{r: off[r+1] <= tok};
 * past the last expert the output is written 0; lane l sums k = l, l+128, ...;
 * then a tree of strides 64, 32, ..., 1. */
static void grouped_matvec_wg(void* vctx, int64_t wg, float* sh) {
    grouped_ctx* c = (grouped_ctx*)vctx;
    const uint32_t K = c->K, N = c->N;
    uint32_t tok = (uint32_t)(wg / N), col = (uint32_t)(wg % N);
    uint32_t e = 0;
    for (uint32_t r = 0; r < c->E; r++)
        if (c->off[r + 1] <= tok) e = e + 1;
    if (e >= c->E) { c->out[tok * N + col] = 0.0f; return; }
    uint32_t base = e * K * N;
    for (uint32_t lid = 0; lid < 128; lid++) {
        float acc = 0.0f;
        for (uint32_t k = lid; k < K; k += 128) {
            float p = c->x[tok * K + k] * grouped_weight(c, base + k * N + col);
            acc = acc + p;
        }
        sh[lid] = acc;
    }
    for (uint32_t stride = 64; stride > 0; stride /= 2)
        for (uint32_t lid = 0; lid < stride; lid++) sh[lid] = sh[lid] + sh[lid + stride];
    c->out[tok * N + col] = sh[0];
}

static void grouped_matvec_run(grouped_ctx* c, int threads) {
    run_grid(grouped_matvec_wg, c, (int64_t)c->T * c->N, threads, 128);
}

void orc_grouped_matvec(uint32_t E, uint32_t T, uint32_t K, uint32_t N, const float* x,
                        const float* w, const uint32_t* off, float* out, int threads) {
    grouped_ctx c = {E, T, K, N, x, w, NULL, NULL, NULL, off, out};
    grouped_matvec_run(&c, threads);
}

void orc_int4_grouped_matvec(uint32_t E, uint32_t T, uint32_t K, uint32_t N,
                             const float* x, const uint32_t* bq, const uint16_t* bs,
                             const uint16_t* bz, const uint32_t* off, float* out,
                             int threads) {
    grouped_ctx c = {E, T, K, N, x, NULL, bq, bs, bz, off, out};
    grouped_matvec_run(&c, threads);
}

/* GroupedMatMul, one workgroup per (16-column tile, expert)
 * (internal/kernels/groupedtiled.go:77-134): rows [off[e], min(off[e+1], T))
 * in blocks of 8, each block through the K tiles of 16 as the tiled GEMM;
 * rows outside every segment are never written. */
static void grouped_matmul_wg(void* vctx, int64_t wg, float* scratch) {
    grouped_ctx* c = (grouped_ctx*)vctx;
    const uint32_t K = c->K, N = c->N;
    uint32_t gxn = (N + 15) / 16;
    uint32_t gx = (uint32_t)(wg % gxn), e = (uint32_t)(wg / gxn);
    float* tileA = scratch;
    float* tileB = scratch + 128;
    float* acc = scratch + 384;
    uint32_t first = c->off[e], last = c->off[e + 1];
    if (last > c->T) last = c->T;
    uint32_t base = e * K * N;
    for (uint32_t r0 = first; r0 < last; r0 += 8) {
        for (int i = 0; i < 128; i++) acc[i] = 0.0f;
        for (uint32_t k0 = 0; k0 < K; k0 += 16) {
            for (uint32_t ly = 0; ly < 8; ly++)
                for (uint32_t lx = 0; lx < 16; lx++) {
                    uint32_t row = r0 + ly;
                    tileA[ly * 16 + lx] =
                        (row < last && k0 + lx < K) ? c->x[row * K + k0 + lx] : 0.0f;
                }
            for (uint32_t kk = 0; kk < 16; kk++)
                for (uint32_t nn = 0; nn < 16; nn++) {
                    uint32_t n = gx * 16 + nn;
                    tileB[kk * 16 + nn] = (k0 + kk < K && n < N)
                        ? grouped_weight(c, base + (k0 + kk) * N + n) : 0.0f;
                }
            for (uint32_t ly = 0; ly < 8; ly++)
                for (uint32_t lx = 0; lx < 16; lx++) {
                    float s = acc[ly * 16 + lx];
                    for (uint32_t k = 0; k < 16; k++) {
                        float p = tileA[ly * 16 + k] * tileB[k * 16 + lx];
                        s = s + p;
                    }
                    acc[ly * 16 + lx] = s;
                }
        }
        for (uint32_t ly = 0; ly < 8; ly++)
            for (uint32_t lx = 0; lx < 16; lx++) {
                uint32_t row = r0 + ly, col = gx * 16 + lx;
                if (row < last && col < N) c->out[row * N + col] = acc[ly * 16 + lx];
            }
    }
}

static void grouped_matmul_run(grouped_ctx* c, int threads) {
    run_grid(grouped_matmul_wg, c, (int64_t)((c->N + 15) / 16) * c->E, threads, 512);
}

void orc_grouped_matmul(uint32_t E, uint32_t T, uint32_t K, uint32_t N, const float* x,
                        const float* w, const uint32_t* off, float* out, int threads) {
    grouped_ctx c = {E, T, K, N, x, w, NULL, NULL, NULL, off, out};
    grouped_matmul_run(&c, threads);
}

void orc_int4_grouped_matmul(uint32_t E, uint32_t T, uint32_t K, uint32_t N,
                             const float* x, const uint32_t* bq, const uint16_t* bs,
                             const uint16_t* bz, const uint32_t* off, float* out,
                             int threads) {
    grouped_ctx c = {E, T, K, N, x, NULL, bq, bs, bz, off, out};
    grouped_matmul_run(&c, threads);
}

/* ------------------------------------------------------------------------ */
/* Decode-step neighbours of the int4 products.                              */
/* ------------------------------------------------------------------------ */

/* kmath.Exp and kmath.RSqrt (kmath/kmath.go:52,55): the f64 function, rounded
 * once to f32. */
static inline float kmath_exp(float x) { return (float)exp((double)x); }
static inline float kmath_rsqrt(float x) { return (float)(1.0 / sqrt((double)x)); }

/* SwiGLU (internal/kernels/elementwise.go:85-91):
 * out[i] = a[i] / (1 + Exp(-a[i])) * b[i], each operation rounded to f32. */
void orc_swiglu(const float* a, const float* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const float x = a[i];
        const float e = kmath_exp(-x);
        const float d = 1.0f + e;
        const float q = x / d;
        out[i] = q * b[i];
    }
}

/* Published 4-bit layers, dequantized (the unpack side of the published
 * formats; the reference names reading them as unbuilt,
 * specs/048-int4.md:126-131,167).  fmt 1 = AWQ (AutoAWQ 0.2 "gemm"): the
 * unpacker takes nibble i of word (k, j) in packing order, position 8j + i,
 * then reverses the packer's column order {0,2,4,6,1,3,5,7}: column 8j + c is
 * packing position 8j + {0,4,1,5,2,6,3,7}[c]; zeros likewise; g = k / G.
 * fmt 2 = GPTQ (AutoGPTQ 0.7): row 8i + j is nibble j of word (i, n); zero
 * column 8j + c is nibble c of word (g, j), plus one; g = g_idx[k] or k / G.
 * fmt 3 = GPTQ v2: as 2 without the plus one.  w = (q - z) * s in f32, which
 * is exact.  w is [K, N]. */
void orc_foreign_dequant(int32_t fmt, int64_t K, int64_t N, int64_t G, const uint32_t* qweight,
                         const uint32_t* qzeros, const uint16_t* scales, const int32_t* g_idx,
                         float* w) {
    static const int reverse_order[8] = {0, 4, 1, 5, 2, 6, 3, 7};
    const int64_t wpr = N / 8;
    for (int64_t k = 0; k < K; k++) {
        const int64_t g = g_idx ? (int64_t)g_idx[k] : k / G;
        for (int64_t j = 0; j < wpr; j++) {
            uint32_t q[8], z[8];
            if (fmt == 1) {
                uint32_t qp[8], zp[8];   /* packing order */
                for (int i = 0; i < 8; i++) {
                    qp[i] = (qweight[k * wpr + j] >> (4 * i)) & 15u;
                    zp[i] = (qzeros[g * wpr + j] >> (4 * i)) & 15u;
                }
                for (int c = 0; c < 8; c++) {
                    q[c] = qp[reverse_order[c]];
                    z[c] = zp[reverse_order[c]];
                }
            } else {
                for (int c = 0; c < 8; c++) {
                    q[c] = (qweight[(k / 8) * N + 8 * j + c] >> (4 * (k % 8))) & 15u;
                    z[c] = ((qzeros[g * wpr + j] >> (4 * c)) & 15u) + (fmt == 2 ? 1u : 0u);
                }
            }
            for (int c = 0; c < 8; c++) {
                const int64_t n = 8 * j + c;
                const float s = orc_f16_to_f32(scales[g * N + n]);
                w[k * N + n] = (float)((int32_t)q[c] - (int32_t)z[c]) * s;
            }
        }
    }
}

/* ElemAdd (internal/kernels/elementwise.go:19-27) of a [rows, cols] matrix
 * and a [cols] vector under the tensor layer's broadcasting
 * (tensor/elementwise.go:60-90): out[r][c] = x[r][c] + v[c], one f32 add. */
void orc_add_rows(uint32_t rows, uint32_t cols, const float* x, const float* v, float* out) {
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t c = 0; c < cols; c++)
            out[(size_t)r * cols + c] = x[(size_t)r * cols + c] + v[c];
}

/* RMSNorm (internal/kernels/norm.go:47-80), one 128-invocation workgroup a
 * row: invocation l sums x[i]^2 over i = l, l+128, ... in increasing i; the
 * 128 partials are added by the halving tree (stride 64, 32, ..., 1; slot l
 * += slot l+stride); mean = total / width, scale = RSqrt(mean + eps), and
 * out[i] = (x[i] * scale) * w[i]. */
void orc_rmsnorm(uint32_t rows, uint32_t width, float eps, const float* x, const float* w,
                 float* out) {
    for (uint32_t r = 0; r < rows; r++) {
        const float* xr = x + (size_t)r * width;
        float* orow = out + (size_t)r * width;
        float sh[128];
        for (uint32_t l = 0; l < 128; l++) {
            float acc = 0.0f;
            for (uint32_t i = l; i < width; i += 128) {
                const float v = xr[i];
                const float sq = v * v;
                acc = acc + sq;
            }
            sh[l] = acc;
        }
        for (uint32_t stride = 64; stride > 0; stride /= 2)
            for (uint32_t l = 0; l < stride; l++) sh[l] = sh[l] + sh[l + stride];
        const float mean = sh[0] / (float)width;
        const float scale = kmath_rsqrt(mean + eps);
        for (uint32_t i = 0; i < width; i++) {
            const float t = xr[i] * scale;
            orow[i] = t * w[i];
        }
    }
}

/* MatVecF32F16 (internal/kernels/matvec.go:79-105): 32 columns x 16 phases a
 * workgroup; phase p accumulates acc = acc + a[k] * F32(b[k*N+col]) over
 * k = p, p+16, ...; the column is the sum of the 16 partials in phase order. */
void orc_matvec_f32_f16(uint32_t K, uint32_t N, const float* a, const uint16_t* b,
                        float* out) {
    for (uint32_t col = 0; col < N; col++) {
        float ph[16];
        for (uint32_t p = 0; p < 16; p++) {
            float acc = 0.0f;
            for (uint32_t k = p; k < K; k += 16) {
                const float prod = a[k] * orc_f16_to_f32(b[(size_t)k * N + col]);
                acc = acc + prod;
            }
            ph[p] = acc;
        }
        float sum = 0.0f;
        for (uint32_t p = 0; p < 16; p++) sum = sum + ph[p];
        out[col] = sum;
    }
}

/* ------------------------------------------------------------------------ */
/* int8 weights (quant/quant.go; internal/kernels/matvec.go, quant.go).      */
/* ------------------------------------------------------------------------ */

/* One int8 weight as the kernels read it: float32(q) * F32(s), one f16 scale
 * per 32 flat weights (QuantBlock, internal/kernels/quant.go:16). */
static inline float int8_weight(const int8_t* bq, const uint16_t* bs, uint64_t w) {
    const float q = (float)bq[w];
    const float s = orc_f16_to_f32(bs[w / 32]);
    return q * s;
}

/* QuantMatVecF32 / QuantMatVec (internal/kernels/matvec.go:157-235): 32
 * columns x 16 phases; phase p accumulates acc = acc + a[k] * (q * s) over
 * k = p, p+16, ...; the column adds the 16 partials in phase order.  `a` is
 * f32 (the f16 variant's activations are widened exactly by the caller). */
void orc_quant_matvec_i8(uint32_t K, uint32_t N, const float* a, const int8_t* bq,
                         const uint16_t* bs, float* out) {
    for (uint32_t col = 0; col < N; col++) {
        float ph[16];
        for (uint32_t p = 0; p < 16; p++) {
            float acc = 0.0f;
            for (uint32_t k = p; k < K; k += 16) {
                const float wv = int8_weight(bq, bs, (uint64_t)k * N + col);
                const float prod = a[k] * wv;
                acc = acc + prod;
            }
            ph[p] = acc;
        }
        float sum = 0.0f;
        for (uint32_t p = 0; p < 16; p++) sum = sum + ph[p];
        out[col] = sum;
    }
}

/* QuantMatMulTiledF32 / QuantMatMulTiled (internal/kernels/quant.go:126-238),
 * which accumulate exactly as QuantMatMul(F32) (:43-124): per output,
 * acc = acc + a[m,k] * (q * s) in increasing k. */
void orc_quant_matmul_i8(uint32_t M, uint32_t K, uint32_t N, const float* a, const int8_t* bq,
                         const uint16_t* bs, float* out) {
    for (uint32_t m = 0; m < M; m++)
        for (uint32_t col = 0; col < N; col++) {
            float acc = 0.0f;
            for (uint32_t k = 0; k < K; k++) {
                const float wv = int8_weight(bq, bs, (uint64_t)k * N + col);
                const float prod = a[(size_t)m * K + k] * wv;
                acc = acc + prod;
            }
            out[(size_t)m * N + col] = acc;
        }
}
