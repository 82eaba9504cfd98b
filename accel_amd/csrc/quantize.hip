// quant.Int4Quantize on the device (quant/int4.go:71-138), bit-identical to
// the host packer.  One wave per group of 128 weights, two per lane.
//
// Bit-exactness rests on three facts: f32 and f64 division and rint are IEEE
// round-to-nearest-even on gfx950 (the divisions are spelled __fdiv_rn /
// __ddiv_rn to say so); the f16 narrowing and widening are integer code
// (the reference's, including its flush of (2^-25, 2^-24) to zero); and the
// group's minimum and maximum reproduce the reference's sequential scan --
// which starts from the group's first weight, replaces only on a strict
// comparison, so a NaN first weight sticks, any later NaN is skipped, and of
// equal values (+0 and -0 included) the earliest is kept.
#include <hip/hip_runtime.h>

#include "internal.hpp"

namespace accel {
namespace {

typedef uint32_t u32x4_q __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t rne_shift(uint32_t v, uint32_t n) {
    if (n == 0) return v;
    if (n > 31) return 0;
    const uint32_t q = v >> n;
    const uint32_t rem = v & ((1u << n) - 1u);
    const uint32_t half = 1u << (n - 1);
    return q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
}

__device__ uint16_t narrow_f16(float x) {
    const uint32_t b = __float_as_uint(x);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7e00;
    const int e = (int)((b >> 23) & 0xffu) - 127;
    const uint32_t mant = b & 0x7fffffu;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    if (e < -24) return sign;
    if (e < -14) return (uint16_t)(sign | rne_shift(mant | 0x800000u, (uint32_t)(-e - 1)));
    return (uint16_t)(sign | (((uint32_t)(e + 15) << 10) + rne_shift(mant, 13)));
}

__device__ float widen_f16(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return __uint_as_float(sign | 0x7f800000u | (m << 13));
    if (e != 0) return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return __uint_as_float(sign);
    const int shift = __clz(m) - 21;
    m = (m << shift) & 0x3ffu;
    return __uint_as_float(sign | ((uint32_t)(113 - shift) << 23) | (m << 13));
}

// The code of one weight: RoundToEven(f64(v) / f64(s) + f64(z)) clamped to
// [0, 15], a NaN giving 0 (quant/int4.go:121-129).  Most weights are settled
// in f32: e = fma(v, rs, z) with rs = 1/s correctly rounded is within
// 2^-23 (|v/s| + |z|) of the exact sum, and the f64 result within
// 2^-52 (|v/s| + |z|), so when e lies farther than `slack` (a group-wide
// bound 4x that) from every half-integer, both round to the same integer.
// The rest -- near a tie, or with a NaN, an infinity or a slack of 1/2 or
// more, all of which fail the comparison -- take the f64 division.
struct CodeRule {
    float s, z, rs, slack;
};

__device__ __forceinline__ CodeRule code_rule(float s16, float z16, float least, float most) {
    CodeRule r;
    r.s = s16;
    r.z = z16;
    r.rs = __fdiv_rn(1.0f, s16);
    r.slack = fmaf(fmaxf(fabsf(least), fabsf(most)), r.rs, fabsf(z16)) * 0x1p-20f;
    if (least != least || most != most) r.slack = __uint_as_float(0x7fc00000u);
    return r;
}

__device__ __forceinline__ uint32_t code_exact(float v, const CodeRule& r) {
    const double q = rint(__ddiv_rn((double)v, (double)r.s) + (double)r.z);
    if (q != q) return 0u;
    return q > 15.0 ? 15u : (q < 0.0 ? 0u : (uint32_t)q);
}

// Sets bit 0 of *open when the f32 estimate leaves the code to the f64 rule.
__device__ __forceinline__ uint32_t code_estimate(float v, const CodeRule& r, uint32_t* open) {
    const float e = fmaf(v, r.rs, r.z);
    const float m = rintf(e);
    *open = fabsf(e - m) < 0.5f - r.slack ? 0u : 1u;
    return (uint32_t)fminf(fmaxf(m, 0.0f), 15.0f);
}

__device__ __forceinline__ uint32_t code_of_weight(float v, const CodeRule& r) {
    uint32_t open;
    const uint32_t code = code_estimate(v, r, &open);
    return open ? code_exact(v, r) : code;
}

// Eight codes estimated in f32 as one word, nibble c for w[c]; bit 8 jj + c
// of *open set for each code left to the f64 rule.
__device__ __forceinline__ uint32_t code_word_estimate(const float* w, const CodeRule& r,
                                                       uint32_t* open, int jj = 0) {
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        uint32_t o;
        word |= code_estimate(w[c], r, &o) << (4 * c);
        *open |= o << (8 * jj + c);
    }
    return word;
}

// Eight codes as one word, nibble c for w[c]: all estimated in f32, then the
// f64 rule for the open ones behind one branch that waves skip when no lane
// has any.
__device__ __forceinline__ uint32_t code_word(const float* w, const CodeRule& r) {
    uint32_t word = 0, open = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        uint32_t o;
        word |= code_estimate(w[c], r, &o) << (4 * c);
        open |= o << c;
    }
    if (open) {
#pragma unroll
        for (int c = 0; c < 8; c++)
            if ((open >> c) & 1u)
                word = (word & ~(15u << (4 * c))) | (code_exact(w[c], r) << (4 * c));
    }
    return word;
}

// (value, index) candidates; `ok` is false for a NaN that cannot win.
struct Cand {
    float v;
    int i;
    bool ok;
};

// a beats b for the minimum (want_min) or maximum: strictly better value,
// or an equal value at an earlier index.
__device__ __forceinline__ bool beats(const Cand& a, const Cand& b, bool want_min) {
    if (!a.ok) return false;
    if (!b.ok) return true;
    const bool better = want_min ? (a.v < b.v) : (a.v > b.v);
    const bool worse = want_min ? (b.v < a.v) : (b.v > a.v);
    return better || (!worse && a.i < b.i);
}

__device__ Cand wave_pick(Cand c, bool want_min) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        Cand o;
        o.v = __shfl_xor(c.v, d, 64);
        o.i = __shfl_xor(c.i, d, 64);
        o.ok = __shfl_xor((int)c.ok, d, 64) != 0;
        if (beats(o, c, want_min)) c = o;
    }
    return c;
}

// Int4Quantize of group g (flat weights lo = 128 g .. lo + 127 of n) by one
// wave: lane l holds weights lo + l (v0) and lo + 64 + l (v1).
__device__ __forceinline__ void quantize_group(float v0, float v1, int lane, int64_t g,
                                               int64_t n, uint32_t* packed, uint16_t* scales,
                                               uint16_t* zeros) {
    const int64_t lo = g * 128;
    const bool in0 = lo + lane < n, in1 = lo + 64 + lane < n;
    const float first = __shfl(v0, 0, 64);  // the scan's starting value
    float least, most;
    if (first != first) {
        least = most = first;  // a NaN first weight is never replaced
    } else {
        // candidate per lane: its better of two weights
        Cand a0 = {v0, lane, in0 && v0 == v0};
        Cand a1 = {v1, 64 + lane, in1 && v1 == v1};
        Cand mn = beats(a1, a0, true) ? a1 : a0;
        Cand mx = beats(a1, a0, false) ? a1 : a0;
        least = wave_pick(mn, true).v;
        most = wave_pick(mx, false).v;
    }

    uint16_t s_bits, z_bits;
    float s16 = 0.0f, z16 = 0.0f;
    bool coded = false;
    if (most == least) {
        s_bits = narrow_f16(0.0f);
        z_bits = narrow_f16(least);
    } else {
        s_bits = narrow_f16(__fdiv_rn(most - least, 15.0f));
        s16 = widen_f16(s_bits);
        if (s16 == 0.0f) {
            z_bits = narrow_f16(least);
        } else {
            z_bits = narrow_f16(__fdiv_rn(-least, s16));
            z16 = widen_f16(z_bits);
            coded = true;
        }
    }
    const CodeRule rule = code_rule(s16, z16, least, most);
    auto code_of = [&](float v, bool in) -> uint32_t {
        if (!coded || !in) return 0u;
        return code_of_weight(v, rule);
    };
    // Pack: lane's weight lo+lane is nibble lane%8 of word lane/8; OR across
    // each run of eight lanes.
    uint32_t p0 = code_of(v0, in0) << (4 * (lane & 7));
    uint32_t p1 = code_of(v1, in1) << (4 * (lane & 7));
#pragma unroll
    for (int d = 1; d < 8; d <<= 1) {
        p0 |= __shfl_xor(p0, d, 64);
        p1 |= __shfl_xor(p1, d, 64);
    }
    const int64_t words = (n + 7) / 8;
    if ((lane & 7) == 0) {
        const int64_t wi0 = (lo >> 3) + (lane >> 3);
        const int64_t wi1 = wi0 + 8;
        if (wi0 < words) packed[wi0] = p0;
        if (wi1 < words) packed[wi1] = p1;
    }
    if (lane == 0) {
        scales[g] = s_bits;
        zeros[g] = z_bits;
    }
}

__global__ __launch_bounds__(256) void int4_quantize_kernel(const float* __restrict__ w,
                                                            int64_t n, uint32_t* packed,
                                                            uint16_t* scales, uint16_t* zeros,
                                                            int64_t groups) {
    const int lane = threadIdx.x & 63;
    const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (g >= groups) return;
    const int64_t i0 = g * 128 + lane, i1 = i0 + 64;
    const float v0 = i0 < n ? w[i0] : 0.0f;
    const float v1 = i1 < n ? w[i1] : 0.0f;
    quantize_group(v0, v1, lane, g, n, packed, scales, zeros);
}

// ---- repacking a published AWQ / GPTQ layer --------------------------------
//
// One wave per reference group of 128 flat weights: each lane dequantizes its
// two weights from the published planes, w = (q - z) * s exactly in f32, and
// the group is quantized as above.  The packings are the published ones (AWQ:
// column 8j + c of a word in nibble {0,4,1,5,2,6,3,7}[c]; GPTQ: eight input
// rows a word, zeros stored z - 1 in its first checkpoint format).  A g_idx
// entry outside the layer's groups is read as group 0 and reported in *bad.

// The published group of input row k (k < 2^31: 32-bit arithmetic).
__device__ __forceinline__ int64_t foreign_group(const accel_foreign_int4_t& f, int64_t k,
                                                 uint32_t* bad) {
    if (f.g_idx) {
        const int64_t g = f.g_idx[k];
        if (g < 0 || g >= f.groups) {
            *bad = 1u;
            return 0;
        }
        return g;
    }
    return (int64_t)((uint32_t)k / (uint32_t)f.group_size);
}

// w(k, n) of the published layer, dequantized exactly; g is row k's group.
__device__ __forceinline__ float foreign_weight(const accel_foreign_int4_t& f, int64_t k,
                                                int64_t n, int64_t g) {
    const int64_t wpr = f.N >> 3;
    uint32_t q, z;
    if (f.format == ACCEL_QFMT_AWQ) {
        // column c of a word sits in nibble c / 2 (c even) or 4 + c / 2 (c odd)
        const int c = (int)(n & 7);
        const int sh = 4 * ((c >> 1) + ((c & 1) << 2));
        q = (f.qweight[k * wpr + (n >> 3)] >> sh) & 15u;
        z = (f.qzeros[g * wpr + (n >> 3)] >> sh) & 15u;
    } else {
        q = (f.qweight[(k >> 3) * f.N + n] >> (4 * (k & 7))) & 15u;
        z = ((f.qzeros[g * wpr + (n >> 3)] >> (4 * (n & 7))) & 15u) +
            (f.format == ACCEL_QFMT_GPTQ ? 1u : 0u);
    }
    return (float)((int)q - (int)z) * widen_f16(f.scales[g * f.N + n]);
}

__global__ __launch_bounds__(256) void int4_repack_kernel(accel_foreign_int4_t f, int64_t n,
                                                          int64_t groups, int groups_per_row,
                                                          uint32_t* packed,
                                                          uint16_t* scales, uint16_t* zeros,
                                                          uint32_t* bad) {
    const int lane = threadIdx.x & 63;
    const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (g >= groups) return;
    const int64_t i0 = g * 128 + lane, i1 = i0 + 64;
    float v0 = 0.0f, v1 = 0.0f;
    if (groups_per_row) {
        // N % 128 == 0: the group lies in one row, found with one 32-bit
        // division a wave (the row count and groups a row are below 2^31)
        const uint32_t gi = (uint32_t)g;
        const uint32_t k = gi / (uint32_t)groups_per_row;
        const int64_t n0 = (int64_t)(gi - k * (uint32_t)groups_per_row) * 128 + lane;
        const int64_t pg = foreign_group(f, k, bad);
        v0 = foreign_weight(f, k, n0, pg);
        v1 = foreign_weight(f, k, n0 + 64, pg);
    } else {
        if (i0 < n) {
            const int64_t k = i0 / f.N;
            v0 = foreign_weight(f, k, i0 - k * f.N, foreign_group(f, k, bad));
        }
        if (i1 < n) {
            const int64_t k = i1 / f.N;
            v1 = foreign_weight(f, k, i1 - k * f.N, foreign_group(f, k, bad));
        }
    }
    quantize_group(v0, v1, lane, g, n, packed, scales, zeros);
}

// Rows that hold whole groups (N % 128 == 0): one lane per reference group,
// 64 groups to a wave, each lane running the reference's two walks over its
// 128 weights -- the sequential scan for the range, then the codes -- so the
// range needs no cross-lane reduction and the scale and zero are worked out
// once per lane.  AWQ: the lane loads its group's planes at once with 16-byte
// loads (sixteen code words, sixteen zero words, 256 bytes of scales) and
// dequantizes the 128 weights into registers; lanes run along a row of
// groups, so a wave's loads and its 64-byte stores of codes are contiguous.
// Every row offset is a multiple of sixteen bytes when N % 128 == 0 and the
// planes start 16-byte aligned.
typedef uint16_t u16x8_q __attribute__((ext_vector_type(8)));

__device__ __forceinline__ void awq_group_weights(const accel_foreign_int4_t& f, uint32_t k,
                                                  int64_t n0, int64_t pg, float* w) {
    const int64_t wpr = f.N >> 3;
    const u32x4_q* zrow = reinterpret_cast<const u32x4_q*>(f.qzeros + pg * wpr + (n0 >> 3));
    const u16x8_q* srow = reinterpret_cast<const u16x8_q*>(f.scales + pg * f.N + n0);
    const u32x4_q* qrow = reinterpret_cast<const u32x4_q*>(f.qweight + (int64_t)k * wpr + (n0 >> 3));
#pragma unroll
    for (int j4 = 0; j4 < 4; j4++) {
        const u32x4_q zv = zrow[j4], qv = qrow[j4];
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const u16x8_q sc = srow[4 * j4 + jj];
#pragma unroll
            for (int c = 0; c < 8; c++) {
                // column c of a word sits in nibble {0,4,1,5,2,6,3,7}[c]
                const int sh = 4 * ((c >> 1) + ((c & 1) << 2));
                const int q = (int)((qv[jj] >> sh) & 15u), z = (int)((zv[jj] >> sh) & 15u);
                w[8 * (4 * j4 + jj) + c] = (float)(q - z) * widen_f16(sc[c]);
            }
        }
    }
}

// GPTQ packs eight input rows a word, so a group's 128 codes are spread over
// 128 words: too many to hold, they are walked eight weights at a time, twice.
template <int FMT>
__device__ __forceinline__ void foreign_eight(const accel_foreign_int4_t& f, uint32_t k,
                                              int64_t n, int64_t pg, float* w) {
    const int64_t wpr = f.N >> 3;
    const uint32_t zw = f.qzeros[pg * wpr + (n >> 3)];
    typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
    const u16x8 sc = *reinterpret_cast<const u16x8*>(f.scales + pg * f.N + n);
    if constexpr (FMT == ACCEL_QFMT_AWQ) {
        const uint32_t qw = f.qweight[(int64_t)k * wpr + (n >> 3)];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int sh = 4 * ((c >> 1) + ((c & 1) << 2));
            const int q = (int)((qw >> sh) & 15u), z = (int)((zw >> sh) & 15u);
            w[c] = (float)(q - z) * widen_f16(sc[c]);
        }
    } else {
        const uint32_t* row = f.qweight + (int64_t)(k >> 3) * f.N + n;
        const int rs = 4 * (int)(k & 7);
        const int plus = FMT == ACCEL_QFMT_GPTQ ? 1 : 0;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            const int q = (int)((row[c] >> rs) & 15u);
            const int z = (int)((zw >> (4 * c)) & 15u) + plus;
            w[c] = (float)(q - z) * widen_f16(sc[c]);
        }
    }
}

// GPTQ lanes walk the groups down a column of groups (lane i takes row k0 + i
// of the same 128 columns): rows of one published group share its scales and
// zeros, and eight rows share a code word, so a wave's loads coincide.
template <int FMT>
__global__ __launch_bounds__(256) void int4_repack_rows_kernel(accel_foreign_int4_t f,
                                                               int64_t groups, int gpr,
                                                               uint32_t* packed,
                                                               uint16_t* scales,
                                                               uint16_t* zeros, uint32_t* bad) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= groups) return;
    const uint32_t ti = (uint32_t)t;
    constexpr bool kAwq = FMT == ACCEL_QFMT_AWQ;
    const uint32_t cb = kAwq ? ti % (uint32_t)gpr : ti / (uint32_t)f.K;
    const uint32_t k = kAwq ? ti / (uint32_t)gpr : ti - cb * (uint32_t)f.K;
    const int64_t g = (int64_t)k * gpr + cb;
    const int64_t n0 = (int64_t)cb * 128;
    const int64_t pg = foreign_group(f, k, bad);

    // the reference's scan: from the first weight, replacing on a strict
    // comparison (a NaN first weight sticks, later NaNs are skipped)
    float w[kAwq ? 128 : 8];
    float least, most;
    if constexpr (kAwq) {
        awq_group_weights(f, k, n0, pg, w);
        least = most = w[0];
#pragma unroll
        for (int i = 1; i < 128; i++) {
            if (w[i] < least) least = w[i];
            if (w[i] > most) most = w[i];
        }
    } else {
        foreign_eight<FMT>(f, k, n0, pg, w);
        least = most = w[0];
#pragma unroll 1
        for (int j = 0; j < 16; j++) {
            if (j) foreign_eight<FMT>(f, k, n0 + 8 * j, pg, w);
#pragma unroll
            for (int c = 0; c < 8; c++) {
                if (w[c] < least) least = w[c];
                if (w[c] > most) most = w[c];
            }
        }
    }
    uint16_t s_bits, z_bits;
    float s16 = 0.0f, z16 = 0.0f;
    bool coded = false;
    if (most == least) {
        s_bits = narrow_f16(0.0f);
        z_bits = narrow_f16(least);
    } else {
        s_bits = narrow_f16(__fdiv_rn(most - least, 15.0f));
        s16 = widen_f16(s_bits);
        if (s16 == 0.0f) {
            z_bits = narrow_f16(least);
        } else {
            z_bits = narrow_f16(__fdiv_rn(-least, s16));
            z16 = widen_f16(z_bits);
            coded = true;
        }
    }
    scales[g] = s_bits;
    zeros[g] = z_bits;
    u32x4_q* out = reinterpret_cast<u32x4_q*>(packed + g * 16);
    if (!coded) {
#pragma unroll
        for (int j4 = 0; j4 < 4; j4++) out[j4] = (u32x4_q){0, 0, 0, 0};
        return;
    }
    const CodeRule rule = code_rule(s16, z16, least, most);
    if constexpr (kAwq) {
#pragma unroll
        for (int j4 = 0; j4 < 4; j4++) {
            u32x4_q words;
            uint32_t open = 0;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) words[jj] = code_word_estimate(w + 32 * j4 + 8 * jj,
                                                                      rule, &open, jj);
            // the f64 rule for the weights the estimate left open, each
            // dequantized again from the planes: one short loop, not 128
            // inlined divisions
            while (open) {
                const int b = __builtin_ctz(open);
                open &= open - 1u;
                const int i = 32 * j4 + b, sh = 4 * (b & 7);
                const uint32_t code = code_exact(foreign_weight(f, k, n0 + i, pg), rule);
                words[b >> 3] = (words[b >> 3] & ~(15u << sh)) | (code << sh);
            }
            out[j4] = words;
        }
    } else {
#pragma unroll 1
        for (int j4 = 0; j4 < 4; j4++) {
            u32x4_q words;
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                foreign_eight<FMT>(f, k, n0 + 8 * (4 * j4 + jj), pg, w);
                words[jj] = code_word(w, rule);
            }
            out[j4] = words;
        }
    }
}

}  // namespace

hipError_t launch_int4_quantize(hipStream_t st, const float* w, int64_t n, uint32_t* packed,
                                uint16_t* scales, uint16_t* zeros) {
    const int64_t groups = (n + 127) / 128;
    const int64_t blocks = (groups + 3) / 4;
    hipLaunchKernelGGL(int4_quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, st, w, n,
                       packed, scales, zeros, groups);
    return hipGetLastError();
}

hipError_t launch_int4_repack(hipStream_t st, const accel_foreign_int4_t& f, uint32_t* codes,
                              uint16_t* scales, uint16_t* zeros, uint32_t* bad) {
    const int64_t n = f.K * f.N;
    const int64_t groups = (n + 127) / 128;
    const int64_t blocks = (groups + 3) / 4;
    if (blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
    // one 32-bit division a wave finds a group's row where rows hold whole
    // groups and the group index fits 32 bits
    const int gpr = (f.N % 128 == 0 && groups < (int64_t(1) << 32)) ? (int)(f.N / 128) : 0;
    const bool aligned = ((reinterpret_cast<uintptr_t>(f.scales) |
                           reinterpret_cast<uintptr_t>(f.qweight) |
                           reinterpret_cast<uintptr_t>(f.qzeros) |
                           reinterpret_cast<uintptr_t>(codes)) & 15) == 0;
    if (gpr && aligned) {
        const int64_t lane_blocks = (groups + 255) / 256;
        const dim3 grid((unsigned)lane_blocks), block(256);
        if (f.format == ACCEL_QFMT_AWQ)
            hipLaunchKernelGGL(int4_repack_rows_kernel<ACCEL_QFMT_AWQ>, grid, block, 0, st, f,
                               groups, gpr, codes, scales, zeros, bad);
        else if (f.format == ACCEL_QFMT_GPTQ)
            hipLaunchKernelGGL(int4_repack_rows_kernel<ACCEL_QFMT_GPTQ>, grid, block, 0, st, f,
                               groups, gpr, codes, scales, zeros, bad);
        else
            hipLaunchKernelGGL(int4_repack_rows_kernel<ACCEL_QFMT_GPTQ_V2>, grid, block, 0, st,
                               f, groups, gpr, codes, scales, zeros, bad);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(int4_repack_kernel, dim3((unsigned)blocks), dim3(256), 0, st, f, n,
                       groups, gpr, codes, scales, zeros, bad);
    return hipGetLastError();
}

}  // namespace accel
