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

__global__ __launch_bounds__(256) void int4_quantize_kernel(const float* __restrict__ w,
                                                            int64_t n, uint32_t* packed,
                                                            uint16_t* scales, uint16_t* zeros,
                                                            int64_t groups) {
    const int lane = threadIdx.x & 63;
    const int64_t g = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (g >= groups) return;
    const int64_t lo = g * 128;
    const int64_t i0 = lo + lane, i1 = lo + 64 + lane;
    const bool in0 = i0 < n, in1 = i1 < n;
    const float v0 = in0 ? w[i0] : 0.0f;
    const float v1 = in1 ? w[i1] : 0.0f;

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
    auto code_of = [&](float v, bool in) -> uint32_t {
        if (!coded || !in) return 0u;
        const double q = rint(__ddiv_rn((double)v, (double)s16) + (double)z16);
        if (q != q) return 0u;
        return q > 15.0 ? 15u : (q < 0.0 ? 0u : (uint32_t)q);
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

}  // namespace

hipError_t launch_int4_quantize(hipStream_t st, const float* w, int64_t n, uint32_t* packed,
                                uint16_t* scales, uint16_t* zeros) {
    const int64_t groups = (n + 127) / 128;
    const int64_t blocks = (groups + 3) / 4;
    hipLaunchKernelGGL(int4_quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, st, w, n,
                       packed, scales, zeros, groups);
    return hipGetLastError();
}

}  // namespace accel
