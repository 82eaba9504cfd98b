// Host side of the int4 format: quant.Int4Quantize and Int4Dequantize
// (quant/int4.go:71-175) with the reference's f16 narrowing
// (internal/kernel/narrow.go:67-139).
//
// The packer is bit-exact with the reference: the range arithmetic is f32,
// the scale and zero point are narrowed to f16 and read back before use, and
// each code is round-half-even of an f64 quotient, clamped to [0, 15].
#include <algorithm>
#include <cmath>
#include <cstring>

#include "internal.hpp"

namespace accel {

namespace {

inline uint32_t bits_of(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    return b;
}
inline float float_of(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// Round-half-even right shift of a mantissa by n bits.
inline uint32_t shift_rne(uint32_t v, uint32_t n) {
    if (n == 0) return v;
    if (n > 31) return 0;
    const uint32_t q = v >> n;
    const uint32_t rem = v & ((1u << n) - 1u);
    const uint32_t half = 1u << (n - 1);
    return q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u);
}

// f32 -> f16 bits as the reference narrows: RNE; overflow and infinity to a
// signed infinity; NaN to 0x7e00; magnitudes below 2^-24 to a signed zero
// (so (2^-25, 2^-24) flushes where IEEE would round up).
uint16_t narrow_f16(float x) {
    const uint32_t b = bits_of(x);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7e00;
    const int e = (int)((b >> 23) & 0xffu) - 127;
    uint32_t mant = b & 0x7fffffu;
    if (e > 15) return (uint16_t)(sign | 0x7c00u);  // includes infinity (e == 128)
    if (e < -24) return sign;
    if (e < -14) return (uint16_t)(sign | shift_rne(mant | 0x800000u, (uint32_t)(-e - 1)));
    return (uint16_t)(sign | (((uint32_t)(e + 15) << 10) + shift_rne(mant, 13)));
}

// f16 bits -> f32, exact.
float widen_f16(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return float_of(sign | 0x7f800000u | (m << 13));
    if (e != 0) return float_of(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return float_of(sign);
    // subnormal: normalise the mantissa
    int shift = __builtin_clz(m) - 21;  // leading zeros within the 11-bit field
    m = (m << shift) & 0x3ffu;
    return float_of(sign | ((uint32_t)(113 - shift) << 23) | (m << 13));
}

}  // namespace

float widen_f16_host(uint16_t h) { return widen_f16(h); }

void int4_quantize_host(const float* w, int64_t n, uint32_t* packed, uint16_t* scales,
                        uint16_t* zeros) {
    const int64_t kGroup = 128;
    const int64_t words = (n + 7) / 8;
    std::memset(packed, 0, sizeof(uint32_t) * (size_t)words);
    for (int64_t g = 0, lo = 0; lo < n; g++, lo += kGroup) {
        const int64_t hi = lo + kGroup < n ? lo + kGroup : n;
        float least = w[lo], most = w[lo];
        for (int64_t i = lo + 1; i < hi; i++) {
            if (w[i] < least) least = w[i];
            if (w[i] > most) most = w[i];
        }
        if (most == least) {  // constant group: the zero point carries it
            scales[g] = narrow_f16(0.0f);
            zeros[g] = narrow_f16(least);
            continue;
        }
        scales[g] = narrow_f16((most - least) / 15.0f);
        const float s16 = widen_f16(scales[g]);
        if (s16 == 0.0f) {  // scale underflowed f16
            zeros[g] = narrow_f16(least);
            continue;
        }
        zeros[g] = narrow_f16(-least / s16);
        const double z16 = (double)widen_f16(zeros[g]);
        const double sd = (double)s16;
        for (int64_t i = lo; i < hi; i++) {
            double q = std::nearbyint((double)w[i] / sd + z16);
            uint32_t code;
            if (q != q) code = 0;  // NaN passes the clamp; Go converts it to 0
            else code = q > 15.0 ? 15u : (q < 0.0 ? 0u : (uint32_t)q);
            packed[i >> 3] |= code << (4 * (i & 7));
        }
    }
}

void int4_dequantize_host(const uint32_t* packed, const uint16_t* scales,
                          const uint16_t* zeros, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) {
        const float s = widen_f16(scales[i / 128]);
        const float z = widen_f16(zeros[i / 128]);
        if (s == 0.0f) {
            out[i] = z;
            continue;
        }
        const uint32_t code = (packed[i >> 3] >> (4 * (i & 7))) & 0xfu;
        out[i] = ((float)code - z) * s;
    }
}

// quant.Int8Quantize (quant/quant.go:60-123): per block of 32 flat weights
// the peak magnitude (f32), s = f16(peak / 127) read back as f32, each quant
// the round-half-even of the f64 quotient w / s clamped to [-127, 127].  A
// zero peak, or a scale that narrows to zero, leaves the block's quants 0.
void int8_quantize_host(const float* w, int64_t n, int8_t* quants, uint16_t* scales) {
    const int64_t blocks = (n + 31) / 32;
    for (int64_t b = 0; b < blocks; b++) {
        const int64_t lo = b * 32, hi = std::min(lo + 32, n);
        float peak = 0.0f;
        for (int64_t i = lo; i < hi; i++) {
            const float a = std::fabs(w[i]);
            if (a > peak) peak = a;   // a NaN never compares greater
        }
        for (int64_t i = lo; i < hi; i++) quants[i] = 0;
        if (peak == 0.0f) {
            scales[b] = narrow_f16(0.0f);
            continue;
        }
        const float s = peak / 127.0f;
        scales[b] = narrow_f16(s);
        const float s16 = widen_f16(scales[b]);
        if (s16 == 0.0f) continue;
        for (int64_t i = lo; i < hi; i++) {
            double q = std::nearbyint((double)w[i] / (double)s16);
            if (q > 127.0) q = 127.0;
            if (q < -127.0) q = -127.0;
            // a NaN weight: Go's int8 conversion on amd64 gives 0
            quants[i] = q == q ? (int8_t)q : 0;
        }
    }
}

// quant.Int8Dequantize (quant/quant.go:129-135).
void int8_dequantize_host(const int8_t* quants, const uint16_t* scales, int64_t n, float* out) {
    for (int64_t i = 0; i < n; i++) out[i] = (float)quants[i] * widen_f16(scales[i / 32]);
}

}  // namespace accel

#define ACCEL_API extern "C" __attribute__((visibility("default")))

ACCEL_API int accel_int8_quantize(const float* w, int64_t n, int8_t* quants,
                                  uint16_t* scales) {
    accel::clear_error();
    if (n < 0) return accel::fail(ACCEL_E_INVALID, "accel_int8_quantize: negative count");
    if (n == 0) return ACCEL_OK;
    if (!w || !quants || !scales)
        return accel::fail(ACCEL_E_INVALID, "accel_int8_quantize: NULL pointer");
    accel::int8_quantize_host(w, n, quants, scales);
    return ACCEL_OK;
}

ACCEL_API int accel_int8_dequantize(const int8_t* quants, const uint16_t* scales, int64_t n,
                                    float* out) {
    accel::clear_error();
    if (n < 0) return accel::fail(ACCEL_E_INVALID, "accel_int8_dequantize: negative count");
    if (n == 0) return ACCEL_OK;
    if (!quants || !scales || !out)
        return accel::fail(ACCEL_E_INVALID, "accel_int8_dequantize: NULL pointer");
    accel::int8_dequantize_host(quants, scales, n, out);
    return ACCEL_OK;
}

ACCEL_API int accel_int4_quantize(const float* w, int64_t n, uint32_t* packed,
                                  uint16_t* scales, uint16_t* zeros) {
    accel::clear_error();
    if (n < 0) return accel::fail(ACCEL_E_INVALID, "accel_int4_quantize: negative count");
    if (n == 0) return ACCEL_OK;
    if (!w || !packed || !scales || !zeros)
        return accel::fail(ACCEL_E_INVALID, "accel_int4_quantize: NULL pointer");
    accel::int4_quantize_host(w, n, packed, scales, zeros);
    return ACCEL_OK;
}

// BASELINE config 1's literal format (no counterpart in the reference, whose
// groups are 128 flat weights with an f16 scale and zero): groups of 32 rows
// of one column, s = f32(amax / 7), q = clamp(rne(f32(w / s)), -8, 7) + 8,
// packed as quant/int4 packs (element k*N + n, low nibble first); a group of
// zeros has s = 0 and codes 8.  Finite weights.
ACCEL_API int accel_int4_g32_quantize(const float* w, int64_t K, int64_t N, uint32_t* packed,
                                      float* scales) {
    accel::clear_error();
    if (K < 0 || N < 0 || K % 32 != 0 || (K * N) % 8 != 0)
        return accel::fail(ACCEL_E_INVALID,
                           "accel_int4_g32_quantize: K=%lld, N=%lld (K must be a multiple of "
                           "32 and K*N of 8)",
                           (long long)K, (long long)N);
    if (K == 0 || N == 0) return ACCEL_OK;
    if (!w || !packed || !scales)
        return accel::fail(ACCEL_E_INVALID, "accel_int4_g32_quantize: NULL pointer");
    std::fill(packed, packed + K * N / 8, 0u);
    for (int64_t g = 0; g < K / 32; g++) {
        for (int64_t n = 0; n < N; n++) {
            float amax = 0.0f;
            for (int64_t r = 0; r < 32; r++) amax = std::fmax(amax, std::fabs(w[(g * 32 + r) * N + n]));
            const float sc = amax / 7.0f;
            scales[g * N + n] = sc;
            for (int64_t r = 0; r < 32; r++) {
                const int64_t i = (g * 32 + r) * N + n;
                float rq = 0.0f;
                if (sc != 0.0f) rq = std::nearbyint(w[i] / sc);
                rq = std::fmin(std::fmax(rq, -8.0f), 7.0f);
                const uint32_t q = (uint32_t)(int)(rq + 8.0f);
                packed[i >> 3] |= q << (4 * (i & 7));
            }
        }
    }
    return ACCEL_OK;
}

ACCEL_API int accel_int4_dequantize(const uint32_t* packed, const uint16_t* scales,
                                    const uint16_t* zeros, int64_t n, float* out) {
    accel::clear_error();
    if (n < 0) return accel::fail(ACCEL_E_INVALID, "accel_int4_dequantize: negative count");
    if (n == 0) return ACCEL_OK;
    if (!packed || !scales || !zeros || !out)
        return accel::fail(ACCEL_E_INVALID, "accel_int4_dequantize: NULL pointer");
    accel::int4_dequantize_host(packed, scales, zeros, n, out);
    return ACCEL_OK;
}
