// Published 4-bit checkpoints (AWQ, GPTQ) into the reference int4 format.
//
// The reference names reading these files as the unbuilt next step of its
// int4 format (specs/048-int4.md:126-131,167): the 4-bit codes, the f16 scale
// and the zero point are the same idea, the layout is not.  AWQ and GPTQ keep
// one (scale, zero) per output column per group of input rows; the reference
// keeps one per 128 consecutive weights of the flat [K, N] array, which runs
// along a row.  So a repack is: dequantize every weight exactly in f32,
// w = (q - z) * s (an integer of at most five bits times an f16 is exact in
// f32), then quantize each group of 128 flat weights with the reference's
// Int4Quantize (quant/int4.go:71-138), here the library's host packer, which
// is bit-identical to it.
//
// The packings restated (from the published packers, whose files are not part
// of the reference):
//   AWQ (AutoAWQ 0.2, "gemm" version): qweight u32 [K, N/8]; the packer ORs
//     column 8j + order[i] into nibble i of word (k, j) with
//     order = {0, 2, 4, 6, 1, 3, 5, 7}, so column 8j + c sits in nibble
//     {0, 4, 1, 5, 2, 6, 3, 7}[c]; qzeros u32 [groups, N/8] the same way;
//     scales f16 [groups, N]; row k belongs to group k / group_size.
//   GPTQ (AutoGPTQ 0.7, checkpoint format "gptq"): qweight u32 [K/8, N], row
//     8i + j in nibble j of word (i, n); qzeros u32 [groups, N/8], column
//     8j + c in nibble c, holding z - 1 (the packer subtracts one; readers add
//     it back); scales f16 [groups, N]; row k belongs to group g_idx[k]
//     (act-order checkpoints) or k / group_size.
//   GPTQ v2 (GPTQModel's "gptq_v2"): as GPTQ with qzeros holding z.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "internal.hpp"

#define ACCEL_API extern "C" __attribute__((visibility("default")))

namespace accel {

void int4_quantize_host(const float* w, int64_t n, uint32_t* packed, uint16_t* scales,
                        uint16_t* zeros);
float widen_f16_host(uint16_t h);

namespace {

constexpr int kAwqNibble[8] = {0, 4, 1, 5, 2, 6, 3, 7};

// Why a published layer cannot be repacked, or "" (pointers not included).
std::string check_foreign_dims(const accel_foreign_int4_t* f) {
    char buf[320];
    if (!f) return "no layer was given";
    if (f->format != ACCEL_QFMT_AWQ && f->format != ACCEL_QFMT_GPTQ &&
        f->format != ACCEL_QFMT_GPTQ_V2) {
        snprintf(buf, sizeof buf, "format %d is none of AWQ (1), GPTQ (2) and GPTQ v2 (3)",
                 (int)f->format);
        return buf;
    }
    if (f->K < 1 || f->N < 1 || f->K > INT32_MAX || f->N > INT32_MAX ||
        (uint64_t)f->K * (uint64_t)f->N >= (1ull << 40)) {
        snprintf(buf, sizeof buf, "the layer is [%lld, %lld], outside this library's extents",
                 (long long)f->K, (long long)f->N);
        return buf;
    }
    if (f->N % 8 != 0) {
        snprintf(buf, sizeof buf,
                 "N = %lld is not a multiple of 8; both formats pack eight columns' zeros a word",
                 (long long)f->N);
        return buf;
    }
    if (f->group_size < 1) {
        snprintf(buf, sizeof buf, "group_size %d; a group spans at least one input row",
                 (int)f->group_size);
        return buf;
    }
    if (f->format == ACCEL_QFMT_AWQ) {
        if (f->g_idx) return "AWQ has no g_idx; its rows are grouped by k / group_size";
        if (f->K % f->group_size != 0 || f->groups != f->K / f->group_size) {
            snprintf(buf, sizeof buf,
                     "AWQ layer with K = %lld and group_size %d has %lld groups; it needs K a "
                     "multiple of group_size and K / group_size groups",
                     (long long)f->K, (int)f->group_size, (long long)f->groups);
            return buf;
        }
        return "";
    }
    if (f->K % 8 != 0) {
        snprintf(buf, sizeof buf,
                 "GPTQ layer with K = %lld; GPTQ packs eight input rows a word, so K is a "
                 "multiple of 8",
                 (long long)f->K);
        return buf;
    }
    const int64_t need = (f->K + f->group_size - 1) / f->group_size;
    if (!f->g_idx && f->groups != need) {
        snprintf(buf, sizeof buf,
                 "GPTQ layer with K = %lld and group_size %d has %lld groups and no g_idx; "
                 "rows grouped by k / group_size need %lld",
                 (long long)f->K, (int)f->group_size, (long long)f->groups, (long long)need);
        return buf;
    }
    if (f->groups < 1) return "the layer has no groups";
    return "";
}

// w(k, n) of a published layer, dequantized exactly; g is k's group.
inline float foreign_weight(const accel_foreign_int4_t& f, int64_t k, int64_t n, int64_t g) {
    const int64_t wpr = f.N / 8;
    uint32_t q, z;
    if (f.format == ACCEL_QFMT_AWQ) {
        const int sh = 4 * kAwqNibble[n & 7];
        q = (f.qweight[k * wpr + (n >> 3)] >> sh) & 15u;
        z = (f.qzeros[g * wpr + (n >> 3)] >> sh) & 15u;
    } else {
        q = (f.qweight[(k >> 3) * f.N + n] >> (4 * (k & 7))) & 15u;
        z = ((f.qzeros[g * wpr + (n >> 3)] >> (4 * (n & 7))) & 15u) +
            (f.format == ACCEL_QFMT_GPTQ ? 1u : 0u);
    }
    return (float)((int)q - (int)z) * widen_f16_host(f.scales[g * f.N + n]);
}

int refuse_repack(const std::string& why) {
    return fail(ACCEL_E_INVALID, "accel/quant: Int4Repack: %s", why.c_str());
}

}  // namespace

hipError_t launch_int4_repack(hipStream_t st, const accel_foreign_int4_t& f, uint32_t* codes,
                              uint16_t* scales, uint16_t* zeros, uint32_t* bad);

}  // namespace accel

using namespace accel;

ACCEL_API int accel_int4_repack_host(const accel_foreign_int4_t* src, uint32_t* codes,
                                     uint16_t* scales, uint16_t* zeros) {
    clear_error();
    std::string why = check_foreign_dims(src);
    if (!why.empty()) return refuse_repack(why);
    if (!src->qweight || !src->qzeros || !src->scales)
        return refuse_repack("the layer needs qweight, qzeros and scales");
    if (!codes || !scales || !zeros) return refuse_repack("an output plane is NULL");
    const accel_foreign_int4_t& f = *src;
    std::vector<int64_t> group(f.K);
    for (int64_t k = 0; k < f.K; k++) {
        const int64_t g = f.g_idx ? (int64_t)f.g_idx[k] : k / f.group_size;
        if (g < 0 || g >= f.groups) {
            char buf[160];
            snprintf(buf, sizeof buf, "g_idx[%lld] = %lld is outside the layer's %lld groups",
                     (long long)k, (long long)g, (long long)f.groups);
            return refuse_repack(buf);
        }
        group[k] = g;
    }
    // Chunks of whole reference groups: each is dequantized into a buffer
    // and quantized in place of the whole matrix at once.
    const int64_t n = f.K * f.N;
    const int64_t chunk = (int64_t)128 * 4096;
    std::vector<float> w((size_t)std::min(n, chunk));
    for (int64_t lo = 0; lo < n; lo += chunk) {
        const int64_t hi = std::min(n, lo + chunk);
        int64_t k = lo / f.N, c = lo % f.N;
        for (int64_t i = lo; i < hi; i++) {
            w[(size_t)(i - lo)] = foreign_weight(f, k, c, group[k]);
            if (++c == f.N) {
                c = 0;
                k++;
            }
        }
        int4_quantize_host(w.data(), hi - lo, codes + lo / 8, scales + lo / 128,
                           zeros + lo / 128);
    }
    return ACCEL_OK;
}

ACCEL_API int accel_int4_repack(int dev, void* stream, const accel_foreign_int4_t* src,
                                accel_int4_t* dst) {
    clear_error();
    std::string why = check_foreign_dims(src);
    if (!why.empty()) return refuse_repack(why);
    if (!src->qweight || !src->qzeros || !src->scales)
        return refuse_repack("the layer needs qweight, qzeros and scales");
    const int64_t n = src->K * src->N;
    if (!dst || !dst->codes || !dst->scales || !dst->zeros || dst->weights != n ||
        dst->codes_len != (n + 7) / 8 || dst->scales_len != (n + 127) / 128 ||
        dst->zeros_len != (n + 127) / 128) {
        char buf[200];
        snprintf(buf, sizeof buf,
                 "the destination must hold %lld weights: %lld code words and %lld scales and "
                 "zeros",
                 (long long)n, (long long)((n + 7) / 8), (long long)((n + 127) / 128));
        return refuse_repack(buf);
    }
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    hipStream_t st = (hipStream_t)stream;
    void* ws = workspace(d, st, sizeof(uint32_t), &status);
    if (!ws) return status;
    uint32_t* bad = reinterpret_cast<uint32_t*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    hipError_t e = hipMemsetAsync(bad, 0, sizeof(uint32_t), st);
    if (e == hipSuccess)
        e = launch_int4_repack(st, *src, const_cast<uint32_t*>(dst->codes),
                               const_cast<uint16_t*>(dst->scales),
                               const_cast<uint16_t*>(dst->zeros), bad);
    // the repack is done before the flag is read, with a blocking copy: no
    // transfer into this frame can outlive the call
    uint32_t flag = 0;
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess) e = hipMemcpy(&flag, bad, sizeof flag, hipMemcpyDeviceToHost);
    status = classify(d, e, "Int4Repack");
    if (status != ACCEL_OK) return status;
    if (flag)
        return refuse_repack("a g_idx entry is outside the layer's groups (the rows it names "
                             "were repacked against group 0)");
    return ACCEL_OK;
}
