// The operator layer of the C ABI: the tensor package's int4 and grouped
// entry points with the reference's validation and refusal messages
// (tensor/int4.go:41-212, tensor/grouped.go:48-212, tensor/segment.go:31-50),
// and kernel-record dispatch for the backend seam.
//
// Kernel selection (the analogue of a plan's selection report,
// tensor/compile.go:36-42, tensor/plan.go:36-41): choose_int4 below picks a
// product's route and says why, and names every route it turned down; the
// launches it becomes are recorded as they are made (accel_hip_last_selection)
// or planned without running (accel_int4_select).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <string>

#include "internal.hpp"

namespace accel {
hipError_t launch_zero_tail_bf16(hipStream_t st, const uint32_t* off, uint16_t* out, int E,
                                 int T, int N);
}

using namespace accel;

#define ACCEL_API extern "C" __attribute__((visibility("default")))

namespace {

const char* dtype_name(int32_t d) {
    switch (d) {
        case ACCEL_F32: return "f32";
        case ACCEL_F16: return "f16";
        case ACCEL_BF16: return "bf16";
        case ACCEL_U32: return "u32";
        case ACCEL_I8: return "i8";
        default: return "an unknown dtype";
    }
}

std::string shape_str(const accel_tensor_t* t) {
    std::string s = "[";
    for (int i = 0; i < t->rank && i < 4; i++) {
        if (i) s += ' ';
        s += std::to_string((long long)t->shape[i]);
    }
    return s + "]";
}

int64_t elements(const accel_tensor_t* t) {
    int64_t n = 1;
    for (int i = 0; i < t->rank && i < 4; i++) n *= t->shape[i];
    return n;
}

int refuse(const char* op, const std::string& why) {
    return fail(ACCEL_E_INVALID, "accel/tensor: %s: %s", op, why.c_str());
}

bool valid_tensor(const accel_tensor_t* t) {
    return t && t->rank >= 0 && t->rank <= 4;
}

// checkInt4 (tensor/int4.go:41-78): why a packed matrix is not usable, or "".
std::string check_int4(const accel_int4_t* q, const char* what) {
    char buf[512];
    if (!q || !q->codes || !q->scales || !q->zeros) {
        snprintf(buf, sizeof buf,
                 "%s needs a code plane, a scale plane and a zero plane; the zero point is "
                 "what makes four bits usable and is not optional",
                 what);
        return buf;
    }
    if (q->weights <= 0) {
        snprintf(buf, sizeof buf,
                 "%s declares %lld weights; the count cannot be derived from the word count, "
                 "because eight weights per word makes several matrices pack into the same "
                 "words",
                 what, (long long)q->weights);
        return buf;
    }
    const int64_t want = (q->weights + 7) / 8;
    if (q->codes_len != want) {
        snprintf(buf, sizeof buf,
                 "%s declares %lld weights, which is %lld words, and the code plane holds %lld",
                 what, (long long)q->weights, (long long)want, (long long)q->codes_len);
        return buf;
    }
    const int64_t groups = (q->weights + 127) / 128;
    if (q->scales_len != groups) {
        snprintf(buf, sizeof buf, "%s has %lld weights, which is %lld groups of 128, and %lld scales",
                 what, (long long)q->weights, (long long)groups, (long long)q->scales_len);
        return buf;
    }
    if (q->zeros_len != groups) {
        snprintf(buf, sizeof buf, "%s has %lld weights, which is %lld groups of 128, and %lld zeros",
                 what, (long long)q->weights, (long long)groups, (long long)q->zeros_len);
        return buf;
    }
    return "";
}

Int4Planes planes(const accel_int4_t* w) { return {w->codes, w->scales, w->zeros}; }

// Runs a launch and classifies its outcome.
int finish(Device* d, hipError_t e, int status, const char* what) {
    if (status != ACCEL_OK) return status;
    return classify(d, e, what);
}

int check_out(const char* op, const accel_tensor_t* out, int32_t dtype, int64_t rows,
              int64_t cols, bool vector) {
    char buf[256];
    if (!valid_tensor(out) || !out->data)
        return refuse(op, "the output tensor is missing");
    if (out->dtype != dtype) {
        snprintf(buf, sizeof buf, "the output is %s and this product writes %s",
                 dtype_name(out->dtype), dtype_name(dtype));
        return refuse(op, buf);
    }
    const bool ok = vector ? (out->rank == 1 && out->shape[0] == cols)
                           : (out->rank == 2 && out->shape[0] == rows && out->shape[1] == cols);
    if (!ok) {
        if (vector)
            snprintf(buf, sizeof buf, "the output is %s and the product is [%lld]",
                     shape_str(out).c_str(), (long long)cols);
        else
            snprintf(buf, sizeof buf, "the output is %s and the product is [%lld %lld]",
                     shape_str(out).c_str(), (long long)rows, (long long)cols);
        return refuse(op, buf);
    }
    return ACCEL_OK;
}

// The routes of an int4 product, in the order they are tried.
enum class Int4Route {
    kNone,          // an empty product: nothing to launch
    kDecodeF32,     // M <= 16 f32 rows: the decode kernels
    kGemmF32x3,     // M > 16 f32 rows on the matrix cores, three-term split
    kGemmF32,       // M > 16 f32 rows, fp32 VALU tiles
    kGenericF32,    // one lane per output element
    kDecodeBf16Row, // one bf16 row: the VALU decode kernel
    kDecodeBf16Rows,// 2..16 bf16 rows: the matrix-core decode kernel
    kGemmBf16,      // bf16 rows on the matrix-core tiles
    kGenericBf16,   // one lane per output element
};

struct Int4Choice {
    Int4Route route = Int4Route::kNone;
    std::string reason;
    std::vector<std::string> rejected;
};

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Which route an int4 product of M x K x N takes, why, and what it turned
// down (KernelSelection's Reason and Rejected).  The shape limits are the
// launchers' own predicates, so the answer is the route run_int4_product
// takes.
Int4Choice choose_int4(int32_t dtype, const void* a, const void* codes, int M, int K, int N) {
    Int4Choice c;
    char buf[320];
    if (M == 0 || N == 0) {
        c.reason = "an empty product: there is nothing to launch";
        return c;
    }
    const bool aligned128 = N % 128 == 0 && (uint64_t)K * (uint64_t)N < (1ull << 32);
    auto reject = [&](const char* route, const char* why) {
        snprintf(buf, sizeof buf, "%s: %s", route, why);
        c.rejected.push_back(buf);
    };
    if (dtype == ACCEL_F32) {
        const bool decode = int4_decode_f32_supported(M, K, N, codes);
        if (decode) {
            c.route = Int4Route::kDecodeF32;
            if (M == 1)
                c.reason = "one f32 row: the VALU decode kernel streams the weights once, K "
                           "split across workgroups so every CU reads";
            else if (K % 32 == 0 && N < (1 << 27) && aligned16(a))
                c.reason = "2..16 f32 rows: the matrix-core decode kernel (x*512s in three bf16 "
                           "terms against the exact codes) reads the weights once for all rows";
            else
                c.reason = "2..16 f32 rows whose K is not a multiple of 32 or whose rows are "
                           "not 16-byte aligned: the VALU decode kernel, rows in passes of up "
                           "to eight";
            if (M > 1) reject("the matrix-core tiles", "a 32-row band would be mostly empty");
            return c;
        }
        if (M <= 16)
            reject("the decode kernels",
                   "they take N a multiple of 128 and 16-byte aligned codes");
        else
            reject("the decode kernels", "they take at most 16 rows a launch");
        if (M > 16 && int4_gemm_f32x3_supported(K, N) && aligned16(a)) {
            c.route = Int4Route::kGemmF32x3;
            c.reason = "more than 16 f32 rows: the bf16 matrix-core tiles to f32 accuracy "
                       "(x*512s in three bf16 terms against the exact codes), a short band "
                       "running only the 32-row m-tiles it has rows for; K split when the "
                       "tiles leave CUs idle";
            if (M <= 48)
                reject("16-row matrix-core decode products",
                       "the tiles' short bands beat them from 17 rows (4096 x 4096 at 32 "
                       "rows: 15.7 against 21.3 us)");
            return c;
        }
        if (M > 16)
            reject("the f32 matrix-core tiles",
                   "they take K % 64 == 0, N % 128 == 0 and 16-byte aligned rows");
        if (M > 16 && aligned128) {
            c.route = Int4Route::kGemmF32;
            c.reason = "more than 16 f32 rows that the matrix-core tiles cannot take: fp32 "
                       "VALU tiles";
            return c;
        }
        if (M > 16) reject("the fp32 VALU tiles", "they take N % 128 == 0 and K*N < 2^32");
        c.route = Int4Route::kGenericF32;
        c.reason = "no tiled kernel takes this shape: one lane per output element, decoding "
                   "with the flat index (correct everywhere, not a speed path)";
        return c;
    }
    if (M == 1 && int4_decode_f32_supported(1, K, N, codes)) {
        c.route = Int4Route::kDecodeBf16Row;
        c.reason = "one bf16 row: the VALU decode kernel reading bf16, f32 arithmetic, one "
                   "rounding of each sum to bf16";
        reject("the matrix-core tiles", "a 32-row band for one row would be mostly empty");
        return c;
    }
    if (M == 1)
        reject("the VALU decode kernel", "it takes N a multiple of 128 and 16-byte aligned codes");
    if (int4_decode_bf16_rows_supported(M, K, N, a, codes)) {
        c.route = Int4Route::kDecodeBf16Rows;
        c.reason = "2..16 bf16 rows: the matrix-core decode kernel (bf16 staged, f32 "
                   "arithmetic, one rounding to bf16) reads the weights once for all rows";
        reject("the matrix-core tiles", "a 32-row band would be mostly empty");
        return c;
    }
    if (M >= 2 && M <= 16)
        reject("the matrix-core decode kernel",
               "it takes K % 32 == 0, N a multiple of 128, 16-byte aligned rows and codes");
    if (int4_gemm_bf16_supported(M, K, N) && aligned16(a)) {
        c.route = Int4Route::kGemmBf16;
        c.reason = "bf16 rows: the matrix-core tiles (codes dequantised to bf16 in registers, "
                   "f32 accumulation); K split when the tiles leave CUs idle";
        return c;
    }
    reject("the matrix-core tiles",
           aligned16(a) ? "they take K % 64 == 0, N % 128 == 0, K < 2^22 and N < 2^26"
                        : "the activations are not 16-byte aligned, and the tiles load them "
                          "16 bytes at a time");
    c.route = Int4Route::kGenericBf16;
    c.reason = "no tiled kernel takes this shape or alignment: one lane per output element, "
               "decoding with the flat index (correct everywhere, not a speed path)";
    return c;
}

// Runs the launches of a chosen route.
hipError_t launch_int4_route(Device* d, hipStream_t st, Int4Route r, const void* a,
                             const Int4Planes& p, void* out, int M, int K, int N, Epilogue ep,
                             int* status) {
    const float* af = static_cast<const float*>(a);
    const uint16_t* ab = static_cast<const uint16_t*>(a);
    uint16_t* ob = static_cast<uint16_t*>(out);
    switch (r) {
        case Int4Route::kNone: return hipSuccess;
        case Int4Route::kDecodeF32:
            return launch_int4_decode_f32(d, st, af, p, out, M, K, N, status, ep);
        case Int4Route::kGemmF32x3:
            return launch_int4_gemm_f32x3(d, st, af, p, out, M, K, N, ep, status);
        case Int4Route::kGemmF32: return launch_int4_gemm_f32(d, st, af, p, out, M, K, N, ep);
        case Int4Route::kGenericF32: return launch_int4_generic_f32(st, af, p, out, M, K, N, ep);
        case Int4Route::kDecodeBf16Row:
            return launch_int4_decode_bf16_row(d, st, ab, p, ob, K, N, status, ep.bias);
        case Int4Route::kDecodeBf16Rows:
            return launch_int4_decode_bf16_rows(d, st, ab, p, ob, M, K, N, status, ep.bias);
        case Int4Route::kGemmBf16:
            return launch_int4_gemm_bf16(d, st, ab, p, ob, M, K, N, ep.bias, status);
        case Int4Route::kGenericBf16:
            return launch_int4_generic_bf16(st, ab, p, ob, M, K, N, ep.bias);
    }
    return hipSuccess;
}

std::string join(const std::vector<std::string>& v, const char* sep) {
    std::string s;
    for (size_t i = 0; i < v.size(); i++) {
        if (i) s += sep;
        s += v[i];
    }
    return s;
}

void fill_selection(accel_selection_t* out, const std::string& op, const std::string& kernel,
                    const std::string& reason, const std::string& rejected) {
    memset(out, 0, sizeof *out);
    snprintf(out->op, sizeof out->op, "%s", op.c_str());
    snprintf(out->kernel, sizeof out->kernel, "%s", kernel.c_str());
    snprintf(out->reason, sizeof out->reason, "%s", reason.c_str());
    snprintf(out->rejected, sizeof out->rejected, "%s", rejected.c_str());
}

// Keeps what a call launched as the device's last selection.
void keep_selection(Device* d, const char* op, const LaunchRecord& rec, const std::string& reason,
                    const std::string& rejected) {
    std::lock_guard<std::mutex> lk(d->mu);
    d->sel_valid = true;
    d->sel_op = op;
    d->sel_kernel = rec.joined();
    d->sel_reason = reason;
    d->sel_rejected = rejected;
}

// The shared core of Int4MatVec, Int4MatMul and Int4Linear once validated.
// `ep` is the fused epilogue (bias, bf16 result); bf16 activations always
// give a bf16 result.  The launches made are kept as the device's last
// selection.
int run_int4_product(Device* d, hipStream_t st, const char* op, const void* a, int32_t dtype,
                     const accel_int4_t* w, void* out, int M, int K, int N,
                     Epilogue ep = Epilogue{}) {
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    const Int4Choice c = choose_int4(dtype, a, w->codes, M, K, N);
    LaunchRecord rec(false);
    const hipError_t e = launch_int4_route(d, st, c.route, a, planes(w), out, M, K, N, ep,
                                           &status);
    keep_selection(d, op, rec, c.reason, join(c.rejected, "; "));
    return finish(d, e, status, "int4 product launch");
}

}  // namespace

// Int4MatVec's checks (tensor/int4.go:99-147); on success fills K and N.
static int check_matvec(const char* op, const accel_tensor_t* a, const accel_int4_t* w,
                        const accel_tensor_t* out, int64_t* K, int64_t* N);

ACCEL_API int accel_int4_matvec(int dev, void* stream, const accel_tensor_t* a,
                                const accel_int4_t* w, accel_tensor_t* out) {
    clear_error();
    int64_t k = 0, n = 0;
    const int rc = check_matvec("Int4MatVec", a, w, out, &k, &n);
    if (rc != ACCEL_OK) return rc;
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    return run_int4_product(d, (hipStream_t)stream, "Int4MatVec", a->data, ACCEL_F32, w,
                            out->data, 1, (int)k, (int)n);
}

// BASELINE config 1's literal format (32-row groups along K, f32 scale, no
// zero): no counterpart in the reference; Int4MatVec's checks on a and out.
ACCEL_API int accel_int4_g32_matvec(int dev, void* stream, const accel_tensor_t* a,
                                    const accel_int4_g32_t* w, accel_tensor_t* out) {
    clear_error();
    const char* op = "Int4G32MatVec";
    if (!w || !w->codes || !w->scales) return refuse(op, "the weight matrix is missing");
    if (!valid_tensor(a) || !a->data) return refuse(op, "the activations are missing");
    char buf[256];
    if (a->dtype != ACCEL_F32 || a->rank != 1) {
        snprintf(buf, sizeof buf, "activations are %s %s; this kernel reads an f32 vector",
                 dtype_name(a->dtype), shape_str(a).c_str());
        return refuse(op, buf);
    }
    const int64_t K = w->K, N = w->N;
    if (a->shape[0] != K) {
        snprintf(buf, sizeof buf, "activations are %lld long and the matrix is [%lld, %lld]",
                 (long long)a->shape[0], (long long)K, (long long)N);
        return refuse(op, buf);
    }
    if (K > INT32_MAX || N > INT32_MAX || !int4_g32_matvec_supported((int)K, (int)N)) {
        snprintf(buf, sizeof buf,
                 "[%lld, %lld]: this kernel takes K a multiple of 32 and N of 256",
                 (long long)K, (long long)N);
        return refuse(op, buf);
    }
    if (((reinterpret_cast<uintptr_t>(w->codes) | reinterpret_cast<uintptr_t>(w->scales) |
          reinterpret_cast<uintptr_t>(a->data)) & 15) != 0)
        return refuse(op, "codes, scales and activations must be 16-byte aligned");
    int rc = check_out(op, out, ACCEL_F32, 1, N, true);
    if (rc != ACCEL_OK) return rc;
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    const hipError_t e = launch_int4_g32_matvec(
        d, (hipStream_t)stream, static_cast<const float*>(a->data), w->codes, w->scales,
        static_cast<float*>(out->data), (int)K, (int)N, &status);
    return finish(d, e, status, "Int4G32MatVec launch");
}

// Int4MatVec without allocating: the same checks and kernels, with the
// split-K buffers in the library's static scratch.
ACCEL_API int accel_int4_matvec_noalloc(int dev, void* stream, const accel_tensor_t* a,
                                        const accel_int4_t* w, accel_tensor_t* out) {
    clear_error();
    int64_t k = 0, n = 0;
    const int rc = check_matvec("Int4MatVecNoAlloc", a, w, out, &k, &n);
    if (rc != ACCEL_OK) return rc;
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    if (n == 0) return ACCEL_OK;
    LaunchRecord rec(false);
    const hipError_t e = launch_int4_matvec_noalloc(
        d, (hipStream_t)stream, static_cast<const float*>(a->data), planes(w),
        static_cast<float*>(out->data), (int)k, (int)n, &status);
    keep_selection(d, "Int4MatVecNoAlloc", rec,
                   "Int4MatVec's kernels and plan, the split-K sums in the static scratch",
                   "the workspace: it may call hipMalloc to grow");
    return finish(d, e, status, "Int4MatVecNoAlloc launch");
}

const char* const kSetReason =
    "matrices that share their input and all take the decode kernels: one launch per tile "
    "width, each matrix with its own launch's plan, so each result is its own product's";

// Int4MatVec over several matrices that share one input vector, in one
// launch where they all take the decode kernel (the q, k, v or gate, up
// products of a decode step); each result is its own Int4MatVec's.
ACCEL_API int accel_int4_matvec_set(int dev, void* stream, const accel_tensor_t* a,
                                    const accel_int4_t* w, accel_tensor_t* out, int count) {
    clear_error();
    const char* op = "Int4MatVecSet";
    if (count < 1 || count > 4 || !w || !out) {
        char buf[160];
        snprintf(buf, sizeof buf, "%d matrices; a set holds one to four", count);
        return refuse(op, buf);
    }
    int64_t K = 0;
    int N[4];
    Int4Planes p[4];
    float* o[4];
    for (int i = 0; i < count; i++) {
        int64_t k = 0, n = 0;
        const int rc = check_matvec(op, a, &w[i], &out[i], &k, &n);
        if (rc != ACCEL_OK) return rc;
        K = k;
        N[i] = (int)n;
        p[i] = planes(&w[i]);
        o[i] = static_cast<float*>(out[i].data);
    }
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    hipStream_t st = (hipStream_t)stream;
    if (!int4_matvec_set_supported(p, N, count, (int)K)) {
        for (int i = 0; i < count; i++) {
            const int rc = run_int4_product(d, st, "Int4MatVec", a->data, ACCEL_F32, &w[i],
                                            out[i].data, 1,
                                            (int)K, N[i]);
            if (rc != ACCEL_OK) return rc;
        }
        return ACCEL_OK;
    }
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    LaunchRecord rec(false);
    hipError_t e = launch_int4_matvec_set(d, st, static_cast<const float*>(a->data), p, o, N,
                                          count, (int)K, &status);
    keep_selection(d, op, rec, kSetReason, "one Int4MatVec launch per matrix: each would read "
                   "the shared vector and pay its own launch");
    return finish(d, e, status, "Int4MatVecSet launch");
}

// Int4MatMul over several matrices that share one f32 activation block
// [M, K]: one launch per tile width where they all take the matrix-core
// decode kernel (2 <= M <= 16), each with its own launch's plan, so each
// result is its own Int4MatMul's; else one Int4MatMul each.
ACCEL_API int accel_int4_matmul_set(int dev, void* stream, const accel_tensor_t* a,
                                    const accel_int4_t* w, accel_tensor_t* out, int count) {
    clear_error();
    const char* op = "Int4MatMulSet";
    char buf[320];
    if (count < 1 || count > 4 || !w || !out) {
        snprintf(buf, sizeof buf, "%d matrices; a set holds one to four", count);
        return refuse(op, buf);
    }
    if (!valid_tensor(a) || !a->data) return refuse(op, "the activations are missing");
    if (a->dtype != ACCEL_F32 || a->rank != 2) {
        snprintf(buf, sizeof buf, "activations are %s %s; a set takes f32 rows [M, K]",
                 dtype_name(a->dtype), shape_str(a).c_str());
        return refuse(op, buf);
    }
    const int64_t m = a->shape[0], k = a->shape[1];
    int N[4];
    Int4Planes p[4];
    float* o[4];
    for (int i = 0; i < count; i++) {
        std::string why = check_int4(&w[i], "the weight matrix");
        if (!why.empty()) return refuse(op, why);
        if (k == 0 || w[i].weights % k != 0) {
            snprintf(buf, sizeof buf,
                     "activations are %lld wide and matrix %d holds %lld weights; the matrix is "
                     "[K, N] with K the activation width, so the second is a multiple of the "
                     "first",
                     (long long)k, i, (long long)w[i].weights);
            return refuse(op, buf);
        }
        const int64_t n = w[i].weights / k;
        if (m > INT32_MAX || k > INT32_MAX || n > INT32_MAX)
            return refuse(op, "the product is larger than this backend's 32-bit extents");
        const int rc = check_out(op, &out[i], ACCEL_F32, m, n, false);
        if (rc != ACCEL_OK) return rc;
        N[i] = (int)n;
        p[i] = planes(&w[i]);
        o[i] = static_cast<float*>(out[i].data);
    }
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    hipStream_t st = (hipStream_t)stream;
    const float* af = static_cast<const float*>(a->data);
    if (m == 1 && int4_matvec_set_supported(p, N, count, (int)k)) {
        int status = begin_submission(d);
        if (status != ACCEL_OK) return status;
        LaunchRecord rec(false);
        hipError_t e = launch_int4_matvec_set(d, st, af, p, o, N, count, (int)k, &status);
        keep_selection(d, op, rec, kSetReason, "one Int4MatMul launch per matrix: each would "
                       "read the shared rows and pay its own launch");
        return finish(d, e, status, "Int4MatMulSet launch");
    }
    if (int4_matmul_set_supported(af, p, N, count, (int)m, (int)k)) {
        int status = begin_submission(d);
        if (status != ACCEL_OK) return status;
        LaunchRecord rec(false);
        hipError_t e = launch_int4_matmul_set(d, st, af, p, o, N, count, (int)m, (int)k, &status);
        keep_selection(d, op, rec, kSetReason, "one Int4MatMul launch per matrix: each would "
                       "read the shared rows and pay its own launch");
        return finish(d, e, status, "Int4MatMulSet launch");
    }
    for (int i = 0; i < count; i++) {
        const int rc = run_int4_product(d, st, "Int4MatMul", a->data, ACCEL_F32, &w[i],
                                        out[i].data, (int)m,
                                        (int)k, N[i]);
        if (rc != ACCEL_OK) return rc;
    }
    return ACCEL_OK;
}

static int check_matvec(const char* op, const accel_tensor_t* a, const accel_int4_t* w,
                        const accel_tensor_t* out, int64_t* K, int64_t* N) {
    std::string why = check_int4(w, "the weight matrix");
    if (!why.empty()) return refuse(op, why);
    if (!valid_tensor(a) || !a->data) return refuse(op, "the activations are missing");
    char buf[512];
    if (a->dtype != ACCEL_F32) {
        snprintf(buf, sizeof buf, "activations are %s and this kernel reads f32",
                 dtype_name(a->dtype));
        return refuse(op, buf);
    }
    if (a->rank != 1) {
        snprintf(buf, sizeof buf,
                 "activations are %s; a matvec takes a vector, and a batch of them is the "
                 "tiled form, Int4MatMul",
                 shape_str(a).c_str());
        return refuse(op, buf);
    }
    const int64_t k = a->shape[0];
    if (k == 0 || w->weights % k != 0) {
        snprintf(buf, sizeof buf,
                 "activations are %lld long and the matrix holds %lld weights; the matrix is "
                 "[K, N] with K the activation width, so the second is a multiple of the "
                 "first",
                 (long long)k, (long long)w->weights);
        return refuse(op, buf);
    }
    const int64_t n = w->weights / k;
    if (k > INT32_MAX || n > INT32_MAX)
        return refuse(op, "the matrix is larger than this backend's 32-bit extents");
    const int rc = check_out(op, out, ACCEL_F32, 1, n, true);
    if (rc != ACCEL_OK) return rc;
    *K = k;
    *N = n;
    return ACCEL_OK;
}

ACCEL_API int accel_int4_matmul(int dev, void* stream, const accel_tensor_t* a,
                                const accel_int4_t* w, accel_tensor_t* out) {
    clear_error();
    const char* op = "Int4MatMul";
    std::string why = check_int4(w, "the weight matrix");
    if (!why.empty()) return refuse(op, why);
    if (!valid_tensor(a) || !a->data) return refuse(op, "the activations are missing");
    char buf[512];
    if (a->dtype != ACCEL_F32 && a->dtype != ACCEL_BF16) {
        snprintf(buf, sizeof buf, "activations are %s and this kernel reads f32 (or bf16)",
                 dtype_name(a->dtype));
        return refuse(op, buf);
    }
    if (a->rank != 2) {
        snprintf(buf, sizeof buf,
                 "activations are %s; this is the batched form and takes [rows, K]. One row "
                 "is Int4MatVec, which is the decode shape and reads the matrix once per token",
                 shape_str(a).c_str());
        return refuse(op, buf);
    }
    const int64_t m = a->shape[0], k = a->shape[1];
    if (k == 0 || w->weights % k != 0) {
        snprintf(buf, sizeof buf,
                 "activations are %lld wide and the matrix holds %lld weights; the matrix is "
                 "[K, N] with K the activation width, so the second is a multiple of the "
                 "first",
                 (long long)k, (long long)w->weights);
        return refuse(op, buf);
    }
    const int64_t n = w->weights / k;
    if (m > INT32_MAX || k > INT32_MAX || n > INT32_MAX)
        return refuse(op, "the product is larger than this backend's 32-bit extents");
    int rc = check_out(op, out, a->dtype, m, n, false);
    if (rc != ACCEL_OK) return rc;
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    return run_int4_product(d, (hipStream_t)stream, "Int4MatMul", a->data, a->dtype, w,
                            out->data, (int)m, (int)k, (int)n);
}

// The int4 analogue of tensor.Linear (tensor/matmul.go:184-225): the
// product and a per-column f32 bias in one kernel, the bias added while the
// sums are still in registers, and, for f32 activations, an f32 or bf16
// result.  The composed form (Int4MatMul, then an add and a cast) is the
// reference the fused one is checked against.
ACCEL_API int accel_int4_linear(int dev, void* stream, const accel_tensor_t* x,
                                const accel_int4_t* w, const accel_tensor_t* bias,
                                accel_tensor_t* out) {
    clear_error();
    const char* op = "Int4Linear";
    std::string why = check_int4(w, "the weight matrix");
    if (!why.empty()) return refuse(op, why);
    if (!valid_tensor(x) || !x->data) return refuse(op, "the activations are missing");
    char buf[512];
    if (x->dtype != ACCEL_F32 && x->dtype != ACCEL_BF16) {
        snprintf(buf, sizeof buf, "activations are %s and this kernel reads f32 (or bf16)",
                 dtype_name(x->dtype));
        return refuse(op, buf);
    }
    if (x->rank != 1 && x->rank != 2) {
        snprintf(buf, sizeof buf,
                 "activations are %s; the fused product takes one vector [K] or rows [M, K]",
                 shape_str(x).c_str());
        return refuse(op, buf);
    }
    const bool vector = x->rank == 1;
    const int64_t m = vector ? 1 : x->shape[0], k = x->shape[x->rank - 1];
    if (k == 0 || w->weights % k != 0) {
        snprintf(buf, sizeof buf,
                 "activations are %lld wide and the matrix holds %lld weights; the matrix is "
                 "[K, N] with K the activation width, so the second is a multiple of the "
                 "first",
                 (long long)k, (long long)w->weights);
        return refuse(op, buf);
    }
    const int64_t n = w->weights / k;
    if (m > INT32_MAX || k > INT32_MAX || n > INT32_MAX)
        return refuse(op, "the product is larger than this backend's 32-bit extents");
    // the bias (matmul.go:211-218); no bias tensor at all is a product whose
    // epilogue only narrows
    if (bias) {
        if (!valid_tensor(bias) || !bias->data)
            return refuse(op, "the bias tensor has no data; a product without a bias passes "
                              "no bias tensor");
        if (bias->dtype != ACCEL_F32) {
            snprintf(buf, sizeof buf, "the bias is %s and the epilogue adds in f32",
                     dtype_name(bias->dtype));
            return refuse(op, buf);
        }
        if (bias->rank != 1 || bias->shape[0] != n) {
            snprintf(buf, sizeof buf,
                     "the bias is %s and the output is %lld wide; a bias is one value per "
                     "output column",
                     shape_str(bias).c_str(), (long long)n);
            return refuse(op, buf);
        }
    }
    if (!valid_tensor(out) || !out->data) return refuse(op, "the output tensor is missing");
    if (out->dtype != ACCEL_F32 && out->dtype != ACCEL_BF16) {
        snprintf(buf, sizeof buf, "the output is %s and the epilogue writes f32 or bf16",
                 dtype_name(out->dtype));
        return refuse(op, buf);
    }
    if (x->dtype == ACCEL_BF16 && out->dtype != ACCEL_BF16)
        return refuse(op, "the output is f32 and bf16 activations give a bf16 result");
    int rc = check_out(op, out, out->dtype, m, n, vector);
    if (rc != ACCEL_OK) return rc;
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    Epilogue ep;
    ep.bias = bias ? static_cast<const float*>(bias->data) : nullptr;
    ep.bf16 = out->dtype == ACCEL_BF16;
    return run_int4_product(d, (hipStream_t)stream, "Int4Linear", x->data, x->dtype, w,
                            out->data, (int)m, (int)k, (int)n, ep);
}

ACCEL_API int accel_segment_offsets(int dev, void* stream, const accel_tensor_t* counts,
                                    accel_tensor_t* offsets) {
    clear_error();
    const char* op = "SegmentOffsets";
    if (!valid_tensor(counts) || !counts->data) return refuse(op, "counts is nil");
    if (counts->dtype != ACCEL_U32) return refuse(op, "counts must be u32");
    const int64_t rows = elements(counts);
    if (!valid_tensor(offsets) || !offsets->data || offsets->dtype != ACCEL_U32 ||
        elements(offsets) != rows + 1)
        return refuse(op, "offsets must be u32 with one more entry than counts");
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    hipError_t e = launch_segment_offsets((hipStream_t)stream,
                                          static_cast<const uint32_t*>(counts->data),
                                          static_cast<uint32_t*>(offsets->data), (int)rows);
    return classify(d, e, "SegmentOffsets launch");
}

namespace {

// Shape checks shared by the two grouped operators (tensor/grouped.go:48-96).
// On success fills T, K, N, E.
int check_grouped(const char* op, const accel_tensor_t* x, const accel_tensor_t* w,
                  const accel_tensor_t* counts, int64_t* T, int64_t* K, int64_t* N,
                  int64_t* E) {
    char buf[512];
    if (!valid_tensor(counts) || !counts->data)
        return refuse(op, "counts is nil; it is one token count per expert and is what says "
                          "which rows belong to which weight matrix");
    if (!valid_tensor(x) || !x->data || !valid_tensor(w) || !w->data)
        return refuse(op, "an operand is missing");
    struct {
        const char* name;
        const accel_tensor_t* t;
        int32_t want;
    } cs[] = {{"x", x, ACCEL_F32}, {"w", w, ACCEL_F32}, {"counts", counts, ACCEL_U32}};
    for (auto& c : cs)
        if (c.t->dtype != c.want) {
            snprintf(buf, sizeof buf, "%s is %s and this kernel reads %s", c.name,
                     dtype_name(c.t->dtype), dtype_name(c.want));
            return refuse(op, buf);
        }
    if (x->rank != 2) {
        snprintf(buf, sizeof buf,
                 "x is %s; it is [tokens, K] with the tokens of every expert end to end",
                 shape_str(x).c_str());
        return refuse(op, buf);
    }
    if (w->rank != 3) {
        snprintf(buf, sizeof buf, "w is %s; it is [experts, K, N], one matrix per expert",
                 shape_str(w).c_str());
        return refuse(op, buf);
    }
    *T = x->shape[0];
    *K = x->shape[1];
    *E = w->shape[0];
    *N = w->shape[2];
    if (w->shape[1] != *K) {
        snprintf(buf, sizeof buf,
                 "x is %s and w is %s; every expert contracts against the same width, so w's "
                 "second axis is x's second",
                 shape_str(x).c_str(), shape_str(w).c_str());
        return refuse(op, buf);
    }
    if (elements(counts) != *E) {
        snprintf(buf, sizeof buf,
                 "counts holds %lld entries and w has %lld experts; it is one token count per "
                 "expert",
                 (long long)elements(counts), (long long)*E);
        return refuse(op, buf);
    }
    if (*E == 0) return refuse(op, "w declares no experts");
    return ACCEL_OK;
}

// Offsets for `experts` counts into the workspace; returns the device
// pointer or nullptr with status set.  The workspace is laid out as its
// counters, the offsets [experts + 1] (rounded up to 256 bytes), then
// `area_bytes` for the product's own sums (*area, when asked for).  It is
// sized for all of that here, once, before the offsets are written, so no
// later request can grow it and move them.
uint32_t* offsets_in_workspace(Device* d, hipStream_t st, const uint32_t* counts,
                               int64_t experts, int* status, size_t area_bytes = 0,
                               void** area = nullptr) {
    const size_t off_bytes = ((size_t)(experts + 1) * sizeof(uint32_t) + 255) / 256 * 256;
    void* ws = workspace(d, st, off_bytes + area_bytes, status);
    if (!ws) return nullptr;
    char* data = static_cast<char*>(ws) + kWorkspaceCounterBytes;
    uint32_t* off = reinterpret_cast<uint32_t*>(data);
    if (area) *area = area_bytes ? data + off_bytes : nullptr;
    hipError_t e = launch_segment_offsets(st, counts, off, (int)experts);
    if (e != hipSuccess) {
        *status = classify(d, e, "SegmentOffsets launch");
        return nullptr;
    }
    return off;
}

int run_grouped_f32(const char* op, int dev, void* stream, const accel_tensor_t* x,
                    const accel_tensor_t* w, const accel_tensor_t* counts, accel_tensor_t* out,
                    bool matvec) {
    clear_error();
    int64_t T, K, N, E;
    int rc = check_grouped(op, x, w, counts, &T, &K, &N, &E);
    if (rc != ACCEL_OK) return rc;
    rc = check_out(op, out, ACCEL_F32, T, N, false);
    if (rc != ACCEL_OK) return rc;
    if (T > INT32_MAX || K > INT32_MAX || N > INT32_MAX || E > INT32_MAX)
        return refuse(op, "the product is larger than this backend's 32-bit extents");
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    hipStream_t st = (hipStream_t)stream;
    uint32_t* off = offsets_in_workspace(d, st, static_cast<const uint32_t*>(counts->data), E,
                                         &status);
    if (!off) return status;
    hipError_t e = launch_grouped_f32(st, static_cast<const float*>(x->data),
                                      static_cast<const float*>(w->data), off,
                                      static_cast<float*>(out->data), (int)E, (int)T, (int)K,
                                      (int)N, matvec);
    return classify(d, e, "grouped launch");
}

int run_grouped_int4(const char* op, int dev, void* stream, const accel_tensor_t* x,
                     const accel_int4_t* w, int64_t experts, const accel_tensor_t* counts,
                     accel_tensor_t* out, bool matvec, const uint16_t* side = nullptr,
                     const void* panels = nullptr, size_t panel_stride = 0) {
    clear_error();
    char buf[512];
    std::string why = check_int4(w, "the expert weights");
    if (!why.empty()) return refuse(op, why);
    if (!valid_tensor(counts) || !counts->data)
        return refuse(op, "counts is nil; it is one token count per expert and is what says "
                          "which rows belong to which weight matrix");
    if (counts->dtype != ACCEL_U32) {
        snprintf(buf, sizeof buf, "counts is %s and this kernel reads u32",
                 dtype_name(counts->dtype));
        return refuse(op, buf);
    }
    if (!valid_tensor(x) || !x->data) return refuse(op, "x is missing");
    if (x->dtype != ACCEL_F32 && x->dtype != ACCEL_BF16) {
        snprintf(buf, sizeof buf, "x is %s and this kernel reads f32 (or bf16)",
                 dtype_name(x->dtype));
        return refuse(op, buf);
    }
    if (x->rank != 2) {
        snprintf(buf, sizeof buf,
                 "x is %s; it is [tokens, K] with the tokens of every expert end to end",
                 shape_str(x).c_str());
        return refuse(op, buf);
    }
    if (experts <= 0) return refuse(op, "w declares no experts");
    if (elements(counts) != experts) {
        snprintf(buf, sizeof buf,
                 "counts holds %lld entries and w has %lld experts; it is one token count per "
                 "expert",
                 (long long)elements(counts), (long long)experts);
        return refuse(op, buf);
    }
    const int64_t T = x->shape[0], K = x->shape[1];
    if (K == 0 || w->weights % (experts * K) != 0) {
        snprintf(buf, sizeof buf,
                 "x is %lld wide and the %lld experts hold %lld weights; each expert is [K, N] "
                 "with K x's width",
                 (long long)K, (long long)experts, (long long)w->weights);
        return refuse(op, buf);
    }
    const int64_t N = w->weights / (experts * K);
    if ((K * N) % 128 != 0)
        return refuse(op, "each expert's K*N must be a multiple of 128, so no quantisation "
                          "group straddles two experts");
    if (T > INT32_MAX || K > INT32_MAX || N > INT32_MAX || experts > INT32_MAX ||
        (uint64_t)w->weights >= (1ull << 40))
        return refuse(op, "the product is larger than this backend's extents");
    int rc = check_out(op, out, x->dtype, T, N, false);
    if (rc != ACCEL_OK) return rc;
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    hipStream_t st = (hipStream_t)stream;
    // the path, and the workspace it needs past the offsets
    const bool f32 = x->dtype == ACCEL_F32;
    if (!f32 && !(int4_gemm_bf16_supported(1, (int)K, (int)N) &&
                  (reinterpret_cast<uintptr_t>(x->data) & 15) == 0))
        return refuse(op, "bf16 grouped products need K % 64 == 0, N % 128 == 0, K < 2^22 and "
                          "N < 2^26");
    // many f32 rows: the f32 matrix-core tiles; few routed rows (f32 or
    // bf16): the decode kernels; the rest of bf16: the bf16 tiles
    const bool tiles_f32 = f32 && T > kGroupedDecodeRowsF32 &&
                           int4_gemm_f32x3_supported((int)K, (int)N) &&
                           (reinterpret_cast<uintptr_t>(x->data) & 15) == 0 &&
                           (uint64_t)experts * (uint64_t)K * (uint64_t)N < (1ull << 40);
    const bool decode = !tiles_f32 &&
                        int4_grouped_decode_supported((int)T, (int)K, (int)N, w->codes, !f32) &&
                        (uint64_t)experts * (uint64_t)K * (uint64_t)N < (1ull << 40);
    const bool tiles = tiles_f32 || (!decode && !f32);
    // prepared experts: the matrix-core decode reads their side copies
    Int4Planes p = planes(w);
    p.side = side;
    p.panels = panels;
    p.panel_stride = panel_stride;
    // the tiles walk segments: the matvec form's rows follow e(t), whose
    // bounds are the offsets sorted (segment_bounds), in the area
    const size_t bounds_bytes = ((size_t)(experts + 1) * sizeof(uint32_t) + 255) / 256 * 256;
    const size_t area_bytes =
        decode ? int4_grouped_decode_area(d, x->data, !f32, p, (int)experts, (int)T, (int)K,
                                          (int)N)
               : (tiles && matvec ? bounds_bytes : 0);
    void* area = nullptr;
    uint32_t* off = offsets_in_workspace(d, st, static_cast<const uint32_t*>(counts->data),
                                         experts, &status, area_bytes, &area);
    if (!off) return status;
    uint32_t* tickets = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(off) -
                                                    kWorkspaceCounterBytes);
    hipError_t e = hipSuccess;
    const uint32_t* seg = off;
    LaunchRecord rec(false);
    std::string reason, rejected;
    if (decode && grouped_panel_route(x->data, p, !f32, (int)experts, (int)T, (int)K)) {
        reason = "few routed f32 rows of experts prepared into the panel layout: workgroup "
                 "(expert, 16-column panel) runs the expert's rows over all of K in passes of "
                 "up to four, no K split and no hand-off (the VALU decode kernel for the "
                 "padding rows, on the planes)";
        rejected = "the matrix-core blocks: their time is set by load latency, the K split "
                   "and its hand-off at one to four rows an expert; the grouped tiles: a "
                   "128- or 256-row block for a few rows would be mostly empty";
    } else if (decode && side) {
        reason = "few routed rows of prepared experts: each expert's rows in blocks of up to "
                 "16 on the matrix-core decode kernel, each 32-row step's scales and zeros "
                 "one contiguous block of the expert's side copy (the VALU decode kernel for "
                 "the rest, on the planes)";
        rejected = "the grouped tiles: a 128- or 256-row block for a few rows would be "
                   "mostly empty; the reference planes: a step's scales and zeros are a piece "
                   "of each of its 32 rows of the two planes";
    } else if (decode) {
        reason = "few routed rows: each expert's rows in blocks of up to 16 on the "
                 "matrix-core decode kernel (and the VALU decode kernel for the rest), the "
                 "weights read once a block";
        rejected = "the grouped tiles: a 128- or 256-row block for a few rows would be "
                   "mostly empty";
    } else if (tiles_f32) {
        reason = "f32 rows: the f32 matrix-core tiles (x*512s in three bf16 terms) walking "
                 "each expert's 128-row blocks";
        rejected = "the decode kernels: they take at most 1024 f32 rows";
    } else if (f32) {
        reason = "no tiled kernel takes this shape or alignment: one lane per (row, column)";
        rejected = "the f32 matrix-core tiles: they take K % 64 == 0, N % 128 == 0 and "
                   "16-byte aligned rows; the decode kernels: at most 1024 rows";
    } else {
        reason = "bf16 rows: the matrix-core tiles walking each expert's blocks of up to 256 "
                 "rows";
        rejected = "the decode kernels: they take at most 64 bf16 rows";
    }
    if (tiles && matvec) {
        uint32_t* bounds = static_cast<uint32_t*>(area);
        e = launch_segment_bounds(st, off, bounds, (int)experts);
        seg = bounds;
    }
    if (e != hipSuccess) {
    } else if (decode) {
        e = launch_int4_grouped_decode(d, st, x->data, !f32, p, off, out->data, (int)experts,
                                       (int)T, (int)K, (int)N, matvec, &status, tickets,
                                       static_cast<float*>(area));
        if (e == hipSuccess && status != ACCEL_OK) return status;
    } else if (tiles_f32) {
        e = launch_int4_grouped_f32x3(st, static_cast<const float*>(x->data), p, seg,
                                      static_cast<float*>(out->data), (int)experts, (int)T,
                                      (int)K, (int)N);
        if (e == hipSuccess && matvec)
            e = launch_zero_tail_f32(st, seg, static_cast<float*>(out->data), (int)experts,
                                     (int)T, (int)N);
    } else if (f32) {
        e = launch_int4_grouped_f32(st, static_cast<const float*>(x->data), p, off,
                                    static_cast<float*>(out->data), (int)experts, (int)T,
                                    (int)K, (int)N, matvec);
    } else {
        e = launch_int4_grouped_bf16(d, st, static_cast<const uint16_t*>(x->data), p, seg,
                                     static_cast<uint16_t*>(out->data), (int)experts, (int)T,
                                     (int)K, (int)N, matvec);
        if (e == hipSuccess && matvec)
            e = launch_zero_tail_bf16(st, seg, static_cast<uint16_t*>(out->data),
                                      (int)experts, (int)T, (int)N);
    }
    keep_selection(d, op, rec, reason, rejected);
    return classify(d, e, "grouped int4 launch");
}

}  // namespace

ACCEL_API int accel_grouped_matvec(int dev, void* stream, const accel_tensor_t* x,
                                   const accel_tensor_t* w, const accel_tensor_t* counts,
                                   accel_tensor_t* out) {
    return run_grouped_f32("GroupedMatVec", dev, stream, x, w, counts, out, true);
}

ACCEL_API int accel_grouped_matmul(int dev, void* stream, const accel_tensor_t* x,
                                   const accel_tensor_t* w, const accel_tensor_t* counts,
                                   accel_tensor_t* out) {
    return run_grouped_f32("GroupedMatMul", dev, stream, x, w, counts, out, false);
}

ACCEL_API int accel_int4_grouped_matvec(int dev, void* stream, const accel_tensor_t* x,
                                        const accel_int4_t* w, int64_t experts,
                                        const accel_tensor_t* counts, accel_tensor_t* out) {
    return run_grouped_int4("Int4GroupedMatVec", dev, stream, x, w, experts, counts, out,
                            true);
}

ACCEL_API int accel_int4_grouped_matmul(int dev, void* stream, const accel_tensor_t* x,
                                        const accel_int4_t* w, int64_t experts,
                                        const accel_tensor_t* counts, accel_tensor_t* out) {
    return run_grouped_int4("Int4GroupedMatMul", dev, stream, x, w, experts, counts, out,
                            false);
}

ACCEL_API int accel_int4_quantize_device(int dev, void* stream, const float* w, int64_t n,
                                         uint32_t* packed, uint16_t* scales, uint16_t* zeros) {
    clear_error();
    if (n < 0) return fail(ACCEL_E_INVALID, "accel_int4_quantize_device: negative count");
    if (n == 0) return ACCEL_OK;
    if (!w || !packed || !scales || !zeros)
        return fail(ACCEL_E_INVALID, "accel_int4_quantize_device: NULL pointer");
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    return classify(d, launch_int4_quantize((hipStream_t)stream, w, n, packed, scales, zeros),
                    "quantize launch");
}

// ---- decode-step neighbours -------------------------------------------------

namespace {

bool same_shape(const accel_tensor_t* a, const accel_tensor_t* b) {
    if (a->rank != b->rank) return false;
    for (int i = 0; i < a->rank; i++)
        if (a->shape[i] != b->shape[i]) return false;
    return true;
}

}  // namespace

// tensor.SwiGLU (tensor/elementwise.go:161-188) over the registered f32
// kernel: gate, value and out share one shape.
ACCEL_API int accel_swiglu(int dev, void* stream, const accel_tensor_t* gate,
                           const accel_tensor_t* value, accel_tensor_t* out) {
    clear_error();
    const char* op = "SwiGLU";
    char buf[256];
    if (!valid_tensor(gate) || !gate->data || !valid_tensor(value) || !value->data)
        return refuse(op, "an operand is missing");
    if (gate->dtype != value->dtype) {
        snprintf(buf, sizeof buf, "operands are %s and %s", dtype_name(gate->dtype),
                 dtype_name(value->dtype));
        return refuse(op, buf);
    }
    if (gate->dtype != ACCEL_F32) {
        snprintf(buf, sizeof buf, "%s has no SwiGLU kernel here; the registered kernel reads f32",
                 dtype_name(gate->dtype));
        return refuse(op, buf);
    }
    if (!same_shape(gate, value)) {
        snprintf(buf, sizeof buf,
                 "shapes %s and %s differ; the fused kernel indexes both operands together, so "
                 "broadcasting one would need the composed form",
                 shape_str(gate).c_str(), shape_str(value).c_str());
        return refuse(op, buf);
    }
    if (!valid_tensor(out) || !out->data || out->dtype != ACCEL_F32 || !same_shape(out, gate))
        return refuse(op, "the output must be f32 with the operands' shape");
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    hipError_t e = launch_swiglu((hipStream_t)stream, static_cast<const float*>(gate->data),
                                 static_cast<const float*>(value->data),
                                 static_cast<float*>(out->data), elements(gate));
    return classify(d, e, "SwiGLU launch");
}

// tensor.RMSNorm (tensor/ops.go:105-135): x f32 of any rank >= 1, gain f32
// [width] with width x's last axis, eps positive and finite.
ACCEL_API int accel_rmsnorm(int dev, void* stream, const accel_tensor_t* x,
                            const accel_tensor_t* gain, float eps, accel_tensor_t* out) {
    clear_error();
    const char* op = "RMSNorm";
    char buf[256];
    if (!valid_tensor(x) || !x->data || !valid_tensor(gain) || !gain->data)
        return refuse(op, "an operand is missing");
    if (x->dtype != ACCEL_F32 || gain->dtype != ACCEL_F32) {
        snprintf(buf, sizeof buf,
                 "x is %s and gain is %s; the registered kernel reads f32",
                 dtype_name(x->dtype), dtype_name(gain->dtype));
        return refuse(op, buf);
    }
    if (x->rank < 1) return refuse(op, "x has no shape");
    const int64_t width = x->shape[x->rank - 1];
    if (gain->rank != 1 || gain->shape[0] != width) {
        snprintf(buf, sizeof buf,
                 "gain is %s and x's last axis is %lld; the gain is one value per feature",
                 shape_str(gain).c_str(), (long long)width);
        return refuse(op, buf);
    }
    if (!(eps > 0) || !(eps < INFINITY)) {
        snprintf(buf, sizeof buf,
                 "eps is %g and must be positive and finite: it is what keeps a row of zeros "
                 "from dividing by zero",
                 (double)eps);
        return refuse(op, buf);
    }
    if (!valid_tensor(out) || !out->data || out->dtype != ACCEL_F32 || !same_shape(out, x))
        return refuse(op, "the output must be f32 with x's shape");
    const int64_t rows = width ? elements(x) / width : 0;
    if (width > INT32_MAX || rows > INT32_MAX)
        return fail(ACCEL_E_UNSUPPORTED, "accel/tensor: RMSNorm: %lld rows of %lld are more than "
                    "this kernel's 32-bit grid indexes", (long long)rows, (long long)width);
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    hipError_t e = launch_rmsnorm((hipStream_t)stream, static_cast<const float*>(x->data),
                                  static_cast<const float*>(gain->data),
                                  static_cast<float*>(out->data), (int)rows, (int)width, eps);
    return classify(d, e, "RMSNorm launch");
}

// tensor.MatMul's M = 1 selection for f32 activations against f16 weights
// (tensor/matmul.go:113-121 -> MatVecF32F16): x f32 [1,K] or [K], w f16
// [K,N] (raw f16 bits) -> out f32 [1,N] or [N].  Larger M selects the mixed
// tiled GEMM in the reference, which is not built here.
ACCEL_API int accel_matvec_f32_f16(int dev, void* stream, const accel_tensor_t* x,
                                   const accel_tensor_t* w, accel_tensor_t* out) {
    clear_error();
    const char* op = "MatMul";
    char buf[256];
    if (!valid_tensor(x) || !x->data || !valid_tensor(w) || !w->data)
        return refuse(op, "an operand is missing");
    if (x->dtype != ACCEL_F32 || w->dtype != ACCEL_F16) {
        snprintf(buf, sizeof buf,
                 "operands are %s and %s; this entry point is the f32-activation, f16-weight "
                 "pair", dtype_name(x->dtype), dtype_name(w->dtype));
        return refuse(op, buf);
    }
    if (w->rank != 2) return refuse(op, "w must be [K N]");
    const int64_t K = w->shape[0], N = w->shape[1];
    const bool vec = x->rank == 1;
    if (!(vec ? x->shape[0] == K : (x->rank == 2 && x->shape[1] == K))) {
        snprintf(buf, sizeof buf, "x is %s and w is %s; the inner dimensions must agree",
                 shape_str(x).c_str(), shape_str(w).c_str());
        return refuse(op, buf);
    }
    if (!vec && x->shape[0] != 1)
        return fail(ACCEL_E_UNSUPPORTED,
                    "accel/tensor: MatMul: x has %lld rows; the f32 x f16 product is built for "
                    "M = 1 (MatVecF32F16) only",
                    (long long)x->shape[0]);
    const int rc = check_out(op, out, ACCEL_F32, 1, N, vec);
    if (rc != ACCEL_OK) return rc;
    if (K > INT32_MAX || N > INT32_MAX)
        return fail(ACCEL_E_UNSUPPORTED, "accel/tensor: MatMul: dimensions past 2^31");
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    hipError_t e = launch_matvec_f32_f16(d, (hipStream_t)stream, static_cast<const float*>(x->data),
                                         static_cast<const uint16_t*>(w->data),
                                         static_cast<float*>(out->data), (int)K, (int)N, &status);
    return finish(d, e, status, "MatVecF32F16 launch");
}

// ---- int8 weights ------------------------------------------------------------

// tensor.QuantMatMul (tensor/quantized.go:72-163) with checkQuantized
// (:32-52): the reference's validation order and wording.
ACCEL_API int accel_quant_matmul(int dev, void* stream, const accel_tensor_t* x,
                                 const accel_tensor_t* quants, const accel_tensor_t* scales,
                                 accel_tensor_t* out) {
    clear_error();
    const char* op = "QuantMatMul";
    char buf[320];
    if (!valid_tensor(quants) || !quants->data || !valid_tensor(scales) || !scales->data)
        return refuse(op, "the weight needs both a quant plane and a scale plane");
    if (quants->dtype != ACCEL_I8) {
        snprintf(buf, sizeof buf, "the weight quants are %s and must be i8",
                 dtype_name(quants->dtype));
        return refuse(op, buf);
    }
    if (scales->dtype != ACCEL_F16) {
        snprintf(buf, sizeof buf, "the weight scales are %s and must be f16",
                 dtype_name(scales->dtype));
        return refuse(op, buf);
    }
    const int64_t nq = elements(quants);
    const int64_t want = (nq + 31) / 32;
    if (elements(scales) != want) {
        snprintf(buf, sizeof buf, "the weight has %lld quants, which is %lld blocks of 32, and "
                 "%lld scales", (long long)nq, (long long)want, (long long)elements(scales));
        return refuse(op, buf);
    }
    if (!valid_tensor(x) || !x->data) return refuse(op, "the activations are missing");
    if (x->dtype != ACCEL_F16 && x->dtype != ACCEL_F32) {
        snprintf(buf, sizeof buf, "activations are %s; specs/010-kernel-corpus.md registers f16 "
                 "and f32 activations against int8 weights", dtype_name(x->dtype));
        return refuse(op, buf);
    }
    if (x->rank != 2 || quants->rank != 2) {
        snprintf(buf, sizeof buf, "operands are %s and %s; v0 multiplies two matrices",
                 shape_str(x).c_str(), shape_str(quants).c_str());
        return refuse(op, buf);
    }
    if (x->shape[1] != quants->shape[0]) {
        snprintf(buf, sizeof buf, "%s times %s: the contracted axes are %lld and %lld",
                 shape_str(x).c_str(), shape_str(quants).c_str(), (long long)x->shape[1],
                 (long long)quants->shape[0]);
        return refuse(op, buf);
    }
    const int64_t M = x->shape[0], K = x->shape[1], N = quants->shape[1];
    const int rc = check_out(op, out, ACCEL_F32, M, N, false);
    if (rc != ACCEL_OK) return rc;
    if (M > INT32_MAX || K > INT32_MAX || N > INT32_MAX || (uint64_t)K * N >= (1ull << 40))
        return fail(ACCEL_E_UNSUPPORTED, "accel/tensor: QuantMatMul: dimensions past this "
                    "library's indexing");
    if (M == 0 || N == 0) return ACCEL_OK;
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    hipError_t e = launch_int8_product(d, (hipStream_t)stream, x->data, x->dtype == ACCEL_F16,
                                       static_cast<const int8_t*>(quants->data),
                                       static_cast<const uint16_t*>(scales->data),
                                       static_cast<float*>(out->data), (int)M, (int)K, (int)N,
                                       &status);
    return finish(d, e, status, "QuantMatMul launch");
}

// ---- backend seam: kernel records ------------------------------------------

namespace {

struct Record {
    const char* name;
    int bindings;
};
const Record kRecords[] = {
    {"QuantMatVecInt4", 5}, {"QuantMatMulInt4", 5}, {"GroupedMatVec", 4},
    {"GroupedMatMul", 4},   {"SegmentOffsets", 2},  {"SwiGLU", 3},
    {"RMSNorm", 3},         {"MatVecF32F16", 3},    {"QuantMatVecF32", 4},
    {"QuantMatVec", 4},     {"QuantMatMulTiledF32", 4}, {"QuantMatMulTiled", 4},
};

uint32_t u32_at(const void* p, size_t off) {
    uint32_t v;
    std::memcpy(&v, static_cast<const char*>(p) + off, 4);
    return v;
}

}  // namespace

// ---- prepared (bind-time) weights ----------------------------------------

// An Int4 weight bound once for one-row products: its planes copied into the
// K-major panel layout (panel.hip).  Owned by the caller; freed with
// accel_int4_prepared_free.
struct accel_int4_prepared {
    uint32_t magic;
    int dev;
    int64_t K, N;
    void* data;
    size_t bytes;
    int layout;        // kPanelLayout, kTilesLayout or kGroupedLayout
    size_t side_off;   // tiles, grouped: the side copy's offset in data
    int64_t experts = 0;                   // grouped: the expert count
    size_t scales_off = 0, zeros_off = 0;  // grouped: the planes' offsets in data
    size_t panel_stride = 0;               // grouped panels: bytes per expert's copy
};
static constexpr int kPanelLayout = 0;   // accel_int4_prepare: K-major panels
static constexpr int kTilesLayout = 1;   // accel_int4_prepare_tiles: codes + side copy
static constexpr int kGroupedLayout = 2;  // accel_int4_prepare_grouped: planes + side copies
static constexpr int kGroupedPanelLayout = 3;  // accel_int4_prepare_grouped_panels: planes +
                                               // each expert's panel copy
static constexpr uint32_t kPreparedMagic = 0x34544e49u;   // "INT4"
static bool is_grouped(const accel_int4_prepared_t* w) {
    return w->layout == kGroupedLayout || w->layout == kGroupedPanelLayout;
}

ACCEL_API int accel_int4_prepare(int dev, void* stream, const accel_int4_t* w, int64_t K,
                                 int64_t N, accel_int4_prepared_t** out) {
    clear_error();
    const char* op = "Int4Prepare";
    if (!out) return refuse(op, "no handle to return the prepared weight in");
    *out = nullptr;
    std::string why = check_int4(w, "the weight matrix");
    if (!why.empty()) return refuse(op, why);
    char buf[320];
    if (K < 1 || N < 1 || w->weights != K * N) {
        snprintf(buf, sizeof buf, "[%lld, %lld] is %lld weights and the matrix holds %lld",
                 (long long)K, (long long)N, (long long)(K * N), (long long)w->weights);
        return refuse(op, buf);
    }
    if (!int4_panel_supported(K, N)) {
        snprintf(buf, sizeof buf,
                 "[%lld, %lld]: the panel layout takes N a multiple of 128 (whole groups in "
                 "a row) and K, N below 2^30",
                 (long long)K, (long long)N);
        return refuse(op, buf);
    }
    if ((reinterpret_cast<uintptr_t>(w->codes) & 7) != 0)
        return refuse(op, "the code plane must be 8-byte aligned");
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    const size_t bytes = int4_panel_bytes((int)K, (int)N, nullptr);
    void* data = nullptr;
    hipError_t e = hipMalloc(&data, bytes);
    if (e != hipSuccess) return classify(d, e, "prepared weight allocation");
    hipStream_t st = (hipStream_t)stream;
    e = launch_int4_panel_prepare(st, planes(w), data, (int)K, (int)N);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipFree(data);
        return classify(d, e, "prepared weight copy");
    }
    auto* p = new accel_int4_prepared{kPreparedMagic, dev, K, N, data, bytes, kPanelLayout, 0};
    *out = p;
    return ACCEL_OK;
}

// The matrix-core decode's prepared form: the code plane copied as it is and
// a side copy of the scales and zeros, one contiguous block per (group,
// 32-row step) (int4_side_prepare_kernel).
ACCEL_API int accel_int4_prepare_tiles(int dev, void* stream, const accel_int4_t* w,
                                       int64_t K, int64_t N, accel_int4_prepared_t** out) {
    clear_error();
    const char* op = "Int4PrepareTiles";
    if (!out) return refuse(op, "no handle to return the prepared weight in");
    *out = nullptr;
    std::string why = check_int4(w, "the weight matrix");
    if (!why.empty()) return refuse(op, why);
    char buf[320];
    if (K < 1 || N < 1 || w->weights != K * N) {
        snprintf(buf, sizeof buf, "[%lld, %lld] is %lld weights and the matrix holds %lld",
                 (long long)K, (long long)N, (long long)(K * N), (long long)w->weights);
        return refuse(op, buf);
    }
    if (!int4_side_supported(K, N)) {
        snprintf(buf, sizeof buf,
                 "[%lld, %lld]: the matrix-core decode takes K a multiple of 32, N a multiple "
                 "of 128 and N below 2^27",
                 (long long)K, (long long)N);
        return refuse(op, buf);
    }
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    const size_t code_bytes = (size_t)K * N / 2;
    const size_t side_off = (code_bytes + 255) / 256 * 256;
    const size_t bytes = side_off + int4_side_bytes((int)K, (int)N);
    void* data = nullptr;
    hipError_t e = hipMalloc(&data, bytes);
    if (e != hipSuccess) return classify(d, e, "prepared weight allocation");
    hipStream_t st = (hipStream_t)stream;
    e = hipMemcpyAsync(data, w->codes, code_bytes, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess)
        e = launch_int4_side_prepare(st, planes(w),
                                     reinterpret_cast<uint16_t*>(static_cast<char*>(data) +
                                                                 side_off),
                                     (int)K, (int)N);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipFree(data);
        return classify(d, e, "prepared weight copy");
    }
    *out = new accel_int4_prepared{kPreparedMagic, dev, K, N, data, bytes, kTilesLayout,
                                   side_off};
    return ACCEL_OK;
}

// Grouped experts prepared for the matrix-core decode: the three planes
// copied as they are (the routes that read planes) and each expert's side
// copy of its scales and zeros (int4_side_prepare_kernel), end to end.
ACCEL_API int accel_int4_prepare_grouped(int dev, void* stream, const accel_int4_t* w,
                                         int64_t experts, int64_t K, int64_t N,
                                         accel_int4_prepared_t** out) {
    clear_error();
    const char* op = "Int4PrepareGrouped";
    if (!out) return refuse(op, "no handle to return the prepared weight in");
    *out = nullptr;
    std::string why = check_int4(w, "the expert weights");
    if (!why.empty()) return refuse(op, why);
    char buf[320];
    if (experts < 1 || K < 1 || N < 1 || w->weights / experts != K * N ||
        w->weights % experts != 0) {
        snprintf(buf, sizeof buf,
                 "%lld experts of [%lld, %lld] are %lld weights and the matrix holds %lld",
                 (long long)experts, (long long)K, (long long)N, (long long)(experts * K * N),
                 (long long)w->weights);
        return refuse(op, buf);
    }
    if (!int4_side_supported(K, N) || experts > INT32_MAX ||
        (uint64_t)w->weights >= (1ull << 40)) {
        snprintf(buf, sizeof buf,
                 "%lld experts of [%lld, %lld]: the matrix-core decode takes K a multiple of "
                 "32, N a multiple of 128, N below 2^27 and under 2^40 weights",
                 (long long)experts, (long long)K, (long long)N);
        return refuse(op, buf);
    }
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t per = (size_t)K * N;
    const size_t code_bytes = (size_t)w->weights / 2;
    const size_t plane_bytes = (size_t)w->weights / 128 * 2;
    const size_t side_per = int4_side_bytes((int)K, (int)N);
    const size_t scales_off = up(code_bytes);
    const size_t zeros_off = scales_off + up(plane_bytes);
    const size_t side_off = zeros_off + up(plane_bytes);
    const size_t bytes = side_off + side_per * (size_t)experts;
    void* data = nullptr;
    hipError_t e = hipMalloc(&data, bytes);
    if (e != hipSuccess) return classify(d, e, "prepared weight allocation");
    hipStream_t st = (hipStream_t)stream;
    char* base = static_cast<char*>(data);
    e = hipMemcpyAsync(base, w->codes, code_bytes, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(base + scales_off, w->scales, plane_bytes, hipMemcpyDeviceToDevice,
                           st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(base + zeros_off, w->zeros, plane_bytes, hipMemcpyDeviceToDevice,
                           st);
    for (int64_t i = 0; i < experts && e == hipSuccess; i++) {
        const Int4Planes pi{w->codes + i * (per >> 3), w->scales + i * (per >> 7),
                            w->zeros + i * (per >> 7)};
        e = launch_int4_side_prepare(st, pi,
                                     reinterpret_cast<uint16_t*>(base + side_off +
                                                                 side_per * (size_t)i),
                                     (int)K, (int)N);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipFree(data);
        return classify(d, e, "prepared weight copy");
    }
    auto* p = new accel_int4_prepared{kPreparedMagic, dev, K, N, data, bytes, kGroupedLayout,
                                      side_off};
    p->experts = experts;
    p->scales_off = scales_off;
    p->zeros_off = zeros_off;
    *out = p;
    return ACCEL_OK;
}

// Grouped experts prepared for few routed rows: the three planes copied as
// they are and, after them, each expert's copy in the panel layout
// (int4_panel_prepare_*_kernel), 256-byte aligned.
ACCEL_API int accel_int4_prepare_grouped_panels(int dev, void* stream, const accel_int4_t* w,
                                                int64_t experts, int64_t K, int64_t N,
                                                accel_int4_prepared_t** out) {
    clear_error();
    const char* op = "Int4PrepareGroupedPanels";
    if (!out) return refuse(op, "no handle to return the prepared weight in");
    *out = nullptr;
    std::string why = check_int4(w, "the expert weights");
    if (!why.empty()) return refuse(op, why);
    char buf[320];
    if (experts < 1 || K < 1 || N < 1 || w->weights % experts != 0 ||
        w->weights / experts != K * N) {
        snprintf(buf, sizeof buf,
                 "%lld experts of [%lld, %lld] are %lld weights and the matrix holds %lld",
                 (long long)experts, (long long)K, (long long)N, (long long)(experts * K * N),
                 (long long)w->weights);
        return refuse(op, buf);
    }
    if (!int4_panel_supported(K, N) || experts > INT32_MAX ||
        (uint64_t)w->weights >= (1ull << 40) || (reinterpret_cast<uintptr_t>(w->codes) & 7) != 0) {
        snprintf(buf, sizeof buf,
                 "%lld experts of [%lld, %lld]: the panel layout takes N a multiple of 128, K "
                 "and N below 2^30, under 2^40 weights and 8-byte aligned codes",
                 (long long)experts, (long long)K, (long long)N);
        return refuse(op, buf);
    }
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    auto up = [](size_t b) { return (b + 255) / 256 * 256; };
    const size_t per = (size_t)K * N;
    const size_t code_bytes = (size_t)w->weights / 2;
    const size_t plane_bytes = (size_t)w->weights / 128 * 2;
    const size_t stride = up(int4_panel_bytes((int)K, (int)N, nullptr));
    const size_t scales_off = up(code_bytes);
    const size_t zeros_off = scales_off + up(plane_bytes);
    const size_t panels_off = zeros_off + up(plane_bytes);
    const size_t bytes = panels_off + stride * (size_t)experts;
    void* data = nullptr;
    hipError_t e = hipMalloc(&data, bytes);
    if (e != hipSuccess) return classify(d, e, "prepared weight allocation");
    hipStream_t st = (hipStream_t)stream;
    char* base = static_cast<char*>(data);
    e = hipMemcpyAsync(base, w->codes, code_bytes, hipMemcpyDeviceToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(base + scales_off, w->scales, plane_bytes, hipMemcpyDeviceToDevice,
                           st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(base + zeros_off, w->zeros, plane_bytes, hipMemcpyDeviceToDevice,
                           st);
    for (int64_t i = 0; i < experts && e == hipSuccess; i++) {
        const Int4Planes pi{w->codes + i * (per >> 3), w->scales + i * (per >> 7),
                            w->zeros + i * (per >> 7)};
        e = launch_int4_panel_prepare(st, pi, base + panels_off + stride * (size_t)i, (int)K,
                                      (int)N);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) {
        (void)hipFree(data);
        return classify(d, e, "prepared weight copy");
    }
    auto* p = new accel_int4_prepared{kPreparedMagic, dev, K, N, data, bytes,
                                      kGroupedPanelLayout, panels_off};
    p->experts = experts;
    p->scales_off = scales_off;
    p->zeros_off = zeros_off;
    p->panel_stride = stride;
    *out = p;
    return ACCEL_OK;
}

ACCEL_API int accel_int4_prepared_free(int dev, accel_int4_prepared_t* p) {
    clear_error();
    if (!p) return ACCEL_OK;
    if (p->magic != kPreparedMagic || p->dev != dev)
        return fail(ACCEL_E_INVALID, "accel_int4_prepared_free: not a prepared weight of "
                                     "device %d", dev);
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    const hipError_t e = hipFree(p->data);
    p->magic = 0;
    delete p;
    return classify(d, e, "prepared weight free");
}

ACCEL_API int accel_int4_prepared_bytes(const accel_int4_prepared_t* p, uint64_t* bytes) {
    clear_error();
    if (!p || p->magic != kPreparedMagic || !bytes)
        return fail(ACCEL_E_INVALID, "accel_int4_prepared_bytes: not a prepared weight");
    *bytes = p->bytes;
    return ACCEL_OK;
}

namespace {

// Int4GroupedMatVec / Int4GroupedMatMul over experts prepared with
// accel_int4_prepare_grouped: the same checks, routes and results, the
// matrix-core decode reading the side copies.
int run_grouped_prepared(const char* op, int dev, void* stream, const accel_tensor_t* x,
                         const accel_int4_prepared_t* w, const accel_tensor_t* counts,
                         accel_tensor_t* out, bool matvec) {
    clear_error();
    if (!w || w->magic != kPreparedMagic) return refuse(op, "the prepared weight is missing");
    if (!is_grouped(w))
        return refuse(op, "the weight was prepared as one matrix; grouped products take "
                          "experts prepared with accel_int4_prepare_grouped[_panels]");
    if (w->dev != dev) {
        char b[128];
        snprintf(b, sizeof b, "the weight was prepared on device %d", w->dev);
        return refuse(op, b);
    }
    const char* base = static_cast<const char*>(w->data);
    const int64_t n = w->experts * w->K * w->N;
    accel_int4_t q{reinterpret_cast<const uint32_t*>(base), n / 8,
                   reinterpret_cast<const uint16_t*>(base + w->scales_off), n / 128,
                   reinterpret_cast<const uint16_t*>(base + w->zeros_off), n / 128, n};
    if (w->layout == kGroupedPanelLayout)
        return run_grouped_int4(op, dev, stream, x, &q, w->experts, counts, out, matvec, nullptr,
                                base + w->side_off, w->panel_stride);
    return run_grouped_int4(op, dev, stream, x, &q, w->experts, counts, out, matvec,
                            reinterpret_cast<const uint16_t*>(base + w->side_off));
}

}  // namespace

ACCEL_API int accel_int4_grouped_matvec_prepared(int dev, void* stream,
                                                 const accel_tensor_t* x,
                                                 const accel_int4_prepared_t* w,
                                                 const accel_tensor_t* counts,
                                                 accel_tensor_t* out) {
    return run_grouped_prepared("Int4GroupedMatVecPrepared", dev, stream, x, w, counts, out,
                                true);
}

ACCEL_API int accel_int4_grouped_matmul_prepared(int dev, void* stream,
                                                 const accel_tensor_t* x,
                                                 const accel_int4_prepared_t* w,
                                                 const accel_tensor_t* counts,
                                                 accel_tensor_t* out) {
    return run_grouped_prepared("Int4GroupedMatMulPrepared", dev, stream, x, w, counts, out,
                                false);
}

namespace {

const char* kTilesReason =
    "weights prepared for the matrix cores: the matrix-core decode kernel (x*512s in three "
    "bf16 terms against the exact codes), each 32-row step's scales and zeros one contiguous "
    "block of the side copy";
const char* kTilesRejected =
    "the same kernel on the reference planes: a step's scales and zeros are a piece of each "
    "of its 32 rows of the two planes";

// M rows of a (f32, 16-byte aligned) against count tiles-prepared weights,
// passes of up to 16 rows; outputs [M, N_i] f32.
int run_prepared_tiles(const char* op, Device* d, int dev, void* stream, const float* af,
                       int64_t M, const accel_int4_prepared_t* const* w, void* const* o,
                       int count, int status) {
    (void)dev;
    const uint32_t* codes[kMaxPreparedSet];
    const uint16_t* side[kMaxPreparedSet];
    int N[kMaxPreparedSet];
    for (int i = 0; i < count; i++) {
        codes[i] = static_cast<const uint32_t*>(w[i]->data);
        side[i] = reinterpret_cast<const uint16_t*>(static_cast<const char*>(w[i]->data) +
                                                    w[i]->side_off);
        N[i] = (int)w[i]->N;
    }
    const int K = (int)w[0]->K;
    LaunchRecord rec(false);
    hipError_t e = hipSuccess;
    for (int64_t r0 = 0; r0 < M && e == hipSuccess && status == ACCEL_OK; r0 += 16) {
        const int rows = (int)std::min<int64_t>(16, M - r0);
        float* outs[kMaxPreparedSet];
        for (int i = 0; i < count; i++)
            outs[i] = static_cast<float*>(o[i]) + (size_t)r0 * N[i];
        e = launch_int4_decode_side(d, (hipStream_t)stream, af + (size_t)r0 * K, codes, side,
                                    outs, N, count, rows, K, &status);
    }
    keep_selection(d, op, rec, kTilesReason, kTilesRejected);
    return finish(d, e, status, "prepared matrix-core launch");
}

}  // namespace

// Int4MatVec over a prepared weight: Int4MatVec's checks on a and out, the
// product from the panel layout (one launch, no workspace).
ACCEL_API int accel_int4_matvec_prepared(int dev, void* stream, const accel_tensor_t* a,
                                         const accel_int4_prepared_t* w, accel_tensor_t* out) {
    clear_error();
    const char* op = "Int4MatVecPrepared";
    if (!w || w->magic != kPreparedMagic) return refuse(op, "the prepared weight is missing");
    if (is_grouped(w))
        return refuse(op, "the weight was prepared as grouped experts (accel_int4_prepare_grouped); "
                          "its products are Int4GroupedMatVecPrepared and "
                          "Int4GroupedMatMulPrepared");
    if (w->dev != dev) {
        char b[128];
        snprintf(b, sizeof b, "the weight was prepared on device %d", w->dev);
        return refuse(op, b);
    }
    if (!valid_tensor(a) || !a->data) return refuse(op, "the activations are missing");
    char buf[320];
    if (a->dtype != ACCEL_F32 || a->rank != 1) {
        snprintf(buf, sizeof buf,
                 "activations are %s %s; a matvec takes an f32 vector, and a batch of them is "
                 "the tiled form, Int4MatMul",
                 dtype_name(a->dtype), shape_str(a).c_str());
        return refuse(op, buf);
    }
    if (a->shape[0] != w->K) {
        snprintf(buf, sizeof buf, "activations are %lld long and the matrix is [%lld, %lld]",
                 (long long)a->shape[0], (long long)w->K, (long long)w->N);
        return refuse(op, buf);
    }
    int rc = check_out(op, out, ACCEL_F32, 1, w->N, true);
    if (rc != ACCEL_OK) return rc;
    if (w->layout == kTilesLayout &&
        !int4_decode_side_rows_supported(1, static_cast<const float*>(a->data)))
        return refuse(op, "weights prepared for the matrix cores take 16-byte aligned "
                          "activations");
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    if (w->layout == kTilesLayout) {
        void* o1 = out->data;
        return run_prepared_tiles(op, d, dev, stream, static_cast<const float*>(a->data), 1, &w,
                                  &o1, 1, status);
    }
    LaunchRecord rec(false);
    const void* data = w->data;
    void* o = out->data;
    const int n = (int)w->N;
    const hipError_t e = launch_int4_panel_matvec((hipStream_t)stream,
                                                  static_cast<const float*>(a->data), &data, &o,
                                                  &n, 1, (int)w->K, Epilogue{});
    keep_selection(d, op, rec,
                   "a prepared weight: one workgroup a 16-column K-major panel over all of K, "
                   "no K split and no hand-off",
                   "the reference-format decode kernel: a column tile of those planes reads a "
                   "narrow strip of every row, so K is split across workgroups and the slices "
                   "meet in a hand-off");
    return finish(d, e, status, "Int4MatVecPrepared launch");
}

// Int4MatVec over up to four prepared weights that share one input vector,
// in one launch (a decode step's q, k, v or gate, up); each out[i] is exactly
// accel_int4_matvec_prepared(a, w[i]).
ACCEL_API int accel_int4_matvec_prepared_set(int dev, void* stream, const accel_tensor_t* a,
                                             const accel_int4_prepared_t* const* w,
                                             accel_tensor_t* out, int count) {
    clear_error();
    const char* op = "Int4MatVecPreparedSet";
    char buf[320];
    if (count < 1 || count > kMaxPreparedSet || !w || !out) {
        snprintf(buf, sizeof buf, "%d matrices; a set holds one to %d", count, kMaxPreparedSet);
        return refuse(op, buf);
    }
    if (!valid_tensor(a) || !a->data) return refuse(op, "the activations are missing");
    if (a->dtype != ACCEL_F32 || a->rank != 1) {
        snprintf(buf, sizeof buf, "activations are %s %s; a matvec takes an f32 vector",
                 dtype_name(a->dtype), shape_str(a).c_str());
        return refuse(op, buf);
    }
    const void* data[kMaxPreparedSet];
    void* o[kMaxPreparedSet];
    int N[kMaxPreparedSet];
    for (int i = 0; i < count; i++) {
        if (!w[i] || w[i]->magic != kPreparedMagic) {
            snprintf(buf, sizeof buf, "prepared weight %d is missing", i);
            return refuse(op, buf);
        }
        if (w[i]->dev != dev) {
            snprintf(buf, sizeof buf, "weight %d was prepared on device %d", i, w[i]->dev);
            return refuse(op, buf);
        }
        if (is_grouped(w[i]))
            return refuse(op, "the weight was prepared as grouped experts (accel_int4_prepare_grouped); "
                              "its products are Int4GroupedMatVecPrepared and "
                              "Int4GroupedMatMulPrepared");
        if (a->shape[0] != w[i]->K) {
            snprintf(buf, sizeof buf, "activations are %lld long and matrix %d is [%lld, %lld]",
                     (long long)a->shape[0], i, (long long)w[i]->K, (long long)w[i]->N);
            return refuse(op, buf);
        }
        const int rc = check_out(op, &out[i], ACCEL_F32, 1, w[i]->N, true);
        if (rc != ACCEL_OK) return rc;
        if (w[i]->layout != w[0]->layout)
            return refuse(op, "the weights of a set are prepared the same way (all "
                              "accel_int4_prepare or all accel_int4_prepare_tiles)");
        data[i] = w[i]->data;
        o[i] = out[i].data;
        N[i] = (int)w[i]->N;
    }
    if (w[0]->layout == kTilesLayout &&
        !int4_decode_side_rows_supported(1, static_cast<const float*>(a->data)))
        return refuse(op, "weights prepared for the matrix cores take 16-byte aligned "
                          "activations");
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    if (w[0]->layout == kTilesLayout)
        return run_prepared_tiles(op, d, dev, stream, static_cast<const float*>(a->data), 1, w,
                                  o, count, status);
    LaunchRecord rec(false);
    const hipError_t e = launch_int4_panel_matvec((hipStream_t)stream,
                                                  static_cast<const float*>(a->data), data, o, N,
                                                  count, (int)a->shape[0], Epilogue{});
    keep_selection(d, op, rec,
                   "prepared weights that share their input: their panels side by side in one "
                   "launch, each matrix's results those of its own launch",
                   "one launch per matrix: each would read the shared vector and pay its own "
                   "launch");
    return finish(d, e, status, "Int4MatVecPreparedSet launch");
}

// SwiGLU(a . gate, a . up) over two weights prepared into the panel layout:
// Int4MatVecPreparedSet of {gate, up} followed by SwiGLU, in one launch and
// with the same result bit for bit.
ACCEL_API int accel_int4_matvec_prepared_swiglu(int dev, void* stream, const accel_tensor_t* a,
                                                const accel_int4_prepared_t* gate,
                                                const accel_int4_prepared_t* up,
                                                accel_tensor_t* out) {
    clear_error();
    const char* op = "Int4MatVecPreparedSwiGLU";
    char buf[320];
    const accel_int4_prepared_t* w[2] = {gate, up};
    const char* names[2] = {"gate", "up"};
    for (int i = 0; i < 2; i++) {
        if (!w[i] || w[i]->magic != kPreparedMagic) {
            snprintf(buf, sizeof buf, "the prepared %s weight is missing", names[i]);
            return refuse(op, buf);
        }
        if (w[i]->dev != dev) {
            snprintf(buf, sizeof buf, "the %s weight was prepared on device %d", names[i],
                     w[i]->dev);
            return refuse(op, buf);
        }
        if (w[i]->layout != kPanelLayout) {
            snprintf(buf, sizeof buf,
                     "the %s weight was not prepared with accel_int4_prepare; this product "
                     "reads the panel layout",
                     names[i]);
            return refuse(op, buf);
        }
    }
    if (gate->K != up->K || gate->N != up->N) {
        snprintf(buf, sizeof buf, "gate is [%lld, %lld] and up is [%lld, %lld]; they share a shape",
                 (long long)gate->K, (long long)gate->N, (long long)up->K, (long long)up->N);
        return refuse(op, buf);
    }
    if (!valid_tensor(a) || !a->data) return refuse(op, "the activations are missing");
    if (a->dtype != ACCEL_F32 || a->rank != 1 || a->shape[0] != gate->K) {
        snprintf(buf, sizeof buf, "activations are %s %s and the matrices are [%lld, %lld]",
                 dtype_name(a->dtype), shape_str(a).c_str(), (long long)gate->K,
                 (long long)gate->N);
        return refuse(op, buf);
    }
    int rc = check_out(op, out, ACCEL_F32, 1, gate->N, true);
    if (rc != ACCEL_OK) return rc;
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    LaunchRecord rec(false);
    const hipError_t e = launch_int4_panel_swiglu(
        (hipStream_t)stream, static_cast<const float*>(a->data), gate->data, up->data,
        static_cast<float*>(out->data), (int)gate->N, (int)gate->K);
    keep_selection(d, op, rec,
                   "two prepared weights of one shape read by SwiGLU: one workgroup a "
                   "16-column panel of both, SwiGLU of the two sums written, nothing else",
                   "Int4MatVecPreparedSet and SwiGLU: the two results make a round trip "
                   "through memory and the elementwise product is a launch of its own");
    return finish(d, e, status, "Int4MatVecPreparedSwiGLU launch");
}

namespace {

const char* kRowsReason =
    "2..8 f32 rows of prepared weights: one workgroup a 16-column panel over all of K, each "
    "lane the panel's columns for every row, no K split and no hand-off (passes of eight "
    "rows past eight)";
const char* kRowsRejected =
    "the matrix-core decode kernel on the reference planes: its time is set by load latency, "
    "its K split and the hand-off, about the same from two rows to sixteen";

// Int4MatMul's checks of a ([M, K] f32) and out ([M, N_i] f32) against count
// prepared weights, then the product: one row as Int4MatVecPrepared, more in
// passes of up to eight rows on the rows kernel.
int run_prepared_rows(const char* op, int dev, void* stream, const accel_tensor_t* a,
                      const accel_int4_prepared_t* const* w, accel_tensor_t* out, int count) {
    char buf[320];
    if (count < 1 || count > kMaxPreparedSet || !w || !out) {
        snprintf(buf, sizeof buf, "%d matrices; a set holds one to %d", count, kMaxPreparedSet);
        return refuse(op, buf);
    }
    if (!valid_tensor(a) || !a->data) return refuse(op, "the activations are missing");
    if (a->dtype != ACCEL_F32 || a->rank != 2) {
        snprintf(buf, sizeof buf, "activations are %s %s; this product takes f32 [M, K]",
                 dtype_name(a->dtype), shape_str(a).c_str());
        return refuse(op, buf);
    }
    const int64_t M = a->shape[0], K = a->shape[1];
    const void* data[kMaxPreparedSet];
    void* o[kMaxPreparedSet];
    int N[kMaxPreparedSet];
    for (int i = 0; i < count; i++) {
        if (!w[i] || w[i]->magic != kPreparedMagic) {
            snprintf(buf, sizeof buf, "prepared weight %d is missing", i);
            return refuse(op, buf);
        }
        if (w[i]->dev != dev) {
            snprintf(buf, sizeof buf, "weight %d was prepared on device %d", i, w[i]->dev);
            return refuse(op, buf);
        }
        if (is_grouped(w[i]))
            return refuse(op, "the weight was prepared as grouped experts (accel_int4_prepare_grouped); "
                              "its products are Int4GroupedMatVecPrepared and "
                              "Int4GroupedMatMulPrepared");
        if (K != w[i]->K) {
            snprintf(buf, sizeof buf, "activations are [%lld, %lld] and matrix %d is [%lld, %lld]",
                     (long long)M, (long long)K, i, (long long)w[i]->K, (long long)w[i]->N);
            return refuse(op, buf);
        }
        const int rc = check_out(op, &out[i], ACCEL_F32, M, w[i]->N, false);
        if (rc != ACCEL_OK) return rc;
        if (w[i]->layout != w[0]->layout)
            return refuse(op, "the weights of a set are prepared the same way (all "
                              "accel_int4_prepare or all accel_int4_prepare_tiles)");
        data[i] = w[i]->data;
        o[i] = out[i].data;
        N[i] = (int)w[i]->N;
    }
    if (M > INT32_MAX) return refuse(op, "the product is larger than this backend's extents");
    const float* af = static_cast<const float*>(a->data);
    if (w[0]->layout == kTilesLayout) {
        if (M > 0 && !int4_decode_side_rows_supported(1, af))
            return refuse(op, "weights prepared for the matrix cores take 16-byte aligned "
                              "activations");
        Device* dt = device(dev);
        if (!dt) return ACCEL_E_NO_DEVICE;
        if (M == 0) return ACCEL_OK;
        int st2 = begin_submission(dt);
        if (st2 != ACCEL_OK) return st2;
        return run_prepared_tiles(op, dt, dev, stream, af, M, w, o, count, st2);
    }
    if (M > 1 && !int4_panel_rows_supported((int)M, (int)K, af)) {
        snprintf(buf, sizeof buf,
                 "[%lld, %lld] activations: the rows kernel takes K even and 8-byte aligned "
                 "rows (one row of any K: Int4MatVecPrepared)",
                 (long long)M, (long long)K);
        return refuse(op, buf);
    }
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (M == 0) return ACCEL_OK;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    LaunchRecord rec(false);
    hipError_t e;
    if (M == 1) {
        e = launch_int4_panel_matvec((hipStream_t)stream, af, data, o, N, count, (int)K,
                                     Epilogue{});
        keep_selection(d, op, rec,
                       "one row of prepared weights: Int4MatVecPrepared's kernel, one "
                       "workgroup a 16-column K-major panel over all of K",
                       kRowsRejected);
    } else {
        e = launch_int4_panel_rows((hipStream_t)stream, af, (int)M, data, o, N, count, (int)K,
                                   Epilogue{});
        keep_selection(d, op, rec, kRowsReason, kRowsRejected);
    }
    return finish(d, e, status, "Int4MatMulPrepared launch");
}

}  // namespace

// Int4MatMul over a prepared weight: a f32 [M, K] -> out f32 [M, N].
ACCEL_API int accel_int4_matmul_prepared(int dev, void* stream, const accel_tensor_t* a,
                                         const accel_int4_prepared_t* w, accel_tensor_t* out) {
    clear_error();
    return run_prepared_rows("Int4MatMulPrepared", dev, stream, a, &w, out, 1);
}

// The same over up to four prepared weights that share a; each out[i] is
// exactly accel_int4_matmul_prepared(a, w[i]).
ACCEL_API int accel_int4_matmul_prepared_set(int dev, void* stream, const accel_tensor_t* a,
                                             const accel_int4_prepared_t* const* w,
                                             accel_tensor_t* out, int count) {
    clear_error();
    return run_prepared_rows("Int4MatMulPreparedSet", dev, stream, a, w, out, count);
}

// ---- the selection report ------------------------------------------------

namespace {

// The device a selection is planned for: an open device, or (dev < 0) an
// MI355X as this library models it, so the question can be asked on a host
// without a GPU.
Device* selection_device(int dev) {
    if (dev >= 0) return device(dev);
    static Device model;
    model.cu_count = 256;
    // a placeholder for the static scratch's address: a dry plan computes
    // offsets from it and launches nothing
    model.scratch = reinterpret_cast<void*>(uintptr_t(1) << 41);
    return &model;
}

}  // namespace

// Which kernels an int4 product would become on device dev (dev < 0: the
// modelled MI355X), and why, without launching or allocating anything.
// op names the entry point: "Int4MatVec", "Int4MatMul", "Int4Linear" or
// "Int4MatVecNoAlloc" (NULL: Int4MatVec for M = 1, else Int4MatMul).
ACCEL_API int accel_int4_select(int dev, const char* op, int32_t dtype, int64_t M, int64_t K,
                                int64_t N, const void* a, const accel_int4_t* w, int32_t flags,
                                accel_selection_t* sel) {
    clear_error();
    if (!sel) return fail(ACCEL_E_INVALID, "accel_int4_select: no selection to fill");
    if (dtype != ACCEL_F32 && dtype != ACCEL_BF16)
        return fail(ACCEL_E_INVALID, "accel_int4_select: activations are %s; int4 products "
                                     "read f32 or bf16", dtype_name(dtype));
    if (M < 0 || K < 1 || N < 0 || M > INT32_MAX || K > INT32_MAX || N > INT32_MAX)
        return fail(ACCEL_E_INVALID, "accel_int4_select: [%lld, %lld] x [%lld, %lld] is not a "
                    "product this backend takes", (long long)M, (long long)K, (long long)K,
                    (long long)N);
    std::string name = op ? op : (M == 1 ? "Int4MatVec" : "Int4MatMul");
    Device* d = selection_device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    // plane addresses matter only for their alignment
    const void* fake = reinterpret_cast<const void*>(uintptr_t(1) << 20);
    Int4Planes p{static_cast<const uint32_t*>(w && w->codes ? w->codes : fake),
                 static_cast<const uint16_t*>(w && w->scales ? w->scales : fake),
                 static_cast<const uint16_t*>(w && w->zeros ? w->zeros : fake)};
    if (!a) a = fake;
    Epilogue ep;
    ep.bias = (flags & ACCEL_SELECT_BIAS) ? static_cast<const float*>(fake) : nullptr;
    ep.bf16 = dtype == ACCEL_BF16 || (flags & ACCEL_SELECT_BF16_OUT) != 0;
    void* out = const_cast<void*>(fake);
    int status = ACCEL_OK;
    LaunchRecord rec(true);
    if (name == "Int4MatVecPrepared") {
        if (dtype != ACCEL_F32 || M != 1)
            return fail(ACCEL_E_INVALID, "accel_int4_select: Int4MatVecPrepared takes one f32 "
                                         "row");
        if (!int4_panel_supported(K, N))
            return fail(ACCEL_E_INVALID, "accel_int4_select: [%lld, %lld] cannot be prepared "
                        "(N a multiple of 128)", (long long)K, (long long)N);
        const int n = (int)N;
        const void* data = fake;
        void* o = out;
        (void)launch_int4_panel_matvec(nullptr, static_cast<const float*>(a), &data, &o, &n, 1,
                                       (int)K, Epilogue{});
        fill_selection(sel, name, rec.joined(),
                       "a prepared weight: one workgroup a 16-column K-major panel over all of "
                       "K, no K split and no hand-off",
                       "the reference-format decode kernel: a column tile of those planes reads "
                       "a narrow strip of every row, so K is split across workgroups and the "
                       "slices meet in a hand-off");
        return ACCEL_OK;
    }
    if (name == "Int4MatMulPreparedTiles") {
        if (dtype != ACCEL_F32 || M < 1)
            return fail(ACCEL_E_INVALID, "accel_int4_select: Int4MatMulPreparedTiles takes f32 "
                                         "rows");
        if (!int4_side_supported(K, N))
            return fail(ACCEL_E_INVALID, "accel_int4_select: [%lld, %lld] cannot be prepared "
                        "for the matrix cores (K a multiple of 32, N of 128)", (long long)K,
                        (long long)N);
        if (!int4_decode_side_rows_supported(1, static_cast<const float*>(a)))
            return fail(ACCEL_E_INVALID, "accel_int4_select: weights prepared for the matrix "
                                         "cores take 16-byte aligned activations");
        const uint32_t* c = static_cast<const uint32_t*>(fake);
        const uint16_t* sd = static_cast<const uint16_t*>(fake);
        const int n = (int)N;
        for (int64_t r0 = 0; r0 < M && status == ACCEL_OK; r0 += 16) {
            float* o = static_cast<float*>(out);
            (void)launch_int4_decode_side(d, nullptr, static_cast<const float*>(a), &c, &sd, &o,
                                          &n, 1, (int)std::min<int64_t>(16, M - r0), (int)K,
                                          &status);
        }
        if (status != ACCEL_OK) return status;
        fill_selection(sel, name, rec.joined(), kTilesReason, kTilesRejected);
        return ACCEL_OK;
    }
    if (name == "Int4MatMulPrepared") {
        if (dtype != ACCEL_F32 || M < 1)
            return fail(ACCEL_E_INVALID, "accel_int4_select: Int4MatMulPrepared takes f32 "
                                         "rows");
        if (!int4_panel_supported(K, N))
            return fail(ACCEL_E_INVALID, "accel_int4_select: [%lld, %lld] cannot be prepared "
                        "(N a multiple of 128)", (long long)K, (long long)N);
        const int n = (int)N;
        const void* data = fake;
        void* o = out;
        if (M == 1) {
            (void)launch_int4_panel_matvec(nullptr, static_cast<const float*>(a), &data, &o, &n,
                                           1, (int)K, Epilogue{});
        } else {
            if (!int4_panel_rows_supported((int)M, (int)K, static_cast<const float*>(a)))
                return fail(ACCEL_E_INVALID, "accel_int4_select: the rows kernel takes K even "
                                             "and 8-byte aligned rows");
            (void)launch_int4_panel_rows(nullptr, static_cast<const float*>(a), (int)M, &data,
                                         &o, &n, 1, (int)K, Epilogue{});
        }
        fill_selection(sel, name, rec.joined(), M == 1 ? "one row of prepared weights: "
                       "Int4MatVecPrepared's kernel" : kRowsReason, kRowsRejected);
        return ACCEL_OK;
    }
    if (name == "Int4MatVecNoAlloc") {
        if (dtype != ACCEL_F32 || M != 1)
            return fail(ACCEL_E_INVALID, "accel_int4_select: Int4MatVecNoAlloc takes one f32 "
                                         "row");
        (void)launch_int4_matvec_noalloc(d, nullptr, static_cast<const float*>(a), p,
                                         static_cast<float*>(out), (int)K, (int)N, &status);
        if (status != ACCEL_OK) return status;
        fill_selection(sel, name, rec.joined(),
                       "Int4MatVec's kernels and plan, the split-K sums in the static scratch",
                       "the workspace: it may call hipMalloc to grow");
        return ACCEL_OK;
    }
    const Int4Choice c = choose_int4(dtype, a, p.codes, (int)M, (int)K, (int)N);
    (void)launch_int4_route(d, nullptr, c.route, a, p, out, (int)M, (int)K, (int)N, ep,
                            &status);
    if (status != ACCEL_OK) return status;
    fill_selection(sel, name, rec.joined(), c.reason, join(c.rejected, "; "));
    return ACCEL_OK;
}

// What the last int4 product on device dev became (any int4 product entry
// point; the set entry points and Int4MatVecNoAlloc included).
ACCEL_API int accel_hip_last_selection(int dev, accel_selection_t* sel) {
    clear_error();
    if (!sel) return fail(ACCEL_E_INVALID, "accel_hip_last_selection: no selection to fill");
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    std::lock_guard<std::mutex> lk(d->mu);
    if (!d->sel_valid)
        return fail(ACCEL_E_INVALID, "accel_hip_last_selection: device %d has run no int4 "
                                     "product since it was opened", dev);
    fill_selection(sel, d->sel_op, d->sel_kernel, d->sel_reason, d->sel_rejected);
    return ACCEL_OK;
}

ACCEL_API int accel_hip_supports_kernel(const char* kernel) {
    if (!kernel) return 0;
    for (const Record& r : kRecords)
        if (std::strcmp(r.name, kernel) == 0) return 1;
    return 0;
}

ACCEL_API int accel_hip_dispatch(int dev, void* stream, const char* kernel,
                                 const void* const* bindings, const uint64_t* lens,
                                 int32_t nbindings, const void* uniform, size_t uniform_bytes,
                                 const uint32_t count[3]) {
    clear_error();
    (void)count;
    if (!kernel) return fail(ACCEL_E_INVALID, "accel_hip_dispatch: no kernel named");
    const Record* rec = nullptr;
    for (const Record& r : kRecords)
        if (std::strcmp(r.name, kernel) == 0) rec = &r;
    if (!rec)
        return fail(ACCEL_E_UNSUPPORTED,
                    "accel_hip: kernel %s has no gfx950 implementation in this backend", kernel);
    if (nbindings != rec->bindings || !bindings || !lens)
        return fail(ACCEL_E_INVALID, "accel_hip: %s takes %d bindings, got %d", kernel,
                    rec->bindings, nbindings);
    std::string name = kernel;
    if (name == "SwiGLU") {
        // no uniform: the length is out's (elementwise.go:85-91)
        const uint64_t n = lens[2];
        if (lens[0] < n || lens[1] < n)
            return fail(ACCEL_E_INVALID, "accel_hip: SwiGLU bindings are shorter than out");
        accel_tensor_t g = {const_cast<void*>(bindings[0]), ACCEL_F32, 1, {(int64_t)n, 0, 0, 0}};
        accel_tensor_t v = {const_cast<void*>(bindings[1]), ACCEL_F32, 1, {(int64_t)n, 0, 0, 0}};
        accel_tensor_t o = {const_cast<void*>(bindings[2]), ACCEL_F32, 1, {(int64_t)n, 0, 0, 0}};
        return accel_swiglu(dev, stream, &g, &v, &o);
    }
    if (!uniform || uniform_bytes < 16)
        return fail(ACCEL_E_INVALID, "accel_hip: %s needs its 16-byte uniform block", kernel);
    if (name == "RMSNorm") {
        // RowDims {Rows@0, Width@4, Eps@8} (norm.go:13-22)
        const uint32_t rows = u32_at(uniform, 0), width = u32_at(uniform, 4);
        float eps;
        std::memcpy(&eps, static_cast<const char*>(uniform) + 8, 4);
        if (lens[0] < (uint64_t)rows * width || lens[1] < width || lens[2] < (uint64_t)rows * width)
            return fail(ACCEL_E_INVALID, "accel_hip: RMSNorm bindings are shorter than its dims");
        accel_tensor_t x = {const_cast<void*>(bindings[0]), ACCEL_F32, 2, {rows, width, 0, 0}};
        accel_tensor_t g = {const_cast<void*>(bindings[1]), ACCEL_F32, 1, {width, 0, 0, 0}};
        accel_tensor_t o = {const_cast<void*>(bindings[2]), ACCEL_F32, 2, {rows, width, 0, 0}};
        return accel_rmsnorm(dev, stream, &x, &g, eps, &o);
    }
    if (name == "QuantMatVecF32" || name == "QuantMatVec" || name == "QuantMatMulTiledF32" ||
        name == "QuantMatMulTiled") {
        // GEMMDims {M@0, N@4, K@8}; the M = 1 records ignore M
        const bool vec = name == "QuantMatVecF32" || name == "QuantMatVec";
        const bool f16 = name == "QuantMatVec" || name == "QuantMatMulTiled";
        const uint32_t M = vec ? 1u : u32_at(uniform, 0);
        const uint32_t N = u32_at(uniform, 4), K = u32_at(uniform, 8);
        const uint64_t W = (uint64_t)K * N;
        if (lens[0] < (uint64_t)M * K || lens[1] < W || lens[2] < (W + 31) / 32 ||
            lens[3] < (uint64_t)M * N)
            return fail(ACCEL_E_INVALID, "accel_hip: %s bindings are shorter than its dims",
                        kernel);
        accel_tensor_t a = {const_cast<void*>(bindings[0]), f16 ? ACCEL_F16 : ACCEL_F32, 2,
                            {M, K, 0, 0}};
        accel_tensor_t q = {const_cast<void*>(bindings[1]), ACCEL_I8, 2, {K, N, 0, 0}};
        accel_tensor_t sc = {const_cast<void*>(bindings[2]), ACCEL_F16, 1,
                             {(int64_t)((W + 31) / 32), 0, 0, 0}};
        accel_tensor_t o = {const_cast<void*>(bindings[3]), ACCEL_F32, 2, {M, N, 0, 0}};
        return accel_quant_matmul(dev, stream, &a, &q, &sc, &o);
    }
    if (name == "MatVecF32F16") {
        // GEMMDims {M@0, N@4, K@8}
        const uint32_t N = u32_at(uniform, 4), K = u32_at(uniform, 8);
        if (lens[0] < K || lens[1] < (uint64_t)K * N || lens[2] < N)
            return fail(ACCEL_E_INVALID,
                        "accel_hip: MatVecF32F16 bindings are shorter than its dims");
        accel_tensor_t a = {const_cast<void*>(bindings[0]), ACCEL_F32, 1, {K, 0, 0, 0}};
        accel_tensor_t wt = {const_cast<void*>(bindings[1]), ACCEL_F16, 2, {K, N, 0, 0}};
        accel_tensor_t o = {const_cast<void*>(bindings[2]), ACCEL_F32, 1, {N, 0, 0, 0}};
        return accel_matvec_f32_f16(dev, stream, &a, &wt, &o);
    }
    if (name == "QuantMatVecInt4" || name == "QuantMatMulInt4") {
        // GEMMDims std140: M@0, N@4, K@8.  The matvec's M is unused (0).
        const uint32_t M = name == "QuantMatVecInt4" ? 1u : u32_at(uniform, 0);
        const uint32_t N = u32_at(uniform, 4), K = u32_at(uniform, 8);
        const uint64_t weights = (uint64_t)K * N;
        accel_int4_t w = {static_cast<const uint32_t*>(bindings[1]), (int64_t)lens[1],
                          static_cast<const uint16_t*>(bindings[2]), (int64_t)lens[2],
                          static_cast<const uint16_t*>(bindings[3]), (int64_t)lens[3],
                          (int64_t)weights};
        if (lens[0] < (uint64_t)M * K || lens[4] < (uint64_t)M * N)
            return fail(ACCEL_E_INVALID, "accel_hip: %s bindings are shorter than its dims",
                        kernel);
        accel_tensor_t a = {const_cast<void*>(bindings[0]), ACCEL_F32, 2, {M, K, 0, 0}};
        accel_tensor_t o = {const_cast<void*>(bindings[4]), ACCEL_F32, 2, {M, N, 0, 0}};
        if (name == "QuantMatVecInt4") {
            a.rank = 1;
            a.shape[0] = K;
            o.rank = 1;
            o.shape[0] = N;
            return accel_int4_matvec(dev, stream, &a, &w, &o);
        }
        return accel_int4_matmul(dev, stream, &a, &w, &o);
    }
    if (name == "SegmentOffsets") {
        const uint32_t rows = u32_at(uniform, 0);
        if (lens[0] < rows || lens[1] < (uint64_t)rows + 1)
            return fail(ACCEL_E_INVALID, "accel_hip: SegmentOffsets bindings are too short");
        accel_tensor_t c = {const_cast<void*>(bindings[0]), ACCEL_U32, 1, {rows, 0, 0, 0}};
        accel_tensor_t o = {const_cast<void*>(bindings[1]), ACCEL_U32, 1, {rows + 1, 0, 0, 0}};
        return accel_segment_offsets(dev, stream, &c, &o);
    }
    // Grouped records take the offsets directly (the plan's SegmentOffsets
    // node already ran).  GroupedDims {E@0,K@4,N@8}: tokens from out's length.
    // GroupedTiledDims {E@0,Tokens@4,K@8,N@12}.
    const bool tiled = name == "GroupedMatMul";
    const uint32_t E = u32_at(uniform, 0);
    uint32_t T, K, N;
    if (tiled) {
        T = u32_at(uniform, 4);
        K = u32_at(uniform, 8);
        N = u32_at(uniform, 12);
    } else {
        K = u32_at(uniform, 4);
        N = u32_at(uniform, 8);
        T = N ? (uint32_t)(lens[3] / N) : 0;
    }
    if (lens[0] < (uint64_t)T * K || lens[1] < (uint64_t)E * K * N || lens[2] < (uint64_t)E + 1 ||
        lens[3] < (uint64_t)T * N)
        return fail(ACCEL_E_INVALID, "accel_hip: %s bindings are shorter than its dims", kernel);
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int status = begin_submission(d);
    if (status != ACCEL_OK) return status;
    hipError_t e = launch_grouped_f32((hipStream_t)stream, static_cast<const float*>(bindings[0]),
                                      static_cast<const float*>(bindings[1]),
                                      static_cast<const uint32_t*>(bindings[2]),
                                      static_cast<float*>(const_cast<void*>(bindings[3])),
                                      (int)E, (int)T, (int)K, (int)N, !tiled);
    return classify(d, e, "grouped launch");
}
