// Decode-shape int4 products (M <= 16 rows of f32 activations), the
// counterpart of the reference's QuantMatVecInt4
// (internal/kernels/int4.go:59-101).
//
// Layout (the reference's, unchanged): W is [K, N], weight (k, n) is nibble
// (k*N+n) % 8 of u32 word (k*N+n) / 8, low nibble first; group
// g = (k*N+n) / 128 carries an f16 scale s and zero z, and
// w = s == 0 ? z : (code - z) * s.  With N % 128 == 0 a group is 128
// consecutive columns of one row k.
//
// Kernel shape.  A workgroup of 512 lanes (eight waves) owns a tile of TILE
// columns and a slice of K rows.  Each lane owns CPL adjacent columns (CPL/8
// words: one 4-, 8- or 16-byte load per row) and kBatch rows of its row
// phase; the TILE/CPL lanes of a row read it as one contiguous segment (128
// bytes for a 256-column tile).  A lane issues all its loads -- codes, then
// the scale, zero and activations of each of its rows -- before it uses
// any, branch free, so a workgroup waits for one memory latency; the slice
// count grows with K instead of a loop (only past kMaxSlices slices does a
// workgroup loop over batches).  Per (row, group) the dequantisation folds
// into two scalars,
//     x*w = (x*s)*code + b,   b = -(x*s)*z   (or x*z for a zero scale),
// so the inner loop is one conversion per two weights and one FMA per
// weight, and b is summed per lane and added once to each of its column
// sums.  Nibbles become floats through the fp8 converter: a byte 0000qqqq
// read as OCP e4m3 is exactly q * 2^-9 (codes 0..7 are the subnormals
// q/8 * 2^-6, codes 8..15 the first binade (1 + (q-8)/8) * 2^-6), so
// v_cvt_pk_f32_fp8 turns two nibbles into two exact floats and the 2^9 is
// folded into x*s.
//
// Reduction.  The row phases of a workgroup are summed through LDS.  With
// one slice those sums are the output.  Otherwise every workgroup stores its
// column sums to the workspace with device-scope stores, waits until they
// are acknowledged, and draws a ticket for its tile with a device-scope
// atomic; the workgroup that draws the last ticket reads all slices' sums
// with device-scope loads, adds them in slice order -- so the result does not
// depend on scheduling -- writes the output and returns the ticket to zero.
// Device-scope ("sc1") stores and loads go through the device's coherence
// point, so only the data of the hand-off pays for it: no L2-wide writeback
// or invalidate (what an agent-scope release/acquire fence costs on CDNA) is
// issued.
//
// Placement.  Workgroups are dealt to the eight XCDs round robin by launch
// index.  Logical workgroups are renumbered so that consecutive ones -- the
// tiles of one K slice, which share scale and zero rows, activations and
// 128-byte code lines -- run on one XCD and its L2 fetches those once.  The
// placement affects speed only: every cross-workgroup access above is
// device-coherent.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.hpp"

namespace accel {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;           // lanes per workgroup of the matrix-core kernel
constexpr int kDecThreads = 512;        // lanes per workgroup of the VALU kernel
constexpr int kBatch = 4;               // rows per lane per fetch batch
constexpr int kMaxSlices = 64;          // K slices of a VALU decode launch, at most
constexpr float kNibbleScale = 512.0f;  // 1 / (e4m3 value of code 1)

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

// Eight nibbles of one word -> eight floats q * 2^-9, in column order.
__device__ __forceinline__ void unpack8(uint32_t w, float* f) {
    const uint32_t lo = w & 0x0F0F0F0Fu;          // nibbles 0,2,4,6 in bytes 0..3
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // nibbles 1,3,5,7
    const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
    const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
    const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
    const f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
    f[0] = a.x; f[2] = a.y; f[4] = b.x; f[6] = b.y;
    f[1] = c.x; f[3] = c.y; f[5] = d.x; f[7] = d.y;
}

// WPL consecutive code words of one row, streamed past the caches.
template <int WPL>
__device__ __forceinline__ void load_words(const uint32_t* p, uint32_t* w) {
    if constexpr (WPL == 4) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (WPL == 2) {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        w[0] = v.x; w[1] = v.y;
    } else {
        w[0] = __builtin_nontemporal_load(p);
    }
}

__device__ __forceinline__ void store_device(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_device(float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K hand-off, called by every lane of a workgroup after it stored its
// sums for columns [col0, col0 + cols) of slice `slice` with store_device:
// the stores are acknowledged by the device coherence point before the
// tile's ticket is drawn (each tile's ticket has a 128-byte line of its own
// where the workspace allows, so the atomics of different tiles do not queue
// behind each other), and the workgroup drawing the last ticket reads all
// slices' sums with device-scope loads, adds them in slice order (so the
// result does not depend on scheduling), writes `out` and returns the ticket
// to zero for the next launch.
__device__ __forceinline__ void split_k_finish(float* partial, uint32_t* ticket, float* out,
                                               int col0, int cols, int M, int N, int slices,
                                               int* last_flag) {
    const int tid = threadIdx.x;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        *last_flag = prev == (uint32_t)(slices - 1);
    }
    __syncthreads();
    if (!*last_flag) return;
    const size_t slice_stride = (size_t)M * N;
    for (int idx = tid; idx < M * cols; idx += blockDim.x) {
        const int m = idx / cols;
        const int col = col0 + idx % cols;
        float* p = partial + (size_t)m * N + col;
        float sum = 0.0f;
        int sl = 0;
        // up to sixteen slices' loads in flight at once
        for (; sl + 16 <= slices; sl += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = load_device(p + (size_t)(sl + u) * slice_stride);
#pragma unroll
            for (int u = 0; u < 16; u++) sum += v[u];
        }
        if (sl < slices) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++)
                v[u] = sl + u < slices ? load_device(p + (size_t)(sl + u) * slice_stride) : 0.0f;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (sl + u < slices) sum += v[u];
        }
        out[(size_t)m * N + col] = sum;
    }
    if (tid == 0)
        __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-lane sums over the row phases of a wave.  A wave holds 64 / LPR row
// phases of LPR lanes each (lane l belongs to row phase l / LPR); every lane
// has n accumulators for its columns.  Each stage halves the values a lane
// holds and doubles the row phases they cover: lanes whose bit D is clear
// keep the first half of the columns, the others the second half, and each
// adds its partner's (lane l ^ D) copy of the half it keeps.  D = 32 and 16
// use the swap-permutes (one instruction moves a pair of values between the
// two halves of the wave, or between adjacent 16-lane rows), D = 8 a DPP
// rotation within 16-lane rows, smaller D a cross-lane read.  Stages run
// from D = 32 down to D = LPR, so the result sums all row phases of the
// wave; lane l ends with n * LPR / 64 values, the columns given by
// reduced_offset.
template <int D>
__device__ __forceinline__ float xor_partner(float x, int l) {
    if constexpr (D == 8) {
        // row_ror:8 within 16-lane rows: lane l reads lane l ^ 8
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf,
                                                          false));
    } else {
        return __int_as_float(__builtin_amdgcn_ds_bpermute((l ^ D) << 2, __float_as_int(x)));
    }
}
template <int n, int D, int LPR>
__device__ __forceinline__ void transpose_reduce(float* v, int l) {
    if constexpr (D >= LPR) {
        constexpr int h = n / 2;
        if constexpr (D == 32 || D == 16) {
#pragma unroll
            for (int j = 0; j < h; j++) {
                const auto r = D == 32 ? __builtin_amdgcn_permlane32_swap(
                                             __float_as_uint(v[j]), __float_as_uint(v[h + j]),
                                             false, false)
                                       : __builtin_amdgcn_permlane16_swap(
                                             __float_as_uint(v[j]), __float_as_uint(v[h + j]),
                                             false, false);
                v[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
            }
        } else {
            const bool upper = (l & D) != 0;
#pragma unroll
            for (int j = 0; j < h; j++) {
                const float keep = upper ? v[h + j] : v[j];
                const float send = upper ? v[j] : v[h + j];
                v[j] = keep + xor_partner<D>(send, l);
            }
        }
        transpose_reduce<h, D / 2, LPR>(v, l);
    }
}
// Column offset (within the lane's CPL columns) of the values transpose_reduce
// leaves in lane l.
template <int n, int D, int LPR>
__device__ __forceinline__ int reduced_offset(int l) {
    if constexpr (D >= LPR) {
        return ((l & D) ? n / 2 : 0) + reduced_offset<n / 2, D / 2, LPR>(l);
    } else {
        return 0;
    }
}

// M rows of activations; TILE columns per workgroup, CPL per lane.
//
// A workgroup of eight waves owns TILE columns and the rows
// [k_begin, k_end) of its slice, kBatch rows per lane: lane (row phase rp,
// segment lane) decodes rows k_begin + rp + i * RP, i < kBatch.  All of a
// lane's loads -- its codes, then the scale, zero and activations of each
// of its rows -- are issued at once, before any is used, and are branch
// free (rows past the end are clamped into the slice, loaded again and
// given a zero factor), so the workgroup waits for one memory latency.
// Matrices longer than the slices the launch can take loop over such
// batches.
template <int M, int TILE, int CPL>
__global__ __launch_bounds__(kDecThreads) void int4_decode_f32_kernel(
    const float* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    float* __restrict__ out, float* partial, uint32_t* tickets, int ticket_stride, int K, int N,
    int rows_per_slice, int slices) {
    constexpr int LPR = TILE / CPL;        // lanes per row
    constexpr int RP = kDecThreads / LPR;  // row phases
    constexpr int RPW = 64 / LPR;          // row phases per wave
    constexpr int WPL = CPL / 8;           // code words per lane per row
    constexpr int NWAVE = kDecThreads / 64;
    __shared__ __attribute__((aligned(16))) float red[NWAVE][TILE];
    __shared__ int last_flag;

    const int tiles = N / TILE;
    const int grid = tiles * slices;
    int b = blockIdx.x;
    if ((grid & 7) == 0) b = (b & 7) * (grid >> 3) + (b >> 3);
    const int tile = b % tiles;
    const int slice = b / tiles;

    const int tid = threadIdx.x;
    const int l64 = tid & 63;
    const int wave = tid >> 6;
    const int lane = tid % LPR;
    const int rp = tid / LPR;
    const int col0 = tile * TILE + lane * CPL;
    const size_t groups_per_row = (size_t)(N >> 7);
    const size_t words_per_row = (size_t)(N >> 3);
    const size_t group = (size_t)((col0) >> 7);
    const int k_begin = slice * rows_per_slice;
    const int k_end = min(K, k_begin + rows_per_slice);
    const uint32_t* qcol = codes + (col0 >> 3);

    float acc[M][CPL];
    float bsum[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        bsum[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; j++) acc[m][j] = 0.0f;
    }

    for (int kb = k_begin; kb < k_end; kb += kBatch * RP) {
        uint32_t q[kBatch][WPL];
        uint16_t sb[kBatch], zb[kBatch];
        float xv[kBatch][M];
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const int row = min(kb + rp + i * RP, k_end - 1);
            load_words<WPL>(qcol + (size_t)row * words_per_row, q[i]);
        }
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const int row = min(kb + rp + i * RP, k_end - 1);
            sb[i] = scales[(size_t)row * groups_per_row + group];
            zb[i] = zeros[(size_t)row * groups_per_row + group];
#pragma unroll
            for (int m = 0; m < M; m++) xv[i][m] = a[(size_t)m * K + row];
        }
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const bool valid = kb + rp + i * RP < k_end;
            const float s = half_bits_to_float(sb[i]);
            const float z = half_bits_to_float(zb[i]);
            float c[M];
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float xs = xv[i][m] * s;
                const float bterm = (s == 0.0f) ? xv[i][m] * z : -(xs * z);
                c[m] = valid ? xs * kNibbleScale : 0.0f;
                bsum[m] += valid ? bterm : 0.0f;
            }
#pragma unroll
            for (int wi = 0; wi < WPL; wi++) {
                float f[8];
                unpack8(q[i][wi], f);
#pragma unroll
                for (int m = 0; m < M; m++)
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        acc[m][wi * 8 + j] = __builtin_fmaf(c[m], f[j], acc[m][wi * 8 + j]);
            }
        }
    }

    // Row-phase sums: across the wave's RPW row phases in registers
    // (transpose_reduce), then across the waves through LDS.  A lane's
    // zero-point sum is a constant of each of its columns.
    const bool split = slices > 1;
    constexpr int NV = CPL / RPW;  // column sums a lane holds after the wave stage
#pragma unroll
    for (int m = 0; m < M; m++) {
        float v[CPL];
#pragma unroll
        for (int j = 0; j < CPL; j++) v[j] = acc[m][j] + bsum[m];
        transpose_reduce<CPL, 64 / 2, LPR>(v, l64);
        const int c0 = lane * CPL + reduced_offset<CPL, 64 / 2, LPR>(l64);
#pragma unroll
        for (int e = 0; e < NV; e++) red[wave][c0 + e] = v[e];
        __syncthreads();
        for (int c = tid; c < TILE; c += kDecThreads) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < NWAVE; w++) sum += red[w][c];
            const int col = tile * TILE + c;
            if (split)
                store_device(&partial[((size_t)slice * M + m) * N + col], sum);
            else
                out[(size_t)m * N + col] = sum;
        }
        __syncthreads();
    }
    if (!split) return;

    split_k_finish(partial, tickets + (size_t)tile * ticket_stride, out, tile * TILE, TILE, M, N,
                   slices, &last_flag);
}

// Spacing of the tiles' tickets in u32 words: 32 (one 128-byte line each)
// when the counter area holds that many, else the widest power of two that
// fits; 0 when not even one word per tile fits.
int ticket_stride(int tiles) {
    const size_t words = kWorkspaceCounterBytes / sizeof(uint32_t);
    for (int stride = 32; stride >= 1; stride >>= 1)
        if ((size_t)tiles * stride <= words) return stride;
    return 0;
}

// Slices: one batch (kBatch rows a lane) per workgroup, so every workgroup
// waits for one memory latency; past kMaxSlices slices a workgroup loops
// over several batches instead, which bounds the partial sums and the
// hand-off's reads.
template <int M, int TILE, int CPL>
hipError_t launch_decode(Device* d, hipStream_t st, const float* a, Int4Planes w,
                         float* out, int K, int N, int* status) {
    constexpr int LPR = TILE / CPL;
    constexpr int RP = kDecThreads / LPR;
    constexpr int kRowsPerBatch = kBatch * RP;
    const int tiles = N / TILE;
    const int batches = (K + kRowsPerBatch - 1) / kRowsPerBatch;
    const int per_slice = (batches + kMaxSlices - 1) / kMaxSlices;
    const int rows = per_slice * kRowsPerBatch;
    const int slices = (K + rows - 1) / rows;
    float* partial = nullptr;
    uint32_t* tickets = nullptr;
    int stride = 0;
    if (slices > 1) {
        stride = ticket_stride(tiles);
        if (stride == 0) {
            *status = fail(ACCEL_E_INVALID,
                           "decode product: N=%d needs more tickets than the workspace holds", N);
            return hipSuccess;
        }
        void* ws = workspace(d, (size_t)slices * M * N * sizeof(float), status);
        if (!ws) return hipSuccess;
        tickets = static_cast<uint32_t*>(ws);
        partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    }
    hipLaunchKernelGGL((int4_decode_f32_kernel<M, TILE, CPL>), dim3(tiles * slices),
                       dim3(kDecThreads), 0, st, a, w.codes, w.scales, w.zeros, out, partial,
                       tickets, stride, K, N, rows, slices);
    return hipGetLastError();
}

// Columns per lane by row count: the accumulators (M * CPL) stay near 64.
template <int M>
hipError_t launch_decode_m(Device* d, hipStream_t st, const float* a, Int4Planes w,
                           float* out, int K, int N, int* status) {
    constexpr int CPL = M <= 2 ? 32 : (M <= 4 ? 16 : 8);
    if (N % 256 == 0) return launch_decode<M, 256, CPL>(d, st, a, w, out, K, N, status);
    return launch_decode<M, 128, CPL>(d, st, a, w, out, K, N, status);
}

// Any shape: one lane per output element, decoding with the flat index.
__global__ void int4_generic_f32_kernel(const float* __restrict__ a,
                                        const uint32_t* __restrict__ codes,
                                        const uint16_t* __restrict__ scales,
                                        const uint16_t* __restrict__ zeros,
                                        float* __restrict__ out, int M, int K, int N) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * N) return;
    const int m = (int)(i / N), n = (int)(i % N);
    float acc = 0.0f;
    for (int k = 0; k < K; k++) {
        const uint64_t idx = (uint64_t)k * N + n;
        const uint32_t code = (codes[idx >> 3] >> (4 * (idx & 7))) & 0xfu;
        const float s = half_bits_to_float(scales[idx >> 7]);
        const float z = half_bits_to_float(zeros[idx >> 7]);
        const float wv = s == 0.0f ? z : ((float)code - z) * s;
        acc = __builtin_fmaf(a[(size_t)m * K + k], wv, acc);
    }
    out[i] = acc;
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
    const uint32_t b = __float_as_uint(f);
    if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

__global__ void int4_generic_bf16_kernel(const uint16_t* __restrict__ a,
                                         const uint32_t* __restrict__ codes,
                                         const uint16_t* __restrict__ scales,
                                         const uint16_t* __restrict__ zeros,
                                         uint16_t* __restrict__ out, int M, int K, int N) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * N) return;
    const int m = (int)(i / N), n = (int)(i % N);
    float acc = 0.0f;
    for (int k = 0; k < K; k++) {
        const uint64_t idx = (uint64_t)k * N + n;
        const uint32_t code = (codes[idx >> 3] >> (4 * (idx & 7))) & 0xfu;
        const float s = half_bits_to_float(scales[idx >> 7]);
        const float z = half_bits_to_float(zeros[idx >> 7]);
        const float wv = s == 0.0f ? z : ((float)code - z) * s;
        acc = __builtin_fmaf(bf16_bits_to_float(a[(size_t)m * K + k]), wv, acc);
    }
    out[i] = float_to_bf16_bits(acc);
}

// ---- 3..16 rows: the matrix cores ------------------------------------------
//
// With M rows of activations every weight feeds M FMAs, and past two rows the
// VALU (not HBM) bounds the product.  This kernel moves the arithmetic onto
// v_mfma_f32_16x16x32_bf16 and keeps f32 accuracy:
//   * the activation rows are the MFMA's A side (16 rows; rows >= M are zero),
//     scaled per (row k, group) to v = x * (512 s) and split exactly into three
//     bf16 terms hi + mid + lo (each the RNE rounding of what is left; the
//     residue is below 2^-27 |v|), so three MFMAs per tile give the product of
//     v with an exact B to f32 accuracy;
//   * B is the code itself, q * 2^-9, exact in bf16 (fp8 converter), so
//     A' * B = x * s * q;
//   * the zero point is the per-(row m, group) bias sum_k x * add,
//     add = s == 0 ? z : -z*s, accumulated in f32 on the VALU.
// A workgroup owns one 128-column group and a K slice; its four waves take
// the slice's 32-k steps in turn and are summed through LDS.  The MFMA column
// c of n-tile j is the physical column 8c + j, so lane c's eight n-tiles are
// the eight nibbles of code word c, read straight from HBM (one u32 per row)
// and paired (row, row+1) with v_perm for the bf16x2 operand.  Slices are
// combined by split_k_finish.

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMfmaCols = 128;      // one quantisation group
constexpr int kMfmaMaxRows = 2048;  // rows of a slice whose fold fits in LDS

struct MfmaDecodeLds {
    f32x2 fold[kMfmaMaxRows];            // (512 s, add) per row of the slice
    float red[4][16][kMfmaCols];         // per-wave sums
    float bias[4][16];
};

__global__ __launch_bounds__(kThreads) void int4_decode_mfma_kernel(
    const float* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    float* __restrict__ out, float* partial, uint32_t* tickets, int ticket_stride, int M, int K,
    int N,
    int rows_per_slice, int slices) {
    __shared__ __attribute__((aligned(16))) MfmaDecodeLds lds;
    __shared__ int last_flag;

    const int tiles = N / kMfmaCols;
    const int grid = tiles * slices;
    int b = blockIdx.x;
    if ((grid & 7) == 0) b = (b & 7) * (grid >> 3) + (b >> 3);
    const int tile = b % tiles;
    const int slice = b / tiles;
    const int n0 = tile * kMfmaCols;
    const size_t g = (size_t)(n0 >> 7);
    const size_t groups_per_row = (size_t)(N >> 7);
    const size_t words_per_row = (size_t)(N >> 3);
    const int k_begin = slice * rows_per_slice;
    const int k_end = min(K, k_begin + rows_per_slice);
    const int nrows = k_end - k_begin;
    const int tid = threadIdx.x;

    for (int r = tid; r < nrows; r += kThreads) {
        const float s = half_bits_to_float(scales[(size_t)(k_begin + r) * groups_per_row + g]);
        const float z = half_bits_to_float(zeros[(size_t)(k_begin + r) * groups_per_row + g]);
        f32x2 f;
        f.x = s * kNibbleScale;
        f.y = (s == 0.0f) ? z : -(z * s);
        lds.fold[r] = f;
    }
    __syncthreads();

    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int c16 = lane & 15;   // A row (activation row m) / B and D column
    const int kg = lane >> 4;    // k-group: 8 consecutive k of a 32-k step
    const bool mrow = c16 < M;
    const float* arow = a + (size_t)(mrow ? c16 : 0) * K;
    const uint32_t* qcol = codes + (n0 >> 3) + c16;

    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float bias = 0.0f;

    // One step's global operands; the next step's are in flight while the
    // current one is converted and multiplied.
    struct StepRegs {
        uint32_t wv[8];
        f32x4 x0, x1;
    };
    auto fetch = [&](StepRegs& r, int stp) {
        const int k = k_begin + stp * 32 + 8 * kg;
#pragma unroll
        for (int e = 0; e < 8; e++)
            r.wv[e] = __builtin_nontemporal_load(qcol + (size_t)(k + e) * words_per_row);
        r.x0 = (f32x4){0.f, 0.f, 0.f, 0.f};
        r.x1 = r.x0;
        if (mrow) {
            r.x0 = *reinterpret_cast<const f32x4*>(arow + k);
            r.x1 = *reinterpret_cast<const f32x4*>(arow + k + 4);
        }
    };
    auto compute = [&](const StepRegs& r, int stp) {
        const int r0 = stp * 32 + 8 * kg;          // first row of this lane, in the slice
        const f32x4* fp = reinterpret_cast<const f32x4*>(&lds.fold[r0]);
        const f32x4 f01 = fp[0], f23 = fp[1], f45 = fp[2], f67 = fp[3];
        const float xv[8] = {r.x0.x, r.x0.y, r.x0.z, r.x0.w, r.x1.x, r.x1.y, r.x1.z, r.x1.w};
        const float mul[8] = {f01.x, f01.z, f23.x, f23.z, f45.x, f45.z, f67.x, f67.z};
        const float add[8] = {f01.y, f01.w, f23.y, f23.w, f45.y, f45.w, f67.y, f67.w};
        bf16x8 ah, am, al;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float v = xv[e] * mul[e];
            bias = __builtin_fmaf(xv[e], add[e], bias);
            const __bf16 h = (__bf16)v;
            const float r1 = v - (float)h;
            const __bf16 md = (__bf16)r1;
            const float r2 = r1 - (float)md;
            ah[e] = h;
            am[e] = md;
            al[e] = (__bf16)r2;
        }
        // B: the code itself as bf16 pairs (row 2p, row 2p+1) straight from
        // the fp8 bytes (scale 1).
        uint32_t bw[8][4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint32_t w0 = r.wv[2 * p], w1 = r.wv[2 * p + 1];
            const uint32_t t01 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);  // bytes 0,1
            const uint32_t t23 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);  // bytes 2,3
            const uint32_t q[4] = {t01 & 0x0F0F0F0Fu, (t01 >> 4) & 0x0F0F0F0Fu,
                                   t23 & 0x0F0F0F0Fu, (t23 >> 4) & 0x0F0F0F0Fu};
            // q[0]: columns 0, 2; q[1]: 1, 3; q[2]: 4, 6; q[3]: 5, 7
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const int c0 = (h >> 1) * 4 + (h & 1);   // 0, 1, 4, 5
                bw[c0][p] = __builtin_bit_cast(
                    uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[h], 1.0f, false));
                bw[c0 + 2][p] = __builtin_bit_cast(
                    uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[h], 1.0f, true));
            }
        }
        bf16x8 bfr[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            bfr[j] = __builtin_bit_cast(bf16x8, (u32x4){bw[j][0], bw[j][1], bw[j][2], bw[j][3]});
        // All hi products, then all mid, then all lo: each accumulator's
        // consecutive MFMAs are eight apart.
#pragma unroll
        for (int j = 0; j < 8; j++)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bfr[j], acc[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 8; j++)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bfr[j], acc[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 8; j++)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bfr[j], acc[j], 0, 0, 0);
    };

    // A ring of kDepth steps in flight per wave: the loads of a step go out
    // kDepth steps (of this wave) before it is used, which covers HBM
    // latency with a wave's own strided row loads.
    constexpr int kDepth = 4;
    const int nsteps = nrows / 32;   // slices are whole 32-k steps
    StepRegs ring[kDepth];
#pragma unroll
    for (int i = 0; i < kDepth; i++)
        if (wave + 4 * i < nsteps) fetch(ring[i], wave + 4 * i);
    for (int base = wave; base < nsteps; base += 4 * kDepth) {
#pragma unroll
        for (int i = 0; i < kDepth; i++) {
            const int stp = base + 4 * i;
            if (stp < nsteps) {
                compute(ring[i], stp);
                if (stp + 4 * kDepth < nsteps) fetch(ring[i], stp + 4 * kDepth);
            }
        }
    }

    // D of a 16 x 16 tile: lane holds column lane % 16, rows 4*(lane/16)+i.
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) lds.red[wave][kg * 4 + i][8 * c16 + j] = acc[j][i];
    bias += __shfl_xor(bias, 16, 64);
    bias += __shfl_xor(bias, 32, 64);
    if (kg == 0) lds.bias[wave][c16] = bias;
    __syncthreads();

    const bool split = slices > 1;
    for (int idx = tid; idx < M * kMfmaCols; idx += kThreads) {
        const int m = idx / kMfmaCols;
        const int c = idx % kMfmaCols;
        const float v = ((lds.red[0][m][c] + lds.red[1][m][c]) +
                         (lds.red[2][m][c] + lds.red[3][m][c])) +
                        ((lds.bias[0][m] + lds.bias[1][m]) + (lds.bias[2][m] + lds.bias[3][m]));
        if (split)
            store_device(&partial[((size_t)slice * M + m) * N + n0 + c], v);
        else
            out[(size_t)m * N + n0 + c] = v;
    }
    if (!split) return;
    split_k_finish(partial, tickets + (size_t)tile * ticket_stride, out, n0, kMfmaCols, M, N,
                   slices, &last_flag);
}

// Slices: two workgroups per CU, partial sums within 1/8 of the codes, and
// every slice a whole number of 32-k steps for each of the four waves.
hipError_t launch_decode_mfma(Device* d, hipStream_t st, const float* a, Int4Planes w,
                              float* out, int M, int K, int N, int* status) {
    const int tiles = N / kMfmaCols;
    constexpr int kQuantum = 32 * 4;
    int slices = std::max(1, (2 * d->cu_count + tiles - 1) / tiles);
    slices = std::min(slices, std::max(1, K / (64 * M)));
    slices = std::min(slices, std::max(1, K / kQuantum));
    slices = std::max(slices, (K + kMfmaMaxRows - 1) / kMfmaMaxRows);
    int rows = (K + slices - 1) / slices;
    rows = (rows + kQuantum - 1) / kQuantum * kQuantum;
    if (rows > kMfmaMaxRows) rows = kMfmaMaxRows;
    slices = (K + rows - 1) / rows;
    float* partial = nullptr;
    uint32_t* tickets = nullptr;
    int stride = 0;
    if (slices > 1) {
        stride = ticket_stride(tiles);
        if (stride == 0) {
            *status = fail(ACCEL_E_INVALID,
                           "decode product: N=%d needs more tickets than the workspace holds", N);
            return hipSuccess;
        }
        void* ws = workspace(d, (size_t)slices * M * N * sizeof(float), status);
        if (!ws) return hipSuccess;
        tickets = static_cast<uint32_t*>(ws);
        partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    }
    hipLaunchKernelGGL(int4_decode_mfma_kernel, dim3(tiles * slices), dim3(kThreads), 0, st, a,
                       w.codes, w.scales, w.zeros, out, partial, tickets, stride, M, K, N, rows,
                       slices);
    return hipGetLastError();
}

}  // namespace

bool int4_decode_f32_supported(int M, int K, int N, const void* codes) {
    return M >= 1 && M <= 16 && K >= 1 && N >= 128 && N % 128 == 0 &&
           (reinterpret_cast<uintptr_t>(codes) & 15) == 0 && K < (1 << 30) && N < (1 << 30);
}

hipError_t launch_int4_decode_f32(Device* d, hipStream_t st, const float* a, Int4Planes w,
                                  float* out, int M, int K, int N, int* status) {
    *status = ACCEL_OK;
    // Three or more rows: the matrix-core kernel, where its shape holds.
    if (M >= 3 && K % 32 == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0)
        return launch_decode_mfma(d, st, a, w, out, M, K, N, status);
    switch (M) {
        case 1: return launch_decode_m<1>(d, st, a, w, out, K, N, status);
        case 2: return launch_decode_m<2>(d, st, a, w, out, K, N, status);
        case 3: return launch_decode_m<3>(d, st, a, w, out, K, N, status);
        case 4: return launch_decode_m<4>(d, st, a, w, out, K, N, status);
        case 5: return launch_decode_m<5>(d, st, a, w, out, K, N, status);
        case 6: return launch_decode_m<6>(d, st, a, w, out, K, N, status);
        case 7: return launch_decode_m<7>(d, st, a, w, out, K, N, status);
        case 8: return launch_decode_m<8>(d, st, a, w, out, K, N, status);
        default: break;
    }
    // 9..16 rows: eight, then the rest.
    hipError_t e = launch_decode_m<8>(d, st, a, w, out, K, N, status);
    if (e != hipSuccess || *status != ACCEL_OK) return e;
    return launch_int4_decode_f32(d, st, a + (size_t)8 * K, w, out + (size_t)8 * N, M - 8, K,
                                  N, status);
}

hipError_t launch_int4_generic_f32(hipStream_t st, const float* a, Int4Planes w, float* out,
                                   int M, int K, int N) {
    const int64_t total = (int64_t)M * N;
    if (total == 0) return hipSuccess;
    const int threads = 256;
    const int64_t blocks = (total + threads - 1) / threads;
    hipLaunchKernelGGL(int4_generic_f32_kernel, dim3((unsigned)blocks), dim3(threads), 0, st,
                       a, w.codes, w.scales, w.zeros, out, M, K, N);
    return hipGetLastError();
}

hipError_t launch_int4_generic_bf16(hipStream_t st, const uint16_t* a, Int4Planes w,
                                    uint16_t* out, int M, int K, int N) {
    const int64_t total = (int64_t)M * N;
    if (total == 0) return hipSuccess;
    const int threads = 256;
    const int64_t blocks = (total + threads - 1) / threads;
    hipLaunchKernelGGL(int4_generic_bf16_kernel, dim3((unsigned)blocks), dim3(threads), 0,
                       st, a, w.codes, w.scales, w.zeros, out, M, K, N);
    return hipGetLastError();
}

}  // namespace accel
