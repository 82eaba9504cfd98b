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
// count grows with K instead of a loop (only past 64 slices at one row, 32 at
// more, does a workgroup loop over batches, the next batch's loads then
// issued before the current one is computed).  Per (row, group) the dequantisation folds
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
#include <type_traits>

#include "internal.hpp"
#include "splitk.hpp"

namespace accel {
namespace {

constexpr float kNibbleScale = 512.0f;  // 1 / (e4m3 value of code 1)

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
// One workgroup's share: column tile `tile` of the matrix, K slice `slice`;
// `ticket` is this tile's split-K ticket.
// An activation as f32: f32 as is, bf16 bits widened exactly.
__device__ __forceinline__ float x_value(float v) { return v; }
__device__ __forceinline__ float x_value(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

template <int M, int TILE, int CPL, bool PIPE, typename XT = float>
__device__ __forceinline__ void decode_tile(
    const XT* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    void* __restrict__ out, float* partial, uint32_t* ticket, int K, int N, int tile, int slice,
    int rows_per_slice, int slices, const Epilogue& ep) {
    constexpr int LPR = TILE / CPL;        // lanes per row
    constexpr int RP = kDecThreads / LPR;  // row phases
    constexpr int RPW = 64 / LPR;          // row phases per wave
    constexpr int WPL = CPL / 8;           // code words per lane per row
    constexpr int NWAVE = kDecThreads / 64;
    __shared__ __attribute__((aligned(16))) float red[NWAVE][TILE];
    __shared__ int last_flag;

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

    uint32_t q[kBatch][WPL];
    uint16_t sb[kBatch], zb[kBatch];
    XT xv[kBatch][M];   // raw: widened where used, so no load waits early
    auto fetch = [&](int kb, uint32_t (&qq)[kBatch][WPL], uint16_t (&ss)[kBatch],
                     uint16_t (&zz)[kBatch], XT (&xx)[kBatch][M]) {
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const int row = min(kb + rp + i * RP, k_end - 1);
            load_words<WPL>(qcol + (size_t)row * words_per_row, qq[i]);
        }
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const int row = min(kb + rp + i * RP, k_end - 1);
            ss[i] = scales[(size_t)row * groups_per_row + group];
            zz[i] = zeros[(size_t)row * groups_per_row + group];
#pragma unroll
            for (int m = 0; m < M; m++) xx[i][m] = a[(size_t)m * K + row];
        }
    };
    auto compute = [&](int kb) {
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const bool valid = kb + rp + i * RP < k_end;
            const float s = half_bits_to_float(sb[i]);
            const float z = half_bits_to_float(zb[i]);
            float c[M];
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float x = x_value(xv[i][m]);
                const float xs = x * s;
                const float bterm = (s == 0.0f) ? x * z : -(xs * z);
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
    };
    if constexpr (PIPE) {
        // Several batches a workgroup: the next batch's loads are issued
        // before the current batch is computed.
        if (k_begin < k_end) fetch(k_begin, q, sb, zb, xv);
        for (int kb = k_begin; kb < k_end; kb += kBatch * RP) {
            uint32_t qn[kBatch][WPL];
            uint16_t sn[kBatch], zn[kBatch];
            XT xn[kBatch][M];
            const bool more = kb + kBatch * RP < k_end;
            if (more) fetch(kb + kBatch * RP, qn, sn, zn, xn);
            compute(kb);
            if (more) {
#pragma unroll
                for (int i = 0; i < kBatch; i++) {
#pragma unroll
                    for (int w = 0; w < WPL; w++) q[i][w] = qn[i][w];
                    sb[i] = sn[i];
                    zb[i] = zn[i];
#pragma unroll
                    for (int m = 0; m < M; m++) xv[i][m] = xn[i][m];
                }
            }
        }
    } else {
        for (int kb = k_begin; kb < k_end; kb += kBatch * RP) {
            fetch(kb, q, sb, zb, xv);
            compute(kb);
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
                store_out(out, (size_t)m * N + col, col, sum, ep);
        }
        __syncthreads();
    }
    if (!split) return;

    split_k_finish(partial, ticket, out, tile * TILE, TILE, M, N, slices, &last_flag, ep);
}

// Workgroup b's (tile, K slice): consecutive workgroups -- the tiles of one
// K slice, which share scale and zero rows, activations and 128-byte code
// lines -- are placed on one XCD (workgroups are dealt to the XCDs round
// robin); the placement matters for speed only.
__device__ __forceinline__ void place(int b, int tiles, int slices, int& tile, int& slice) {
    const int grid = tiles * slices;
    if ((grid & 7) == 0) b = (b & 7) * (grid >> 3) + (b >> 3);
    tile = b % tiles;
    slice = b / tiles;
}

// XT: the activations' type, f32 or bf16 bits (one-row bf16 products).
template <int M, int TILE, int CPL, bool PIPE, typename XT = float>
__global__ __launch_bounds__(kDecThreads) void int4_decode_f32_kernel(
    const XT* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    void* __restrict__ out, float* partial, uint32_t* tickets, int ticket_stride, int K, int N,
    int rows_per_slice, int slices, Epilogue ep) {
    int tile, slice;
    place(blockIdx.x, N / TILE, slices, tile, slice);
    decode_tile<M, TILE, CPL, PIPE, XT>(a, codes, scales, zeros, out, partial,
                                    tickets + (size_t)tile * ticket_stride, K, N, tile, slice,
                                    rows_per_slice, slices, ep);
}

// Several matrices against one input in one launch (the q, k, v or gate, up
// products of a decode step): the grid is the matrices' column tiles side by
// side, times the K slices; a workgroup finds its matrix from its global
// tile.  Each matrix's results are those of its own launch, bit for bit.
constexpr int kMaxSet = 4;
struct DecodeSet {
    const uint32_t* codes[kMaxSet];
    const uint16_t* scales[kMaxSet];
    const uint16_t* zeros[kMaxSet];
    void* out[kMaxSet];
    float* partial[kMaxSet];
    int n[kMaxSet];
    int tile0[kMaxSet + 1];   // first global tile of each matrix; tile0[count] = all
    int count;
};

template <int M, int TILE, int CPL, bool PIPE>
__global__ __launch_bounds__(kDecThreads) void int4_decode_set_kernel(
    const float* __restrict__ a, DecodeSet set, uint32_t* tickets, int ticket_stride, int K,
    int rows_per_slice, int slices) {
    int tg, slice;
    place(blockIdx.x, set.tile0[set.count], slices, tg, slice);
    int i = 0;
#pragma unroll
    for (int j = 1; j < kMaxSet; j++)
        if (j < set.count && tg >= set.tile0[j]) i = j;
    decode_tile<M, TILE, CPL, PIPE>(a, set.codes[i], set.scales[i], set.zeros[i], set.out[i],
                                    set.partial[i], tickets + (size_t)tg * ticket_stride, K,
                                    set.n[i], tg - set.tile0[i], slice, rows_per_slice, slices,
                                    Epilogue{});
}

// Slices: one batch (kBatch rows a lane) per workgroup, so every workgroup
// waits for one memory latency; past the slice cap a workgroup loops over
// several batches instead (pipelined), which bounds the partial sums and the
// hand-off's reads.
template <int M, int TILE, int CPL, typename XT = float>
hipError_t launch_decode(Device* d, hipStream_t st, const XT* a, Int4Planes w,
                         void* out, int K, int N, int* status, Epilogue ep,
                         void* fixed_scratch = nullptr) {
    constexpr int LPR = TILE / CPL;
    constexpr int RP = kDecThreads / LPR;
    constexpr int kRowsPerBatch = kBatch * RP;
    const int tiles = N / TILE;
    const int batches = (K + kRowsPerBatch - 1) / kRowsPerBatch;
    // One row: up to 64 slices of one batch each.  More rows: up to 32
    // slices, past which a workgroup takes several batches, pipelined (the
    // next batch's loads before the current one's arithmetic).  Measured at
    // K = 14336, N = 4096: M = 1 56 single-batch slices 12.7 us against 28
    // pipelined pairs 13.0; M = 2 19.8 against 18.9; M = 8 55.6 against
    // 42.3.  The pipelined kernel holds more registers, so it is used only
    // where a workgroup has more than one batch.
    const int max_slices = M == 1 ? kMaxSlices : 32;
    const int per_slice = (batches + max_slices - 1) / max_slices;
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
        const size_t bytes = (size_t)slices * M * N * sizeof(float);
        void* ws = nullptr;
        if (fixed_scratch) {
            if (kWorkspaceCounterBytes + bytes > kScratchBytes) {
                *status = fail(ACCEL_E_INVALID,
                               "Int4MatVecNoAlloc: K=%d, N=%d needs %zu bytes of split-K sums "
                               "and the static scratch holds %zu",
                               K, N, bytes, kScratchBytes - kWorkspaceCounterBytes);
                return hipSuccess;
            }
            ws = fixed_scratch;
        } else {
            ws = workspace(d, st, bytes, status);
            if (!ws) return hipSuccess;
        }
        tickets = static_cast<uint32_t*>(ws);
        partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    }
    if (per_slice > 1)
        ACCEL_LAUNCH(tname("int4_decode_f32_kernel", M, TILE, CPL, true, type_name<XT>()) +
                         grid_note(tiles, slices),
                     (int4_decode_f32_kernel<M, TILE, CPL, true, XT>),
                           dim3(tiles * slices), dim3(kDecThreads), 0, st, a, w.codes, w.scales,
                           w.zeros, out, partial, tickets, stride, K, N, rows, slices, ep);
    else
        ACCEL_LAUNCH(tname("int4_decode_f32_kernel", M, TILE, CPL, false, type_name<XT>()) +
                         grid_note(tiles, slices),
                     (int4_decode_f32_kernel<M, TILE, CPL, false, XT>),
                           dim3(tiles * slices), dim3(kDecThreads), 0, st, a, w.codes, w.scales,
                           w.zeros, out, partial, tickets, stride, K, N, rows, slices, ep);
    return launch_status();
}

// Column tile of a one-row product: 512 columns for wide matrices (a row's
// scale and zero lines then serve 256 code bytes instead of 128; measured
// 12.8 -> 12.1 us at K = 4096, N = 14336 and 20.9 -> 18.7 at N = 28672),
// 256 where N allows (at N = 4096 the 512 tile's 32 slices make the hand-off
// longer than the lines it saves: 6.64 against 6.26 us), else 128.  Every
// one-row launch of a matrix -- alone, in a set or without allocation --
// takes the same width, so their results agree bit for bit.
int matvec_tile(int N) {
    if (N >= 8192 && N % 512 == 0) return 512;
    return N % 256 == 0 ? 256 : 128;
}

// Columns per lane by row count: the accumulators (M * CPL) stay near 64.
template <int M, typename XT = float>
hipError_t launch_decode_m(Device* d, hipStream_t st, const XT* a, Int4Planes w,
                           void* out, int K, int N, int* status, Epilogue ep) {
    constexpr int CPL = M <= 2 ? 32 : (M <= 4 ? 16 : 8);
    if constexpr (M == 1) {
        if (matvec_tile(N) == 512)
            return launch_decode<M, 512, CPL, XT>(d, st, a, w, out, K, N, status, ep);
    }
    if (N % 256 == 0)
        return launch_decode<M, 256, CPL, XT>(d, st, a, w, out, K, N, status, ep);
    return launch_decode<M, 128, CPL, XT>(d, st, a, w, out, K, N, status, ep);
}

// ---- MatVecF32F16: f32 activations against f16 weights --------------------
//
// The reference's MatVecF32F16 (internal/kernels/matvec.go:79-105) is the
// M = 1 product a transformer decode step has besides the int4 ones (f16
// weights such as an output projection).  HBM-bound like the int4 matvec and
// built the same way: a 512-lane workgroup owns TILE columns and a K slice;
// a lane owns eight adjacent columns (one 16-byte load a row) and kBatch rows
// of its row phase, all its loads issued before any is used; the row phases
// meet through the same cross-lane and LDS stages, and the slices through
// the same deterministic hand-off.  The f32 sums are formed in a different
// order from the reference's 16-phase one, so results agree to f32 rounding,
// not bit for bit.
template <int TILE>
__global__ __launch_bounds__(kDecThreads) void matvec_f16_kernel(
    const float* __restrict__ a, const uint16_t* __restrict__ w, float* __restrict__ out,
    float* partial, uint32_t* tickets, int ticket_stride, int K, int N, int rows_per_slice,
    int slices) {
    constexpr int CPL = 8;
    constexpr int LPR = TILE / CPL;
    constexpr int RP = kDecThreads / LPR;
    constexpr int RPW = 64 / LPR;
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
    const int k_begin = slice * rows_per_slice;
    const int k_end = min(K, k_begin + rows_per_slice);
    const uint16_t* wcol = w + col0;

    float acc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; j++) acc[j] = 0.0f;
    for (int kb = k_begin; kb < k_end; kb += kBatch * RP) {
        u32x4 q[kBatch];
        float xv[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const int row = min(kb + rp + i * RP, k_end - 1);
            q[i] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(wcol + (size_t)row * N));
        }
#pragma unroll
        for (int i = 0; i < kBatch; i++) xv[i] = a[min(kb + rp + i * RP, k_end - 1)];
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const float c = kb + rp + i * RP < k_end ? xv[i] : 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t pair = q[i][j];
                acc[2 * j] = __builtin_fmaf(c, half_bits_to_float((uint16_t)pair), acc[2 * j]);
                acc[2 * j + 1] =
                    __builtin_fmaf(c, half_bits_to_float((uint16_t)(pair >> 16)), acc[2 * j + 1]);
            }
        }
    }

    constexpr int NV = CPL / RPW;
    transpose_reduce<CPL, 64 / 2, LPR>(acc, l64);
    const int c0 = lane * CPL + reduced_offset<CPL, 64 / 2, LPR>(l64);
#pragma unroll
    for (int e = 0; e < NV; e++) red[wave][c0 + e] = acc[e];
    __syncthreads();
    const bool split = slices > 1;
    for (int c = tid; c < TILE; c += kDecThreads) {
        float sum = 0.0f;
#pragma unroll
        for (int wv = 0; wv < NWAVE; wv++) sum += red[wv][c];
        const int col = tile * TILE + c;
        if (split)
            store_device(&partial[(size_t)slice * N + col], sum);
        else
            out[col] = sum;
    }
    if (!split) return;
    split_k_finish(partial, tickets + (size_t)tile * ticket_stride, out, tile * TILE, TILE, 1, N,
                   slices, &last_flag, Epilogue{});
}

// Any shape: one lane per column, the reference's 16-phase order.
__global__ void matvec_f16_generic_kernel(const float* __restrict__ a,
                                          const uint16_t* __restrict__ w,
                                          float* __restrict__ out, int K, int N) {
    const int col = blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= N) return;
    float sum = 0.0f;
    for (int p = 0; p < 16; p++) {
        float acc = 0.0f;
        for (int k = p; k < K; k += 16)
            acc = __builtin_fmaf(a[k], half_bits_to_float(w[(size_t)k * N + col]), acc);
        sum += acc;
    }
    out[col] = sum;
}

template <int TILE>
hipError_t launch_matvec_f16_tiled(Device* d, hipStream_t st, const float* a, const uint16_t* w,
                                   float* out, int K, int N, int* status) {
    constexpr int LPR = TILE / 8;
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
                           "matvec: N=%d needs more tickets than the workspace holds", N);
            return hipSuccess;
        }
        void* ws = workspace(d, st, (size_t)slices * N * sizeof(float), status);
        if (!ws) return hipSuccess;
        tickets = static_cast<uint32_t*>(ws);
        partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    }
    ACCEL_LAUNCH(tname("matvec_f16_kernel", TILE) + grid_note(tiles, slices), (matvec_f16_kernel<TILE>), dim3(tiles * slices), dim3(kDecThreads), 0, st,
                       a, w, out, partial, tickets, stride, K, N, rows, slices);
    return launch_status();
}

// Any shape: one lane per output element, decoding with the flat index.
__global__ void int4_generic_f32_kernel(const float* __restrict__ a,
                                        const uint32_t* __restrict__ codes,
                                        const uint16_t* __restrict__ scales,
                                        const uint16_t* __restrict__ zeros,
                                        void* __restrict__ out, int M, int K, int N,
                                        Epilogue ep) {
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
    store_out(out, (size_t)i, n, acc, ep);
}

__device__ __forceinline__ float bf16_bits_to_float(uint16_t h) {
    return __uint_as_float((uint32_t)h << 16);
}

__global__ void int4_generic_bf16_kernel(const uint16_t* __restrict__ a,
                                         const uint32_t* __restrict__ codes,
                                         const uint16_t* __restrict__ scales,
                                         const uint16_t* __restrict__ zeros,
                                         uint16_t* __restrict__ out, int M, int K, int N,
                                         const float* __restrict__ bias) {
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
    if (bias) acc = acc + bias[n];
    out[i] = float_to_bf16_bits(acc);
}

// ---- 2..16 rows: the matrix cores ------------------------------------------
//
// With M rows of activations every weight feeds M FMAs, and from two rows the
// VALU (not HBM) bounds a VALU product.  This kernel moves the arithmetic
// onto v_mfma_f32_16x16x32_bf16 and keeps f32 accuracy:
//   * the activation rows are the MFMA's A side (16 rows; rows >= M are
//     clamped copies whose results are never stored), scaled per (row k,
//     group) to v = x * (512 s) and split exactly into three bf16 terms
//     hi + mid + lo (each the RNE rounding of what is left; the residue is
//     below 2^-27 |v|), so three MFMAs per tile give the product of v with
//     an exact B to f32 accuracy;
//   * B is the code itself, q * 2^-9, exact in bf16 (fp8 converter), so
//     A' * B = x * s * q;
//   * the zero point is the per-(row m, group) bias sum_k x * add,
//     add = s == 0 ? z : -z*s, accumulated in f32 on the VALU.
// The MFMA column c of n-tile j of group g is the tile column
// 128 g + 8 c + j, so a lane's eight n-tiles of a group are the eight
// nibbles of one code word (word 16 g + c of a tile row), and the sixteen
// columns of every n-tile lie in one quantisation group, as the A side's
// per-group scale requires.
//
// Memory.  A workgroup (eight waves) owns a tile of 128 G columns (64 G bytes
// of every code row) and a K slice; its waves take the slice's 32-row steps
// in turn.  A step's codes reach LDS with global_load_lds_dwordx4 (no
// registers: each lane's 16 bytes land at the instruction's LDS base + 16 *
// lane, and every lane may name any global chunk), so each instruction reads
// whole 64 G-byte row segments, and the MFMA layout -- one word of eight rows
// per lane -- is read back with ds_read2(st64)_b32.  Rows are placed (row
// slot, XOR of the 16-byte chunk) so that those reads are free of bank
// conflicts.  The step's scales and zeros arrive the same way; one lane per
// (row, group) folds them into (512 s, add) in LDS for the whole wave.  Each
// wave keeps kDepth steps in flight in its own LDS ring, so no barrier is
// needed until the epilogue.  The compiler does not order LDS reads after
// LDS-direct loads, so each step waits for its own loads explicitly
// (s_waitcnt vmcnt counting the loads issued after it).
//
// The waves' sums meet in LDS; with one slice they are the output, else the
// split-K hand-off below combines the slices (in slice order).

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kMfLdsBytes = 155648;   // 152 KiB of the 160 KiB a workgroup may hold

// Geometry of a tile of G quantisation groups (128 G columns) worked by NW
// waves.  A step is 32 rows; its LDS buffer holds the codes, the 16 x 32
// activations, the raw scales and zeros and their fold.
// SIDE: the step's scales and zeros come from a bind-time side copy
// (int4_side_prepare_kernel), one contiguous 128-byte block per (group,
// step) -- 32 scales, then 32 zeros -- instead of one 2- or 4-byte piece from
// each of the step's 32 rows of the two planes.  With two groups a step then
// takes one block per group, each its own 256-byte raw area.
template <int G, int NW, bool SIDE = false>
struct MfTile {
    static constexpr int kThreads = 64 * NW;
    static constexpr int kCols = 128 * G;
    static constexpr int kRowBytes = 64 * G;            // codes of one tile row
    static constexpr int kChunks = 4 * G;               // 16-byte chunks per tile row
    static constexpr int kCodeBytes = 32 * kRowBytes;
    static constexpr int kXBytes = 16 * 32 * 4;
    static constexpr int kRawBytes = SIDE ? 256 * G : 256;   // scales, then zeros: a dword a row
    static constexpr int kFoldBytes = 256 * G;          // (512 s, add) per (row, group)
    static constexpr int kXOff = kCodeBytes;
    static constexpr int kRawOff = kXOff + kXBytes;
    static constexpr int kFoldOff = kRawOff + kRawBytes;
    static constexpr int kStepBytes = kFoldOff + kFoldBytes;
    static constexpr int kDepth = kMfLdsBytes / (NW * kStepBytes);
    static constexpr int kCodeDma = kCodeBytes / 1024;  // 1 KiB per instruction
    static constexpr int kVmemPerStep = kCodeDma + 2 + (SIDE ? G : 1);   // + activations, scale/zero
    static constexpr int kItems = 16 * kCols / 4 / kThreads;  // f32x4 outputs per lane
    static_assert(kDepth >= 2 && kDepth <= 8, "ring depth");
    static_assert(NW * 16 * (kCols + 4 + G) * 4 <= kMfLdsBytes, "reduction LDS");
    static_assert(kItems >= 1 && 16 * kCols / 4 == kItems * kThreads, "items");
};

// LDS row slot of step row r (0..31) and the XOR applied to its 16-byte
// chunk index.  Lane (c, kg) reads word 16 g + c of rows 8 kg + e; these
// place the four kg rows of one read in four different 16-bank ranges (and
// two different ones within each half wave).
template <int G>
__device__ __forceinline__ int mf_row_slot(int r) {
    if constexpr (G == 1) return r ^ ((r >> 3) & 3);
    else return r ^ ((r >> 4) & 1);
}
template <int G>
__device__ __forceinline__ int mf_chunk_xor(int r) {
    if constexpr (G == 1) return 0;
    else return 4 * ((r >> 3) & 1);
}
// Position of 16-byte chunk q (0..7) of activation row m in its 128-byte LDS
// row: the sixteen rows' reads of one chunk fall in sixteen bank groups.
__device__ __forceinline__ int mf_x_pos(int m, int q) { return q ^ ((m >> 1) & 7); }

// LDS-direct loads: `bytes` per lane from `src` to lds_dst + bytes * lane
// (lds_dst uniform).  Non-template wrappers, so that host compilation of
// the kernel templates never instantiates the LDS address-space casts.
__device__ __forceinline__ void lds_load16(const void* src, uint8_t* lds_dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_dst, 16, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void* src, uint8_t* lds_dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_dst, 4, 0, 0);
}
__device__ __forceinline__ void lds_load2(const void* src, uint8_t* lds_dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_dst, 2, 0, 0);
}
// Byte address of an LDS location, as ds_* instructions take it.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return (uint32_t)(uintptr_t)(lds_void*)p;
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waits until at most V * q vector-memory loads are outstanding, q < D.
template <int V, int D>
__device__ __forceinline__ void wait_vmem_steps(int q) {
    if constexpr (D > 1) {
        if (q == D - 1) {
            wait_vmem<V * (D - 1)>();
            return;
        }
        wait_vmem_steps<V, D - 1>(q);
    } else {
        wait_vmem<0>();
    }
}

// Two values -> three bf16 pairs whose sum is (v0, v1) to 2^-27 relative:
// each term is the RNE bf16 of what the previous ones leave, and the
// remainder v - term is exact in f32, taken with one v_dot2 (-1 * term + v).
// The pairs (-1, 0) and (0, -1) come in as SGPRs: the compiler would encode
// the first as the inline constant -1.0, which the hardware does not expand
// to bf16 -1 in the low half.
__device__ __forceinline__ bf16x2 bf16_pair_bits(uint32_t bits) {
    uint32_t r;
    asm("s_mov_b32 %0, %1" : "=s"(r) : "i"(bits));
    return __builtin_bit_cast(bf16x2, r);
}
__device__ __forceinline__ void split3(float v0, float v1, uint32_t& hi, uint32_t& mid,
                                       uint32_t& lo) {
    const bf16x2 m10 = bf16_pair_bits(0x0000BF80u);   // (-1, 0)
    const bf16x2 m01 = bf16_pair_bits(0xBF800000u);   // (0, -1)
    const bf16x2 h = __builtin_convertvector((f32x2){v0, v1}, bf16x2);
    const float r0 = __builtin_amdgcn_fdot2_f32_bf16(h, m10, v0, false);
    const float r1 = __builtin_amdgcn_fdot2_f32_bf16(h, m01, v1, false);
    const bf16x2 m = __builtin_convertvector((f32x2){r0, r1}, bf16x2);
    const float s0 = __builtin_amdgcn_fdot2_f32_bf16(m, m10, r0, false);
    const float s1 = __builtin_amdgcn_fdot2_f32_bf16(m, m01, r1, false);
    const bf16x2 l = __builtin_convertvector((f32x2){s0, s1}, bf16x2);
    hi = __builtin_bit_cast(uint32_t, h);
    mid = __builtin_bit_cast(uint32_t, m);
    lo = __builtin_bit_cast(uint32_t, l);
}

// Eight code words (rows 2p, 2p+1 paired) -> the B operands of the eight
// n-tiles (nibble j of each word), as bf16 q * 2^-9.
__device__ __forceinline__ void codes_to_b(const uint32_t (&w)[8], bf16x8 (&b)[8]) {
    uint32_t bw[8][4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t w0 = w[2 * p], w1 = w[2 * p + 1];
        const uint32_t t01 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);  // bytes 0,1
        const uint32_t t23 = __builtin_amdgcn_perm(w1, w0, 0x07030602u);  // bytes 2,3
        const uint32_t q[4] = {t01 & 0x0F0F0F0Fu, (t01 >> 4) & 0x0F0F0F0Fu,
                               t23 & 0x0F0F0F0Fu, (t23 >> 4) & 0x0F0F0F0Fu};
        // q[0]: nibbles 0, 2; q[1]: 1, 3; q[2]: 4, 6; q[3]: 5, 7
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const int c0 = (h >> 1) * 4 + (h & 1);
            bw[c0][p] = __builtin_bit_cast(
                uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[h], 1.0f, false));
            bw[c0 + 2][p] = __builtin_bit_cast(
                uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[h], 1.0f, true));
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++)
        b[j] = __builtin_bit_cast(bf16x8, (u32x4){bw[j][0], bw[j][1], bw[j][2], bw[j][3]});
}

// One workgroup's share: column tile `tile`, K slice `slice`; `ticket` is
// the tile's pair of hand-off counters.
// XT: the activations' type, f32 or bf16 bits (a bf16 step is one 16-byte
// chunk a lane, eight values, widened in registers).
template <int G, int NW, typename XT = float, bool SIDE = false>
__device__ __forceinline__ void decode_mfma_tile(
    const XT* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    void* __restrict__ out, float* partial, uint32_t* ticket, int M, int K, int N, int tile,
    int slice, int rows_per_slice, int slices, const Epilogue& ep, uint32_t* fault,
    int wait_limit, const uint16_t* __restrict__ side = nullptr) {
    using T = MfTile<G, NW, SIDE>;
    constexpr bool kBf16X = sizeof(XT) == 2;
    constexpr int kXDma = kBf16X ? 1 : 2;                 // activation loads a step
    constexpr int D = T::kDepth;
    constexpr int V = T::kVmemPerStep - 2 + kXDma;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kMfLdsBytes];
    __shared__ int last_flag;
    __shared__ int waited;

    const int n0 = tile * T::kCols;
    const int g0 = tile * G;
    const size_t gpr = (size_t)(N >> 7);           // groups per row
    const size_t row_bytes = (size_t)(N >> 1);
    const int k_begin = slice * rows_per_slice;
    const int k_end = min(K, k_begin + rows_per_slice);
    const int nsteps = (k_end - k_begin) >> 5;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int c16 = lane & 15;
    const int kg = lane >> 4;
    const int my_steps = wave < nsteps ? (nsteps - wave + NW - 1) / NW : 0;

    uint8_t* ring = lds + wave * (D * T::kStepBytes);

    // This lane's global sources, relative to a step's first row.
    const uint8_t* code_tile = reinterpret_cast<const uint8_t*>(codes) + (size_t)n0 / 2;
    uint32_t code_off[T::kCodeDma];
#pragma unroll
    for (int i = 0; i < T::kCodeDma; i++) {
        const int s = 64 * i + lane;
        const int r = mf_row_slot<G>(s / T::kChunks);   // the slot map is an involution
        const int ch = (s % T::kChunks) ^ mf_chunk_xor<G>(r);
        code_off[i] = (uint32_t)r * (uint32_t)row_bytes + 16u * (uint32_t)ch;
    }
    // activations: instruction j, lane l fills position (64 j + l) % 8 of row
    // (64 j + l) / 8 of the step's 16 x 32 block (rows >= M repeat row M - 1);
    // bf16: one instruction, lane l fills chunk l % 4 (eight values) of row l / 4
    const XT* x_src[2];
    if constexpr (kBf16X) {
        x_src[0] = x_src[1] = a + (size_t)min(lane >> 2, M - 1) * K + 8 * (lane & 3);
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int s = 64 * j + lane;
            const int m = s >> 3;
            x_src[j] = a + (size_t)min(m, M - 1) * K + 4 * mf_x_pos(m, s & 7);
        }
    }
    // scales (lanes 0..31) or zeros (32..63) of row lane % 32: G f16 values,
    // landing in dword `lane` of the step's raw block
    const uint16_t* raw_src =
        SIDE ? nullptr : (lane < 32 ? scales : zeros) + (size_t)(lane & 31) * gpr + g0;
    // side copy: the blocks of group g0 (group g's are side_group further),
    // lane l taking entry l of a block
    const size_t side_group = (size_t)(K >> 5) * 64;
    const uint16_t* side_src = SIDE ? side + (size_t)g0 * side_group + lane : nullptr;

    auto issue = [&](int i, int slot) {
        const int row0 = k_begin + 32 * (wave + NW * i);
        uint8_t* buf = ring + slot * T::kStepBytes;
        const uint8_t* src = code_tile + (size_t)row0 * row_bytes;
#pragma unroll
        for (int c = 0; c < T::kCodeDma; c++) lds_load16(src + code_off[c], buf + 1024 * c);
#pragma unroll
        for (int j = 0; j < kXDma; j++) lds_load16(x_src[j] + row0, buf + T::kXOff + 1024 * j);
        if constexpr (SIDE) {
            // group g's block of this step: 32 scales, then 32 zeros
#pragma unroll
            for (int g = 0; g < G; g++)
                lds_load2(side_src + (size_t)g * side_group + (size_t)(row0 >> 5) * 64,
                          buf + T::kRawOff + 256 * g);
        } else if constexpr (G == 1) {
            lds_load2(raw_src + (size_t)row0 * gpr, buf + T::kRawOff);
        } else {
            lds_load4(raw_src + (size_t)row0 * gpr, buf + T::kRawOff);
        }
    };

    // LDS byte addresses (within a step buffer) of this lane's reads.
    // Codes: row 8 kg + e of word 16 g + c16 (see mf_row_slot); two bases
    // per group whose rows sit 256 bytes apart.
    const uint32_t ring_lds = lds_address(ring);
    uint32_t cbase[4];
    if constexpr (G == 1) {
        // row 8 kg + 4 h + l sits in slot 8 kg + 4 h + (l ^ kg): base l, + 256 h
#pragma unroll
        for (int l = 0; l < 4; l++) cbase[l] = 512 * kg + 64 * (l ^ kg) + 4 * c16;
    } else {
        // row 8 kg + e sits in slot 8 kg + (e ^ (kg >> 1)), its chunks XOR
        // 4 (kg & 1): even e from one base, odd e from the other, + 256 (e / 2)
        const int bb = kg >> 1;
#pragma unroll
        for (int g = 0; g < 2; g++) {
            const uint32_t goff = 64 * (g ^ (kg & 1)) + 4 * c16 + 1024 * kg;
            cbase[2 * g] = goff + 128 * bb;
            cbase[2 * g + 1] = goff + 128 * (1 - bb);
        }
    }
    // activations: row c16, columns 8 kg .. 8 kg + 7 (bf16: one chunk, read
    // twice so that the read sequence stays that of f32)
    const uint32_t xoff0 = kBf16X ? T::kXOff + 64 * c16 + 16 * kg
                                  : T::kXOff + 128 * c16 + 16 * mf_x_pos(c16, 2 * kg);
    const uint32_t xoff1 = kBf16X ? xoff0
                                  : T::kXOff + 128 * c16 + 16 * mf_x_pos(c16, 2 * kg + 1);
    // fold: rows 8 kg .. 8 kg + 7, all groups; the lane folding (row, group)
    // pair `fold_p` (G == 1: lanes 16 r + e, e < 8, fold row 8 r + e)
    const uint32_t foff = T::kFoldOff + 64 * G * kg;
    const int fold_p = G == 2 ? lane : 8 * (lane >> 4) + (lane & 7);
    // LDS-direct loads of fewer than 16 bytes land one dword per lane: the
    // scales of row r at 4 r (group g at + 2 g), the zeros 128 bytes on
    // (with the side copy and two groups, group g's pieces sit in raw area g)
    const uint32_t raw_off = G == 2 ? (SIDE ? 256 * (fold_p & 1) + 4 * (fold_p >> 1) : 2 * fold_p)
                                    : 4 * fold_p;
    const bool folds = G == 2 || (lane & 15) < 8;

    f32x4 acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[g][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float bias[G];
#pragma unroll
    for (int g = 0; g < G; g++) bias[g] = 0.0f;

    // Reads of LDS-direct data are inline asm with their own lgkmcnt wait:
    // the compiler cannot tell LDS-direct loads' addresses from other LDS
    // accesses and would wait for every outstanding load (vmcnt(0)) before
    // them, which drains the ring.  Their order is fixed by the asm blocks;
    // LDS operations of one wave complete in order.
    auto compute = [&](int slot) {
        const uint32_t sb = ring_lds + slot * T::kStepBytes;
        // one lane per (row, group): (512 s, add), written back for the wave
        if (folds) {
            uint32_t sr, zr;
            asm volatile(
                "ds_read_u16 %0, %2\n\t"
                "ds_read_u16 %1, %2 offset:128\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(sr), "=&v"(zr)
                : "v"(sb + T::kRawOff + raw_off));
            const float s = half_bits_to_float((uint16_t)sr);
            const float z = half_bits_to_float((uint16_t)zr);
            const f32x2 f = {s * kNibbleScale, s == 0.0f ? z : -(z * s)};
            asm volatile("ds_write_b64 %0, %1" ::"v"(sb + T::kFoldOff + 8 * fold_p),
                         "v"(__builtin_bit_cast(uint64_t, f))
                         : "memory");
        }
        f32x4 x0, x1;
        f32x4 fv[4 * G];
        u32x2 wp[G][4];   // (rows e, e + 2) for G == 2, (l, l + 4) for G == 1
        if constexpr (G == 1) {
            asm volatile(
                "ds_read_b128 %0, %10\n\t"
                "ds_read_b128 %1, %11\n\t"
                "ds_read_b128 %2, %12\n\t"
                "ds_read_b128 %3, %12 offset:16\n\t"
                "ds_read_b128 %4, %12 offset:32\n\t"
                "ds_read_b128 %5, %12 offset:48\n\t"
                "ds_read2_b32 %6, %13 offset1:64\n\t"
                "ds_read2_b32 %7, %14 offset1:64\n\t"
                "ds_read2_b32 %8, %15 offset1:64\n\t"
                "ds_read2_b32 %9, %16 offset1:64\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(x0), "=&v"(x1), "=&v"(fv[0]), "=&v"(fv[1]), "=&v"(fv[2]),
                  "=&v"(fv[3]), "=&v"(wp[0][0]), "=&v"(wp[0][1]), "=&v"(wp[0][2]),
                  "=&v"(wp[0][3])
                : "v"(sb + xoff0), "v"(sb + xoff1), "v"(sb + foff), "v"(sb + cbase[0]),
                  "v"(sb + cbase[1]), "v"(sb + cbase[2]), "v"(sb + cbase[3])
                : "memory");
        } else {
            asm volatile(
                "ds_read_b128 %0, %18\n\t"
                "ds_read_b128 %1, %19\n\t"
                "ds_read_b128 %2, %20\n\t"
                "ds_read_b128 %3, %20 offset:16\n\t"
                "ds_read_b128 %4, %20 offset:32\n\t"
                "ds_read_b128 %5, %20 offset:48\n\t"
                "ds_read_b128 %6, %20 offset:64\n\t"
                "ds_read_b128 %7, %20 offset:80\n\t"
                "ds_read_b128 %8, %20 offset:96\n\t"
                "ds_read_b128 %9, %20 offset:112\n\t"
                "ds_read2st64_b32 %10, %21 offset1:1\n\t"
                "ds_read2st64_b32 %11, %21 offset0:2 offset1:3\n\t"
                "ds_read2st64_b32 %12, %22 offset1:1\n\t"
                "ds_read2st64_b32 %13, %22 offset0:2 offset1:3\n\t"
                "ds_read2st64_b32 %14, %23 offset1:1\n\t"
                "ds_read2st64_b32 %15, %23 offset0:2 offset1:3\n\t"
                "ds_read2st64_b32 %16, %24 offset1:1\n\t"
                "ds_read2st64_b32 %17, %24 offset0:2 offset1:3\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(x0), "=&v"(x1), "=&v"(fv[0]), "=&v"(fv[1]), "=&v"(fv[2]),
                  "=&v"(fv[3]), "=&v"(fv[4]), "=&v"(fv[5]), "=&v"(fv[6]), "=&v"(fv[7]),
                  "=&v"(wp[0][0]), "=&v"(wp[0][1]), "=&v"(wp[0][2]), "=&v"(wp[0][3]),
                  "=&v"(wp[1][0]), "=&v"(wp[1][1]), "=&v"(wp[1][2]), "=&v"(wp[1][3])
                : "v"(sb + xoff0), "v"(sb + xoff1), "v"(sb + foff), "v"(sb + cbase[0]),
                  "v"(sb + cbase[1]), "v"(sb + cbase[2]), "v"(sb + cbase[3])
                : "memory");
        }
        float xv[8];
        if constexpr (kBf16X) {
            const u32x4 r = __builtin_bit_cast(u32x4, x0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                xv[2 * i] = __uint_as_float(r[i] << 16);
                xv[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
            }
        } else {
            xv[0] = x0.x; xv[1] = x0.y; xv[2] = x0.z; xv[3] = x0.w;
            xv[4] = x1.x; xv[5] = x1.y; xv[6] = x1.z; xv[7] = x1.w;
        }
        f32x2 fe[G][8];
#pragma unroll
        for (int q = 0; q < 4 * G; q++) {
            const int p0 = 2 * q, p1 = 2 * q + 1;   // (row, group) pairs p = e * G + g
            fe[p0 % G][p0 / G] = (f32x2){fv[q].x, fv[q].y};
            fe[p1 % G][p1 / G] = (f32x2){fv[q].z, fv[q].w};
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            uint32_t w[8];
            if constexpr (G == 1) {
#pragma unroll
                for (int l = 0; l < 4; l++) {
                    w[l] = wp[0][l].x;
                    w[l + 4] = wp[0][l].y;
                }
            } else {
                // even base: (0, 2), (4, 6); odd base: (1, 3), (5, 7)
                w[0] = wp[g][0].x; w[2] = wp[g][0].y; w[4] = wp[g][1].x; w[6] = wp[g][1].y;
                w[1] = wp[g][2].x; w[3] = wp[g][2].y; w[5] = wp[g][3].x; w[7] = wp[g][3].y;
            }
            uint32_t ah[4], am[4], al[4];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const float v0 = xv[2 * p] * fe[g][2 * p].x;
                const float v1 = xv[2 * p + 1] * fe[g][2 * p + 1].x;
                bias[g] = __builtin_fmaf(xv[2 * p], fe[g][2 * p].y, bias[g]);
                bias[g] = __builtin_fmaf(xv[2 * p + 1], fe[g][2 * p + 1].y, bias[g]);
                split3(v0, v1, ah[p], am[p], al[p]);
            }
            const bf16x8 Ah = __builtin_bit_cast(bf16x8, (u32x4){ah[0], ah[1], ah[2], ah[3]});
            const bf16x8 Am = __builtin_bit_cast(bf16x8, (u32x4){am[0], am[1], am[2], am[3]});
            const bf16x8 Al = __builtin_bit_cast(bf16x8, (u32x4){al[0], al[1], al[2], al[3]});
            bf16x8 bq[8];
            codes_to_b(w, bq);
#pragma unroll
            for (int j = 0; j < 8; j++)
                acc[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ah, bq[j], acc[g][j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 8; j++)
                acc[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Am, bq[j], acc[g][j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 8; j++)
                acc[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Al, bq[j], acc[g][j], 0, 0, 0);
        }
    };

    // The ring: D - 1 steps in flight ahead of the one being computed.  A
    // slot is refilled only after the step that used it has been computed
    // (its LDS reads have returned: their values fed that step's MFMAs).
    // Every load of a step is issued before any load of a later step, so
    // "at most V * q loads outstanding", q = the steps issued after it,
    // means the step has landed.
#pragma unroll
    for (int u = 0; u < D - 1; u++)
        if (u < my_steps) issue(u, u);
    for (int base = 0; base < my_steps; base += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            const int i = base + u;
            if (i < my_steps) {
                __builtin_amdgcn_sched_barrier(0);
                if (i + D - 1 < my_steps) issue(i + D - 1, (u + D - 1) % D);
                wait_vmem_steps<V, D>(min(D - 1, my_steps - 1 - i));
                __builtin_amdgcn_sched_barrier(0);
                compute(u);
            }
        }
    }

    // ---- epilogue: the waves' sums meet in LDS --------------------------
    constexpr int C4 = T::kCols / 4;
    // the fused bias of this lane's output items, fetched now so that its
    // latency overlaps the reduction
    f32x4 ebias[T::kItems];
#pragma unroll
    for (int u = 0; u < T::kItems; u++) {
        const int it = tid + T::kThreads * u;
        const int c = n0 + 4 * (it % C4);
        ebias[u] = (f32x4){0.f, 0.f, 0.f, 0.f};
        if (ep.bias && it / C4 < M)
            ebias[u] = (f32x4){ep.bias[c], ep.bias[c + 1], ep.bias[c + 2], ep.bias[c + 3]};
    }
    __syncthreads();
    // rows padded by four floats: the four kg rows a store instruction
    // writes land in different banks
    constexpr int RS = T::kCols + 4;
    float* red = reinterpret_cast<float*>(lds);                       // [wave][16][RS]
    float* red_bias = red + NW * 16 * RS;                             // [wave][16][G]
#pragma unroll
    for (int g = 0; g < G; g++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float* dst = red + (size_t)(wave * 16 + 4 * kg + i) * RS + 128 * g + 8 * c16;
            *reinterpret_cast<f32x4*>(dst) =
                (f32x4){acc[g][0][i], acc[g][1][i], acc[g][2][i], acc[g][3][i]};
            *reinterpret_cast<f32x4*>(dst + 4) =
                (f32x4){acc[g][4][i], acc[g][5][i], acc[g][6][i], acc[g][7][i]};
        }
        float bs = bias[g];
        bs += __shfl_xor(bs, 16, 64);
        bs += __shfl_xor(bs, 32, 64);
        if (kg == 0) red_bias[(wave * 16 + c16) * G + g] = bs;
    }
    __syncthreads();

    f32x4 val[T::kItems];
    int item_m[T::kItems], item_c[T::kItems];
#pragma unroll
    for (int u = 0; u < T::kItems; u++) {
        const int it = tid + T::kThreads * u;
        const int m = it / C4;
        const int c = 4 * (it % C4);
        item_m[u] = m;
        item_c[u] = c;
        f32x4 s = (f32x4){0.f, 0.f, 0.f, 0.f};
        float bsum = 0.0f;
        if (m < M) {
#pragma unroll
            for (int w = 0; w < NW; w++)
                s += *reinterpret_cast<const f32x4*>(red + (size_t)(w * 16 + m) * RS + c);
#pragma unroll
            for (int w = 0; w < NW; w++) bsum += red_bias[(w * 16 + m) * G + c / 128];
        }
        val[u] = s + bsum;
    }

    if (slices == 1) {
#pragma unroll
        for (int u = 0; u < T::kItems; u++) {
            if (item_m[u] >= M) continue;
            const size_t o = (size_t)item_m[u] * N + n0 + item_c[u];
            const f32x4 v = ep.bias ? val[u] + ebias[u] : val[u];
            store_value(out, o, v.x, ep.bf16);
            store_value(out, o + 1, v.y, ep.bf16);
            store_value(out, o + 2, v.z, ep.bf16);
            store_value(out, o + 3, v.w, ep.bf16);
        }
        return;
    }

    // ---- split-K hand-off -----------------------------------------------
    // Arrival first: a workgroup draws its tile's arrival ticket as soon as
    // its sums are ready.  Every workgroup but the last stores its sums
    // (device scope), waits until they are acknowledged and then counts
    // itself done.  The last arriver keeps its own sums in registers, waits
    // until the others -- all of which hold tickets, so all are running and
    // none waits on anything -- are done, and adds the slices in slice order.
    // This takes the last arriver's store round trip off the critical path.
    const size_t slice_stride = (size_t)M * N;
    uint32_t* arrive = ticket;
    uint32_t* done = arrive + 1;
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        last_flag = prev == (uint32_t)(slices - 1);
    }
    __syncthreads();
    if (!last_flag) {
#pragma unroll
        for (int u = 0; u < T::kItems; u++) {
            if (item_m[u] >= M) continue;
            uint64_t* p = reinterpret_cast<uint64_t*>(partial + slice * slice_stride +
                                                      (size_t)item_m[u] * N + n0 + item_c[u]);
            __hip_atomic_store(p, __builtin_bit_cast(uint64_t, (f32x2){val[u].x, val[u].y}),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p + 1, __builtin_bit_cast(uint64_t, (f32x2){val[u].z, val[u].w}),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __syncthreads();
        if (tid == 0)
            __hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (tid == 0) {
        // Bounded: every workgroup counted in `arrive` is running toward
        // `done`.  Should the bound run out all the same, the workgroup
        // reports it in the fault word and leaves the output and the
        // counters alone (a late workgroup may still count itself done; the
        // host clears the counters when it reads the fault).
        int ok = 0;
        for (int spin = 0; spin < wait_limit; spin++) {
            if (__hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                (uint32_t)(slices - 1)) {
                ok = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!ok)
            __hip_atomic_fetch_or(fault, kFaultWaitGaveUp, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_SYSTEM);
        waited = ok;
    }
    __syncthreads();
    if (!waited) return;
    // every slice's sums in slice order, eight slices' loads in flight at a
    // time; this workgroup's own come from registers
    f32x4 sum[T::kItems];
#pragma unroll
    for (int u = 0; u < T::kItems; u++) sum[u] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < slices; s0 += 8) {
        f32x4 v[T::kItems][8];
#pragma unroll
        for (int u = 0; u < T::kItems; u++) {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int sl = s0 + q;
                v[u][q] = val[u];
                if (item_m[u] < M && sl < slices && sl != slice) {
                    uint64_t* p = reinterpret_cast<uint64_t*>(
                        partial + sl * slice_stride + (size_t)item_m[u] * N + n0 + item_c[u]);
                    const f32x2 lo = __builtin_bit_cast(
                        f32x2, __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                    const f32x2 hi = __builtin_bit_cast(
                        f32x2,
                        __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                    v[u][q] = (f32x4){lo.x, lo.y, hi.x, hi.y};
                }
            }
        }
#pragma unroll
        for (int u = 0; u < T::kItems; u++)
#pragma unroll
            for (int q = 0; q < 8; q++)
                if (s0 + q < slices) sum[u] += v[u][q];
    }
#pragma unroll
    for (int u = 0; u < T::kItems; u++) {
        if (item_m[u] >= M) continue;
        const size_t o = (size_t)item_m[u] * N + n0 + item_c[u];
        const f32x4 v = ep.bias ? sum[u] + ebias[u] : sum[u];
        store_value(out, o, v.x, ep.bf16);
        store_value(out, o + 1, v.y, ep.bf16);
        store_value(out, o + 2, v.z, ep.bf16);
        store_value(out, o + 3, v.w, ep.bf16);
    }
    if (tid == 0) {
        __hip_atomic_store(arrive, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int G, int NW, typename XT = float>
__global__ __launch_bounds__(64 * NW) void int4_decode_mfma_kernel(
    const XT* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    void* __restrict__ out, float* partial, uint32_t* tickets, int ticket_stride, int M, int K,
    int N, int rows_per_slice, int slices, Epilogue ep, uint32_t* fault, int wait_limit) {
    using T = MfTile<G, NW>;
    const int tiles = N / T::kCols;
    const int grid = tiles * slices;
    int b = blockIdx.x;
    if ((grid & 7) == 0) b = (b & 7) * (grid >> 3) + (b >> 3);
    const int tile = b % tiles;
    const int slice = b / tiles;
    decode_mfma_tile<G, NW, XT>(a, codes, scales, zeros, out, partial,
                                tickets + (size_t)tile * ticket_stride, M, K, N, tile, slice,
                                rows_per_slice, slices, ep, fault, wait_limit);
}

// The same product over prepared weights: the codes in the reference order
// and the scales and zeros from the side copy (see MfTile).
template <int G, int NW>
__global__ __launch_bounds__(64 * NW) void int4_decode_mfma_side_kernel(
    const float* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ side, float* __restrict__ out, float* partial,
    uint32_t* tickets, int ticket_stride, int M, int K, int N, int rows_per_slice, int slices,
    uint32_t* fault, int wait_limit) {
    using T = MfTile<G, NW, true>;
    const int tiles = N / T::kCols;
    const int grid = tiles * slices;
    int b = blockIdx.x;
    if ((grid & 7) == 0) b = (b & 7) * (grid >> 3) + (b >> 3);
    const int tile = b % tiles;
    const int slice = b / tiles;
    decode_mfma_tile<G, NW, float, true>(a, codes, nullptr, nullptr, out, partial,
                                         tickets + (size_t)tile * ticket_stride, M, K, N, tile,
                                         slice, rows_per_slice, slices, Epilogue{}, fault,
                                         wait_limit, side);
}

// Several matrices against one activation block in one launch, each with the
// plan (slices, rows) its own launch would take, so each result is its own
// launch's bit for bit: the grid is the matrices' workgroups side by side.
// The hand-off waits only on workgroups that already hold tickets, so a set
// larger than the chip drains like consecutive launches.
struct MfSet {
    const uint32_t* codes[kMaxSet];
    const uint16_t* scales[kMaxSet];
    const uint16_t* zeros[kMaxSet];
    const uint16_t* side[kMaxSet];   // the side copies (SIDE launches)
    void* out[kMaxSet];
    float* partial[kMaxSet];
    int n[kMaxSet];
    int rows[kMaxSet];
    int slices[kMaxSet];
    int wg0[kMaxSet + 1];    // first workgroup of each matrix; wg0[count] = grid
    int tick0[kMaxSet];      // first ticket pair of each matrix
    int count;
};

template <int G, int NW, bool SIDE>
__device__ __forceinline__ void decode_mfma_set_body(const float* __restrict__ a,
                                                     const MfSet& set, uint32_t* tickets,
                                                     int ticket_stride, int M, int K,
                                                     uint32_t* fault, int wait_limit) {
    using T = MfTile<G, NW, SIDE>;
    const int grid = set.wg0[set.count];
    int b = blockIdx.x;
    if ((grid & 7) == 0) b = (b & 7) * (grid >> 3) + (b >> 3);
    int i = 0;
#pragma unroll
    for (int j = 1; j < kMaxSet; j++)
        if (j < set.count && b >= set.wg0[j]) i = j;
    const int bl = b - set.wg0[i];
    const int tiles = set.n[i] / T::kCols;
    const int tile = bl % tiles;
    const int slice = bl / tiles;
    decode_mfma_tile<G, NW, float, SIDE>(
        a, set.codes[i], set.scales[i], set.zeros[i], set.out[i], set.partial[i],
        tickets + (size_t)(set.tick0[i] + tile) * ticket_stride, M, K, set.n[i], tile, slice,
        set.rows[i], set.slices[i], Epilogue{}, fault, wait_limit, set.side[i]);
}

template <int G, int NW>
__global__ __launch_bounds__(64 * NW) void int4_decode_mfma_set_kernel(
    const float* __restrict__ a, MfSet set, uint32_t* tickets, int ticket_stride, int M, int K,
    uint32_t* fault, int wait_limit) {
    decode_mfma_set_body<G, NW, false>(a, set, tickets, ticket_stride, M, K, fault, wait_limit);
}

// The set over prepared weights (side copies of the scales and zeros).
template <int G, int NW>
__global__ __launch_bounds__(64 * NW) void int4_decode_mfma_side_set_kernel(
    const float* __restrict__ a, MfSet set, uint32_t* tickets, int ticket_stride, int M, int K,
    uint32_t* fault, int wait_limit) {
    decode_mfma_set_body<G, NW, true>(a, set, tickets, ticket_stride, M, K, fault, wait_limit);
}

struct MfPlan {
    int groups;   // G
    int slices;
    int rows;     // per slice, a multiple of 32
};

// Tile width and K slices: at most one workgroup per CU (a workgroup holds
// 152 KiB of LDS, so more would wait for a second round), and the last
// workgroup of a tile reads at most 128 / (G M) slices' sums (64 KiB at
// M = 16).  Two-group tiles (128-byte
// row segments) when the planes allow them and they fill the CUs as well
// as one-group tiles do.
MfPlan plan_decode_mfma(const Device* d, int M, int K, int N, bool planes_4b) {
    MfPlan best{1, 1, K};
    int best_wgs = -1;
    for (int G = 2; G >= 1; G--) {
        if (G == 2 && (N % 256 != 0 || !planes_4b)) continue;
        const int tiles = N / (128 * G);
        // one workgroup per CU: more would run in a second round
        int slices = std::max(1, d->cu_count / tiles);
        slices = std::max(1, std::min(slices, 128 / (G * M)));
        slices = std::min(slices, std::max(1, K / 256));
        const int rows = (K / 32 + slices - 1) / slices * 32;
        slices = (K + rows - 1) / rows;
        const int wgs = std::min(tiles * slices, d->cu_count);
        if (wgs > best_wgs) {
            best_wgs = wgs;
            best = MfPlan{G, slices, rows};
        }
    }
    return best;
}

template <int G, int NW, typename XT = float, bool SIDE = false>
hipError_t launch_mfma(Device* d, hipStream_t st, const XT* a, Int4Planes w, void* out,
                       int M, int K, int N, const MfPlan& p, int* status, Epilogue ep,
                       const uint16_t* side = nullptr) {
    static_assert(!SIDE || std::is_same<XT, float>::value, "prepared products read f32");
    const int tiles = N / (128 * G);
    float* partial = nullptr;
    uint32_t* tickets = nullptr;
    int stride = 0;
    if (p.slices > 1) {
        stride = ticket_stride(tiles);   // two counters a tile: arrivals, stores done
        if (stride < 2) {
            *status = fail(ACCEL_E_INVALID,
                           "decode product: N=%d needs more tickets than the workspace holds", N);
            return hipSuccess;
        }
        void* ws = workspace(d, st, (size_t)p.slices * M * N * sizeof(float), status);
        if (!ws) return hipSuccess;
        tickets = static_cast<uint32_t*>(ws);
        partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    }
    if constexpr (SIDE)
        ACCEL_LAUNCH(tname("int4_decode_mfma_side_kernel", G, NW) + grid_note(tiles, p.slices),
                     (int4_decode_mfma_side_kernel<G, NW>), dim3(tiles * p.slices),
                     dim3(64 * NW), 0, st, reinterpret_cast<const float*>(a), w.codes, side,
                     static_cast<float*>(out), partial, tickets, stride, M, K, N, p.rows,
                     p.slices, d->fault_dev, d->wait_limit);
    else
        ACCEL_LAUNCH(tname("int4_decode_mfma_kernel", G, NW, type_name<XT>()) +
                         grid_note(tiles, p.slices),
                     (int4_decode_mfma_kernel<G, NW, XT>), dim3(tiles * p.slices),
                     dim3(64 * NW), 0, st, a, w.codes, w.scales, w.zeros, out, partial,
                     tickets, stride, M, K, N, p.rows, p.slices, ep, d->fault_dev,
                     d->wait_limit);
    return launch_status();
}

// Matrices of one tile width G in one launch, each with its own plan.
template <int G, bool SIDE = false>
hipError_t launch_mfma_set(Device* d, hipStream_t st, const float* a, const Int4Planes* w,
                           float* const* out, const int* N, const MfPlan* plan, int count, int M,
                           int K, int* status, const uint16_t* const* side = nullptr) {
    MfSet set{};
    set.count = count;
    int wgs = 0, tiles_all = 0;
    size_t partial_floats = 0;
    bool split = false;
    for (int i = 0; i < count; i++) {
        const int tiles = N[i] / (128 * G);
        set.codes[i] = w[i].codes;
        set.scales[i] = w[i].scales;
        set.zeros[i] = w[i].zeros;
        set.side[i] = SIDE ? side[i] : nullptr;
        set.out[i] = out[i];
        set.n[i] = N[i];
        set.rows[i] = plan[i].rows;
        set.slices[i] = plan[i].slices;
        set.wg0[i] = wgs;
        set.tick0[i] = tiles_all;
        wgs += tiles * plan[i].slices;
        tiles_all += tiles;
        partial_floats += (size_t)plan[i].slices * M * N[i];
        split = split || plan[i].slices > 1;
    }
    set.wg0[count] = wgs;
    uint32_t* tickets = nullptr;
    int stride = 0;
    if (split) {
        stride = ticket_stride(tiles_all);
        if (stride < 2) {
            *status = fail(ACCEL_E_INVALID,
                           "decode product: %d tiles need more tickets than the workspace holds",
                           tiles_all);
            return hipSuccess;
        }
        void* ws = workspace(d, st, partial_floats * sizeof(float), status);
        if (!ws) return hipSuccess;
        tickets = static_cast<uint32_t*>(ws);
        float* p = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
        for (int i = 0; i < count; i++) {
            set.partial[i] = p;
            p += (size_t)plan[i].slices * M * N[i];
        }
    }
    if constexpr (SIDE)
        ACCEL_LAUNCH(tname("int4_decode_mfma_side_set_kernel", G, 8) + grid_note(wgs, 0),
                     (int4_decode_mfma_side_set_kernel<G, 8>), dim3(wgs), dim3(64 * 8), 0, st,
                     a, set, tickets, stride, M, K, d->fault_dev, d->wait_limit);
    else
        ACCEL_LAUNCH(tname("int4_decode_mfma_set_kernel", G, 8) + grid_note(wgs, 0),
                     (int4_decode_mfma_set_kernel<G, 8>), dim3(wgs), dim3(64 * 8), 0, st, a,
                     set, tickets, stride, M, K, d->fault_dev, d->wait_limit);
    return launch_status();
}

template <typename XT = float>
hipError_t launch_decode_mfma(Device* d, hipStream_t st, const XT* a, Int4Planes w,
                              void* out, int M, int K, int N, int* status, Epilogue ep) {
    const bool planes_4b = ((reinterpret_cast<uintptr_t>(w.scales) |
                             reinterpret_cast<uintptr_t>(w.zeros)) & 3) == 0;
    const MfPlan p = plan_decode_mfma(d, M, K, N, planes_4b);
    if (p.groups == 2) return launch_mfma<2, 8, XT>(d, st, a, w, out, M, K, N, p, status, ep);
    return launch_mfma<1, 8, XT>(d, st, a, w, out, M, K, N, p, status, ep);
}

template <int TILE>
hipError_t launch_matvec_set(Device* d, hipStream_t st, const float* a, const Int4Planes* w,
                             float* const* out, const int* N, int count, int K, int* status) {
    constexpr int CPL = 32;
    constexpr int LPR = TILE / CPL;
    constexpr int RP = kDecThreads / LPR;
    constexpr int kRowsPerBatch = kBatch * RP;
    const int batches = (K + kRowsPerBatch - 1) / kRowsPerBatch;
    const int per_slice = (batches + kMaxSlices - 1) / kMaxSlices;   // as a lone M = 1 launch
    const int rows = per_slice * kRowsPerBatch;
    const int slices = (K + rows - 1) / rows;
    DecodeSet set{};
    set.count = count;
    int tiles = 0;
    size_t partial_floats = 0;
    for (int i = 0; i < count; i++) {
        set.codes[i] = w[i].codes;
        set.scales[i] = w[i].scales;
        set.zeros[i] = w[i].zeros;
        set.out[i] = out[i];
        set.n[i] = N[i];
        set.tile0[i] = tiles;
        tiles += N[i] / TILE;
        partial_floats += (size_t)slices * N[i];
    }
    set.tile0[count] = tiles;
    uint32_t* tickets = nullptr;
    int stride = 0;
    if (slices > 1) {
        stride = ticket_stride(tiles);
        if (stride == 0) {
            *status = fail(ACCEL_E_INVALID,
                           "decode product: %d tiles need more tickets than the workspace holds",
                           tiles);
            return hipSuccess;
        }
        void* ws = workspace(d, st, partial_floats * sizeof(float), status);
        if (!ws) return hipSuccess;
        tickets = static_cast<uint32_t*>(ws);
        float* p = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
        for (int i = 0; i < count; i++) {
            set.partial[i] = p;
            p += (size_t)slices * N[i];
        }
    }
    if (per_slice > 1)
        ACCEL_LAUNCH(tname("int4_decode_set_kernel", 1, TILE, CPL, true) + grid_note(tiles, slices),
                     (int4_decode_set_kernel<1, TILE, CPL, true>), dim3(tiles * slices),
                           dim3(kDecThreads), 0, st, a, set, tickets, stride, K, rows, slices);
    else
        ACCEL_LAUNCH(tname("int4_decode_set_kernel", 1, TILE, CPL, false) + grid_note(tiles, slices),
                     (int4_decode_set_kernel<1, TILE, CPL, false>), dim3(tiles * slices),
                           dim3(kDecThreads), 0, st, a, set, tickets, stride, K, rows, slices);
    return launch_status();
}

}  // namespace

hipError_t launch_matvec_f32_f16(Device* d, hipStream_t st, const float* a, const uint16_t* w,
                                 float* out, int K, int N, int* status) {
    *status = ACCEL_OK;
    if (K <= 0 || N <= 0) return hipSuccess;
    const bool aligned = (reinterpret_cast<uintptr_t>(w) & 15) == 0;
    if (aligned && N % 256 == 0 && N < (1 << 30))
        return launch_matvec_f16_tiled<256>(d, st, a, w, out, K, N, status);
    if (aligned && N % 128 == 0 && N < (1 << 30))
        return launch_matvec_f16_tiled<128>(d, st, a, w, out, K, N, status);
    ACCEL_LAUNCH(std::string("matvec_f16_generic_kernel"), matvec_f16_generic_kernel, dim3((N + 255) / 256), dim3(256), 0, st, a, w,
                       out, K, N);
    return launch_status();
}

bool int4_matmul_set_supported(const float* a, const Int4Planes* w, const int* N, int count,
                               int M, int K) {
    if (count < 1 || count > kMaxSet || M < 2 || M > 16 || K % 32 != 0 ||
        (reinterpret_cast<uintptr_t>(a) & 15) != 0)
        return false;
    for (int i = 0; i < count; i++)
        if (!int4_decode_f32_supported(M, K, N[i], w[i].codes) || N[i] >= (1 << 27))
            return false;
    return true;
}

hipError_t launch_int4_matmul_set(Device* d, hipStream_t st, const float* a, const Int4Planes* w,
                                  float* const* out, const int* N, int count, int M, int K,
                                  int* status) {
    *status = ACCEL_OK;
    // each matrix with the plan its own launch would take; one launch per G
    Int4Planes wg[2][kMaxSet];
    float* og[2][kMaxSet];
    int ng[2][kMaxSet], cnt[2] = {0, 0};
    MfPlan pg[2][kMaxSet];
    for (int i = 0; i < count; i++) {
        const bool planes_4b = ((reinterpret_cast<uintptr_t>(w[i].scales) |
                                 reinterpret_cast<uintptr_t>(w[i].zeros)) & 3) == 0;
        const MfPlan p = plan_decode_mfma(d, M, K, N[i], planes_4b);
        const int g = p.groups == 2 ? 0 : 1;
        wg[g][cnt[g]] = w[i];
        og[g][cnt[g]] = out[i];
        pg[g][cnt[g]] = p;
        ng[g][cnt[g]++] = N[i];
    }
    hipError_t e = hipSuccess;
    if (cnt[0]) e = launch_mfma_set<2>(d, st, a, wg[0], og[0], ng[0], pg[0], cnt[0], M, K, status);
    if (e != hipSuccess || *status != ACCEL_OK) return e;
    if (cnt[1]) e = launch_mfma_set<1>(d, st, a, wg[1], og[1], ng[1], pg[1], cnt[1], M, K, status);
    return e;
}

// ---- prepared weights for the matrix-core decode ------------------------------
//
// The side copy of a weight's scales and zeros: for group g and 32-row step
// s, 64 f16 values -- the scales of rows 32 s .. 32 s + 31, then their zeros
// -- so that a step's are one contiguous 128-byte block (MfTile, SIDE).  The
// codes stay in the reference order.  Measured with contiguous blocks in
// place of the planes' pieces (timing only): config 2 18.7-19.0 -> 16.8-17.0
// us, the decode MoE 92-93 -> 83.5 us.
namespace {
__global__ __launch_bounds__(256) void int4_side_prepare_kernel(
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    uint16_t* __restrict__ side, int K, int groups) {
    const size_t per_group = (size_t)(K >> 5) * 64;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= per_group * groups) return;
    const int g = (int)(i / per_group);
    const size_t r = i % per_group;
    const int j = (int)(r & 63);
    const size_t row = (r >> 6) * 32 + (j & 31);
    side[i] = (j < 32 ? scales : zeros)[row * groups + g];
}
}  // namespace

bool int4_side_supported(int64_t K, int64_t N) {
    return K >= 32 && K % 32 == 0 && N >= 128 && N % 128 == 0 && N < (1 << 27) &&
           K < (1 << 30);
}

size_t int4_side_bytes(int K, int N) { return (size_t)(N / 128) * (K / 32) * 64 * 2; }

hipError_t launch_int4_side_prepare(hipStream_t st, Int4Planes w, uint16_t* side, int K, int N) {
    const size_t n = (size_t)(N / 128) * (K / 32) * 64;
    ACCEL_LAUNCH(std::string("int4_side_prepare_kernel"), int4_side_prepare_kernel,
                 dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w.scales, w.zeros, side,
                 K, N / 128);
    return launch_status();
}

bool int4_decode_side_rows_supported(int M, const float* a) {
    return M >= 1 && M <= 16 && (reinterpret_cast<uintptr_t>(a) & 15) == 0;
}

// M (1..16) f32 rows against count (1..kMaxSet) prepared matrices: each with
// the plan its own launch on the planes would take (so its result is that
// launch's bit for bit), one launch per tile width present.
hipError_t launch_int4_decode_side(Device* d, hipStream_t st, const float* a,
                                   const uint32_t* const* codes, const uint16_t* const* side,
                                   float* const* out, const int* N, int count, int M, int K,
                                   int* status) {
    *status = ACCEL_OK;
    if (count == 1) {
        const MfPlan p = plan_decode_mfma(d, M, K, N[0], true);
        const Int4Planes w{codes[0], nullptr, nullptr};
        if (p.groups == 2)
            return launch_mfma<2, 8, float, true>(d, st, a, w, out[0], M, K, N[0], p, status,
                                                  Epilogue{}, side[0]);
        return launch_mfma<1, 8, float, true>(d, st, a, w, out[0], M, K, N[0], p, status,
                                              Epilogue{}, side[0]);
    }
    Int4Planes wg[2][kMaxSet];
    const uint16_t* sg[2][kMaxSet];
    float* og[2][kMaxSet];
    int ng[2][kMaxSet], cnt[2] = {0, 0};
    MfPlan pg[2][kMaxSet];
    for (int i = 0; i < count; i++) {
        const MfPlan p = plan_decode_mfma(d, M, K, N[i], true);
        const int g = p.groups == 2 ? 0 : 1;
        wg[g][cnt[g]] = Int4Planes{codes[i], nullptr, nullptr};
        sg[g][cnt[g]] = side[i];
        og[g][cnt[g]] = out[i];
        pg[g][cnt[g]] = p;
        ng[g][cnt[g]++] = N[i];
    }
    hipError_t e = hipSuccess;
    if (cnt[0])
        e = launch_mfma_set<2, true>(d, st, a, wg[0], og[0], ng[0], pg[0], cnt[0], M, K, status,
                                     sg[0]);
    if (e != hipSuccess || *status != ACCEL_OK) return e;
    if (cnt[1])
        e = launch_mfma_set<1, true>(d, st, a, wg[1], og[1], ng[1], pg[1], cnt[1], M, K, status,
                                     sg[1]);
    return e;
}

bool int4_matvec_set_supported(const Int4Planes* w, const int* N, int count, int K) {
    if (count < 1 || count > kMaxSet) return false;
    for (int i = 0; i < count; i++)
        if (!int4_decode_f32_supported(1, K, N[i], w[i].codes)) return false;
    return true;
}

hipError_t launch_int4_matvec_set(Device* d, hipStream_t st, const float* a, const Int4Planes* w,
                                  float* const* out, const int* N, int count, int K,
                                  int* status) {
    *status = ACCEL_OK;
    // Each matrix keeps the tile width its own launch would take
    // (matvec_tile), so its sums are added in the same order and its result
    // is its own Int4MatVec's: one launch per width present.
    Int4Planes wg[3][kMaxSet];
    float* og[3][kMaxSet];
    int ng[3][kMaxSet], cnt[3] = {0, 0, 0};
    for (int i = 0; i < count; i++) {
        const int tw = matvec_tile(N[i]);
        const int g = tw == 512 ? 0 : (tw == 256 ? 1 : 2);
        wg[g][cnt[g]] = w[i];
        og[g][cnt[g]] = out[i];
        ng[g][cnt[g]++] = N[i];
    }
    hipError_t e = hipSuccess;
    if (cnt[0]) e = launch_matvec_set<512>(d, st, a, wg[0], og[0], ng[0], cnt[0], K, status);
    if (e != hipSuccess || *status != ACCEL_OK) return e;
    if (cnt[1]) e = launch_matvec_set<256>(d, st, a, wg[1], og[1], ng[1], cnt[1], K, status);
    if (e != hipSuccess || *status != ACCEL_OK) return e;
    if (cnt[2]) e = launch_matvec_set<128>(d, st, a, wg[2], og[2], ng[2], cnt[2], K, status);
    return e;
}

bool int4_decode_f32_supported(int M, int K, int N, const void* codes) {
    return M >= 1 && M <= 16 && K >= 1 && N >= 128 && N % 128 == 0 &&
           (reinterpret_cast<uintptr_t>(codes) & 15) == 0 && K < (1 << 30) && N < (1 << 30);
}

hipError_t launch_int4_decode_f32(Device* d, hipStream_t st, const float* a, Int4Planes w,
                                  void* out, int M, int K, int N, int* status, Epilogue ep) {
    *status = ACCEL_OK;
    // Two or more rows: the matrix-core kernel, where its shape holds (its
    // per-lane code offsets within a 32-row step are 32-bit).  Two rows
    // measured against the VALU kernel (us): K x N = 4096 x 1024 7.9 / 9.8,
    // 1024 x 4096 7.2 / 9.7, 2048 x 2048 7.4 / 9.8, 4096 x 14336 16.6 / 20.9,
    // 14336 x 4096 16.1 / 19.0, 4096 x 28672 25.2 / 34.8; 4096 x 4096 10.4 / 10.0.
    if (M >= 2 && K % 32 == 0 && N < (1 << 27) && (reinterpret_cast<uintptr_t>(a) & 15) == 0)
        return launch_decode_mfma(d, st, a, w, out, M, K, N, status, ep);
    switch (M) {
        case 1: return launch_decode_m<1>(d, st, a, w, out, K, N, status, ep);
        case 2: return launch_decode_m<2>(d, st, a, w, out, K, N, status, ep);
        case 3: return launch_decode_m<3>(d, st, a, w, out, K, N, status, ep);
        case 4: return launch_decode_m<4>(d, st, a, w, out, K, N, status, ep);
        case 5: return launch_decode_m<5>(d, st, a, w, out, K, N, status, ep);
        case 6: return launch_decode_m<6>(d, st, a, w, out, K, N, status, ep);
        case 7: return launch_decode_m<7>(d, st, a, w, out, K, N, status, ep);
        case 8: return launch_decode_m<8>(d, st, a, w, out, K, N, status, ep);
        default: break;
    }
    // 9..16 rows: eight, then the rest.
    hipError_t e = launch_decode_m<8>(d, st, a, w, out, K, N, status, ep);
    if (e != hipSuccess || *status != ACCEL_OK) return e;
    char* rest = static_cast<char*>(out) + (size_t)8 * N * (ep.bf16 ? 2 : 4);
    return launch_int4_decode_f32(d, st, a + (size_t)8 * K, w, rest, M - 8, K, N, status, ep);
}

// One row of bf16 activations: the VALU decode kernel reading bf16 (widened
// exactly to f32), the f32 arithmetic of a one-row f32 product, and one
// rounding of each sum (plus bias) to bf16.  The bf16 tiles take a 32-row
// band for it; measured (us, this / the tiles / a one-row f32 product):
// K x N = 4096 x 4096 6.24 / 10.6 / 6.11, 4096 x 14336 13.5 / 23.1 / 12.0,
// 14336 x 4096 14.0 / 19.8 / 12.8.  The activations stay raw bf16 in
// registers until they are used: widened as they were loaded, they made the
// compiler wait for each load before issuing the next (7.0, 14.6, 14.8 us).
hipError_t launch_int4_decode_bf16_row(Device* d, hipStream_t st, const uint16_t* a,
                                       Int4Planes w, uint16_t* out, int K, int N, int* status,
                                       const float* bias) {
    *status = ACCEL_OK;
    Epilogue ep;
    ep.bias = bias;
    ep.bf16 = true;
    return launch_decode_m<1, uint16_t>(d, st, a, w, out, K, N, status, ep);
}

// 2..16 rows of bf16 activations on the matrix-core decode kernel (bf16
// staged, widened in registers, the f32 product's arithmetic), one rounding
// to bf16: where the bf16 tiles would run a mostly empty 32-row band.
bool int4_decode_bf16_rows_supported(int M, int K, int N, const void* a, const void* codes) {
    return M >= 2 && M <= 16 && K % 32 == 0 && int4_decode_f32_supported(M, K, N, codes) &&
           N < (1 << 27) && (reinterpret_cast<uintptr_t>(a) & 15) == 0;
}

hipError_t launch_int4_decode_bf16_rows(Device* d, hipStream_t st, const uint16_t* a,
                                        Int4Planes w, uint16_t* out, int M, int K, int N,
                                        int* status, const float* bias) {
    *status = ACCEL_OK;
    Epilogue ep;
    ep.bias = bias;
    ep.bf16 = true;
    return launch_decode_mfma<uint16_t>(d, st, a, w, out, M, K, N, status, ep);
}

namespace {

// ---- ragged int4 GEMV: the decode form of the grouped product -------------
//
// The counterpart of GroupedMatVec / GroupedMatMul (internal/kernels/
// grouped.go:47-97, groupedtiled.go:77-134) over per-expert int4 weights when
// there are few routed rows (decode MoE): the rows t of an expert,
// e(t) = #{r : off[r+1] <= t}, are decode products against its matrix two at
// a time (an odd one out alone), with the same batches and split-K hand-off
// as Int4MatVec.  A pair runs 16 columns a lane, which keeps the kernel at
// two workgroups a CU; a lone row runs the matvec's 32.  Rows past
// every segment (t >= off[E]) are written 0 by the matvec form and left alone
// by the matmul form.  Workgroups are ordered (K slice, column tile, row) with
// the row fastest and dealt to the XCDs in contiguous runs, so the rows of one
// expert -- adjacent, rows being sorted by expert -- read the same code lines
// together through one L2.
//
// With sorted offsets and enough rows, an expert's rows are cut into blocks
// of 16 from its first row and every block goes to the matrix-core decode
// kernel (one read of the expert's weights for up to 16 rows,
// int4_grouped_decode_mfma_kernel, a second launch); this kernel then only
// writes the padding rows, or takes every row when the offsets wrapped.
// Measured at 4, 8, 16 and 32 tokens routed top-2 over config 4's experts
// (us): rows alone or in pairs here 78.8, 119.4, 208.3, 372; blocks of 3..16
// rows on the matrix cores 78.7, 102.1, 154.1, 140.8; of 2..16 78.6, 98.6,
// 154.5, 140.7; of 1..16, with this launch at one K slice and 512-column
// tiles, 79.1, 93.9, 116.1, 123.8.
constexpr int kMfBlockRows = 16;   // rows of a matrix-core block, at most
constexpr int kMfBlockMin = 1;     // and at least

// Matrix-core blocks of an expert with c rows (a block of kMfBlockMin rows
// or more past the full ones).
__device__ __forceinline__ uint32_t grouped_mfma_blocks(uint32_t c) {
    return c / kMfBlockRows + (c % kMfBlockRows >= (uint32_t)kMfBlockMin ? 1u : 0u);
}

__device__ __forceinline__ int grouped_expert_of(const uint32_t* off, int E, uint32_t t) {
    int e = 0;
    for (int r = 0; r < E; r++) e += (off[r + 1] <= t) ? 1 : 0;
    return e;
}

// Offsets that never decrease (every count sum short of the u32 wrap): then
// the rows of expert e are exactly [off[e], min(off[e+1], T)).
__device__ __forceinline__ bool grouped_offsets_sorted(const uint32_t* off, int E) {
    bool ok = true;
    for (int r = 0; r < E; r++) ok = ok && off[r] <= off[r + 1];
    return ok;
}

// XT: f32 or bf16 bits; the result is written in the same type.
//
// Workgroup b takes row t = b % T, and, when the rows are this launch's
// alone, column tile (b / T) % tiles and K slice b / (T tiles).  When the
// matrix-core launch takes the rows (mfma_blocks), this launch is left the
// padding rows, and every row should the offsets have wrapped: then one
// workgroup a row walks the row's column tiles with K whole (the host plans
// one slice), so that the workgroups finding no row are T, not T x tiles
// (1024 f32 rows of N = 14336, all of them the matrix cores': 28 672 such
// workgroups took 106 us).
template <int TILE, int CPL, bool PIPE, typename XT = float>
__global__ __launch_bounds__(kDecThreads) void int4_grouped_decode_kernel(
    const XT* __restrict__ x, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    const uint32_t* __restrict__ off, void* __restrict__ out, float* partial,
    uint32_t* tickets, int ticket_stride, int E, int T, int K, int N, int rows_per_slice,
    int slices, bool write_padding, bool mfma_blocks) {
    const int tiles = N / TILE;
    const int grid = gridDim.x;
    int b = blockIdx.x;
    if ((grid & 7) == 0) b = (b & 7) * (grid >> 3) + (b >> 3);
    const int t = b % T;
    const int tile0 = mfma_blocks ? 0 : (b / T) % tiles;
    const int tile_end = mfma_blocks ? tiles : tile0 + 1;
    const int slice = mfma_blocks ? 0 : b / (T * tiles);
    const int e = grouped_expert_of(off, E, (uint32_t)t);
    if (e >= E) {
        // past every segment: the matvec form writes zeros, once per column tile
        if (write_padding && slice == 0)
            for (int c = tile0 * TILE + threadIdx.x; c < tile_end * TILE; c += kDecThreads) {
                const size_t o = (size_t)t * N + c;
                if constexpr (sizeof(XT) == 2)
                    static_cast<uint16_t*>(out)[o] = 0;
                else
                    static_cast<float*>(out)[o] = 0.0f;
            }
        return;
    }
    // An expert's rows go two at a time (its weights read once for both): the
    // first row of a pair takes both, the second has nothing to do, and an
    // odd one out goes alone.  A pair's split-K sums take the two rows' slots
    // and the first row's ticket.  Offsets that wrapped (no longer sorted)
    // leave every row alone.
    const bool sorted = grouped_offsets_sorted(off, E);
    if (sorted && mfma_blocks) {
        // rows of a block of kMfBlockMin or more are the matrix-core launch's
        const uint32_t i = (uint32_t)t - off[e];
        const uint32_t c = min(off[e + 1], (uint32_t)T) - off[e];
        const uint32_t j = i / kMfBlockRows;
        if (min((uint32_t)kMfBlockRows, c - j * kMfBlockRows) >= (uint32_t)kMfBlockMin) return;
    }
    if (sorted && (((uint32_t)t - off[e]) & 1u) != 0) return;
    const bool pair = sorted && (uint32_t)t + 1 < min(off[e + 1], (uint32_t)T);
    const size_t per = (size_t)K * N;
    const uint32_t* c = codes + (size_t)e * (per >> 3);
    const uint16_t* s = scales + (size_t)e * (per >> 7);
    const uint16_t* z = zeros + (size_t)e * (per >> 7);
    float* p = partial ? partial + (size_t)t * slices * N : nullptr;
    void* o = static_cast<char*>(out) + (size_t)t * N * sizeof(XT);
    Epilogue ep;
    ep.bf16 = sizeof(XT) == 2;
    // (decode_tile ends at a barrier, so its LDS is free for the next tile)
    for (int tile = tile0; tile < tile_end; tile++) {
        uint32_t* tk = tickets + ((size_t)t * tiles + tile) * ticket_stride;
        if (pair)
            decode_tile<2, TILE, CPL / 2, PIPE, XT>(x + (size_t)t * K, c, s, z, o, p, tk, K, N,
                                                    tile, slice, rows_per_slice, slices, ep);
        else
            decode_tile<1, TILE, CPL, PIPE, XT>(x + (size_t)t * K, c, s, z, o, p, tk, K, N,
                                                tile, slice, rows_per_slice, slices, ep);
    }
}

// The matrix-core blocks of a grouped decode product: workgroup b takes
// block u -- the u-th block of 1..16 rows in (expert, first row) order, found
// from the offsets by one wave's prefix sum over the experts' block counts --
// and within it a K slice and column tile, as a lone 16-row matrix-core
// decode launch would.  The grid is sized for the most blocks the rows can
// make; workgroups past the real blocks return at once, as do all when the
// offsets are not sorted (the VALU launch then takes every row).  A block's
// split-K sums sit at slices x (its first row) x N floats into `partial`, so
// blocks never share them; block u's tickets are the tile pairs past the
// earlier blocks'.  (A persistent form, each workgroup looping over the
// blocks, spilled registers and ran 3% slower.)
template <int G, int NW, typename XT, bool SIDE>
__device__ __forceinline__ void grouped_decode_mfma_body(
    const XT* __restrict__ x, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    const uint16_t* __restrict__ side, const uint32_t* __restrict__ off,
    void* __restrict__ out, float* partial, uint32_t* tickets, int ticket_stride, int E, int T,
    int K, int N, int rows_per_slice, int slices, uint32_t* fault, int wait_limit) {
    using Tl = MfTile<G, NW, SIDE>;
    __shared__ int blk_e, blk_row0, blk_rows;
    const int tiles = N / Tl::kCols;
    const int per_block = tiles * slices;
    // Blocks in dispatch order, each dealt to the eight XCDs (workgroups go
    // to them round robin) in contiguous eighths of its (slice, tile) list,
    // as a lone launch places them: the real blocks, which come first, keep
    // every XCD busy, and the grid's surplus workgroups come last.
    const int b = blockIdx.x;
    uint32_t u;
    int r;
    if ((per_block & 7) == 0) {
        const int q = per_block >> 3;
        u = (uint32_t)((b >> 3) / q);
        r = (b & 7) * q + (b >> 3) % q;
    } else {
        u = (uint32_t)(b / per_block);
        r = b % per_block;
    }
    const int tile = r % tiles;
    const int slice = r / tiles;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        if (lane == 0) blk_e = -1;
        if (grouped_offsets_sorted(off, E)) {
            uint32_t base = 0;   // blocks of the experts before this run of 64
            for (int e0 = 0; e0 < E && base <= u; e0 += 64) {
                const int e = e0 + lane;
                uint32_t start = 0, c = 0;
                if (e < E) {
                    start = min(off[e], (uint32_t)T);
                    c = min(off[e + 1], (uint32_t)T) - start;
                }
                const uint32_t n = grouped_mfma_blocks(c);
                uint32_t incl = n;   // inclusive prefix sum over the wave
#pragma unroll
                for (int dd = 1; dd < 64; dd <<= 1) {
                    const uint32_t v = __shfl_up(incl, dd, 64);
                    if (lane >= dd) incl += v;
                }
                const uint32_t first = base + incl - n;
                if (u >= first && u < base + incl) {
                    const uint32_t j = u - first;
                    blk_e = e;
                    blk_row0 = (int)(start + j * kMfBlockRows);
                    blk_rows = (int)min((uint32_t)kMfBlockRows, c - j * kMfBlockRows);
                }
                base += __shfl(incl, 63, 64);
            }
        }
    }
    __syncthreads();
    const int e = blk_e;
    if (e < 0) return;
    const int row0 = blk_row0;
    const size_t per = (size_t)K * N;
    Epilogue ep;
    ep.bf16 = sizeof(XT) == 2;
    decode_mfma_tile<G, NW, XT, SIDE>(x + (size_t)row0 * K, codes + (size_t)e * (per >> 3),
                            SIDE ? nullptr : scales + (size_t)e * (per >> 7),
                            SIDE ? nullptr : zeros + (size_t)e * (per >> 7),
                            static_cast<char*>(out) + (size_t)row0 * N * sizeof(XT),
                            partial ? partial + (size_t)slices * row0 * N : nullptr,
                            tickets ? tickets + ((size_t)u * tiles + tile) * ticket_stride
                                    : nullptr,
                            blk_rows, K, N, tile, slice, rows_per_slice, slices, ep,
                            fault, wait_limit,
                            SIDE ? side + (size_t)e * ((size_t)(N >> 7) * (K >> 5) * 64)
                                 : nullptr);
}

template <int G, int NW, typename XT = float>
__global__ __launch_bounds__(64 * NW) void int4_grouped_decode_mfma_kernel(
    const XT* __restrict__ x, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    const uint32_t* __restrict__ off, void* __restrict__ out, float* partial,
    uint32_t* tickets, int ticket_stride, int E, int T, int K, int N, int rows_per_slice,
    int slices, uint32_t* fault, int wait_limit) {
    grouped_decode_mfma_body<G, NW, XT, false>(x, codes, scales, zeros, nullptr, off, out,
                                              partial, tickets, ticket_stride, E, T, K, N,
                                              rows_per_slice, slices, fault, wait_limit);
}

// The same over prepared experts: each expert's scales and zeros from its
// side copy (see MfTile).
template <int G, int NW, typename XT = float>
__global__ __launch_bounds__(64 * NW) void int4_grouped_decode_mfma_side_kernel(
    const XT* __restrict__ x, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ side, const uint32_t* __restrict__ off,
    void* __restrict__ out, float* partial, uint32_t* tickets, int ticket_stride, int E, int T,
    int K, int N, int rows_per_slice, int slices, uint32_t* fault, int wait_limit) {
    grouped_decode_mfma_body<G, NW, XT, true>(x, codes, nullptr, nullptr, side, off, out,
                                             partial, tickets, ticket_stride, E, T, K, N,
                                             rows_per_slice, slices, fault, wait_limit);
}

// K slices of a grouped decode launch: enough workgroups for two per CU
// across all rows, at most one batch each beyond that (the rows already fill
// the chip).
template <int TILE>
struct GroupedDecodeShape {
    static constexpr int CPL = 32;
    static constexpr int LPR = TILE / CPL;
    static constexpr int RP = kDecThreads / LPR;
    static constexpr int kRowsPerBatch = kBatch * RP;
    int tiles, per_slice, rows, slices;
    long long pairs;
    // singles: the matrix-core launch takes the rows, which leaves this launch
    // the padding rows (or every row, should the offsets have wrapped): one K
    // slice, so that the grid its workgroups without rows return from stays
    // small (8 tokens routed top-2 over config 4's experts: 8.0 us with two
    // slices)
    GroupedDecodeShape(const Device* d, int T, int K, int N, bool singles) {
        tiles = N / TILE;
        const int batches = (K + kRowsPerBatch - 1) / kRowsPerBatch;
        pairs = (long long)T * tiles;
        int want = singles ? 1 : (int)std::max(1LL, (2LL * d->cu_count + pairs - 1) / pairs);
        want = std::min(want, std::min(batches, kMaxSlices));
        per_slice = (batches + want - 1) / want;
        rows = per_slice * kRowsPerBatch;
        slices = (K + rows - 1) / rows;
    }
    size_t area_bytes(int T, int N) const {
        return slices > 1 ? (size_t)T * slices * N * sizeof(float) : 0;
    }
};

// Whether a grouped decode product runs its blocks of up to 16 rows on the
// matrix cores (a second launch), and that launch's plan: a lone 16-row
// product's tile width and K slices, and the most blocks T rows over E
// experts can make (each has a row at least; an expert's blocks past its
// first are full).  The launch is made only when the rows average two or
// more an expert: with fewer, blocks of several rows are rare, and a launch
// that finds none costs a round of workgroups (measured at 4 tokens routed
// top-2 over 8 experts: 78 -> 82.7 us).
struct GroupedMfma {
    bool on = false;
    MfPlan plan{1, 1, 0};
    int blocks = 0;    // blocks the grid and the tickets are sized for
    int stride = 0;    // ticket spacing (two counters a tile)
};
GroupedMfma grouped_mfma(const Device* d, const void* x, Int4Planes w, int E, int T, int K,
                         int N) {
    GroupedMfma g;
    g.blocks = std::min(T / kMfBlockMin, T / kMfBlockRows + E);
    if (g.blocks == 0 || (long long)T < 2LL * E || K % 32 != 0 || N >= (1 << 27) ||
        (reinterpret_cast<uintptr_t>(x) & 15) != 0)
        return g;
    // an expert's scale and zero planes start 4-byte aligned when the base does
    // and K * N / 128 is even
    // (side copies have no such condition)
    const size_t per = (size_t)K * N;
    const bool planes_4b = w.side != nullptr ||
                           (((reinterpret_cast<uintptr_t>(w.scales) |
                              reinterpret_cast<uintptr_t>(w.zeros)) & 3) == 0 &&
                            ((per >> 7) & 1) == 0);
    g.plan = plan_decode_mfma(d, kMfBlockRows, K, N, planes_4b);
    // The plan above fills the CUs from one block.  The rows make at least
    // ceil(T / 16) blocks; once those blocks' column tiles alone fill the
    // CUs, K is not split: no tickets, no sums area, no hand-off.
    const long long min_blocks = (T + kMfBlockRows - 1) / kMfBlockRows;
    if (min_blocks * (N / (128 * g.plan.groups)) >= d->cu_count) {
        g.plan.slices = 1;
        g.plan.rows = K;
    }
    if (g.plan.slices > 1) {
        g.stride = ticket_stride(g.blocks * (N / (128 * g.plan.groups)));
        if (g.stride < 2) return g;
    }
    g.on = true;
    return g;
}

template <int TILE, typename XT>
hipError_t launch_grouped_decode_tile(Device* d, hipStream_t st, const XT* x, Int4Planes w,
                                      const uint32_t* off, void* out, int E, int T, int K,
                                      int N, bool write_padding, int* status,
                                      uint32_t* tickets, float* area, bool mfma_blocks) {
    constexpr int CPL = GroupedDecodeShape<TILE>::CPL;
    const GroupedDecodeShape<TILE> sh(d, T, K, N, mfma_blocks);
    const int tiles = sh.tiles, per_slice = sh.per_slice, rows = sh.rows, slices = sh.slices;
    const long long pairs = sh.pairs;
    if (pairs * slices > (1ll << 31) - 8) {
        *status = fail(ACCEL_E_INVALID, "grouped decode product: %d rows x %d tiles is too large",
                       T, tiles);
        return hipSuccess;
    }
    // tickets only where K is split (rows x tiles then under twice the CUs)
    const int stride = slices > 1 ? ticket_stride((int)pairs) : 0;
    if (slices > 1 && stride == 0) {
        *status = fail(ACCEL_E_INVALID,
                       "grouped decode product: %d rows x %d tiles need more tickets than the "
                       "workspace holds",
                       T, tiles);
        return hipSuccess;
    }
    // the split-K sums live in the caller's area, past the offsets
    float* partial = slices > 1 ? area : nullptr;
    // with the matrix-core launch taking the rows: one workgroup a row, which
    // walks the column tiles with K whole
    if (mfma_blocks && slices != 1) {
        *status = fail(ACCEL_E_INVALID, "grouped decode product: %d K slices planned for the "
                                        "padding launch", slices);
        return hipSuccess;
    }
    const dim3 grid((unsigned)(mfma_blocks ? (long long)T : pairs * slices));
    const std::string note =
        mfma_blocks ? " [" + std::to_string(T) + " rows, each walking " + std::to_string(tiles) +
                          " tiles: the padding rows]"
                    : grid_note(tiles, slices);
    if (per_slice > 1)
        ACCEL_LAUNCH(tname("int4_grouped_decode_kernel", TILE, CPL, true, type_name<XT>()) +
                         note,
                     (int4_grouped_decode_kernel<TILE, CPL, true, XT>), grid,
                           dim3(kDecThreads), 0, st, x, w.codes, w.scales, w.zeros, off, out,
                           partial, tickets, stride, E, T, K, N, rows, slices, write_padding,
                           mfma_blocks);
    else
        ACCEL_LAUNCH(tname("int4_grouped_decode_kernel", TILE, CPL, false, type_name<XT>()) +
                         note,
                     (int4_grouped_decode_kernel<TILE, CPL, false, XT>), grid,
                           dim3(kDecThreads), 0, st, x, w.codes, w.scales, w.zeros, off, out,
                           partial, tickets, stride, E, T, K, N, rows, slices, write_padding,
                           mfma_blocks);
    return launch_status();
}

template <int G, typename XT>
hipError_t launch_grouped_mfma(Device* d, hipStream_t st, const XT* x, Int4Planes w,
                               const uint32_t* off, void* out, int E, int T, int K, int N,
                               const GroupedMfma& g, uint32_t* tickets, float* area) {
    const int tiles = N / (128 * G);
    const bool split = g.plan.slices > 1;
    const dim3 grid((unsigned)(g.blocks * tiles * g.plan.slices));
    if (w.side)
        ACCEL_LAUNCH(tname("int4_grouped_decode_mfma_side_kernel", G, 8, type_name<XT>()) +
                         grid_note(tiles, g.plan.slices),
                     (int4_grouped_decode_mfma_side_kernel<G, 8, XT>), grid, dim3(64 * 8), 0,
                     st, x, w.codes, w.side, off, out, split ? area : nullptr,
                     split ? tickets : nullptr, g.stride, E, T, K, N, g.plan.rows,
                     g.plan.slices, d->fault_dev, d->wait_limit);
    else
        ACCEL_LAUNCH(tname("int4_grouped_decode_mfma_kernel", G, 8, type_name<XT>()) +
                         grid_note(tiles, g.plan.slices),
                     (int4_grouped_decode_mfma_kernel<G, 8, XT>), grid, dim3(64 * 8), 0, st, x,
                     w.codes, w.scales, w.zeros, off, out, split ? area : nullptr,
                     split ? tickets : nullptr, g.stride, E, T, K, N, g.plan.rows,
                     g.plan.slices, d->fault_dev, d->wait_limit);
    return launch_status();
}

}  // namespace

bool int4_grouped_decode_supported(int T, int K, int N, const void* codes, bool bf16) {
    return T >= 1 && T <= (bf16 ? kGroupedDecodeRows : kGroupedDecodeRowsF32) && K >= 1 &&
           N >= 128 && N % 128 == 0 &&
           (reinterpret_cast<uintptr_t>(codes) & 15) == 0 && K < (1 << 30) && N < (1 << 30);
}

// Column tile of the ragged GEMV: 512 columns for wide matrices when the
// rows are few (rows x tiles at most half the CUs, so the launch is mostly
// K slices and the halved scale/zero lines pay), else the matvec's 256 or 128.
// Measured at K = 4096, N = 14336 (decode MoE, top-2 of 8 experts): 1 token
// 27.1 -> 24.1-24.8 us, 2 tokens 45.1 -> 43.4; at 4 tokens (8 rows) 512
// columns lose, 78.6 -> 84.5, and at 8 tokens 120 -> 121-126.
static int grouped_decode_tile(const Device* d, int T, int N) {
    if (N >= 8192 && N % 512 == 0 && (long long)T * (N / 512) <= d->cu_count / 2) return 512;
    return N % 256 == 0 ? 256 : 128;
}

// Experts prepared into the panel layout take f32 rows on the panel kernel
// where the matrix-core blocks are not launched (fewer than two rows an
// expert on average) and there are three rows or more; K even and the rows
// 8-byte aligned.  Measured on config 4's experts (K = 4096, N = 14336,
// top-2 of 8; us, panels in passes of up to four rows / the planes' route,
// matrix-core blocks or VALU): 1 token (2 rows) 32.2 / 28.1, 2 tokens
// 43.7 / 50.5, 4 tokens 55.9 / 96.0, 8 tokens 83.9 / 81.5 (side copies),
// 16 tokens 147.4 / 99.3.
bool grouped_panel_route(const void* x, Int4Planes w, bool bf16, int E, int T, int K) {
    return w.panels && !bf16 && T >= 3 && T <= kGroupedDecodeRows && (long long)T < 2LL * E &&
           K % 2 == 0 && (reinterpret_cast<uintptr_t>(x) & 7) == 0;
}

size_t int4_grouped_decode_area(const Device* d, const void* x, bool bf16, Int4Planes w, int E,
                                int T, int K, int N) {
    // the same rule the launch applies (launch_grouped_decode_t): bf16 rows
    // never take the panels, and then plan their own split-K sums below
    if (grouped_panel_route(x, w, bf16, E, T, K)) {
        // the VALU launch alone uses the area: the padding rows at one slice
        const int tw = N % 512 == 0 ? 512 : grouped_decode_tile(d, T, N);
        if (tw == 512) return GroupedDecodeShape<512>(d, T, K, N, true).area_bytes(T, N);
        if (tw == 256) return GroupedDecodeShape<256>(d, T, K, N, true).area_bytes(T, N);
        return GroupedDecodeShape<128>(d, T, K, N, true).area_bytes(T, N);
    }
    const GroupedMfma g = grouped_mfma(d, x, w, E, T, K, N);
    const int tw = g.on && N % 512 == 0 ? 512 : grouped_decode_tile(d, T, N);
    size_t bytes;
    if (tw == 512)
        bytes = GroupedDecodeShape<512>(d, T, K, N, g.on).area_bytes(T, N);
    else if (tw == 256)
        bytes = GroupedDecodeShape<256>(d, T, K, N, g.on).area_bytes(T, N);
    else
        bytes = GroupedDecodeShape<128>(d, T, K, N, g.on).area_bytes(T, N);
    // the two launches run in turn on one stream, so their sums share the area
    if (g.on && g.plan.slices > 1)
        bytes = std::max(bytes, (size_t)g.plan.slices * T * N * sizeof(float));
    return bytes;
}

template <typename XT>
hipError_t launch_grouped_decode_t(Device* d, hipStream_t st, const XT* x, Int4Planes w,
                                  const uint32_t* off, void* out, int E, int T, int K,
                                      int N, bool write_padding, int* status,
                                      uint32_t* tickets, float* area) {
    *status = ACCEL_OK;
    if constexpr (sizeof(XT) == 4) {
        if (grouped_panel_route(x, w, false, E, T, K)) {
            // the padding rows (and every row should the offsets have
            // wrapped) on the VALU kernel, the experts' rows on the panels;
            // as beside the matrix-core blocks, the widest tile
            const int tw = N % 512 == 0 ? 512 : grouped_decode_tile(d, T, N);
            hipError_t e;
            if (tw == 512)
                e = launch_grouped_decode_tile<512, XT>(d, st, x, w, off, out, E, T, K, N,
                                                        write_padding, status, tickets, area, true);
            else if (tw == 256)
                e = launch_grouped_decode_tile<256, XT>(d, st, x, w, off, out, E, T, K, N,
                                                        write_padding, status, tickets, area, true);
            else
                e = launch_grouped_decode_tile<128, XT>(d, st, x, w, off, out, E, T, K, N,
                                                        write_padding, status, tickets, area, true);
            if (e != hipSuccess || *status != ACCEL_OK) return e;
            return launch_int4_grouped_panel_rows(st, reinterpret_cast<const float*>(x), w.panels,
                                                  w.panel_stride, off, static_cast<float*>(out),
                                                  E, T, K, N);
        }
    }
    const GroupedMfma g = grouped_mfma(d, x, w, E, T, K, N);
    // with the rows on the matrix cores, the widest tile (fewest workgroups)
    const int tw = g.on && N % 512 == 0 ? 512 : grouped_decode_tile(d, T, N);
    hipError_t e;
    if (tw == 512)
        e = launch_grouped_decode_tile<512, XT>(d, st, x, w, off, out, E, T, K, N, write_padding,
                                            status, tickets, area, g.on);
    else if (tw == 256)
        e = launch_grouped_decode_tile<256, XT>(d, st, x, w, off, out, E, T, K, N, write_padding,
                                            status, tickets, area, g.on);
    else
        e = launch_grouped_decode_tile<128, XT>(d, st, x, w, off, out, E, T, K, N, write_padding,
                                            status, tickets, area, g.on);
    if (e != hipSuccess || *status != ACCEL_OK || !g.on) return e;
    if (g.plan.groups == 2)
        return launch_grouped_mfma<2, XT>(d, st, x, w, off, out, E, T, K, N, g, tickets, area);
    return launch_grouped_mfma<1, XT>(d, st, x, w, off, out, E, T, K, N, g, tickets, area);
}

hipError_t launch_int4_grouped_decode(Device* d, hipStream_t st, const void* x, bool bf16,
                                      Int4Planes w, const uint32_t* off, void* out, int E, int T,
                                      int K, int N, bool write_padding, int* status,
                                      uint32_t* tickets, float* area) {
    if (bf16)
        return launch_grouped_decode_t(d, st, static_cast<const uint16_t*>(x), w, off, out, E, T,
                                       K, N, write_padding, status, tickets, area);
    return launch_grouped_decode_t(d, st, static_cast<const float*>(x), w, off, out, E, T, K, N,
                                   write_padding, status, tickets, area);
}

namespace {

// ---- BASELINE config 1's literal format ----------------------------------
//
// int4 with 32-row groups along K, one f32 scale per (group, column) and no
// zero point: w = (q - 8) s.  No counterpart in the reference (its groups run
// along N with an f16 scale and zero); an additive variant, reported
// separately.  A workgroup of eight waves owns 256 columns and a K slice;
// wave w takes the slice's 32-row groups w, w + 8, ...: lane (row phase p,
// column chunk c) decodes rows 4p .. 4p+3 of the group for columns 32c ..
// 32c+31, the wave's eight row phases are summed across lanes, and each
// lane scales its four reduced columns once per group:
//     sum_k x w = s (512 sum_k x (q 2^-9) - 8 sum_k x)
// (codes through the fp8 converter as in the other decode kernels).  Waves
// meet in LDS; K slices through the split-K hand-off.
constexpr int kG32Tile = 256;

__global__ __launch_bounds__(kDecThreads) void int4_g32_matvec_kernel(
    const float* __restrict__ a, const uint32_t* __restrict__ codes,
    const float* __restrict__ scales, float* __restrict__ out, float* partial,
    uint32_t* tickets, int ticket_stride, int K, int N, int rows_per_slice, int slices) {
    constexpr int TILE = kG32Tile, CPL = 32, LPR = 8, NWAVE = kDecThreads / 64;
    __shared__ __attribute__((aligned(16))) float red[NWAVE][TILE];
    __shared__ int last_flag;
    int tile, slice;
    place(blockIdx.x, N / TILE, slices, tile, slice);
    const int tid = threadIdx.x;
    const int l64 = tid & 63;
    const int wave = tid >> 6;
    const int chunk = l64 % LPR;
    const int phase = l64 / LPR;
    const int col0 = tile * TILE + chunk * CPL;
    const int cred = reduced_offset<CPL, 32, LPR>(l64);   // first of this lane's 4 reduced columns
    const size_t words_per_row = (size_t)(N >> 3);
    const int k_begin = slice * rows_per_slice;
    const int k_end = min(K, k_begin + rows_per_slice);
    const uint32_t* qcol = codes + (col0 >> 3);

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int g0 = k_begin + 32 * wave; g0 < k_end; g0 += 32 * NWAVE) {
        const int r0 = g0 + 4 * phase;
        uint32_t q[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++) load_words<4>(qcol + (size_t)(r0 + i) * words_per_row, q[i]);
        const f32x4 xv = *reinterpret_cast<const f32x4*>(a + r0);
        const f32x4 sv =
            *reinterpret_cast<const f32x4*>(scales + (size_t)(g0 >> 5) * N + col0 + cred);
        const float xr[4] = {xv.x, xv.y, xv.z, xv.w};
        float v[CPL];
#pragma unroll
        for (int j = 0; j < CPL; j++) v[j] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int wi = 0; wi < 4; wi++) {
                float f[8];
                unpack8(q[i][wi], f);
#pragma unroll
                for (int j = 0; j < 8; j++) v[wi * 8 + j] = __builtin_fmaf(xr[i], f[j], v[wi * 8 + j]);
            }
        }
        transpose_reduce<CPL, 32, LPR>(v, l64);
        // the group's activation sum: the lane's four rows, then the eight
        // row phases (lanes l ^ 8, ^ 16, ^ 32 hold the other phases)
        float xs = (xr[0] + xr[1]) + (xr[2] + xr[3]);
        xs += __shfl_xor(xs, 8, 64);
        xs += __shfl_xor(xs, 16, 64);
        xs += __shfl_xor(xs, 32, 64);
        const float sc[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
        for (int e = 0; e < 4; e++)
            acc[e] = __builtin_fmaf(sc[e], __builtin_fmaf(kNibbleScale, v[e], -8.0f * xs), acc[e]);
    }
    // after the reduction each lane holds four distinct columns of its wave's
    // sums; the waves meet in LDS
#pragma unroll
    for (int e = 0; e < 4; e++) red[wave][chunk * CPL + cred + e] = acc[e];
    __syncthreads();
    const bool split = slices > 1;
    for (int c = tid; c < TILE; c += kDecThreads) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) sum += red[w][c];
        const int col = tile * TILE + c;
        if (split)
            store_device(&partial[(size_t)slice * N + col], sum);
        else
            out[col] = sum;
    }
    if (!split) return;
    split_k_finish(partial, tickets + (size_t)tile * ticket_stride, out, tile * TILE, TILE, 1, N,
                   slices, &last_flag, Epilogue{});
}

}  // namespace

bool int4_g32_matvec_supported(int K, int N) {
    return K >= 32 && K % 32 == 0 && N >= kG32Tile && N % kG32Tile == 0 && K < (1 << 30) &&
           N < (1 << 30);
}

hipError_t launch_int4_g32_matvec(Device* d, hipStream_t st, const float* a,
                                  const uint32_t* codes, const float* scales, float* out, int K,
                                  int N, int* status) {
    *status = ACCEL_OK;
    const int tiles = N / kG32Tile;
    constexpr int kRowsPerPass = 32 * (kDecThreads / 64);   // one group per wave
    const int passes = (K + kRowsPerPass - 1) / kRowsPerPass;
    // one pass a workgroup up to 64 slices, as the reference-format GEMV
    const int per_slice = (passes + kMaxSlices - 1) / kMaxSlices;
    const int rows = per_slice * kRowsPerPass;
    const int slices = (K + rows - 1) / rows;
    float* partial = nullptr;
    uint32_t* tickets = nullptr;
    int stride = 0;
    if (slices > 1) {
        stride = ticket_stride(tiles);
        if (stride == 0) {
            *status = fail(ACCEL_E_INVALID,
                           "g32 matvec: N=%d needs more tickets than the workspace holds", N);
            return hipSuccess;
        }
        void* ws = workspace(d, st, (size_t)slices * N * sizeof(float), status);
        if (!ws) return hipSuccess;
        tickets = static_cast<uint32_t*>(ws);
        partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    }
    ACCEL_LAUNCH(std::string("int4_g32_matvec_kernel") + grid_note(tiles, slices), int4_g32_matvec_kernel, dim3(tiles * slices), dim3(kDecThreads), 0, st, a,
                       codes, scales, out, partial, tickets, stride, K, N, rows, slices);
    return launch_status();
}

// ---- the no-allocation Int4MatVec -----------------------------------------
//
// A caller that cannot allocate (code under graph capture, a serving loop
// that must not call hipMalloc) gets Int4MatVec with its split-K tickets and
// partial sums in this file-scope array instead of the library's workspace.
// Each GPU holds its own copy until the process ends.  In host code the name
// `scratch` is only a stand-in; the device address of this GPU's copy comes
// from hipGetSymbolAddress (init_scratch, at open) and is what every launch
// receives.  Every call on one GPU shares the array: calls that overlap on a
// GPU race.  The tickets start at zero (cleared at open) and each launch's
// consumer returns its own to zero.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

int init_scratch(Device* d) {
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return classify(d, e, "hipGetSymbolAddress(scratch)");
    e = hipMemset(ptr, 0, kWorkspaceCounterBytes);
    if (e != hipSuccess) return classify(d, e, "scratch ticket clear");
    e = hipDeviceSynchronize();
    if (e != hipSuccess) return classify(d, e, "scratch ticket clear");
    d->scratch = ptr;
    return ACCEL_OK;
}

hipError_t launch_int4_matvec_noalloc(Device* d, hipStream_t st, const float* a, Int4Planes w,
                                      float* out, int K, int N, int* status) {
    *status = ACCEL_OK;
    if (!d->scratch) {
        *status = fail(ACCEL_E_HIP, "Int4MatVecNoAlloc: the device's static scratch was not "
                                    "resolved when it was opened");
        return hipSuccess;
    }
    if (!int4_decode_f32_supported(1, K, N, w.codes))
        return launch_int4_generic_f32(st, a, w, out, 1, K, N, Epilogue{});   // no scratch
    const int tw = matvec_tile(N);
    if (tw == 512)
        return launch_decode<1, 512, 32>(d, st, a, w, out, K, N, status, Epilogue{}, d->scratch);
    if (tw == 256)
        return launch_decode<1, 256, 32>(d, st, a, w, out, K, N, status, Epilogue{}, d->scratch);
    return launch_decode<1, 128, 32>(d, st, a, w, out, K, N, status, Epilogue{}, d->scratch);
}

hipError_t launch_int4_generic_f32(hipStream_t st, const float* a, Int4Planes w, void* out,
                                   int M, int K, int N, Epilogue ep) {
    const int64_t total = (int64_t)M * N;
    if (total == 0) return hipSuccess;
    const int threads = 256;
    const int64_t blocks = (total + threads - 1) / threads;
    ACCEL_LAUNCH(std::string("int4_generic_f32_kernel"), int4_generic_f32_kernel, dim3((unsigned)blocks), dim3(threads), 0, st,
                       a, w.codes, w.scales, w.zeros, out, M, K, N, ep);
    return launch_status();
}

hipError_t launch_int4_generic_bf16(hipStream_t st, const uint16_t* a, Int4Planes w,
                                    uint16_t* out, int M, int K, int N, const float* bias) {
    const int64_t total = (int64_t)M * N;
    if (total == 0) return hipSuccess;
    const int threads = 256;
    const int64_t blocks = (total + threads - 1) / threads;
    ACCEL_LAUNCH(std::string("int4_generic_bf16_kernel"), int4_generic_bf16_kernel, dim3((unsigned)blocks), dim3(threads), 0,
                       st, a, w.codes, w.scales, w.zeros, out, M, K, N, bias);
    return launch_status();
}

}  // namespace accel
