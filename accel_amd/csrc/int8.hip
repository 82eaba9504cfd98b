// int8 weight products: the counterpart of the reference's QuantMatMul
// selections (tensor/quantized.go:72-163): QuantMatVec(F32) at M = 1
// (internal/kernels/matvec.go:157-235) and QuantMatMulTiled(F32) otherwise
// (internal/kernels/quant.go:126-238).
//
// Format (the reference's): quants int8 [K, N] row-major, one f16 scale per
// block of 32 consecutive flat weights (quant/quant.go:45-123), so weight
// (k, n) is q[k N + n] * s[(k N + n) / 32]; symmetric, no zero point.
//
// Decode shapes (M <= 8, N % 32 == 0, 16- or 8-byte aligned quants): the
// int4 matvec's structure on 8-bit weights.  A 512-lane workgroup owns
// TILE = 256 columns (256 bytes of every row) and a K slice; a lane owns CPL
// adjacent columns, which lie in one scale block, and kBatch rows of its row
// phase, all of whose loads (quants, scale, activations) go out before any is
// used.  Per (row, lane) the scale folds into the activations, c = x * s,
// and each weight costs a sign extension, a conversion and one FMA per
// activation row.  The row phases meet through the shared cross-lane and LDS
// stages and the K slices through the deterministic split-K hand-off.
//
// Other shapes: an LDS-tiled fp32 VALU product (64 x 64 tiles, 32-k steps)
// that dequantizes each weight once per tile with the per-element block
// index, so any N works.
//
// Activations are f32 or f16 (the reference's two widths); sums are f32 in
// this library's order, so results agree with the reference to f32 rounding.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.hpp"
#include "splitk.hpp"

namespace accel {
namespace {

template <typename ACT>
__device__ __forceinline__ float act_f32(ACT v) {
    if constexpr (sizeof(ACT) == 2)
        return half_bits_to_float(v);
    else
        return v;
}

// Byte j of a word as a signed integer, converted exactly.
__device__ __forceinline__ float sbyte(uint32_t w, int j) {
    return (float)(int32_t)(int8_t)(w >> (8 * j));
}

template <int M, int TILE, int CPL, typename ACT>
__global__ __launch_bounds__(kDecThreads) void int8_decode_kernel(
    const ACT* __restrict__ a, const int8_t* __restrict__ quants,
    const uint16_t* __restrict__ scales, float* __restrict__ out, float* partial,
    uint32_t* tickets, int ticket_stride, int K, int N, int rows_per_slice, int slices) {
    constexpr int LPR = TILE / CPL;
    constexpr int RP = kDecThreads / LPR;
    constexpr int RPW = 64 / LPR;
    constexpr int WPL = CPL / 4;   // quant words per lane per row
    constexpr int NWAVE = kDecThreads / 64;
    // every row's per-wave column sums at once: one barrier for all M rows
    __shared__ __attribute__((aligned(16))) float red[NWAVE][M][TILE];
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
    const size_t blocks_per_row = (size_t)(N >> 5);
    const size_t block = (size_t)(col0 >> 5);
    const int k_begin = slice * rows_per_slice;
    const int k_end = min(K, k_begin + rows_per_slice);
    const int8_t* qcol = quants + col0;

    float acc[M][CPL];
#pragma unroll
    for (int m = 0; m < M; m++)
#pragma unroll
        for (int j = 0; j < CPL; j++) acc[m][j] = 0.0f;

    for (int kb = k_begin; kb < k_end; kb += kBatch * RP) {
        uint32_t q[kBatch][WPL];
        uint16_t sb[kBatch];
        float xv[kBatch][M];
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const int row = min(kb + rp + i * RP, k_end - 1);
            const int8_t* p = qcol + (size_t)row * N;
            if constexpr (WPL == 4) {
                const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
                q[i][0] = v.x; q[i][1] = v.y; q[i][2] = v.z; q[i][3] = v.w;
            } else {
                const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
                q[i][0] = v.x; q[i][1] = v.y;
            }
        }
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const int row = min(kb + rp + i * RP, k_end - 1);
            sb[i] = scales[(size_t)row * blocks_per_row + block];
#pragma unroll
            for (int m = 0; m < M; m++) xv[i][m] = act_f32(a[(size_t)m * K + row]);
        }
#pragma unroll
        for (int i = 0; i < kBatch; i++) {
            const bool valid = kb + rp + i * RP < k_end;
            const float s = half_bits_to_float(sb[i]);
            float c[M];
#pragma unroll
            for (int m = 0; m < M; m++) c[m] = valid ? xv[i][m] * s : 0.0f;
#pragma unroll
            for (int wi = 0; wi < WPL; wi++)
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float f = sbyte(q[i][wi], j);
#pragma unroll
                    for (int m = 0; m < M; m++)
                        acc[m][wi * 4 + j] = __builtin_fmaf(c[m], f, acc[m][wi * 4 + j]);
                }
        }
    }

    const bool split = slices > 1;
    constexpr int NV = CPL / RPW;
#pragma unroll
    for (int m = 0; m < M; m++) {
        float v[CPL];
#pragma unroll
        for (int j = 0; j < CPL; j++) v[j] = acc[m][j];
        transpose_reduce<CPL, 64 / 2, LPR>(v, l64);
        const int c0 = lane * CPL + reduced_offset<CPL, 64 / 2, LPR>(l64);
#pragma unroll
        for (int e = 0; e < NV; e++) red[wave][m][c0 + e] = v[e];
    }
    __syncthreads();
    for (int idx = tid; idx < M * TILE; idx += kDecThreads) {
        const int m = idx / TILE, cc = idx - m * TILE;
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < NWAVE; w++) sum += red[w][m][cc];
        const int col = tile * TILE + cc;
        if (split)
            store_device(&partial[((size_t)slice * M + m) * N + col], sum);
        else
            out[(size_t)m * N + col] = sum;
    }
    if (!split) return;
    split_k_finish(partial, tickets + (size_t)tile * ticket_stride, out, tile * TILE, TILE, M, N,
                   slices, &last_flag, Epilogue{});
}

constexpr int QM = 64, QN = 64, QK = 32;

template <typename ACT>
__global__ __launch_bounds__(256) void int8_gemm_kernel(const ACT* __restrict__ a,
                                                        const int8_t* __restrict__ quants,
                                                        const uint16_t* __restrict__ scales,
                                                        float* __restrict__ out, int M, int K,
                                                        int N) {
    __shared__ float As[QK][QM + 4];   // k-major: a lane's four rows are adjacent
    __shared__ float Bs[QK][QN + 4];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int n0 = blockIdx.x * QN, m0 = blockIdx.y * QM;
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += QK) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int idx = tid + i * 256;
            const int r = idx >> 5, kk = idx & 31;
            const int row = m0 + r, k = k0 + kk;
            As[kk][r] = (row < M && k < K) ? act_f32(a[(size_t)row * K + k]) : 0.0f;
        }
        {
            // 32 k x 64 n: eight weights of one row per lane, each with its
            // own block index (blocks run over the flat array)
            const int kk = tid >> 3, c8 = tid & 7;
            const int k = k0 + kk;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int n = n0 + c8 * 8 + j;
                float f = 0.0f;
                if (k < K && n < N) {
                    const size_t w = (size_t)k * N + n;
                    f = (float)quants[w] * half_bits_to_float(scales[w >> 5]);
                }
                Bs[kk][c8 * 8 + j] = f;
            }
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < QK; kk++) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) av[i] = As[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; j++) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = m0 + ty * 4 + i;
        if (row >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int col = n0 + tx * 4 + j;
            if (col < N) out[(size_t)row * N + col] = acc[i][j];
        }
    }
}

template <int M, int TILE, int CPL, typename ACT>
hipError_t launch_int8_decode(Device* d, hipStream_t st, const ACT* a, const int8_t* q,
                              const uint16_t* s, float* out, int K, int N, int* status) {
    constexpr int LPR = TILE / CPL;
    constexpr int RP = kDecThreads / LPR;
    constexpr int kRowsPerBatch = kBatch * RP;
    const int tiles = N / TILE;
    const int batches = (K + kRowsPerBatch - 1) / kRowsPerBatch;
    // slices <= K / (16 M): the f32 partials (slices x M x N x 4 bytes) stay
    // within a quarter of the quant bytes they summarise
    const int max_slices = std::max(1, std::min(kMaxSlices, K / (16 * M)));
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
                           "int8 product: N=%d needs more tickets than the workspace holds", N);
            return hipSuccess;
        }
        void* ws = workspace(d, st, (size_t)slices * M * N * sizeof(float), status);
        if (!ws) return hipSuccess;
        tickets = static_cast<uint32_t*>(ws);
        partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    }
    hipLaunchKernelGGL((int8_decode_kernel<M, TILE, CPL, ACT>), dim3(tiles * slices),
                       dim3(kDecThreads), 0, st, a, q, s, out, partial, tickets, stride, K, N,
                       rows, slices);
    return hipGetLastError();
}

// Columns per lane by row count: 16 (one 16-byte load a row) for one or two
// rows, 8 for more, so the accumulators (M * CPL) stay near 64.
template <int M, typename ACT>
hipError_t launch_int8_decode_m(Device* d, hipStream_t st, const ACT* a, const int8_t* q,
                                const uint16_t* s, float* out, int K, int N, int* status) {
    constexpr int CPL = M <= 2 ? 16 : 8;
    return launch_int8_decode<M, 256, CPL, ACT>(d, st, a, q, s, out, K, N, status);
}

template <typename ACT>
hipError_t launch_int8_any(Device* d, hipStream_t st, const ACT* a, const int8_t* q,
                           const uint16_t* s, float* out, int M, int K, int N, int* status) {
    *status = ACCEL_OK;
    if (M <= 0 || N <= 0) return hipSuccess;
    // N <= 2^24 keeps the decode grid (N / 256 tiles x 64 slices x 512
    // lanes) within 2^32 work-items
    const bool decode = M <= 8 && K >= 1 && N % 256 == 0 && N <= (1 << 24) &&
                        (reinterpret_cast<uintptr_t>(q) & 15) == 0;
    if (decode) {
        switch (M) {
            case 1: return launch_int8_decode_m<1>(d, st, a, q, s, out, K, N, status);
            case 2: return launch_int8_decode_m<2>(d, st, a, q, s, out, K, N, status);
            case 3: return launch_int8_decode_m<3>(d, st, a, q, s, out, K, N, status);
            case 4: return launch_int8_decode_m<4>(d, st, a, q, s, out, K, N, status);
            case 5: return launch_int8_decode_m<5>(d, st, a, q, s, out, K, N, status);
            case 6: return launch_int8_decode_m<6>(d, st, a, q, s, out, K, N, status);
            case 7: return launch_int8_decode_m<7>(d, st, a, q, s, out, K, N, status);
            default: return launch_int8_decode_m<8>(d, st, a, q, s, out, K, N, status);
        }
    }
    dim3 grid((N + QN - 1) / QN, (M + QM - 1) / QM);
    if ((uint64_t)grid.x * 256 >= (1ull << 32) || grid.y > 65535) {
        *status = fail(ACCEL_E_UNSUPPORTED,
                       "int8 product: M=%d N=%d is past this library's launch grid", M, N);
        return hipSuccess;
    }
    hipLaunchKernelGGL((int8_gemm_kernel<ACT>), grid, dim3(256), 0, st, a, q, s, out, M, K, N);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_int8_product(Device* d, hipStream_t st, const void* a, bool f16_act,
                               const int8_t* quants, const uint16_t* scales, float* out, int M,
                               int K, int N, int* status) {
    if (f16_act)
        return launch_int8_any(d, st, static_cast<const uint16_t*>(a), quants, scales, out, M,
                               K, N, status);
    return launch_int8_any(d, st, static_cast<const float*>(a), quants, scales, out, M, K, N,
                           status);
}

}  // namespace accel
