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
// Kernel shape.  A workgroup of 256 lanes owns a 256-column tile (two groups,
// 128 bytes of codes per row) and a slice of K.  Each lane owns CPL adjacent
// columns and walks the rows of its row-phase; a row of the tile is read by
// 256/CPL adjacent lanes as one 128-byte segment (16-byte loads for CPL=32).
// Per (row, group) the lane folds the dequantisation into two scalars,
//     x*w = (x*s)*code + b,   b = -(x*s)*z   (or x*z for a zero scale),
// so the inner loop is one conversion and one FMA per weight, and b is summed
// once per row.  Nibbles become floats through the fp8 converter: a byte
// 0000qqqq read as OCP e4m3 is exactly q * 2^-9 (codes 0..7 are subnormals
// q/8 * 2^-6, codes 8..15 the first binade (1 + (q-8)/8) * 2^-6), so
// v_cvt_pk_f32_fp8 turns two nibbles into two exact floats and the 2^9 is
// folded into x*s.
//
// The row-phases of a workgroup are summed through LDS.  When K is split
// across workgroups, each writes its column partials to the workspace and
// the last workgroup of the tile to finish (an atomic ticket) adds the
// partials in slice order and writes the output, so the result does not
// depend on scheduling.  The ticket is reset by that workgroup.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "internal.hpp"

namespace accel {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kTile = 256;     // columns per workgroup
constexpr int kThreads = 256;  // lanes per workgroup
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

template <int CPL>
struct CodeLoad;
template <>
struct CodeLoad<32> {
    static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* w) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    }
};
template <>
struct CodeLoad<16> {
    static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* w) {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        w[0] = v.x; w[1] = v.y;
    }
};
template <>
struct CodeLoad<8> {
    static __device__ __forceinline__ void load(const uint32_t* p, uint32_t* w) {
        w[0] = __builtin_nontemporal_load(p);
    }
};

// M rows of activations, CPL columns per lane.
template <int M, int CPL>
__global__ __launch_bounds__(kThreads) void int4_decode_f32_kernel(
    const float* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    float* __restrict__ out, float* __restrict__ partial, uint32_t* __restrict__ tickets,
    int K, int N, int rows_per_slice) {
    constexpr int LPR = kTile / CPL;       // lanes per row
    constexpr int RP = kThreads / LPR;     // row phases
    constexpr int WPL = CPL / 8;           // words per lane per row
    __shared__ float red[RP][kTile];
    __shared__ int last_flag;

    const int tid = threadIdx.x;
    const int lane = tid % LPR;
    const int rp = tid / LPR;
    const int tile0 = blockIdx.x * kTile;
    const int col0 = tile0 + lane * CPL;
    const bool active = col0 < N;
    const int groups_per_row = N >> 7;
    const int g = col0 >> 7;
    const int k_begin = blockIdx.y * rows_per_slice;
    const int k_end = min(K, k_begin + rows_per_slice);
    const size_t words_per_row = (size_t)(N >> 3);

    float acc[M][CPL];
    float bias[M];
#pragma unroll
    for (int m = 0; m < M; m++) {
        bias[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; j++) acc[m][j] = 0.0f;
    }

    if (active) {
        const uint32_t* qp = codes + (size_t)(k_begin + rp) * words_per_row + (col0 >> 3);
        const uint16_t* sp = scales + (size_t)(k_begin + rp) * groups_per_row + g;
        const uint16_t* zp = zeros + (size_t)(k_begin + rp) * groups_per_row + g;
        const float* ap = a + k_begin + rp;
#pragma unroll 2
        for (int k = k_begin + rp; k < k_end; k += RP) {
            uint32_t w[WPL];
            CodeLoad<CPL>::load(qp, w);
            const float s = half_bits_to_float(*sp);
            const float z = half_bits_to_float(*zp);
            float xs[M];
#pragma unroll
            for (int m = 0; m < M; m++) {
                const float x = ap[(size_t)m * K];
                const float xsm = x * s;
                bias[m] += (s == 0.0f) ? x * z : -(xsm * z);
                xs[m] = xsm * kNibbleScale;
            }
#pragma unroll
            for (int i = 0; i < WPL; i++) {
                float f[8];
                unpack8(w[i], f);
#pragma unroll
                for (int m = 0; m < M; m++)
#pragma unroll
                    for (int j = 0; j < 8; j++)
                        acc[m][i * 8 + j] = __builtin_fmaf(xs[m], f[j], acc[m][i * 8 + j]);
            }
            qp += RP * words_per_row;
            sp += RP * groups_per_row;
            zp += RP * groups_per_row;
            ap += RP;
        }
    }

    const bool split = gridDim.y > 1;
    const int col = tile0 + tid;
#pragma unroll
    for (int m = 0; m < M; m++) {
#pragma unroll
        for (int j = 0; j < CPL; j += 4) {
            float4 v = make_float4(acc[m][j] + bias[m], acc[m][j + 1] + bias[m],
                                   acc[m][j + 2] + bias[m], acc[m][j + 3] + bias[m]);
            *reinterpret_cast<float4*>(&red[rp][lane * CPL + j]) = v;
        }
        __syncthreads();
        float sum = 0.0f;
#pragma unroll
        for (int p = 0; p < RP; p++) sum += red[p][tid];
        if (col < N) {
            if (split)
                partial[((size_t)blockIdx.y * M + m) * N + col] = sum;
            else
                out[(size_t)m * N + col] = sum;
        }
        __syncthreads();
    }
    if (!split) return;

    // Publish this slice's partials, then take a ticket; the last slice of
    // the tile to arrive adds all slices in slice order.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(&tickets[blockIdx.x], 1u);
        last_flag = (prev == gridDim.y - 1);
    }
    __syncthreads();
    if (!last_flag) return;
    __threadfence();
    if (col < N) {
#pragma unroll
        for (int m = 0; m < M; m++) {
            float sum = 0.0f;
            for (int sl = 0; sl < (int)gridDim.y; sl++)
                sum += __builtin_nontemporal_load(&partial[((size_t)sl * M + m) * N + col]);
            out[(size_t)m * N + col] = sum;
        }
    }
    if (tid == 0) tickets[blockIdx.x] = 0;
}

template <int M, int CPL>
hipError_t launch_decode(Device* d, hipStream_t st, const float* a, Int4Planes w,
                         float* out, int K, int N, int* status) {
    constexpr int LPR = kTile / CPL;
    constexpr int RP = kThreads / LPR;
    const int tiles = (N + kTile - 1) / kTile;
    // Enough workgroups to give every CU a few, each slice at least a few rows
    // per lane; the split costs M*N*4 bytes per slice of workspace traffic.
    const int target_blocks = d->cu_count * 2;
    int slices = std::max(1, target_blocks / tiles);
    const int min_rows = RP * 4;
    slices = std::min(slices, std::max(1, K / min_rows));
    int rows = (K + slices - 1) / slices;
    rows = (rows + RP - 1) / RP * RP;
    slices = (K + rows - 1) / rows;
    float* partial = nullptr;
    uint32_t* tickets = nullptr;
    if (slices > 1) {
        if ((size_t)tiles * sizeof(uint32_t) > kWorkspaceCounterBytes) {
            *status = fail(ACCEL_E_INVALID, "decode product: N=%d needs more tickets than "
                                            "the workspace holds", N);
            return hipSuccess;
        }
        void* ws = workspace(d, (size_t)slices * M * N * sizeof(float), status);
        if (!ws) return hipSuccess;
        tickets = static_cast<uint32_t*>(ws);
        partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    }
    dim3 grid(tiles, slices);
    hipLaunchKernelGGL((int4_decode_f32_kernel<M, CPL>), grid, dim3(kThreads), 0, st, a,
                       w.codes, w.scales, w.zeros, out, partial, tickets, K, N, rows);
    return hipGetLastError();
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

}  // namespace

bool int4_decode_f32_supported(int M, int K, int N, const void* codes) {
    return M >= 1 && M <= 16 && K >= 1 && N >= 128 && N % 128 == 0 &&
           (reinterpret_cast<uintptr_t>(codes) & 15) == 0 &&
           (uint64_t)K * (uint64_t)N < (1ull << 32);
}

hipError_t launch_int4_decode_f32(Device* d, hipStream_t st, const float* a, Int4Planes w,
                                  float* out, int M, int K, int N, int* status) {
    *status = ACCEL_OK;
    switch (M) {
        case 1: return launch_decode<1, 32>(d, st, a, w, out, K, N, status);
        case 2: return launch_decode<2, 32>(d, st, a, w, out, K, N, status);
        case 3: return launch_decode<3, 16>(d, st, a, w, out, K, N, status);
        case 4: return launch_decode<4, 16>(d, st, a, w, out, K, N, status);
        case 5: return launch_decode<5, 16>(d, st, a, w, out, K, N, status);
        case 6: return launch_decode<6, 16>(d, st, a, w, out, K, N, status);
        case 7: return launch_decode<7, 8>(d, st, a, w, out, K, N, status);
        case 8: return launch_decode<8, 8>(d, st, a, w, out, K, N, status);
        default: break;
    }
    // 9..16 rows: two passes of up to eight rows each.
    const int first = 8;
    hipError_t e = launch_decode<8, 8>(d, st, a, w, out, K, N, status);
    if (e != hipSuccess || *status != ACCEL_OK) return e;
    return launch_int4_decode_f32(d, st, a + (size_t)first * K, w, out + (size_t)first * N,
                                  M - first, K, N, status);
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
