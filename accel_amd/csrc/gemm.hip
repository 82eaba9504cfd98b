// Prefill-shape int4 products: the counterpart of the reference's tiled
// QuantMatMulInt4 (internal/kernels/int4tiled.go:166-238), rebuilt around
// CDNA4's bf16 matrix cores.
//
// bf16 path (activations and output bf16, fp32 accumulation).  A workgroup
// of 256 lanes (four waves, 2x2) computes a 128x128 output tile; each wave a
// 64x64 block as 4x4 v_mfma_f32_16x16x32_bf16 tiles.  Per K step of 64:
//   * the activation tile (128 rows x 128 bytes) is loaded with 16-byte loads
//     and stored to LDS as rows of 64 k;
//   * the code tile (64 rows x 64 bytes) is loaded as 4-row x 8-column
//     blocks, one per lane, dequantised in registers to bf16 and written to
//     LDS transposed, as columns of 64 k -- the layout the MFMA B operand
//     reads, 8 consecutive k per lane;
// both LDS tiles use a 16-byte XOR swizzle so the operand reads (16 rows x
// 4 chunks per wave) hit every bank slot equally.  LDS is double buffered,
// and the next step's global loads are issued before the current step's
// MFMAs.  The 128-column tile is one quantisation group wide, so a K row of
// the tile has one (scale, zero) pair.
//
// f32 path (the reference API's f32 activations and output, M > 16): an
// LDS-tiled fp32 VALU product, exact up to f32 rounding order.
#include <hip/hip_runtime.h>

#include "internal.hpp"

namespace accel {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kThreads = 256;
constexpr int kRowBytes = BK * 2;  // one LDS row: 64 bf16

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

__device__ __forceinline__ void unpack8(uint32_t w, float* f) {
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
    const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
    const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
    const f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
    f[0] = a.x; f[2] = a.y; f[4] = b.x; f[6] = b.y;
    f[1] = c.x; f[3] = c.y; f[5] = d.x; f[7] = d.y;
}

// Byte offset of 16-byte chunk `c` of LDS row `r` under the swizzle.
__device__ __forceinline__ int swz(int r, int c) {
    return r * kRowBytes + ((c ^ ((r >> 1) & 7)) << 4);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 v;
    v.x = (__bf16)lo;
    v.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
}

// One 128x128 output tile: rows [m0, m_end) of a/out are valid (rows past
// m_end are computed from a clamped row and never stored); the codes,
// scales and zeros pointers are those of the [K, N] matrix in use.
__device__ __forceinline__ void gemm_tile_bf16(
    char (*lds)[2][BM * kRowBytes], const uint16_t* __restrict__ a,
    const uint32_t* __restrict__ codes, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ zeros, uint16_t* __restrict__ out, int m0, int m_end,
    int n0, int K, int N) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int groups_per_row = N >> 7;
    const int g = n0 >> 7;
    const size_t words_per_row = (size_t)(N >> 3);

    // A loader: row t/2, 64 bytes at (t&1)*64.
    const int a_row = tid >> 1;
    const int a_half = tid & 1;
    const int a_grow = min(m0 + a_row, m_end - 1);
    const uint16_t* a_src = a + (size_t)a_grow * K + a_half * 32;
    // B loader: 8 columns (one word) x 4 rows.
    const int b_cw = tid & 15;
    const int b_rq = tid >> 4;
    const uint32_t* b_src = codes + (size_t)(b_rq * 4) * words_per_row + (n0 >> 3) + b_cw;
    const uint16_t* s_src = scales + (size_t)(b_rq * 4) * groups_per_row + g;
    const uint16_t* z_src = zeros + (size_t)(b_rq * 4) * groups_per_row + g;

    uint4 a_reg[4];
    uint32_t b_reg[4];
    uint16_t s_reg[4], z_reg[4];

    auto load_global = [&](int k0) {
        const uint4* ap = reinterpret_cast<const uint4*>(a_src + k0);
#pragma unroll
        for (int i = 0; i < 4; i++) a_reg[i] = ap[i];
        const size_t roff = (size_t)k0 * words_per_row;
        const size_t goff = (size_t)k0 * groups_per_row;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            b_reg[i] = __builtin_nontemporal_load(b_src + roff + i * words_per_row);
            s_reg[i] = s_src[goff + i * groups_per_row];
            z_reg[i] = z_src[goff + i * groups_per_row];
        }
    };

    auto store_lds = [&](int buf) {
        char* As = lds[buf][0];
        char* Bs = lds[buf][1];
#pragma unroll
        for (int i = 0; i < 4; i++)
            *reinterpret_cast<uint4*>(As + swz(a_row, a_half * 4 + i)) = a_reg[i];
        // Dequantise the 4x8 block and write it transposed: column n gets
        // k = 4*b_rq .. 4*b_rq+3 (half of one 16-byte chunk).
        float v[4][8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float s = half_bits_to_float(s_reg[i]);
            const float z = half_bits_to_float(z_reg[i]);
            const float mul = s * 512.0f;
            const float add = (s == 0.0f) ? z : -(z * s);
            float f[8];
            unpack8(b_reg[i], f);
#pragma unroll
            for (int j = 0; j < 8; j++) v[i][j] = __builtin_fmaf(f[j], mul, add);
        }
        const int chunk = b_rq >> 1;
        const int sub = (b_rq & 1) * 8;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int n = b_cw * 8 + j;
            uint2 pr;
            pr.x = pack_bf16x2(v[0][j], v[1][j]);
            pr.y = pack_bf16x2(v[2][j], v[3][j]);
            *reinterpret_cast<uint2*>(Bs + swz(n, chunk) + sub) = pr;
        }
    };

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const int ktiles = K / BK;
    load_global(0);
    store_lds(0);
    __syncthreads();

    const int r16 = lane & 15;
    const int kq = lane >> 4;  // which 8-k chunk within a 32-k MFMA step
    for (int kt = 0; kt < ktiles; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < ktiles) load_global((kt + 1) * BK);
        const char* As = lds[cur][0];
        const char* Bs = lds[cur][1];
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            bf16x8 af[4], bfr[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                af[t] = *reinterpret_cast<const bf16x8*>(
                    As + swz(wm * 64 + t * 16 + r16, ks * 4 + kq));
                bfr[t] = *reinterpret_cast<const bf16x8*>(
                    Bs + swz(wn * 64 + t * 16 + r16, ks * 4 + kq));
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j],
                                                                        acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < ktiles) store_lds(cur ^ 1);
        __syncthreads();
    }

    // D layout of a 16x16 tile: lane holds column lane%16, rows 4*(lane/16)+i.
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int col = n0 + wn * 64 + j * 16 + r16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = m0 + wm * 64 + i * 16 + kq * 4 + r;
                if (row < m_end) {
                    const __bf16 v = (__bf16)acc[i][j][r];
                    out[(size_t)row * N + col] = __builtin_bit_cast(uint16_t, v);
                }
            }
        }
    }
}

__global__ __launch_bounds__(kThreads, 2) void int4_gemm_bf16_kernel(
    const uint16_t* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    uint16_t* __restrict__ out, int M, int K, int N) {
    __shared__ __attribute__((aligned(16))) char lds[2][2][BM * kRowBytes];  // [buf][A|B]
    // Consecutive workgroups walk N within a band of M rows, so the band's
    // activations stay cache-resident while the codes stream.
    const int tiles_n = N / BN;
    const int m0 = (blockIdx.x / tiles_n) * BM;
    const int n0 = (blockIdx.x % tiles_n) * BN;
    gemm_tile_bf16(lds, a, codes, scales, zeros, out, m0, M, n0, K, N);
}

// Ragged grouped form: blockIdx.x is the column tile, blockIdx.y the
// position in the list of (expert, 128-row block) pairs, walked from the
// offsets; blocks past the list's end exit.  Expert e's rows are
// [off[e], min(off[e+1], T)) (groupedtiled.go:184-188).
__global__ __launch_bounds__(kThreads, 2) void int4_grouped_bf16_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    const uint32_t* __restrict__ off, uint16_t* __restrict__ out, int E, int T, int K,
    int N) {
    __shared__ __attribute__((aligned(16))) char lds[2][2][BM * kRowBytes];
    int idx = blockIdx.y;
    int e = 0, m0 = 0, m_end = 0;
    bool found = false;
    for (; e < E; e++) {
        const uint32_t first = off[e];
        uint32_t last = off[e + 1];
        if (last > (uint32_t)T) last = (uint32_t)T;
        const int rows = last > first ? (int)(last - first) : 0;
        const int blocks = (rows + BM - 1) / BM;
        if (idx < blocks) {
            m0 = (int)first + idx * BM;
            m_end = (int)last;
            found = true;
            break;
        }
        idx -= blocks;
    }
    if (!found) return;
    const size_t per_expert = (size_t)K * N;
    gemm_tile_bf16(lds, x, codes + e * (per_expert >> 3), scales + e * (per_expert >> 7),
                   zeros + e * (per_expert >> 7), out, m0, m_end, blockIdx.x * BN, K, N);
}

// ---- f32 activations, fp32 VALU tiles -------------------------------------

constexpr int FM = 64, FN = 64, FK = 32;

__global__ __launch_bounds__(256) void int4_gemm_f32_kernel(
    const float* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    float* __restrict__ out, int M, int K, int N) {
    __shared__ float As[FK][FM + 4];   // k-major so a lane's 4 rows are adjacent
    __shared__ float Bs[FK][FN + 4];
    const int tid = threadIdx.x;
    const int tx = tid & 15, ty = tid >> 4;
    const int n0 = blockIdx.x * FN, m0 = blockIdx.y * FM;
    const int groups_per_row = N >> 7;
    const size_t words_per_row = (size_t)(N >> 3);
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += FK) {
        // A: 64 rows x 32 k, 8 per lane
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int idx = tid + i * 256;
            const int r = idx >> 5, kk = idx & 31;
            const int row = m0 + r, k = k0 + kk;
            As[kk][r] = (row < M && k < K) ? a[(size_t)row * K + k] : 0.0f;
        }
        // B: 32 k x 64 n = 32 rows x 8 words, one word per lane
        {
            const int kk = tid >> 3, cw = tid & 7;
            const int k = k0 + kk;
            const int n = n0 + cw * 8;
            float f[8];
            if (k < K && n < N) {
                const uint32_t w = codes[(size_t)k * words_per_row + (n >> 3)];
                const float s = half_bits_to_float(scales[(size_t)k * groups_per_row + (n >> 7)]);
                const float z = half_bits_to_float(zeros[(size_t)k * groups_per_row + (n >> 7)]);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float code = (float)((w >> (4 * j)) & 0xfu);
                    f[j] = s == 0.0f ? z : (code - z) * s;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 8; j++) f[j] = 0.0f;
            }
#pragma unroll
            for (int j = 0; j < 8; j++) Bs[kk][cw * 8 + j] = f[j];
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < FK; kk++) {
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

}  // namespace

bool int4_gemm_bf16_supported(int M, int K, int N) {
    return M >= 1 && K >= BK && K % BK == 0 && N >= BN && N % BN == 0 &&
           (uint64_t)K * (uint64_t)N < (1ull << 32);
}

hipError_t launch_int4_gemm_bf16(Device*, hipStream_t st, const uint16_t* a, Int4Planes w,
                                 uint16_t* out, int M, int K, int N) {
    const int tiles = ((M + BM - 1) / BM) * (N / BN);
    hipLaunchKernelGGL(int4_gemm_bf16_kernel, dim3(tiles), dim3(kThreads), 0, st, a, w.codes,
                       w.scales, w.zeros, out, M, K, N);
    return hipGetLastError();
}

hipError_t launch_int4_grouped_bf16(Device*, hipStream_t st, const uint16_t* x,
                                    Int4Planes w, const uint32_t* off, uint16_t* out, int E,
                                    int T, int K, int N, bool) {
    // Upper bound on (expert, row block) pairs: every expert can add one
    // partial block.
    const int max_blocks = (T + BM - 1) / BM + E;
    if (max_blocks > 65535) return hipErrorInvalidConfiguration;
    dim3 grid(N / BN, max_blocks);
    hipLaunchKernelGGL(int4_grouped_bf16_kernel, grid, dim3(kThreads), 0, st, x, w.codes,
                       w.scales, w.zeros, off, out, E, T, K, N);
    return hipGetLastError();
}

hipError_t launch_int4_gemm_f32(Device*, hipStream_t st, const float* a, Int4Planes w,
                                float* out, int M, int K, int N) {
    dim3 grid((N + FN - 1) / FN, (M + FM - 1) / FM);
    hipLaunchKernelGGL(int4_gemm_f32_kernel, grid, dim3(256), 0, st, a, w.codes, w.scales,
                       w.zeros, out, M, K, N);
    return hipGetLastError();
}

}  // namespace accel
