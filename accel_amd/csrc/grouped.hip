// Ragged grouped products and their segment offsets: the counterparts of the
// reference's SegmentOffsets (internal/kernels/segment.go:40-50),
// GroupedMatVec (internal/kernels/grouped.go:47-97) and GroupedMatMul
// (internal/kernels/groupedtiled.go:77-134), for f32 weights [E,K,N] and
// for stacked int4 weights.
//
// Token t of x [T,K] belongs to expert e(t) = #{r : off[r+1] <= t}.  The
// matvec form writes 0 for a token past the last segment; the matmul form
// covers rows [off[e], min(off[e+1], T)) per expert and leaves the others
// unwritten.  Both forms compute the same values on the rows they write.
#include <hip/hip_runtime.h>

#include "internal.hpp"

namespace accel {
namespace {

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

// Exclusive prefix sum of `rows` counts: one wave, a carried running total
// over chunks of 64.  u32 arithmetic wraps as the reference's does.
__global__ __launch_bounds__(64) void segment_offsets_kernel(const uint32_t* __restrict__ counts,
                                                             uint32_t* __restrict__ offsets,
                                                             int rows) {
    const int lane = threadIdx.x;
    uint32_t carry = 0;
    for (int base = 0; base < rows; base += 64) {
        const int r = base + lane;
        const uint32_t c = r < rows ? counts[r] : 0u;
        uint32_t incl = c;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t up = __shfl_up(incl, d, 64);
            if (lane >= d) incl += up;
        }
        if (r < rows) offsets[r] = carry + incl - c;
        carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) offsets[rows] = carry;
}

// Expert of token t, or E when t is past every segment.
__device__ __forceinline__ int expert_of(const uint32_t* off, int E, uint32_t t) {
    int e = 0;
    for (int r = 0; r < E; r++) e += (off[r + 1] <= t) ? 1 : 0;
    return e;
}

// Whether row t is inside expert e's clamped segment.
__device__ __forceinline__ bool in_segment(const uint32_t* off, int e, uint32_t t, int T) {
    uint32_t last = off[e + 1];
    if (last > (uint32_t)T) last = (uint32_t)T;
    return t >= off[e] && t < last;
}

// One lane per (token, column); consecutive lanes take consecutive columns,
// so the weight row reads coalesce.  `int4` selects the weight source.
template <bool kInt4>
__global__ __launch_bounds__(256) void grouped_f32_kernel(
    const float* __restrict__ x, const float* __restrict__ wf,
    const uint32_t* __restrict__ codes, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ zeros, const uint32_t* __restrict__ off,
    float* __restrict__ out, int E, int T, int K, int N, bool write_padding) {
    const int col = blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= N) return;
    for (int t = blockIdx.y; t < T; t += gridDim.y) {
        const int e = expert_of(off, E, (uint32_t)t);
        if (e >= E) {  // past every segment: the matvec form writes 0
            if (write_padding) out[(size_t)t * N + col] = 0.0f;
            continue;
        }
        // The matmul form writes only rows its expert's clamped segment covers.
        if (!write_padding && !in_segment(off, e, (uint32_t)t, T)) continue;
        const uint64_t base = (uint64_t)e * K * N;
        const float* xr = x + (size_t)t * K;
        float acc = 0.0f;
        for (int k = 0; k < K; k++) {
            const uint64_t idx = base + (uint64_t)k * N + col;
            float wv;
            if (kInt4) {
                const uint32_t code = (codes[idx >> 3] >> (4 * (idx & 7))) & 0xfu;
                const float s = half_bits_to_float(scales[idx >> 7]);
                const float z = half_bits_to_float(zeros[idx >> 7]);
                wv = s == 0.0f ? z : ((float)code - z) * s;
            } else {
                wv = wf[idx];
            }
            acc = __builtin_fmaf(xr[k], wv, acc);
        }
        out[(size_t)t * N + col] = acc;
    }
}

// Zero rows [start, T) of a [T, N] output, start = min(off[E], T): the
// matvec form's padding rows (off: the segment bounds below).
template <typename OT>
__global__ void zero_tail_kernel(const uint32_t* __restrict__ off, OT* out, int E, int T,
                                 int N) {
    uint32_t start = off[E];
    if (start > (uint32_t)T) start = (uint32_t)T;
    const size_t begin = (size_t)start * N, end = (size_t)T * N;
    for (size_t i = begin + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < end;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = 0;
}

// The matvec form's segment bounds: token t belongs to expert
// e(t) = #{r : off[r+1] <= t}, which never decreases as t grows, so expert
// e's tokens are [S(e-1), S(e)) for S the offsets off[1..E] in increasing
// order (S(-1) = 0), and the tokens from S(E-1) on are padding.  bounds[0] =
// 0 and bounds[1 + rank of off[j+1]] = off[j+1], ties in index order.  For
// offsets that do not wrap (sorted) the bounds are the offsets themselves;
// counts whose sum wraps u32 leave them unsorted, and the tiled products
// then walk the bounds rather than the offsets.
__global__ __launch_bounds__(256) void segment_bounds_kernel(const uint32_t* __restrict__ off,
                                                             uint32_t* __restrict__ bounds,
                                                             int E) {
    for (int j = blockIdx.x * blockDim.x + threadIdx.x; j < E; j += gridDim.x * blockDim.x) {
        const uint32_t v = off[j + 1];
        int rank = 0;
        for (int i = 0; i < E; i++) {
            const uint32_t u = off[i + 1];
            rank += (u < v || (u == v && i < j)) ? 1 : 0;
        }
        bounds[rank + 1] = v;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) bounds[0] = 0;
}

}  // namespace

hipError_t launch_segment_offsets(hipStream_t st, const uint32_t* counts, uint32_t* offsets,
                                  int rows) {
    ACCEL_LAUNCH(std::string("segment_offsets_kernel"), segment_offsets_kernel, dim3(1),
                 dim3(64), 0, st, counts, offsets, rows);
    return launch_status();
}

hipError_t launch_grouped_f32(hipStream_t st, const float* x, const float* w,
                              const uint32_t* off, float* out, int E, int T, int K, int N,
                              bool write_padding) {
    if (T == 0 || N == 0) return hipSuccess;
    dim3 grid((N + 255) / 256, T < 65535 ? T : 65535);
    ACCEL_LAUNCH(tname("grouped_f32_kernel", false), (grouped_f32_kernel<false>), grid,
                 dim3(256), 0, st, x, w, nullptr, nullptr, nullptr, off, out, E, T, K, N,
                 write_padding);
    return launch_status();
}

hipError_t launch_int4_grouped_f32(hipStream_t st, const float* x, Int4Planes w,
                                   const uint32_t* off, float* out, int E, int T, int K,
                                   int N, bool write_padding) {
    if (T == 0 || N == 0) return hipSuccess;
    dim3 grid((N + 255) / 256, T < 65535 ? T : 65535);
    ACCEL_LAUNCH(tname("grouped_f32_kernel", true), (grouped_f32_kernel<true>), grid,
                 dim3(256), 0, st, x, nullptr, w.codes, w.scales, w.zeros, off, out, E, T, K,
                 N, write_padding);
    return launch_status();
}

hipError_t launch_zero_tail_bf16(hipStream_t st, const uint32_t* off, uint16_t* out, int E,
                                 int T, int N) {
    if (T == 0 || N == 0) return hipSuccess;
    ACCEL_LAUNCH(tname("zero_tail_kernel", "unsigned short"), zero_tail_kernel<uint16_t>,
                 dim3(256), dim3(256), 0, st, off, out, E, T, N);
    return launch_status();
}

hipError_t launch_zero_tail_f32(hipStream_t st, const uint32_t* off, float* out, int E, int T,
                                int N) {
    if (T == 0 || N == 0) return hipSuccess;
    ACCEL_LAUNCH(tname("zero_tail_kernel", "float"), zero_tail_kernel<float>, dim3(256),
                 dim3(256), 0, st, off, out, E, T, N);
    return launch_status();
}

hipError_t launch_segment_bounds(hipStream_t st, const uint32_t* off, uint32_t* bounds, int E) {
    ACCEL_LAUNCH(std::string("segment_bounds_kernel"), segment_bounds_kernel,
                 dim3((E + 255) / 256), dim3(256), 0, st, off, bounds, E);
    return launch_status();
}

}  // namespace accel
