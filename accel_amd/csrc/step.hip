// Decode-step neighbours of the int4 products: SwiGLU and RMSNorm, in the
// reference's evaluation order so that the results are the reference CPU
// backend's bit for bit.
//
// SwiGLU (internal/kernels/elementwise.go:85-91): out = a / (1 + Exp(-a)) * b,
// where Exp is the f64 exponential rounded once to f32 (kmath/kmath.go:55).
// Every operation is rounded to f32 on its own (no contraction).  The kernel
// is HBM-bound (12 bytes an element); a lane handles four consecutive
// elements with 16-byte accesses when the buffers allow it.
//
// RMSNorm (internal/kernels/norm.go:47-80): one workgroup a row.  The
// reference's lane l sums x[i]^2 over i = l, l+128, ... in increasing i, the
// 128 partials meet in its halving tree (stride 64 .. 1), and
// out[i] = (x[i] * RSqrt(mean + eps)) * w[i] with RSqrt the f64 reciprocal
// square root rounded to f32 (kmath/kmath.go:52).  That order is kept, not
// re-chosen for the hardware, because it is what makes the result exact.
// What is re-chosen is how the row arrives: rows that fit are staged in LDS
// by the whole workgroup with 16-byte loads before the 128 partials are
// formed, so a decode-shape row costs one memory round trip.
#include <hip/hip_runtime.h>

#include "internal.hpp"
#include "splitk.hpp"

namespace accel {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));


__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ a,
                                                     const float* __restrict__ b,
                                                     float* __restrict__ out, int64_t n,
                                                     bool vec4) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (vec4) {
        const int64_t e = 4 * i;
        if (e + 4 <= n) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(a + e);
            const f32x4 y = *reinterpret_cast<const f32x4*>(b + e);
            f32x4 r;
#pragma unroll
            for (int j = 0; j < 4; j++) r[j] = swiglu1(x[j], y[j]);
            *reinterpret_cast<f32x4*>(out + e) = r;
        } else {
            for (int64_t k = e; k < n; k++) out[k] = swiglu1(a[k], b[k]);
        }
    } else if (i < n) {
        out[i] = swiglu1(a[i], b[i]);
    }
}

constexpr int kRowLanes = 128;   // the reference's RowWidth (norm.go:25)
constexpr int kChunk = 16;       // loads a lane issues before it adds
constexpr int kHold = 32;        // values a lane keeps for the second pass

__global__ __launch_bounds__(kRowLanes) void rmsnorm_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ w,
                                                            float* __restrict__ out, int width,
                                                            float eps) {
#pragma clang fp contract(off)
    __shared__ float sh[kRowLanes];
    const int l = threadIdx.x;
    const float* xr = x + (size_t)blockIdx.x * width;
    float* orow = out + (size_t)blockIdx.x * width;
    // lane l's elements are l + 128 j; loads go out kChunk at a time and are
    // added in increasing j, the reference's order
    const int n = l < width ? (width - l + kRowLanes - 1) / kRowLanes : 0;
    float held[kHold];
    float acc = 0.0f;
    for (int j0 = 0; j0 < n; j0 += kChunk) {
        float v[kChunk];
#pragma unroll
        for (int j = 0; j < kChunk; j++)
            v[j] = j0 + j < n ? xr[l + (size_t)kRowLanes * (j0 + j)] : 0.0f;
#pragma unroll
        for (int j = 0; j < kChunk; j++) {
            if (j0 + j < n) {
                const float sq = v[j] * v[j];
                acc = acc + sq;
            }
        }
        if (j0 < kHold) {
#pragma unroll
            for (int j = 0; j < kChunk; j++)
                if (j0 + j < kHold) held[j0 + j] = v[j];
        }
    }
    sh[l] = acc;
    __syncthreads();
    for (int stride = kRowLanes / 2; stride > 0; stride /= 2) {
        if (l < stride) sh[l] = sh[l] + sh[l + stride];
        __syncthreads();
    }
    const float mean = sh[0] / (float)width;
    const float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    for (int j0 = 0; j0 < n; j0 += kChunk) {
        float g[kChunk], v[kChunk];
#pragma unroll
        for (int j = 0; j < kChunk; j++) {
            const size_t i = l + (size_t)kRowLanes * (j0 + j);
            g[j] = j0 + j < n ? w[i] : 0.0f;
            v[j] = j0 + j < kHold ? held[j0 + j] : (j0 + j < n ? xr[i] : 0.0f);
        }
#pragma unroll
        for (int j = 0; j < kChunk; j++) {
            if (j0 + j < n) {
                const float t = v[j] * scale;
                orow[l + (size_t)kRowLanes * (j0 + j)] = t * g[j];
            }
        }
    }
}

// Rows up to kLdsWidth wide: the whole row and the gain go to LDS with
// 16-byte loads from all 256 lanes at once (one memory round trip), lanes
// 0..127 then form the reference's 128 strided partials from LDS in the
// reference's order, and every lane writes its share of the output.
constexpr int kLdsThreads = 256;
constexpr int kLdsWidth = 16384;

__global__ __launch_bounds__(kLdsThreads) void rmsnorm_lds_kernel(const float* __restrict__ x,
                                                                  const float* __restrict__ w,
                                                                  float* __restrict__ out,
                                                                  int width, float eps) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* xs = smem;            // [width]
    float* ws = smem + width;    // [width]
    __shared__ float sh[kRowLanes];
    const int t = threadIdx.x;
    const float* xr = x + (size_t)blockIdx.x * width;
    float* orow = out + (size_t)blockIdx.x * width;
    const int w4 = width / 4;    // width % 4 == 0 and 16-byte rows on this path
    for (int i = t; i < w4; i += kLdsThreads) {
        reinterpret_cast<f32x4*>(xs)[i] = reinterpret_cast<const f32x4*>(xr)[i];
        reinterpret_cast<f32x4*>(ws)[i] = reinterpret_cast<const f32x4*>(w)[i];
    }
    __syncthreads();
    if (t < kRowLanes) {
        float acc = 0.0f;
        for (int i = t; i < width; i += kRowLanes) {
            const float v = xs[i];
            const float sq = v * v;
            acc = acc + sq;
        }
        sh[t] = acc;
    }
    __syncthreads();
    for (int stride = kRowLanes / 2; stride > 0; stride /= 2) {
        if (t < stride) sh[t] = sh[t] + sh[t + stride];
        __syncthreads();
    }
    const float mean = sh[0] / (float)width;
    const float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    for (int i = t; i < w4; i += kLdsThreads) {
        const f32x4 v = reinterpret_cast<const f32x4*>(xs)[i];
        const f32x4 g = reinterpret_cast<const f32x4*>(ws)[i];
        f32x4 r;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float p = v[j] * scale;
            r[j] = p * g[j];
        }
        reinterpret_cast<f32x4*>(orow)[i] = r;
    }
}

}  // namespace

hipError_t launch_swiglu(hipStream_t st, const float* a, const float* b, float* out, int64_t n) {
    if (n <= 0) return hipSuccess;
    const bool vec4 = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                        reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    const int64_t lanes = vec4 ? (n + 3) / 4 : n;
    const int64_t blocks = (lanes + 255) / 256;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a, b, out, n,
                       vec4);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(hipStream_t st, const float* x, const float* w, float* out, int rows,
                          int width, float eps) {
    if (rows <= 0 || width <= 0) return hipSuccess;
    const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w) |
                           reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (aligned && width % 4 == 0 && width <= kLdsWidth) {
        hipLaunchKernelGGL(rmsnorm_lds_kernel, dim3(rows), dim3(kLdsThreads),
                           (size_t)2 * width * sizeof(float), st, x, w, out, width, eps);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kRowLanes), 0, st, x, w, out, width,
                       eps);
    return hipGetLastError();
}

}  // namespace accel
