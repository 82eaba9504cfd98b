// Device helpers shared by the decode-shape kernels (int4, f16 and int8
// matvecs): the split-K hand-off, the cross-lane row-phase reduction, the
// f16 widening and the reference's SwiGLU of one element.  Included into one
// anonymous namespace per translation unit.
#pragma once

#include <hip/hip_runtime.h>

#include "internal.hpp"

namespace accel {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kDecThreads = 512;        // lanes per workgroup of the VALU kernel
constexpr int kBatch = 4;               // rows per lane per fetch batch
constexpr int kMaxSlices = 64;          // K slices of a VALU decode launch, at most

// SwiGLU of one element (internal/kernels/elementwise.go:85-91):
// a / (1 + Exp(-a)) * b, Exp the f64 exponential rounded once to f32
// (kmath/kmath.go:55), every other operation rounded to f32 on its own.
__device__ __forceinline__ float swiglu1(float x, float b) {
#pragma clang fp contract(off)
    const float e = (float)exp(-(double)x);
    const float d = 1.0f + e;
    const float q = x / d;
    return q * b;
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

// f32 -> bf16 bits, round to nearest even; NaN -> the quiet NaN 0x7fc0.
__device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
    const uint32_t b = __float_as_uint(f);
    if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

// The store of a finished value: f32, or bf16 rounded once.
__device__ __forceinline__ void store_value(void* out, size_t idx, float v, bool bf16) {
    if (bf16)
        static_cast<uint16_t*>(out)[idx] = float_to_bf16_bits(v);
    else
        static_cast<float*>(out)[idx] = v;
}

// The product's last store of element idx (column col) under `ep`.
__device__ __forceinline__ void store_out(void* out, size_t idx, int col, float v,
                                          const Epilogue& ep) {
    if (ep.bias) v = v + ep.bias[col];
    store_value(out, idx, v, ep.bf16);
}

__device__ __forceinline__ void store_device(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_device(float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Split-K hand-off, called by every lane of a workgroup after it stored its
// sums for columns [col0, col0 + cols) of slice `slice` with store_device:
// the stores are acknowledged by the device's coherence point before the
// tile's ticket is drawn (each tile's ticket has a 128-byte line of its own
// where the workspace allows, so the atomics of different tiles do not queue
// behind each other), and the workgroup drawing the last ticket reads all
// slices' sums with device-scope loads, adds them in slice order (so the
// result does not depend on scheduling), writes `out` through the epilogue
// and returns the ticket to zero for the next launch.
__device__ __forceinline__ void split_k_finish(float* partial, uint32_t* ticket, void* out,
                                               int col0, int cols, int M, int N, int slices,
                                               int* last_flag, const Epilogue& ep) {
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
            for (int u = 0; u < 16; u++)
                v[u] = load_device(p + (size_t)(sl + u) * slice_stride);
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
        store_out(out, (size_t)m * N + col, col, sum, ep);
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

// Spacing of the tiles' tickets in u32 words: 32 (one 128-byte line each)
// when the counter area holds that many, else the widest power of two that
// fits; 0 when not even one word per tile fits.
inline int ticket_stride(int tiles) {
    const size_t words = kWorkspaceCounterBytes / sizeof(uint32_t);
    for (int stride = 32; stride >= 1; stride >>= 1)
        if ((size_t)tiles * stride <= words) return stride;
    return 0;
}

}  // namespace
}  // namespace accel
