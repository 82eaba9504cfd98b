// Prepared int4 weights: a bind-time private layout for one-row products.
//
// The reference format (quant/int4.go:55-57,141-153) runs the codes of a
// row k along N, so a one-row product reads each row as N/2 contiguous
// bytes, and a column tile owning all of K reads a narrow strip of every
// row.  The decode kernels therefore split K across workgroups and add the
// slices' sums in a hand-off (about a quarter of config 1's time).  When a
// weight is bound (once, on the device), accel_int4_prepare copies its planes
// into a layout where a column strip is contiguous:
//
//   codes: [N/16 panels][K2 rows][8 bytes]   a panel is 16 columns; a row of
//          it is the two code words the reference stores at word
//          k*N/8 + 2p and the next (K2 = K rounded up to even, a padding row
//          of zero codes);
//   sz:    [N/128 groups][K2 rows] u32        the reference's f16 scale (low
//          half) and zero (high half) of group (k, g) side by side.
//
// Then one workgroup owns one panel over all of K with coalesced 16-byte
// loads (two rows of a panel), and no cross-workgroup hand-off remains.  The
// dequantisation and its fold are the decode kernel's,
//     x*w = (x*s)*code + b,   b = -(x*s)*z   (or x*z for a zero scale),
// codes through the fp8 converter (a byte 0000qqqq as e4m3 is q * 2^-9); only
// the order the f32 sums are added in differs.
#include <hip/hip_runtime.h>

#include "internal.hpp"
#include "splitk.hpp"

namespace accel {
namespace {

constexpr int kPanelCols = 16;       // columns of a panel
constexpr int kPanelThreads = 512;   // lanes of a workgroup: eight waves
// Row pairs a lane loads at once (PPL): a chunk is 512 * PPL pairs.  4 (4096
// rows) in general; 7 (7168 rows) where that makes K whole chunks and 4 does
// not (K = 14336), so no lane's load is clamped.

// Two rows of a panel's codes (16 columns each) -> 32 floats q * 2^-9.
__device__ __forceinline__ void unpack_word(uint32_t w, float* f) {
    const uint32_t lo = w & 0x0F0F0F0Fu;          // nibbles 0,2,4,6
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;   // nibbles 1,3,5,7
    const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);
    const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);
    const f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
    const f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
    f[0] = a.x; f[2] = a.y; f[4] = b.x; f[6] = b.y;
    f[1] = c.x; f[3] = c.y; f[5] = d.x; f[7] = d.y;
}

// Panel of workgroup b: the panels of one group (eight consecutive) and of
// neighbouring groups run on one XCD (workgroups are dealt to the XCDs round
// robin), so its L2 fetches their shared scale/zero rows once.
__device__ __forceinline__ int panel_of(int b, int panels) {
    if ((panels & 63) == 0) return (b & 7) * (panels >> 3) + (b >> 3);
    return b;
}

// One chunk of a lane's row pairs: loads (all issued before any is used).
template <int PPL>
struct PanelChunk {
    u32x4 q[PPL];
    u32x2 sz[PPL];
    float x0[PPL], x1[PPL];
};

// A pair's codes, scale/zero words and activations are issued together, pair
// after pair: loads complete in order, so the arithmetic of the first pairs
// runs while the later ones are in flight (measured at config 1: 4.43 us,
// against 4.92 with every code load issued first).  Each address is a
// uniform base plus an unsigned 32-bit lane offset (one offset register a
// pair, the base in scalar registers), and every load is issued before any
// arithmetic: left to itself the compiler sank the last pair's loads behind a
// wait for the first, a second memory latency.
template <typename T>
__device__ __forceinline__ const T* at_offset(const T* base, uint32_t bytes) {
    return reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + bytes);
}

template <int PPL, bool X2, bool FULL>
__device__ __forceinline__ void panel_fetch(PanelChunk<PPL>& c, const float* __restrict__ a,
                                            const u32x4* __restrict__ qp,
                                            const u32x2* __restrict__ szp, int pair0, int pairs,
                                            int K) {
#pragma unroll
    for (int i = 0; i < PPL; i++) {
        const uint32_t j = FULL ? (uint32_t)(pair0 + i * kPanelThreads)
                                : (uint32_t)min(pair0 + i * kPanelThreads, pairs - 1);
        c.q[i] = __builtin_nontemporal_load(at_offset(qp, j * 16u));
        c.sz[i] = *at_offset(szp, j * 8u);
        if constexpr (X2) {
            const f32x2 v = *at_offset(reinterpret_cast<const f32x2*>(a), j * 8u);
            c.x0[i] = v.x;
            c.x1[i] = v.y;
        } else {
            c.x0[i] = *at_offset(a, (uint32_t)min(2 * (int)j, K - 1) * 4u);
            c.x1[i] = *at_offset(a, (uint32_t)min(2 * (int)j + 1, K - 1) * 4u);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// acc[16] += one row's codes (two words) times x * s * 512; its zero-point
// term into bsum.  valid = false adds nothing (a clamped or padding row).
__device__ __forceinline__ void panel_row(float* acc, float& bsum, uint32_t w0, uint32_t w1,
                                          uint32_t szw, float x, bool valid) {
    const float s = half_bits_to_float((uint16_t)(szw & 0xffffu));
    const float z = half_bits_to_float((uint16_t)(szw >> 16));
    const float xs = x * s;
    const float bterm = (s == 0.0f) ? x * z : -(xs * z);
    const float c = valid ? xs * 512.0f : 0.0f;
    bsum += valid ? bterm : 0.0f;
    float f[16];
    unpack_word(w0, f);
    unpack_word(w1, f + 8);
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = __builtin_fmaf(c, f[j], acc[j]);
}

template <int PPL, bool FULL>
__device__ __forceinline__ void panel_compute(float* acc, float& bsum, const PanelChunk<PPL>& c,
                                              int pair0, int K) {
#pragma unroll
    for (int i = 0; i < PPL; i++) {
        const int row = 2 * (pair0 + i * kPanelThreads);
        panel_row(acc, bsum, c.q[i].x, c.q[i].y, c.sz[i].x, c.x0[i], FULL || row < K);
        panel_row(acc, bsum, c.q[i].z, c.q[i].w, c.sz[i].y, c.x1[i], FULL || row + 1 < K);
    }
}

// Up to four prepared matrices against one input in one launch (a decode
// step's q, k, v or gate, up): the grid is their panels side by side.
constexpr int kMaxPanelSet = 4;
struct PanelSet {
    const u32x4* codes[kMaxPanelSet];
    const u32x2* sz[kMaxPanelSet];
    void* out[kMaxPanelSet];
    int panel0[kMaxPanelSet + 1];   // first global panel of each matrix; [count] = all
    int count;
};

// The matrix of global panel p, its first panel and planes, chosen with
// static indices only: a dynamic index into the kernel arguments would add
// a dependent scalar load ahead of the first global load.
struct PanelPick {
    const u32x4* codes;
    const u32x2* sz;
    void* out;
    int first;
};
__device__ __forceinline__ PanelPick pick_panel(const PanelSet& set, int p) {
    PanelPick r{set.codes[0], set.sz[0], set.out[0], 0};
#pragma unroll
    for (int j = 1; j < kMaxPanelSet; j++) {
        if (j < set.count && p >= set.panel0[j])
            r = PanelPick{set.codes[j], set.sz[j], set.out[j], set.panel0[j]};
    }
    return r;
}

// out_i[16 q .. 16 q + 15] = a[K] . panel q of matrix i, for the global panel
// p of this workgroup.  PIPE: K past one chunk, the next chunk's loads issued
// before the current one is computed.  X2: K even and a 8-byte aligned, so a
// row pair's activations are one 8-byte load.  FULL: K a multiple of the
// chunk, so no lane's pair is clamped and every row is real.  SET: several
// matrices (else the first of `set` only, no selection).
template <int PPL, bool PIPE, bool X2, bool FULL, bool SET>
__global__ __launch_bounds__(kPanelThreads) void int4_panel_matvec_kernel(
    const float* __restrict__ a, PanelSet set, int panels, int K, int K2, Epilogue ep) {
    const int p = panel_of(blockIdx.x, panels);
    const PanelPick m =
        SET ? pick_panel(set, p) : PanelPick{set.codes[0], set.sz[0], set.out[0], 0};
    const int q = p - m.first;
    const int pairs = K2 >> 1;
    const u32x4* qp = m.codes + (size_t)q * pairs;
    const u32x2* szp = m.sz + (size_t)(q >> 3) * pairs;
    const int tid = threadIdx.x;
    float acc[kPanelCols];
#pragma unroll
    for (int j = 0; j < kPanelCols; j++) acc[j] = 0.0f;
    float bsum = 0.0f;

    constexpr int kChunkPairs = kPanelThreads * PPL;
    PanelChunk<PPL> c;
    panel_fetch<PPL, X2, FULL>(c, a, qp, szp, tid, pairs, K);
    if constexpr (PIPE) {
        const int chunks = (pairs + kChunkPairs - 1) / kChunkPairs;
        for (int ci = 0; ci < chunks; ci++) {
            const int pair0 = tid + ci * kChunkPairs;
            PanelChunk<PPL> n;
            const bool more = ci + 1 < chunks;
            if (more) panel_fetch<PPL, X2, FULL>(n, a, qp, szp, pair0 + kChunkPairs, pairs, K);
            panel_compute<PPL, FULL>(acc, bsum, c, pair0, K);
            if (more) c = n;
        }
    } else {
        panel_compute<PPL, FULL>(acc, bsum, c, tid, K);
    }

    // All 512 lanes hold sums of the same 16 columns: across the wave by
    // lane swaps (16 values -> one a lane over 16 lanes, then the last two
    // lane bits), then across the eight waves through LDS.
    __shared__ float red[kPanelThreads / 64][kPanelCols];
    const int l = tid & 63;
    float v[kPanelCols];
#pragma unroll
    for (int j = 0; j < kPanelCols; j++) v[j] = acc[j] + bsum;
    transpose_reduce<kPanelCols, 32, 4>(v, l);
    v[0] += xor_partner<2>(v[0], l);
    v[0] += xor_partner<1>(v[0], l);
    if ((l & 3) == 0) red[tid >> 6][reduced_offset<kPanelCols, 32, 4>(l)] = v[0];
    __syncthreads();
    if (tid < kPanelCols) {
        float sum = 0.0f;
#pragma unroll
        for (int w = 0; w < kPanelThreads / 64; w++) sum += red[w][tid];
        const int col = q * kPanelCols + tid;
        store_out(m.out, col, col, sum, ep);
    }
}

// SwiGLU(a . gate, a . up) for two prepared matrices of one shape (a decode
// step's gate and up projections): a workgroup of twice the lanes computes
// panel p of both, the first half of its waves gate's and the second up's,
// each half with int4_panel_matvec_kernel's loads, sums and reduction (so
// the two 16-value results are that kernel's bit for bit), and writes
// out[16 p + j] = swiglu1(gate_j, up_j), the SwiGLU kernel's function of the
// two.  The two 14336-wide results never leave the workgroup, and the
// elementwise launch between the gate/up products and the down projection
// is gone.  (One half-size workgroup doing both panels took 84 registers a
// lane against 59 and ran slower than the two launches it replaces.)
template <int PPL, bool PIPE, bool X2, bool FULL>
__global__ __launch_bounds__(2 * kPanelThreads) void int4_panel_swiglu_kernel(
    const float* __restrict__ a, PanelSet set, int panels, int K, int K2) {
    const int p = panel_of(blockIdx.x, panels);
    const int pairs = K2 >> 1;
    const int m = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kPanelThreads);
    const int tid = threadIdx.x % kPanelThreads;
    const u32x4* qp = (m ? set.codes[1] : set.codes[0]) + (size_t)p * pairs;
    const u32x2* szp = (m ? set.sz[1] : set.sz[0]) + (size_t)(p >> 3) * pairs;
    float acc[kPanelCols];
#pragma unroll
    for (int j = 0; j < kPanelCols; j++) acc[j] = 0.0f;
    float bsum = 0.0f;

    constexpr int kChunkPairs = kPanelThreads * PPL;
    PanelChunk<PPL> c;
    panel_fetch<PPL, X2, FULL>(c, a, qp, szp, tid, pairs, K);
    if constexpr (PIPE) {
        const int chunks = (pairs + kChunkPairs - 1) / kChunkPairs;
        for (int ci = 0; ci < chunks; ci++) {
            const int pair0 = tid + ci * kChunkPairs;
            PanelChunk<PPL> n;
            const bool more = ci + 1 < chunks;
            if (more) panel_fetch<PPL, X2, FULL>(n, a, qp, szp, pair0 + kChunkPairs, pairs, K);
            panel_compute<PPL, FULL>(acc, bsum, c, pair0, K);
            if (more) c = n;
        }
    } else {
        panel_compute<PPL, FULL>(acc, bsum, c, tid, K);
    }

    __shared__ float red[2][kPanelThreads / 64][kPanelCols];
    const int l = tid & 63;
    float v[kPanelCols];
#pragma unroll
    for (int j = 0; j < kPanelCols; j++) v[j] = acc[j] + bsum;
    transpose_reduce<kPanelCols, 32, 4>(v, l);
    v[0] += xor_partner<2>(v[0], l);
    v[0] += xor_partner<1>(v[0], l);
    if ((l & 3) == 0) red[m][tid >> 6][reduced_offset<kPanelCols, 32, 4>(l)] = v[0];
    __syncthreads();
    if (threadIdx.x < kPanelCols) {
        float g = 0.0f, u = 0.0f;
#pragma unroll
        for (int w = 0; w < kPanelThreads / 64; w++) g += red[0][w][threadIdx.x];
#pragma unroll
        for (int w = 0; w < kPanelThreads / 64; w++) u += red[1][w][threadIdx.x];
        static_cast<float*>(set.out[0])[p * kPanelCols + threadIdx.x] = swiglu1(g, u);
    }
}

// ---- a few rows: 2..8 rows a launch ------------------------------------------
//
// The matrix-core decode kernel (decode.hip) takes about as long at two rows
// as at sixteen (4096 x 14336: 16.5 against 18.7 us): it is set by its load
// latency, its K split and the split's hand-off, not by its arithmetic.  On
// prepared weights the same rows run here with no K split: one workgroup a
// panel over all of K, as the one-row kernel, each lane holding the 16
// columns of its panel for each of the MR rows (16 MR accumulators).  Per row
// pair of the panel a lane unpacks the codes once and folds each row's scale
// and zero once, (512 s, s == 0 ? z : -z s), shared by the MR rows, whose
// activations it reads as one 8-byte load each; then per row m
//     acc[m][j] += (x[m] 512 s) (q_j 2^-9),   bsum[m] += x[m] add
// (the one-row kernel's arithmetic).  Rows past M (MR rounded up) read row
// M - 1 and are not stored.  A set of up to four matrices runs as one grid,
// as for one row.  Measured (us, this kernel / the matrix-core decode on the
// reference planes) at 2, 4 and 8 rows: 4096 x 4096 5.3 / 10.4, 7.1 / 11.2,
// 10.6 / 9.6; 4096 x 14336 11.9 / 16.4, 18.4 / 16.7, 37.2 / 16.9; 14336 x
// 4096 11.0 / 16.1, 16.3 / 16.6, 24.2 / 17.6.  It wins at two rows and loses
// at eight: a 16-column panel re-reads every row's activations, which at
// eight rows are four times the code bytes a workgroup loads, in eight times
// the load instructions, and the address unit sets the time.
template <int MR, int PPL>
struct RowsChunk {
    u32x4 q[PPL];
    u32x2 sz[PPL];
    f32x2 x[PPL][MR];
};

template <int MR, int PPL, bool FULL>
__device__ __forceinline__ void rows_fetch(RowsChunk<MR, PPL>& c, const float* __restrict__ a,
                                           const u32x4* __restrict__ qp,
                                           const u32x2* __restrict__ szp, int pair0, int pairs,
                                           int K, int M) {
#pragma unroll
    for (int i = 0; i < PPL; i++) {
        const uint32_t j = FULL ? (uint32_t)(pair0 + i * kPanelThreads)
                                : (uint32_t)min(pair0 + i * kPanelThreads, pairs - 1);
        c.q[i] = __builtin_nontemporal_load(at_offset(qp, j * 16u));
        c.sz[i] = *at_offset(szp, j * 8u);
#pragma unroll
        for (int m = 0; m < MR; m++) {
            const float* row = a + (size_t)min(m, M - 1) * K;
            c.x[i][m] = *at_offset(reinterpret_cast<const f32x2*>(row), j * 8u);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int MR, int PPL, bool FULL>
__device__ __forceinline__ void rows_compute(float (&acc)[MR][kPanelCols], float (&bsum)[MR],
                                             const RowsChunk<MR, PPL>& c, int pair0, int K) {
#pragma unroll
    for (int i = 0; i < PPL; i++) {
        const int row = 2 * (pair0 + i * kPanelThreads);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t szw = h ? c.sz[i].y : c.sz[i].x;
            const bool valid = FULL || row + h < K;
            const float s = half_bits_to_float((uint16_t)(szw & 0xffffu));
            const float z = half_bits_to_float((uint16_t)(szw >> 16));
            const float mul = valid ? s * 512.0f : 0.0f;
            const float add = valid ? (s == 0.0f ? z : -(z * s)) : 0.0f;
            float f[kPanelCols];
            unpack_word(h ? c.q[i].z : c.q[i].x, f);
            unpack_word(h ? c.q[i].w : c.q[i].y, f + 8);
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const float x = h ? c.x[i][m].y : c.x[i][m].x;
                const float cm = x * mul;
                bsum[m] = __builtin_fmaf(x, add, bsum[m]);
#pragma unroll
                for (int jj = 0; jj < kPanelCols; jj++)
                    acc[m][jj] = __builtin_fmaf(cm, f[jj], acc[m][jj]);
            }
        }
    }
}

// out[m, 16 q + c] (row stride N) = a[m, :] . panel (qp, szp), m < M <= MR,
// c < 16, through ep: the product of one panel and M rows, every lane
// holding the panel's 16 columns for each row, then the one-row kernel's
// reduction per row (lane swaps, then the eight waves through LDS).  Ends at
// a barrier, so a caller may run it again at once.  K even, rows 8-byte
// aligned; FULL: K a multiple of the chunk (512 PPL row pairs).
template <int MR, int PPL, bool FULL>
__device__ __forceinline__ void panel_rows_tile(const float* __restrict__ a,
                                                const u32x4* __restrict__ qp,
                                                const u32x2* __restrict__ szp, void* out, int M,
                                                int K, int N, int q, const Epilogue& ep) {
    const int pairs = K >> 1;
    const int tid = threadIdx.x;
    float acc[MR][kPanelCols];
    float bsum[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) {
        bsum[m] = 0.0f;
#pragma unroll
        for (int j = 0; j < kPanelCols; j++) acc[m][j] = 0.0f;
    }
    constexpr int kChunkPairs = kPanelThreads * PPL;
    const int chunks = (pairs + kChunkPairs - 1) / kChunkPairs;
    for (int ci = 0; ci < chunks; ci++) {
        const int pair0 = tid + ci * kChunkPairs;
        RowsChunk<MR, PPL> c;
        rows_fetch<MR, PPL, FULL>(c, a, qp, szp, pair0, pairs, K, M);
        rows_compute<MR, PPL, FULL>(acc, bsum, c, pair0, K);
    }

    __shared__ float red[kPanelThreads / 64][MR][kPanelCols];
    const int l = tid & 63;
#pragma unroll
    for (int m = 0; m < MR; m++) {
        float v[kPanelCols];
#pragma unroll
        for (int j = 0; j < kPanelCols; j++) v[j] = acc[m][j] + bsum[m];
        transpose_reduce<kPanelCols, 32, 4>(v, l);
        v[0] += xor_partner<2>(v[0], l);
        v[0] += xor_partner<1>(v[0], l);
        if ((l & 3) == 0) red[tid >> 6][m][reduced_offset<kPanelCols, 32, 4>(l)] = v[0];
    }
    __syncthreads();
    if (tid < MR * kPanelCols) {
        const int m = tid / kPanelCols, c = tid % kPanelCols;
        if (m < M) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < kPanelThreads / 64; w++) sum += red[w][m][c];
            const int col = q * kPanelCols + c;
            store_out(out, (size_t)m * N + col, col, sum, ep);
        }
    }
    __syncthreads();
}

// out_i[m, 16 q .. 16 q + 15] = a[m, :] . panel q of matrix i, m < M <= MR,
// for the global panel p of this workgroup.  K even, rows 8-byte aligned.
// FULL: K a multiple of the chunk (512 PPL row pairs).
template <int MR, int PPL, bool FULL, bool SET>
__global__ __launch_bounds__(kPanelThreads) void int4_panel_rows_kernel(
    const float* __restrict__ a, PanelSet set, int panels, int M, int K, Epilogue ep) {
    const int p = panel_of(blockIdx.x, panels);
    const PanelPick pk =
        SET ? pick_panel(set, p) : PanelPick{set.codes[0], set.sz[0], set.out[0], 0};
    const int q = p - pk.first;
    const int pairs = K >> 1;
    // this matrix's width from its panels: [first, next first) of the set
    int n = panels;
    if (SET) {
#pragma unroll
        for (int j = 1; j <= kMaxPanelSet; j++)
            if (j <= set.count && set.panel0[j] > pk.first && set.panel0[j] < n)
                n = set.panel0[j];
    }
    panel_rows_tile<MR, PPL, FULL>(a, pk.codes + (size_t)q * pairs,
                                   pk.sz + (size_t)(q >> 3) * pairs, pk.out, M, K,
                                   (n - pk.first) * kPanelCols, q, ep);
}

// The ragged GEMV (decode MoE) on experts prepared into the panel layout,
// one expert's copy `stride` bytes after the last (codes, then the sz words
// at sz_off): workgroup (expert e, panel p) runs the rows of e,
// [off[e], min(off[e+1], T)), against its panel p in passes of one or two
// rows (panel_rows_tile), K whole and no hand-off.  (Passes of up to four
// rows took more registers, fewer waves, and 55.5 against 53.5 us at 4
// tokens top-2 of config 4's experts.)  Sorted offsets only: when they have wrapped, every
// workgroup returns and the VALU decode launch takes every row; it also
// writes the rows past the last segment.
template <int PPL, bool FULL>
__global__ __launch_bounds__(kPanelThreads) void int4_grouped_panel_rows_kernel(
    const float* __restrict__ x, const char* __restrict__ panels_base, size_t stride,
    size_t sz_off, const uint32_t* __restrict__ off, float* __restrict__ out, int E, int T,
    int K, int N) {
    const int panels = N / kPanelCols;
    const int e = blockIdx.x / panels;
    const int q = panel_of(blockIdx.x % panels, panels);
    __shared__ int s_first, s_count;
    if (threadIdx.x < 64) {
        // the offsets' order checked by the first wave, a pair a lane
        const int lane = threadIdx.x;
        bool ok = true;
        for (int r = lane; r < E; r += 64) ok = ok && off[r] <= off[r + 1];
        const bool sorted = __all(ok);
        if (lane == 0) {
            const uint32_t first = min(off[e], (uint32_t)T);
            const uint32_t last = min(off[e + 1], (uint32_t)T);
            s_first = (int)first;
            s_count = sorted && last > first ? (int)(last - first) : 0;
        }
    }
    __syncthreads();
    const int first = s_first, count = s_count;
    if (count == 0) return;
    const int pairs = K >> 1;
    const char* base = panels_base + (size_t)e * stride;
    const u32x4* qp = reinterpret_cast<const u32x4*>(base) + (size_t)q * pairs;
    const u32x2* szp = reinterpret_cast<const u32x2*>(base + sz_off) + (size_t)(q >> 3) * pairs;
    const Epilogue ep{};
    for (int r0 = 0; r0 < count; r0 += 2) {
        const int rows = min(2, count - r0);
        const float* a = x + (size_t)(first + r0) * K;
        float* o = out + (size_t)(first + r0) * N;
        if (rows == 1)
            panel_rows_tile<1, PPL, FULL>(a, qp, szp, o, 1, K, N, q, ep);
        else
            panel_rows_tile<2, PPL, FULL>(a, qp, szp, o, 2, K, N, q, ep);
    }
}

// ---- the bind-time copy ------------------------------------------------------

// codes: a 64-row x 64-panel tile through LDS, so the reads run along the
// reference's rows and the writes along the panels' rows.
__global__ __launch_bounds__(256) void int4_panel_prepare_codes_kernel(
    const u32x2* __restrict__ src, u32x2* __restrict__ dst, int K, int K2, int panels) {
    __shared__ u32x2 t[64][65];
    const int p0 = blockIdx.x * 64, k0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4) {
        const int k = k0 + r, p = p0 + tx;
        u32x2 v = {0u, 0u};
        if (k < K && p < panels) v = src[(size_t)k * panels + p];
        t[r][tx] = v;
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        const int p = p0 + r, k = k0 + tx;
        if (p < panels && k < K2) dst[(size_t)p * K2 + k] = t[tx][r];
    }
}

__global__ __launch_bounds__(256) void int4_panel_prepare_sz_kernel(
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    uint32_t* __restrict__ dst, int K, int K2, int groups) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)groups * K2) return;
    const int g = (int)(i / K2), k = (int)(i % K2);
    uint32_t v = 0;
    if (k < K) {
        const size_t at = (size_t)k * groups + g;
        v = (uint32_t)scales[at] | ((uint32_t)zeros[at] << 16);
    }
    dst[i] = v;
}

}  // namespace

bool int4_panel_supported(int64_t K, int64_t N) {
    return K >= 1 && N >= 128 && N % 128 == 0 && K < (1 << 30) && N < (1 << 30) &&
           (N / kPanelCols) * ((K + 1) / 2 * 2) < (int64_t(1) << 40);
}

size_t int4_panel_bytes(int K, int N, size_t* sz_offset) {
    const size_t K2 = (size_t)(K + 1) / 2 * 2;
    const size_t code_bytes = (size_t)(N / kPanelCols) * K2 * 8;
    const size_t off = (code_bytes + 255) / 256 * 256;
    if (sz_offset) *sz_offset = off;
    return off + (size_t)(N / 128) * K2 * 4;
}

hipError_t launch_int4_panel_prepare(hipStream_t st, Int4Planes w, void* dst, int K, int N) {
    const int K2 = (K + 1) / 2 * 2;
    const int panels = N / kPanelCols, groups = N / 128;
    size_t sz_off = 0;
    int4_panel_bytes(K, N, &sz_off);
    char* base = static_cast<char*>(dst);
    ACCEL_LAUNCH(std::string("int4_panel_prepare_codes_kernel"),
                 int4_panel_prepare_codes_kernel, dim3((panels + 63) / 64, (K2 + 63) / 64),
                 dim3(256), 0, st, reinterpret_cast<const u32x2*>(w.codes),
                 reinterpret_cast<u32x2*>(base), K, K2, panels);
    const size_t n = (size_t)groups * K2;
    ACCEL_LAUNCH(std::string("int4_panel_prepare_sz_kernel"), int4_panel_prepare_sz_kernel,
                 dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w.scales, w.zeros,
                 reinterpret_cast<uint32_t*>(base + sz_off), K, K2, groups);
    return launch_status();
}

// count (1..4) prepared matrices of K rows (N[i] columns) against one a [K].
hipError_t launch_int4_panel_matvec(hipStream_t st, const float* a, const void* const* prepared,
                                    void* const* out, const int* N, int count, int K,
                                    Epilogue ep) {
    const int K2 = (K + 1) / 2 * 2;
    PanelSet set{};
    set.count = count;
    int panels = 0;
    for (int i = 0; i < count; i++) {
        size_t sz_off = 0;
        int4_panel_bytes(K, N[i], &sz_off);
        const char* base = static_cast<const char*>(prepared[i]);
        set.codes[i] = reinterpret_cast<const u32x4*>(base);
        set.sz[i] = reinterpret_cast<const u32x2*>(base + sz_off);
        set.out[i] = out[i];
        set.panel0[i] = panels;
        panels += N[i] / kPanelCols;
    }
    set.panel0[count] = panels;
    const bool x2 = K % 2 == 0 && (reinterpret_cast<uintptr_t>(a) & 7) == 0;
    // 7 pairs a lane where that makes K whole chunks and 4 does not
    const bool ppl7 = x2 && K % (2 * kPanelThreads * 4) != 0 && K % (2 * kPanelThreads * 7) == 0;
    const int chunk_rows = 2 * kPanelThreads * (ppl7 ? 7 : 4);
    const bool pipe = K2 > chunk_rows;
    const bool full = K % chunk_rows == 0;
    const dim3 grid(panels), block(kPanelThreads);
#define PANEL_LAUNCH(L, P, X, F, S)                                                        \
    ACCEL_LAUNCH(tname("int4_panel_matvec_kernel", L, P, X, F, S) + grid_note(panels, 1), \
                 (int4_panel_matvec_kernel<L, P, X, F, S>), grid, block, 0, st, a, set,    \
                 panels, K, K2, ep)
#define PANEL_PIPE(P, S)                                                                   \
    do {                                                                                   \
        if (ppl7) PANEL_LAUNCH(7, P, true, true, S);                                      \
        else if (full && x2) PANEL_LAUNCH(4, P, true, true, S);                           \
        else if (x2) PANEL_LAUNCH(4, P, true, false, S);                                  \
        else PANEL_LAUNCH(4, P, false, false, S);                                         \
    } while (0)
    if (count > 1) {
        if (pipe) PANEL_PIPE(true, true);
        else PANEL_PIPE(false, true);
    } else {
        if (pipe) PANEL_PIPE(true, false);
        else PANEL_PIPE(false, false);
    }
#undef PANEL_PIPE
#undef PANEL_LAUNCH
    return launch_status();
}

// out [N] = SwiGLU(a . gate, a . up), gate and up prepared [K, N] matrices.
hipError_t launch_int4_panel_swiglu(hipStream_t st, const float* a, const void* gate,
                                    const void* up, float* out, int N, int K) {
    const int K2 = (K + 1) / 2 * 2;
    PanelSet set{};
    set.count = 2;
    size_t sz_off = 0;
    int4_panel_bytes(K, N, &sz_off);
    const void* mats[2] = {gate, up};
    for (int i = 0; i < 2; i++) {
        const char* base = static_cast<const char*>(mats[i]);
        set.codes[i] = reinterpret_cast<const u32x4*>(base);
        set.sz[i] = reinterpret_cast<const u32x2*>(base + sz_off);
    }
    set.out[0] = out;
    const int panels = N / kPanelCols;
    const bool x2 = K % 2 == 0 && (reinterpret_cast<uintptr_t>(a) & 7) == 0;
    const bool ppl7 = x2 && K % (2 * kPanelThreads * 4) != 0 && K % (2 * kPanelThreads * 7) == 0;
    const int chunk_rows = 2 * kPanelThreads * (ppl7 ? 7 : 4);
    const bool pipe = K2 > chunk_rows;
    const bool full = K % chunk_rows == 0;
    const dim3 grid(panels), block(2 * kPanelThreads);
#define SWIGLU_LAUNCH(L, P, X, F)                                                          \
    ACCEL_LAUNCH(tname("int4_panel_swiglu_kernel", L, P, X, F) + grid_note(panels, 1),    \
                 (int4_panel_swiglu_kernel<L, P, X, F>), grid, block, 0, st, a, set, panels, \
                 K, K2)
#define SWIGLU_PIPE(P)                                                                     \
    do {                                                                                   \
        if (ppl7) SWIGLU_LAUNCH(7, P, true, true);                                        \
        else if (full && x2) SWIGLU_LAUNCH(4, P, true, true);                             \
        else if (x2) SWIGLU_LAUNCH(4, P, true, false);                                    \
        else SWIGLU_LAUNCH(4, P, false, false);                                           \
    } while (0)
    if (pipe) SWIGLU_PIPE(true);
    else SWIGLU_PIPE(false);
#undef SWIGLU_PIPE
#undef SWIGLU_LAUNCH
    return launch_status();
}

// The ragged GEMV on panel-prepared experts (int4_grouped_panel_rows_kernel):
// x f32 [T, K] (K even, 8-byte aligned), E experts of [K, N] `stride` bytes
// apart from panels_base, sorted offsets off[E + 1]; out f32 [T, N] for the
// experts' rows (the rest is the VALU launch's).
hipError_t launch_int4_grouped_panel_rows(hipStream_t st, const float* x, const void* panels_base,
                                          size_t stride, const uint32_t* off, float* out, int E,
                                          int T, int K, int N) {
    constexpr int PPL = 2;
    size_t sz_off = 0;
    int4_panel_bytes(K, N, &sz_off);
    const bool full = K % (2 * kPanelThreads * PPL) == 0;
    const long long wgs = (long long)E * (N / kPanelCols);
    if (wgs > INT32_MAX) return hipErrorInvalidConfiguration;
    const char* base = static_cast<const char*>(panels_base);
#define GPR_LAUNCH(F)                                                                        \
    ACCEL_LAUNCH(tname("int4_grouped_panel_rows_kernel", PPL, F) + grid_note(wgs, 1),         \
                 (int4_grouped_panel_rows_kernel<PPL, F>), dim3((unsigned)wgs),              \
                 dim3(kPanelThreads), 0, st, x, base, stride, sz_off, off, out, E, T, K, N)
    if (full) GPR_LAUNCH(true);
    else GPR_LAUNCH(false);
#undef GPR_LAUNCH
    return launch_status();
}

// count (1..4) prepared matrices of K rows against M rows of a ([M, K]),
// out[i] [M, N[i]]: passes of up to eight rows, each one launch.
bool int4_panel_rows_supported(int M, int K, const float* a) {
    return M >= 1 && K % 2 == 0 && (reinterpret_cast<uintptr_t>(a) & 7) == 0;
}

hipError_t launch_int4_panel_rows(hipStream_t st, const float* a, int M,
                                  const void* const* prepared, void* const* out, const int* N,
                                  int count, int K, Epilogue ep) {
    constexpr int PPL = 2;
    const size_t esz = ep.bf16 ? 2 : 4;
    const bool full = K % (2 * kPanelThreads * PPL) == 0;
    for (int r0 = 0; r0 < M; r0 += 8) {
        const int rows = std::min(8, M - r0);
        PanelSet set{};
        set.count = count;
        int panels = 0;
        for (int i = 0; i < count; i++) {
            size_t sz_off = 0;
            int4_panel_bytes(K, N[i], &sz_off);
            const char* base = static_cast<const char*>(prepared[i]);
            set.codes[i] = reinterpret_cast<const u32x4*>(base);
            set.sz[i] = reinterpret_cast<const u32x2*>(base + sz_off);
            set.out[i] = static_cast<char*>(out[i]) + (size_t)r0 * N[i] * esz;
            set.panel0[i] = panels;
            panels += N[i] / kPanelCols;
        }
        set.panel0[count] = panels;
        const float* ar = a + (size_t)r0 * K;
        const dim3 grid(panels), block(kPanelThreads);
#define ROWS_LAUNCH(R, F, S)                                                              \
    ACCEL_LAUNCH(tname("int4_panel_rows_kernel", R, PPL, F, S) + grid_note(panels, 1),   \
                 (int4_panel_rows_kernel<R, PPL, F, S>), grid, block, 0, st, ar, set,    \
                 panels, rows, K, ep)
#define ROWS_PICK(R)                                                                      \
    do {                                                                                  \
        if (count > 1) {                                                                  \
            if (full) ROWS_LAUNCH(R, true, true); else ROWS_LAUNCH(R, false, true);       \
        } else {                                                                          \
            if (full) ROWS_LAUNCH(R, true, false); else ROWS_LAUNCH(R, false, false);     \
        }                                                                                 \
    } while (0)
        if (rows <= 2) ROWS_PICK(2);
        else if (rows <= 4) ROWS_PICK(4);
        else ROWS_PICK(8);
#undef ROWS_PICK
#undef ROWS_LAUNCH
        const hipError_t e = launch_status();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace accel
