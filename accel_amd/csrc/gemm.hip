// Prefill-shape int4 products: the counterpart of the reference's tiled
// QuantMatMulInt4 (internal/kernels/int4tiled.go:66-137), rebuilt around
// CDNA4's bf16 matrix cores.
//
// bf16 path (activations and output bf16, fp32 accumulation).  A workgroup
// of 256 lanes (four waves, one per SIMD) computes an output tile of up to
// 256 rows (MT active 32-row m-tiles) by 128 columns -- one quantisation
// group.  Wave w owns the column half ch = w & 1 (64 columns) and all MT
// m-tiles, as MT x 2 tiles of v_mfma_f32_32x32x16_bf16, for the 16-k
// substeps of parity w >> 1 of every 64-k stage; the two parities'
// accumulators are added through LDS at the end.  Per stage:
//   * the activation rows (MT x 32 rows x 128 bytes) go to LDS through
//     16-byte loads, rows XOR-swizzled in 16-byte chunks so the fragment
//     reads (32 rows x one chunk) spread over the banks;
//   * the packed codes (64 rows x 64 bytes) go to LDS as they are, four
//     bits a weight, transposed in 4 x 4-byte blocks so that each u32 holds
//     one byte (two adjacent columns) of four consecutive rows;
//   * per row the fold (512*s, s == 0 ? z : -z*s) goes to LDS.
// Each wave dequantises its own B fragments in registers: a lane reads one
// code byte of its eight rows, turns the nibbles into exact floats with the
// fp8 converter (byte 0000qqqq as OCP e4m3 is q*2^-9; a converter pair is
// the same column of two rows, the pairing the bf16x2 operand wants),
// applies w = f*(512 s) + add in fp32 and packs to bf16.  The MFMA's n-tile
// j, column c is the tile column 64 ch + 2c + j, so a lane's two n-tiles are
// the two nibbles of one code byte and its outputs two adjacent bf16.
// Every weight is dequantised once and feeds MT m-tiles: with all eight,
// the dequantisation costs about 2.4 VALU instructions per MFMA.
//
// Measured on gfx950 (one wave per SIMD, 16 independent 32x32x16 MFMAs a
// step): the matrix cores sustain about 2.1 PFLOP/s alone; up to ~32 VALU
// instructions per 16 MFMAs are free, ~64 cost a few percent, and more make
// the VALU the bound; LDS reads and vector-memory loads interleaved with the
// MFMAs cost more (eight 16-byte LDS reads per 16 MFMAs: -18%; eight
// L1-hitting global loads: -40%), which is why the activations are shared
// through LDS.
//
// Placement: consecutive logical tiles (the column tiles of one row band,
// which share its activations) are dealt to one XCD so its L2 serves them.
//
// f32 path (the reference API's f32 activations and output, M > 16): an
// LDS-tiled fp32 VALU product, exact up to f32 rounding order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "internal.hpp"
#include "splitk.hpp"

namespace accel {
namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int BM = 256, BN = 128, BK = 64;
constexpr int kThreads = 256;        // four waves, one per SIMD
constexpr int kARowBytes = BK * 2;   // one LDS activation row: 64 bf16
constexpr int kBQuadWords = BN / 2;  // u32 words per row quad: one per code byte
constexpr int MAX_MT = BM / 32;      // 32-row m-tiles of a full tile

// Byte offset of 16-byte chunk `c` of activation row `r` under the swizzle:
// LDS has 64 banks (256 bytes), two rows wide; each row pair puts a chunk
// index on its own 16-byte bank group, so a fragment read (32 rows, one
// chunk) does not conflict.
__device__ __forceinline__ int a_off(int r, int c) {
    return r * kARowBytes + ((c ^ ((r >> 1) & 7)) << 4);
}
// Word offset of code byte `bc` of row quad `rq`: a lane reads quads 2p and
// 2p + 1 (its eight rows); the next pair of quads -- the other k-group of
// the wave -- is shifted by half the banks.
__device__ __forceinline__ int b_off(int rq, int bc) {
    return rq * kBQuadWords + (bc ^ (((rq >> 1) & 1) << 5));
}

// A buffer resource over `base` (raw, no stride): loads through it take a
// workgroup-uniform base in scalar registers and a 32-bit per-lane byte
// offset, so they cost no vector address arithmetic.  Offsets stay below
// the 2^31 - 1 byte extent given here (the callers' shape limits ensure it).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff,
                                             0x00020000);
}

// 4 x 4 byte transpose: out[b] = byte b of r0, r1, r2, r3 (low to high).
__device__ __forceinline__ u32x4 transpose4(uint32_t r0, uint32_t r1, uint32_t r2,
                                            uint32_t r3) {
    const uint32_t lo01 = __builtin_amdgcn_perm(r1, r0, 0x05010400u);  // r0b0 r1b0 r0b1 r1b1
    const uint32_t lo23 = __builtin_amdgcn_perm(r3, r2, 0x05010400u);
    const uint32_t hi01 = __builtin_amdgcn_perm(r1, r0, 0x07030602u);  // r0b2 r1b2 r0b3 r1b3
    const uint32_t hi23 = __builtin_amdgcn_perm(r3, r2, 0x07030602u);
    u32x4 o;
    o.x = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
    o.y = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
    o.z = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
    o.w = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
    return o;
}

// One 64-k stage in LDS.
struct __attribute__((aligned(16))) GemmStage {
    char a[BM * kARowBytes];                  // 32 KB, swizzled rows
    uint32_t b[(BK / 4) * kBQuadWords];       // 4 KB: [row quad][code byte]
    f32x2 fold[BK + 64];                      // (512 s, add) per row of the stage; 64 spare
};
// The stages, and after the last one the accumulator hand-off of the
// k-parity wave pairs: [column half][m-tile][n-tile][register quad][lane],
// 16 KB an m-tile.  MTR: the m-tiles a kernel may run.
template <int MTR>
struct __attribute__((aligned(16))) GemmLds {
    union {
        GemmStage st[2];
        f32x4 red[2][MTR][2][4][64];
    };
};

// One stage's global loads, held in registers until written to LDS: the
// activations (two stages ahead) and the codes with their scale and zero
// (a deeper ring: they come from HBM, the activations from L2).
template <int MT>
struct ARegs {
    u32x4 a[MT];      // 16-byte activation chunks: 32 rows each across the workgroup
};
struct CRegs {
    uint32_t b[4];    // 4 bytes of codes of each of four consecutive rows
    uint16_t s, z;
};
// Stages of codes in flight: as many as the registers allow.
template <int MT>
constexpr int code_depth() {
    return MT >= 7 ? 2 : 4;
}

// One 16-k substep's LDS operands for a wave.
template <int MT>
struct SubstepRegs {
    bf16x8 af[MT];     // A fragments of the m-tiles
    uint32_t tw[2];    // one code byte (two columns) of rows 8*kg .. +3 and +4 .. +7
    f32x4 fr[4];       // (mul, add) of those rows, two per vector
};

// One output tile: rows [m0, m0 + 32 MT) of which [m0, m_end) are valid
// (rows past m_end are computed from a clamped row and not stored), columns
// [n0, n0 + 128).  codes/scales/zeros describe the [K, N] matrix in use.
//
// Stages.  Stage kt (64 k) sits in LDS buffer kt % 2.  At its first
// substep a wave writes its share of stage kt+1 (loaded two stages
// earlier) into the other buffer and issues the global loads of stage
// kt+3; the stage's one barrier, before its second substep, makes stage
// kt+1 visible before that substep reads the next stage's operands.  A
// wave pipelines its substeps: while the MFMAs of one run, it dequantises
// the next one's codes, read from LDS at the start of the current one.
//
// A K slice (split K, for products with too few tiles to fill the chip)
// runs stages [kt0, kt0 + ktiles) and, with PART, stores its f32 sums to
// `part` ([M, N], row stride N) instead of the bf16 result.
template <int MT, bool BIAS, int MTR, bool PART = false>
__device__ __forceinline__ void gemm_tile_bf16(GemmLds<MTR>& lds, const uint16_t* __restrict__ a,
                                               const uint32_t* __restrict__ codes,
                                               const uint16_t* __restrict__ scales,
                                               const uint16_t* __restrict__ zeros,
                                               uint16_t* __restrict__ out, int m0, int m_end,
                                               int n0, int K, int N,
                                               const float* __restrict__ bias, int kt0 = 0,
                                               int kt_count = -1, float* part = nullptr) {
    static_assert(MT <= MTR, "hand-off slots");
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int ch = wave & 1;     // column half
    const int kp = wave >> 1;    // substep parity
    const int lane = tid & 63;
    const int c32 = lane & 31;   // MFMA row (A) / column (B, D) within a 32 x 32 tile
    const int kg = lane >> 5;    // MFMA k-group (8 consecutive k)
    const size_t groups_per_row = (size_t)(N >> 7);
    const size_t words_per_row = (size_t)(N >> 3);
    const int ktiles = kt_count < 0 ? K / BK : kt_count;   // stages of this slice
    auto kofs = [&](int kt) { return (kt0 + min(kt, ktiles - 1)) * BK; };

    // Global loads are buffer loads: a per-stage resource over the tile's
    // first row, column and stage, and a 32-bit per-lane byte offset fixed
    // for the whole tile (below 2^31 for K < 2^22 and N < 2^26,
    // int4_gemm_bf16_supported).
    //
    // Activation staging: 32 rows (256 chunks of 16 bytes) per m-tile a
    // stage, one chunk per lane and m-tile.
    const char* a_tile = reinterpret_cast<const char*>(a + (size_t)m0 * K);
    uint32_t a_src[MT];
    int a_dst[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) {
        const int q = tid + kThreads * i;
        const int r = q >> 3, c = q & 7;
        const int row = min(m0 + r, m_end - 1);
        a_src[i] = (uint32_t)(((size_t)(row - m0) * K + c * 8) * 2);
        a_dst[i] = a_off(r, c);
    }
    // Code staging: row quad tid / 16 and 4-byte column chunk tid % 16 (eight
    // columns) of each of the quad's four rows.
    const int b_rq = tid >> 4;
    const int b_cc = tid & 15;
    const char* b_tile = reinterpret_cast<const char*>(codes + (n0 >> 3));
    const uint32_t b_src = (uint32_t)(((size_t)(4 * b_rq) * words_per_row + b_cc) * 4);
    const int b_dst = b_off(b_rq, 4 * b_cc);
    // Fold staging: wave w folds the stage's rows 16w .. 16w + 15, four lanes
    // a row.  A load whose lanes name many rows costs the address unit about
    // a cycle a row, so the 64 rows are split over the waves rather than
    // loaded by each; lanes 16 .. 63 write their duplicate to spare slots, so
    // the stage code has no branch to cut the schedule.
    const int f_row = 16 * wave + (lane & 15);
    const int f_dst = lane < 16 ? f_row : BK + lane;
    const size_t f_g = (size_t)(n0 >> 7);
    const char* s_tile = reinterpret_cast<const char*>(scales + f_g);
    const char* z_tile = reinterpret_cast<const char*>(zeros + f_g);
    const uint32_t f_src = (uint32_t)((size_t)f_row * groups_per_row * 2);

    // Stage indices past the end are clamped to the last stage: the loads
    // repeat valid data and land in buffers no later stage reads.
    const int row_bytes = (int)(words_per_row * 4);   // one row of codes
    auto a_rsrc = [&](int k0) { return tile_rsrc(a_tile + (size_t)k0 * 2); };
    auto b_rsrc = [&](int k0) { return tile_rsrc(b_tile + (size_t)k0 * row_bytes); };
    auto s_rsrc = [&](int k0) { return tile_rsrc(s_tile + (size_t)k0 * groups_per_row * 2); };
    auto z_rsrc = [&](int k0) { return tile_rsrc(z_tile + (size_t)k0 * groups_per_row * 2); };
    auto load_a = [&](ARegs<MT>& g, int kt) {
        const auto r = a_rsrc(kofs(kt));
#pragma unroll
        for (int i = 0; i < MT; i++) g.a[i] = __builtin_amdgcn_raw_buffer_load_b128(r, a_src[i], 0, 0);
    };
    auto load_c = [&](CRegs& g, int kt) {
        const int k0 = kofs(kt);
        const auto r = b_rsrc(k0);
#pragma unroll
        for (int i = 0; i < 4; i++)
            g.b[i] = __builtin_amdgcn_raw_buffer_load_b32(r, b_src, i * row_bytes, 0);
        g.s = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc(k0), f_src, 0, 0);
        g.z = __builtin_amdgcn_raw_buffer_load_b16(z_rsrc(k0), f_src, 0, 0);
    };
    auto store_lds = [&](const ARegs<MT>& ga, const CRegs& g, int buf) {
        GemmStage& S = lds.st[buf];
#pragma unroll
        for (int i = 0; i < MT; i++) *reinterpret_cast<u32x4*>(S.a + a_dst[i]) = ga.a[i];
        *reinterpret_cast<u32x4*>(&S.b[b_dst]) = transpose4(g.b[0], g.b[1], g.b[2], g.b[3]);
        const float s = half_bits_to_float(g.s);
        const float z = half_bits_to_float(g.z);
        f32x2 f;
        f.x = s * 512.0f;
        f.y = (s == 0.0f) ? z : -(z * s);
        S.fold[f_dst] = f;
    };
    // This lane's code byte: 32*ch + c32 (columns 64ch + 2c32, + 1).
    const int my_bc = 32 * ch + c32;

    auto read_substep = [&](SubstepRegs<MT>& r, int buf, int ks) {
        const GemmStage& S = lds.st[buf];
#pragma unroll
        for (int h = 0; h < 2; h++) r.tw[h] = S.b[b_off(ks * 4 + 2 * kg + h, my_bc)];
        const f32x4* fp = reinterpret_cast<const f32x4*>(&S.fold[ks * 16 + 8 * kg]);
#pragma unroll
        for (int i = 0; i < 4; i++) r.fr[i] = fp[i];   // (mul, add) of rows 2i, 2i+1
#pragma unroll
        for (int t = 0; t < MT; t++)
            r.af[t] = *reinterpret_cast<const bf16x8*>(S.a + a_off(t * 32 + c32, ks * 2 + kg));
    };
    // B fragments of the two n-tiles: the code byte of row i of a quad is
    // byte i of tw[h]; its low nibble is n-tile 0, its high nibble n-tile 1.
    auto dequant = [&](const SubstepRegs<MT>& r, bf16x8 (&bfr)[2]) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t t = r.tw[h];
            const uint32_t lo = t & 0x0F0F0F0Fu;          // n-tile 0, rows 4h .. 4h+3
            const uint32_t hi = (t >> 4) & 0x0F0F0F0Fu;   // n-tile 1
            const f32x2 c0a = __builtin_amdgcn_cvt_pk_f32_fp8(lo, false);  // rows 0, 1
            const f32x2 c0b = __builtin_amdgcn_cvt_pk_f32_fp8(lo, true);   // rows 2, 3
            const f32x2 c1a = __builtin_amdgcn_cvt_pk_f32_fp8(hi, false);
            const f32x2 c1b = __builtin_amdgcn_cvt_pk_f32_fp8(hi, true);
            const f32x4 f01 = r.fr[2 * h], f23 = r.fr[2 * h + 1];
            const int p = 4 * h;
            bfr[0][p + 0] = (__bf16)__builtin_fmaf(c0a.x, f01.x, f01.y);
            bfr[0][p + 1] = (__bf16)__builtin_fmaf(c0a.y, f01.z, f01.w);
            bfr[0][p + 2] = (__bf16)__builtin_fmaf(c0b.x, f23.x, f23.y);
            bfr[0][p + 3] = (__bf16)__builtin_fmaf(c0b.y, f23.z, f23.w);
            bfr[1][p + 0] = (__bf16)__builtin_fmaf(c1a.x, f01.x, f01.y);
            bfr[1][p + 1] = (__bf16)__builtin_fmaf(c1a.y, f01.z, f01.w);
            bfr[1][p + 2] = (__bf16)__builtin_fmaf(c1b.x, f23.x, f23.y);
            bfr[1][p + 3] = (__bf16)__builtin_fmaf(c1b.y, f23.z, f23.w);
        }
    };

    f32x16 acc[MT][2];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[t][j][r] = 0.0f;

    // Prologue: stage 0 in LDS buffer 0; activations of stage 1 in set 1 and
    // stage 2 in flight into set 0; codes of stages 1 .. PD - 1 in code sets
    // 1 .. PD - 1 and stage PD in flight into code set 0 (stage s in set
    // s mod PD); this wave's first substep read and dequantised.
    constexpr int PD = code_depth<MT>();
    ARegs<MT> g[2];
    CRegs cg[PD];
    SubstepRegs<MT> fr[2];
    bf16x8 bq[2][2];
    load_a(g[0], 0);
#pragma unroll
    for (int c = 0; c < PD; c++) load_c(cg[c], c);
    load_a(g[1], 1);
    store_lds(g[0], cg[0], 0);
    load_a(g[0], 2);
    load_c(cg[0], PD);
    __syncthreads();
    read_substep(fr[0], 0, kp);
    dequant(fr[0], bq[0]);

    // Issue order of a substep.  Each of its 2*MT MFMAs is followed by a
    // share of the other work, in this order: the next substep's code bytes
    // and folds (R0-R2); at u = 0 the stage's LDS writes of stage kt+1 and
    // global loads of stage kt+3 (activations) and kt+1+PD (codes, scale and
    // zero), A chunk by chunk (W, L), then the codes and folds; last the next substep's A fragments (RA) with its four
    // dequantisation pieces (D) spread among them, late enough for the code
    // and fold reads to have landed.  A scheduling barrier after every MFMA
    // keeps this order.
    constexpr int kMfmas = 2 * MT;
    constexpr int kTail = MT + 4;   // RA and D
    auto tail_is_d = [](int t) {
        for (int q = 0; q < 4; q++)
            if (t == q * kTail / 4 + 1) return q;
        return -1;
    };
    auto tail_ra = [&](int t) {
        int d = 0;
        for (int q = 0; q < 4; q++) d += (q * kTail / 4 + 1) < t;
        return t - d;
    };

    auto substep = [&](int kt, auto U, auto SET, auto CSET) {
        constexpr int u = decltype(U)::value;
        constexpr int set = decltype(SET)::value;
        constexpr int cset = decltype(CSET)::value;   // code set of stage kt+1
        constexpr int kItems = u == 0 ? 3 * MT + 15 : MT + 7;
        const int buf = kt & 1;
        const int rbuf = u == 0 ? buf : buf ^ 1;   // the next substep's buffer
        const int rks = u == 0 ? 2 + kp : kp;      // and its 16-k step in it
        SubstepRegs<MT>& nx = fr[u ^ 1];
        ARegs<MT>& gs = g[set ^ 1];
        CRegs& cs = cg[cset];
        const GemmStage& RS = lds.st[rbuf];
        GemmStage& WS = lds.st[buf ^ 1];
        const int k0n = kofs(kt + 3);        // activations loaded now
        const int k0c = kofs(kt + 1 + PD);   // codes loaded now
        const f32x4* fp = reinterpret_cast<const f32x4*>(&RS.fold[rks * 16 + 8 * kg]);

        auto dq = [&](int q) {
            const int h = q >> 1, j = q & 1;
            const uint32_t t = nx.tw[h];
            const uint32_t nib = (j ? (t >> 4) : t) & 0x0F0F0F0Fu;
            const f32x2 ca = __builtin_amdgcn_cvt_pk_f32_fp8(nib, false);   // rows 0, 1
            const f32x2 cb = __builtin_amdgcn_cvt_pk_f32_fp8(nib, true);    // rows 2, 3
            const f32x4 f01 = nx.fr[2 * h], f23 = nx.fr[2 * h + 1];
            bf16x8& b = bq[u ^ 1][j];
            b[4 * h + 0] = (__bf16)__builtin_fmaf(ca.x, f01.x, f01.y);
            b[4 * h + 1] = (__bf16)__builtin_fmaf(ca.y, f01.z, f01.w);
            b[4 * h + 2] = (__bf16)__builtin_fmaf(cb.x, f23.x, f23.y);
            b[4 * h + 3] = (__bf16)__builtin_fmaf(cb.y, f23.z, f23.w);
        };
        auto item = [&](int it) {
            if (it == 0) {
#pragma unroll
                for (int h = 0; h < 2; h++) nx.tw[h] = RS.b[b_off(rks * 4 + 2 * kg + h, my_bc)];
                return;
            }
            if (it == 1) { nx.fr[0] = fp[0]; nx.fr[1] = fp[1]; return; }
            if (it == 2) { nx.fr[2] = fp[2]; nx.fr[3] = fp[3]; return; }
            it -= 3;
            if (u == 0) {
                if (it < 2 * MT) {
                    const int p = it >> 1;
                    if ((it & 1) == 0)
                        *reinterpret_cast<u32x4*>(WS.a + a_dst[p]) = gs.a[p];
                    else
                        gs.a[p] = __builtin_amdgcn_raw_buffer_load_b128(a_rsrc(k0n), a_src[p],
                                                                        0, 0);
                    return;
                }
                it -= 2 * MT;
                if (it == 0) {
                    *reinterpret_cast<u32x4*>(&WS.b[b_dst]) =
                        transpose4(cs.b[0], cs.b[1], cs.b[2], cs.b[3]);
                    return;
                }
                if (it <= 4) {
                    cs.b[it - 1] = __builtin_amdgcn_raw_buffer_load_b32(
                        b_rsrc(k0c), b_src, (it - 1) * row_bytes, 0);
                    return;
                }
                if (it == 5) {
                    const float sv = half_bits_to_float(cs.s);
                    const float zv = half_bits_to_float(cs.z);
                    f32x2 f;
                    f.x = sv * 512.0f;
                    f.y = (sv == 0.0f) ? zv : -(zv * sv);
                    WS.fold[f_dst] = f;
                    return;
                }
                if (it == 6) {
                    cs.s = __builtin_amdgcn_raw_buffer_load_b16(s_rsrc(k0c), f_src, 0, 0);
                    return;
                }
                if (it == 7) {
                    cs.z = __builtin_amdgcn_raw_buffer_load_b16(z_rsrc(k0c), f_src, 0, 0);
                    return;
                }
                it -= 8;
            }
            const int q = tail_is_d(it);
            if (q >= 0) {
                dq(q);
            } else {
                const int t = tail_ra(it);
                nx.af[t] = *reinterpret_cast<const bf16x8*>(
                    RS.a + a_off(t * 32 + c32, rks * 2 + kg));
            }
        };

#pragma unroll
        for (int i = 0; i < kMfmas; i++) {
            const int t = i >> 1, j = i & 1;
            acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr[u].af[t], bq[u][j], acc[t][j],
                                                               0, 0, 0);
            if (u == 1 && i == 0) __syncthreads();   // stage kt+1 visible
#pragma unroll
            for (int it = 0; it < kItems; it++)
                if (it * kMfmas / kItems == i) item(it);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // Stage kt = base + j of a group of SU stages (SU a multiple of 2 and of
    // PD) uses activation set j % 2 and code set (j + 1) % PD.
    constexpr int SU = PD == 2 ? 2 : 4;
    auto stage = [&](int kt, auto J) {
        constexpr int j = decltype(J)::value;
        using S = std::integral_constant<int, j % 2>;
        using C = std::integral_constant<int, (j + 1) % PD>;
        substep(kt, I0{}, S{}, C{});
        substep(kt, I1{}, S{}, C{});
    };
    int kt = 0;
    for (; kt + SU <= ktiles; kt += SU) {
        stage(kt, std::integral_constant<int, 0>{});
        stage(kt + 1, std::integral_constant<int, 1>{});
        if constexpr (SU == 4) {
            stage(kt + 2, std::integral_constant<int, 2>{});
            stage(kt + 3, std::integral_constant<int, 3>{});
        }
    }
    if (kt < ktiles) stage(kt, std::integral_constant<int, 0>{});
    if constexpr (SU == 4) {
        if (kt + 1 < ktiles) stage(kt + 1, std::integral_constant<int, 1>{});
        if (kt + 2 < ktiles) stage(kt + 2, std::integral_constant<int, 2>{});
    }

    // The fused bias of this lane's two columns, fetched now so that its
    // latency overlaps the hand-over below.
    const int col = n0 + 64 * ch + 2 * c32;
    float bj[2] = {0.0f, 0.0f};
    if constexpr (BIAS) {
        bj[0] = bias[col];
        bj[1] = bias[col + 1];
    }

    // The two parities of a column half split the m-tiles: parity 0 finishes
    // [0, MT0), parity 1 [MT0, MT).  Each hands the other the partial sums
    // of the m-tiles it does not finish through LDS (one round, every m-tile
    // its own slot), then adds what it received: the sum of the two
    // parities' f32 values, the same whichever wave adds them.
    constexpr int MT0 = (MT + 1) / 2;
    auto give = [&](auto KP) {
        constexpr int p = decltype(KP)::value;
#pragma unroll
        for (int t = p == 0 ? MT0 : 0; t < (p == 0 ? MT : MT0); t++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f32x16& v = acc[t][j];
                    lds.red[ch][t][j][q][lane] =
                        (f32x4){v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                }
            __builtin_amdgcn_sched_barrier(0);   // one m-tile at a time
        }
    };
    // D of a 32 x 32 tile: lane holds column lane % 32; register r is row
    // 8*(r/4) + 4*(lane/32) + r%4.  A lane's two n-tiles are two adjacent
    // columns; the fused bias is one f32 value per column, added before the
    // one rounding.  Row addresses are a uniform row base plus this lane's
    // offset; a tile wholly inside [m0, m_end) stores without row checks.
    const bool whole = m0 + 32 * MT <= m_end;
    const uint32_t lane_off = (uint32_t)(4 * kg) * (uint32_t)N + (uint32_t)col;
    auto take_store = [&](auto KP) {
        constexpr int p = decltype(KP)::value;
#pragma unroll
        for (int t = p == 0 ? 0 : MT0; t < (p == 0 ? MT0 : MT); t++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f32x4 v = lds.red[ch][t][j][q][lane];
                    f32x16& d = acc[t][j];
                    d[4 * q] += v.x;
                    d[4 * q + 1] += v.y;
                    d[4 * q + 2] += v.z;
                    d[4 * q + 3] += v.w;
                }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int dr = t * 32 + 8 * (r >> 2) + (r & 3);   // row - m0 - 4 kg
                const bool keep = whole || m0 + dr + 4 * kg < m_end;
                if constexpr (PART) {
                    float* rowp = part + (size_t)(m0 + dr) * N;
                    if (keep)
                        *reinterpret_cast<f32x2*>(rowp + lane_off) =
                            (f32x2){acc[t][0][r], acc[t][1][r]};
                } else {
                    bf16x2 v;
                    v[0] = (__bf16)(BIAS ? acc[t][0][r] + bj[0] : acc[t][0][r]);
                    v[1] = (__bf16)(BIAS ? acc[t][1][r] + bj[1] : acc[t][1][r]);
                    uint16_t* rowp = out + (size_t)(m0 + dr) * N;
                    if (keep) *reinterpret_cast<bf16x2*>(rowp + lane_off) = v;
                }
            }
            __builtin_amdgcn_sched_barrier(0);   // one m-tile at a time
        }
    };
    __syncthreads();   // every wave is past its last read of the stages
    if (kp == 0) give(I0{}); else give(I1{});
    __syncthreads();
    if (kp == 0) take_store(I0{}); else take_store(I1{});
}

// Row bands of BM rows by column tiles of BN; MT = 8 for the full bands, the
// last band's own count for a partial one (launched separately).
template <int MT, bool BIAS>
__global__ __launch_bounds__(kThreads, 1) void int4_gemm_bf16_kernel(
    const uint16_t* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    uint16_t* __restrict__ out, int m_first, int M, int K, int N,
    const float* __restrict__ bias) {
    __shared__ GemmLds<MT> lds;
    const int tiles_n = N / BN;
    const int grid = gridDim.x;
    int b = blockIdx.x;
    if ((grid & 7) == 0) b = (b & 7) * (grid >> 3) + (b >> 3);
    const int m0 = m_first + (b / tiles_n) * BM;
    const int n0 = (b % tiles_n) * BN;
    gemm_tile_bf16<MT, BIAS>(lds, a, codes, scales, zeros, out, m0, M, n0, K, N, bias);
}

// Split K: workgroup (band, column tile, slice) runs slice `slice` of the
// stages, kt_per stages each (the last takes the rest), into the f32 sums
// part[slice] ([M, N]); int4_gemm_reduce_kernel adds the slices in slice
// order and rounds once to bf16.
template <int MT>
__global__ __launch_bounds__(kThreads, 1) void int4_gemm_bf16_splitk_kernel(
    const uint16_t* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    float* __restrict__ part, int m_first, int M, int K, int N, int slices, int kt_per) {
    __shared__ GemmLds<MT> lds;
    const int tiles_n = N / BN;
    const int grid = gridDim.x;
    int b = blockIdx.x;
    if ((grid & 7) == 0) b = (b & 7) * (grid >> 3) + (b >> 3);
    // the slices of one tile are consecutive (one XCD); measured faster than
    // the column tiles of a slice consecutive (M = 64: 14.9 against 16.5 us)
    const int slice = b % slices;
    const int tile = b / slices;
    const int m0 = m_first + (tile / tiles_n) * BM;
    const int n0 = (tile % tiles_n) * BN;
    const int kt0 = slice * kt_per;
    const int count = slice == slices - 1 ? K / BK - kt0 : kt_per;
    gemm_tile_bf16<MT, false, MT, true>(lds, a, codes, scales, zeros, nullptr, m0, M, n0, K, N,
                                        nullptr, kt0, count,
                                        part + (size_t)slice * M * N);
}

// out[m, n] = sum over s in order of part[s][m, n] (+ bias[n]), rounded once
// to bf16 or stored as f32; four columns a lane.
__global__ __launch_bounds__(256) void int4_gemm_reduce_kernel(const float* __restrict__ part,
                                                               void* __restrict__ out,
                                                               long long quads, int N, int slices,
                                                               long long stride,
                                                               const float* __restrict__ bias,
                                                               bool bf16) {
    const long long q = (long long)blockIdx.x * 256 + threadIdx.x;
    if (q >= quads) return;
    const size_t i = (size_t)q * 4;
    // eight slices' loads in flight at a time, added in slice order
    f32x4 sum = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < slices; s0 += 8) {
        f32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++)
            v[u] = s0 + u < slices
                       ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(
                             part + (size_t)(s0 + u) * stride + i))
                       : (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (s0 + u < slices) sum = s0 + u == 0 ? v[u] : sum + v[u];
    }
    if (bias) {
        const int c = (int)(i % (size_t)N);
        sum += (f32x4){bias[c], bias[c + 1], bias[c + 2], bias[c + 3]};
    }
    if (!bf16) {
        *reinterpret_cast<f32x4*>(static_cast<float*>(out) + i) = sum;
        return;
    }
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 v;
    v[0] = (__bf16)sum.x;
    v[1] = (__bf16)sum.y;
    v[2] = (__bf16)sum.z;
    v[3] = (__bf16)sum.w;
    *reinterpret_cast<bf16x4*>(static_cast<uint16_t*>(out) + i) = v;
}

// Ragged grouped form: the work is the list of (expert, row block, column
// tile) triples, row blocks of up to BM rows walked from the offsets: expert
// e's rows are [off[e], min(off[e+1], T)) (groupedtiled.go:87-91), and a
// block runs as many 32-row m-tiles as it has rows.  The launch is sized for
// the most blocks the offsets can make; every workgroup counts the real
// ones and finds its (block, column tile) by the XCD placement below (the
// dispatcher deals workgroup b to XCD b % 8).  The placement affects speed
// only.  Surplus workgroups exit.
__global__ __launch_bounds__(kThreads, 1) void int4_grouped_bf16_kernel(
    const uint16_t* __restrict__ x, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    const uint32_t* __restrict__ off, uint16_t* __restrict__ out, int E, int T, int K,
    int N) {
    __shared__ GemmLds<MAX_MT> lds;
    const int tiles_n = N / BN;
    auto rows_of = [&](int e, uint32_t& first, uint32_t& last) {
        first = off[e];
        last = off[e + 1];
        if (last > (uint32_t)T) last = (uint32_t)T;
        return last > first ? (int)(last - first) : 0;
    };
    int blocks_all = 0;
    for (int e = 0; e < E; e++) {
        uint32_t f, l;
        blocks_all += (rows_of(e, f, l) + BM - 1) / BM;
    }
    // Each XCD (workgroups are dealt to the eight round robin) takes an eighth
    // of every block's column tiles, block after block: the blocks' differing
    // m-tile counts are spread evenly over the XCDs, and the few blocks an XCD
    // works on at once keep their activation rows in its L2.  (One block's
    // tiles to one XCD left the XCDs with 5-m-tile experts ~10 us behind the
    // others: config 4 221 -> 216-217 us.)  Column counts that are not a
    // multiple of eight tiles: contiguous eighths of the whole list.
    const int work = blocks_all * tiles_n;
    int idx, n0;
    if ((tiles_n & 7) == 0) {
        const int cpx = tiles_n >> 3;
        const int slot = blockIdx.x >> 3;
        if (slot >= blocks_all * cpx) return;
        idx = slot / cpx;
        n0 = ((blockIdx.x & 7) * cpx + slot % cpx) * BN;
    } else {
        const int per_xcd = (work + 7) / 8;
        const int slot = blockIdx.x >> 3;
        if (slot >= per_xcd) return;
        const int li = (blockIdx.x & 7) * per_xcd + slot;
        if (li >= work) return;
        idx = li / tiles_n;
        n0 = (li % tiles_n) * BN;
    }
    int e = 0, m0 = 0, m_end = 0;
    bool found = false;
    for (; e < E; e++) {
        uint32_t first, last;
        const int blocks = (rows_of(e, first, last) + BM - 1) / BM;
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
    const uint32_t* c = codes + e * (per_expert >> 3);
    const uint16_t* s = scales + e * (per_expert >> 7);
    const uint16_t* z = zeros + e * (per_expert >> 7);
    switch ((min(m_end - m0, BM) + 31) / 32) {
        case 1: gemm_tile_bf16<1, false>(lds, x, c, s, z, out, m0, m_end, n0, K, N, nullptr); break;
        case 2: gemm_tile_bf16<2, false>(lds, x, c, s, z, out, m0, m_end, n0, K, N, nullptr); break;
        case 3: gemm_tile_bf16<3, false>(lds, x, c, s, z, out, m0, m_end, n0, K, N, nullptr); break;
        case 4: gemm_tile_bf16<4, false>(lds, x, c, s, z, out, m0, m_end, n0, K, N, nullptr); break;
        case 5: gemm_tile_bf16<5, false>(lds, x, c, s, z, out, m0, m_end, n0, K, N, nullptr); break;
        case 6: gemm_tile_bf16<6, false>(lds, x, c, s, z, out, m0, m_end, n0, K, N, nullptr); break;
        case 7: gemm_tile_bf16<7, false>(lds, x, c, s, z, out, m0, m_end, n0, K, N, nullptr); break;
        default: gemm_tile_bf16<8, false>(lds, x, c, s, z, out, m0, m_end, n0, K, N, nullptr); break;
    }
}

// ---- f32 activations on the matrix cores ---------------------------------
//
// The reference API's own dtype (f32 activations and result) to f32
// accuracy.  Within a 128-column tile every row k has one scale s and zero
// z, so with add = (s == 0 ? z : -z*s) and q the code,
//     sum_k x[m,k] w[k,n] = sum_k (x[m,k] 512 s_k) (q[k,n] 2^-9) + sum_k x[m,k] add_k
// (s_k taken as 0 where it is 0).  The first sum runs on the bf16 matrix
// cores: B is the code itself, q 2^-9, exact in bf16, and A' = x 512 s is
// split exactly into three bf16 terms hi + mid + lo (each the RNE rounding of
// what the previous ones leave; the residue is below 2^-27 |A'|), three MFMAs
// per tile step.  The second sum, one value per row, is accumulated in f32
// while the A tile is staged and added to the row at the end.
//
// A workgroup of four waves computes 128 rows (four 32-row m-tiles) by 128
// columns; wave w owns the column half w & 1 and the 16-k substeps of parity
// w >> 1, as in the bf16 tiles.  Per 64-k stage the workgroup turns the f32
// activations (staged through registers two stages ahead) into the three
// bf16 terms in LDS, each lane eight consecutive k of one row per m-tile,
// reading the (512 s, add) fold of the stage's rows from LDS (published a
// stage earlier); codes go to LDS transposed as in the bf16 tiles.

constexpr int XBM = 128;            // rows of an f32 tile: four m-tiles
constexpr int kXTerms = 3;

struct __attribute__((aligned(16))) XStage {
    char a[kXTerms][XBM * kARowBytes];        // 3 x 16 KB: hi, mid, lo, swizzled rows
    uint32_t b[(BK / 4) * kBQuadWords];       // 4 KB: [row quad][code byte]
};
struct __attribute__((aligned(16))) XLds {
    union {
        XStage st[2];
        // accumulator hand-off of the k-parity wave pairs:
        // [column half][m-tile][n-tile][register quad][lane]
        f32x4 red[2][4][2][4][64];
    };
    f32x2 fold[2][BK + 64];   // (512 s, add) of the stage rows, double-buffered; 64 spare
    float corr[XBM];       // sum_k x add of each row, at the end
};

// Two values -> three bf16 pairs whose sum is (v0, v1) to 2^-27 relative:
// each term is the RNE bf16 of what the previous ones leave, and the
// remainder v - term is exact in f32, taken with one v_dot2 (-1 * term + v).
// The pairs (-1, 0) and (0, -1) come in as SGPRs: the compiler would encode
// the first as the inline constant -1.0, which the hardware does not expand
// to bf16 -1 in the low half.
__device__ __forceinline__ bf16x2 xbf16_pair(uint32_t bits) {
    uint32_t r;
    asm("s_mov_b32 %0, %1" : "=s"(r) : "i"(bits));
    return __builtin_bit_cast(bf16x2, r);
}
__device__ __forceinline__ void xsplit3(float v0, float v1, uint32_t& hi, uint32_t& mid,
                                        uint32_t& lo) {
    const bf16x2 m10 = xbf16_pair(0x0000BF80u);   // (-1, 0)
    const bf16x2 m01 = xbf16_pair(0xBF800000u);   // (0, -1)
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

// One 128-row x 128-column tile: rows [m0, min(m0 + 128, m_end)) of a (rows
// past m_end are clamped copies, never stored), columns [n0, n0 + 128), the
// stages [kt0, kt0 + ktiles) of K.  With `my_part` the f32 sums, row
// corrections included, go to my_part ([M, N] of the slice) and the caller's
// reduction applies the epilogue; else they go to `out` through `ep`.  MT:
// the 32-row m-tiles that hold rows (a short band or block runs only those).
template <int MT>
__device__ __forceinline__ void gemm_tile_f32x3_t(XLds& lds, const float* __restrict__ a,
                                                const uint32_t* __restrict__ codes,
                                                const uint16_t* __restrict__ scales,
                                                const uint16_t* __restrict__ zeros,
                                                void* __restrict__ out, int m0, int m_end,
                                                int n0, int K, int N, const Epilogue& ep,
                                                float* my_part, int kt0, int ktiles) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int ch = wave & 1;
    const int kp = wave >> 1;
    const int lane = tid & 63;
    const int c32 = lane & 31;
    const int kg = lane >> 5;
    const size_t groups_per_row = (size_t)(N >> 7);
    const size_t words_per_row = (size_t)(N >> 3);

    // Activation staging: m-tile i, row (tid >> 3) + 32 i, k 8 (tid & 7) ..
    // + 7 of a stage: two 16-byte loads each.
    const int x_row = tid >> 3;
    const int x_c8 = tid & 7;
    const float* x_src[MT];
    int x_dst[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) {
        const int r = x_row + 32 * i;
        x_src[i] = a + (size_t)min(m0 + r, m_end - 1) * K + 8 * x_c8;
        x_dst[i] = a_off(r, x_c8);
    }
    // codes and fold staging as in the bf16 tiles
    const int b_rq = tid >> 4;
    const int b_cc = tid & 15;
    const uint32_t* b_src = codes + (size_t)(4 * b_rq) * words_per_row + (n0 >> 3) + b_cc;
    const int b_dst = b_off(b_rq, 4 * b_cc);
    const int f_row = 16 * wave + (lane & 15);
    const int f_dst = lane < 16 ? f_row : BK + lane;
    const size_t f_g = (size_t)(n0 >> 7);
    const uint16_t* s_src = scales + (size_t)f_row * groups_per_row + f_g;
    const uint16_t* z_src = zeros + (size_t)f_row * groups_per_row + f_g;
    const int my_bc = 32 * ch + c32;

    struct XRegs { f32x4 x[MT][2]; };
    struct CRegs2 { uint32_t b[4]; };
    struct SZ { uint16_t s, z; };
    auto load_x = [&](XRegs& g, int kt) {
        const int k0 = (kt0 + min(kt, ktiles - 1)) * BK;
#pragma unroll
        for (int i = 0; i < MT; i++) {
            g.x[i][0] = *reinterpret_cast<const f32x4*>(x_src[i] + k0);
            g.x[i][1] = *reinterpret_cast<const f32x4*>(x_src[i] + k0 + 4);
        }
    };
    auto load_b = [&](CRegs2& g, int kt) {
        const int k0 = (kt0 + min(kt, ktiles - 1)) * BK;
        const uint32_t* bp = b_src + (size_t)k0 * words_per_row;
#pragma unroll
        for (int i = 0; i < 4; i++) g.b[i] = bp[(size_t)i * words_per_row];
    };
    auto load_sz = [&](SZ& g, int kt) {
        const int k0 = (kt0 + min(kt, ktiles - 1)) * BK;
        g.s = s_src[(size_t)k0 * groups_per_row];
        g.z = z_src[(size_t)k0 * groups_per_row];
    };
    auto write_fold = [&](const SZ& g, int fb) {
        const float sv = half_bits_to_float(g.s);
        const float zv = half_bits_to_float(g.z);
        f32x2 f;
        f.x = sv * 512.0f;
        f.y = (sv == 0.0f) ? zv : -(zv * sv);
        lds.fold[fb][f_dst] = f;
    };
    float corr[MT];
#pragma unroll
    for (int i = 0; i < MT; i++) corr[i] = 0.0f;
    // The three terms of m-tile i's chunk, from its activations and the
    // stage's fold (fv: the eight k of this lane), into LDS buffer `buf`;
    // `real` is false for the stage past the last, staged (from clamped
    // loads) but never read, whose rows must not reach the corrections.
    auto stage_x = [&](const f32x4 (&xv)[2], const f32x2 (&fv)[8], int i, int buf, bool real) {
        const float x8[8] = {xv[0].x, xv[0].y, xv[0].z, xv[0].w,
                             xv[1].x, xv[1].y, xv[1].z, xv[1].w};
        uint32_t h[4], md[4], lo[4];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const float v0 = x8[2 * p] * fv[2 * p].x;
            const float v1 = x8[2 * p + 1] * fv[2 * p + 1].x;
            const float c0 = __builtin_fmaf(x8[2 * p], fv[2 * p].y, corr[i]);
            corr[i] = real ? __builtin_fmaf(x8[2 * p + 1], fv[2 * p + 1].y, c0) : corr[i];
            xsplit3(v0, v1, h[p], md[p], lo[p]);
        }
        XStage& S = lds.st[buf];
        *reinterpret_cast<u32x4*>(S.a[0] + x_dst[i]) = (u32x4){h[0], h[1], h[2], h[3]};
        *reinterpret_cast<u32x4*>(S.a[1] + x_dst[i]) = (u32x4){md[0], md[1], md[2], md[3]};
        *reinterpret_cast<u32x4*>(S.a[2] + x_dst[i]) = (u32x4){lo[0], lo[1], lo[2], lo[3]};
    };
    auto read_fold = [&](f32x2 (&fv)[8], int fb) {
        const f32x4* fp = reinterpret_cast<const f32x4*>(&lds.fold[fb][8 * x_c8]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const f32x4 t = fp[j];
            fv[2 * j] = (f32x2){t.x, t.y};
            fv[2 * j + 1] = (f32x2){t.z, t.w};
        }
    };

    // One substep's operands: the three terms' A fragments of the MT
    // m-tiles, one code byte of eight rows.
    struct XSub {
        bf16x8 af[kXTerms][MT];
        uint32_t tw[2];
    };
    auto read_sub = [&](XSub& r, int buf, int ks) {
        const XStage& S = lds.st[buf];
#pragma unroll
        for (int h = 0; h < 2; h++) r.tw[h] = S.b[b_off(ks * 4 + 2 * kg + h, my_bc)];
#pragma unroll
        for (int tt = 0; tt < kXTerms; tt++)
#pragma unroll
            for (int t = 0; t < MT; t++)
                r.af[tt][t] = *reinterpret_cast<const bf16x8*>(
                    S.a[tt] + a_off(t * 32 + c32, ks * 2 + kg));
    };
    // B of the two n-tiles: q 2^-9 as bf16, exact (byte 0000qqqq as e4m3).
    auto codes_b = [&](const XSub& r, bf16x8 (&bfr)[2]) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t t = r.tw[h];
            const uint32_t lo = t & 0x0F0F0F0Fu;
            const uint32_t hi = (t >> 4) & 0x0F0F0F0Fu;
            const bf16x2 l01 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
            const bf16x2 l23 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
            const bf16x2 h01 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
            const bf16x2 h23 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
            bfr[0][4 * h + 0] = l01[0];
            bfr[0][4 * h + 1] = l01[1];
            bfr[0][4 * h + 2] = l23[0];
            bfr[0][4 * h + 3] = l23[1];
            bfr[1][4 * h + 0] = h01[0];
            bfr[1][4 * h + 1] = h01[1];
            bfr[1][4 * h + 2] = h23[0];
            bfr[1][4 * h + 3] = h23[1];
        }
    };

    f32x16 acc[MT][2];
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[t][j][r] = 0.0f;

    // Prologue: folds of stages 0 and 1 published; stage 0 staged into LDS
    // buffer 0; activations of stage 1 in set 1 and stage 2 in flight into
    // set 0; codes of stage 1 held, s/z of stages 2 and 3 in flight.
    XRegs gx[2];
    CRegs2 gb[2];
    SZ gz[2];
    {
        SZ z0, z1;
        load_sz(z0, 0);
        load_sz(z1, 1);
        load_x(gx[0], 0);
        load_b(gb[0], 0);
        load_x(gx[1], 1);
        load_b(gb[1], 1);
        load_sz(gz[0], 2);
        load_sz(gz[1], 3);
        write_fold(z0, 0);
        write_fold(z1, 1);
    }
    __syncthreads();
    {
        f32x2 fv[8];
        read_fold(fv, 0);
#pragma unroll
        for (int i = 0; i < MT; i++) stage_x(gx[0].x[i], fv, i, 0, true);
        *reinterpret_cast<u32x4*>(&lds.st[0].b[b_dst]) =
            transpose4(gb[0].b[0], gb[0].b[1], gb[0].b[2], gb[0].b[3]);
    }
    load_x(gx[0], 2);
    load_b(gb[0], 2);
    __syncthreads();
    XSub sub[2];
    bf16x8 bq[2][2];
    read_sub(sub[0], 0, kp);
    codes_b(sub[0], bq[0]);

    auto mfma_all = [&](const XSub& r, const bf16x8 (&bfr)[2]) {
#pragma unroll
        for (int tt = 0; tt < kXTerms; tt++)
#pragma unroll
            for (int t = 0; t < MT; t++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(r.af[tt][t], bfr[j],
                                                                       acc[t][j], 0, 0, 0);
    };

    // Stage kt: substep u = 0 publishes the fold of stage kt+2, stages the
    // activations and codes of stage kt+1 (fold kt+1, published a stage
    // ago), issues the loads of stage kt+3 (activations, codes) and kt+4
    // (scale, zero), and reads its second substep's operands; substep u = 1
    // waits at the stage's barrier and reads the first substep of stage kt+1.
    auto stage = [&](int kt, auto SET) {
        constexpr int set = decltype(SET)::value;   // gx/gb[set ^ 1]: stage kt+1
        const int buf = kt & 1;
        {
            write_fold(gz[kt & 1], kt & 1);           // stage kt+2
            f32x2 fv[8];
            read_fold(fv, (kt + 1) & 1);
            read_sub(sub[1], buf, 2 + kp);
            mfma_all(sub[0], bq[0]);
#pragma unroll
            for (int i = 0; i < MT; i++) stage_x(gx[set ^ 1].x[i], fv, i, buf ^ 1, kt + 1 < ktiles);
            *reinterpret_cast<u32x4*>(&lds.st[buf ^ 1].b[b_dst]) =
                transpose4(gb[set ^ 1].b[0], gb[set ^ 1].b[1], gb[set ^ 1].b[2], gb[set ^ 1].b[3]);
            load_x(gx[set ^ 1], kt + 3);
            load_b(gb[set ^ 1], kt + 3);
            load_sz(gz[kt & 1], kt + 4);
            codes_b(sub[1], bq[1]);
        }
        {
            __syncthreads();                          // stage kt+1 and fold kt+2 visible
            read_sub(sub[0], buf ^ 1, kp);
            mfma_all(sub[1], bq[1]);
            codes_b(sub[0], bq[0]);
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    int kt = 0;
    for (; kt + 2 <= ktiles; kt += 2) {
        stage(kt, I0{});
        stage(kt + 1, I1{});
    }
    if (kt < ktiles) stage(kt, I0{});

    // Row corrections: the eight lanes of a row (x_c8) add theirs; LDS holds
    // one value per tile row.
#pragma unroll
    for (int i = 0; i < MT; i++) {
        float c = corr[i];
        c += __shfl_xor(c, 1, 64);
        c += __shfl_xor(c, 2, 64);
        c += __shfl_xor(c, 4, 64);
        corr[i] = c;
    }
    __syncthreads();
    if (x_c8 == 0) {
#pragma unroll
        for (int i = 0; i < MT; i++) lds.corr[x_row + 32 * i] = corr[i];
    }
    // The two parities of a column half split the m-tiles: parity 0 finishes
    // [0, MT0), parity 1 [MT0, MT), each handing the other its partial sums
    // of the rest through LDS (the sum of the two parities' f32 values, the
    // same whichever wave adds them).
    constexpr int MT0 = (MT + 1) / 2;
    const int col = n0 + 64 * ch + 2 * c32;
    float bj[2] = {0.0f, 0.0f};
    if (ep.bias) {
        bj[0] = ep.bias[col];
        bj[1] = ep.bias[col + 1];
    }
    auto give = [&](auto KP) {
        constexpr int p = decltype(KP)::value;
#pragma unroll
        for (int t = p == 0 ? MT0 : 0; t < (p == 0 ? MT : MT0); t++)
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f32x16& v = acc[t][j];
                    lds.red[ch][t][j][q][lane] =
                        (f32x4){v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                }
    };
    auto take_store = [&](auto KP) {
        constexpr int p = decltype(KP)::value;
#pragma unroll
        for (int t = p == 0 ? 0 : MT0; t < (p == 0 ? MT0 : MT); t++) {
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f32x4 v = lds.red[ch][t][j][q][lane];
                    f32x16& d = acc[t][j];
                    d[4 * q] += v.x;
                    d[4 * q + 1] += v.y;
                    d[4 * q + 2] += v.z;
                    d[4 * q + 3] += v.w;
                }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int rl = t * 32 + 8 * (r >> 2) + 4 * kg + (r & 3);
                const int row = m0 + rl;
                if (row < m_end) {
                    const float cr = lds.corr[rl];
                    const size_t o = (size_t)row * N + col;
                    if (my_part) {
                        *reinterpret_cast<f32x2*>(my_part + o) =
                            (f32x2){acc[t][0][r] + cr, acc[t][1][r] + cr};
                    } else {
                        store_value(out, o, acc[t][0][r] + cr + bj[0], ep.bf16);
                        store_value(out, o + 1, acc[t][1][r] + cr + bj[1], ep.bf16);
                    }
                }
            }
        }
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    if (kp == 0) give(P0{}); else give(P1{});
    __syncthreads();
    if (kp == 0) take_store(P0{}); else take_store(P1{});
}

// The tile of rows [m0, min(m0 + 128, m_end)) with the m-tiles it has rows
// for (uniform across the workgroup).  Measured (us, all four m-tiles / only
// those with rows): M = 64, K = N = 4096 (split K) 26.8 / 20.3; at 17..48
// rows the short bands also beat 16-row matrix-core decode launches, which
// these shapes took before (4096 x 4096 at 32 rows 21.3 / 15.7, 14336 x 4096
// at 48 rows 49.0 / 39.3).
__device__ __forceinline__ void gemm_tile_f32x3(XLds& lds, const float* __restrict__ a,
                                                const uint32_t* __restrict__ codes,
                                                const uint16_t* __restrict__ scales,
                                                const uint16_t* __restrict__ zeros,
                                                void* __restrict__ out, int m0, int m_end,
                                                int n0, int K, int N, const Epilogue& ep,
                                                float* my_part, int kt0, int ktiles) {
    switch ((min(m_end - m0, XBM) + 31) / 32) {
        case 1:
            gemm_tile_f32x3_t<1>(lds, a, codes, scales, zeros, out, m0, m_end, n0, K, N, ep,
                                 my_part, kt0, ktiles);
            break;
        case 2:
            gemm_tile_f32x3_t<2>(lds, a, codes, scales, zeros, out, m0, m_end, n0, K, N, ep,
                                 my_part, kt0, ktiles);
            break;
        case 3:
            gemm_tile_f32x3_t<3>(lds, a, codes, scales, zeros, out, m0, m_end, n0, K, N, ep,
                                 my_part, kt0, ktiles);
            break;
        default:
            gemm_tile_f32x3_t<4>(lds, a, codes, scales, zeros, out, m0, m_end, n0, K, N, ep,
                                 my_part, kt0, ktiles);
            break;
    }
}

// With `part`, split K: workgroup (tile, slice) runs slice `slice` of the
// stages (kt_per each, the last the rest) and stores its f32 sums, row
// corrections included, to part[slice] ([M, N]); int4_gemm_reduce_kernel
// adds the slices in order and applies the epilogue.
__global__ __launch_bounds__(kThreads, 1) void int4_gemm_f32x3_kernel(
    const float* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    void* __restrict__ out, int M, int K, int N, Epilogue ep, float* part, int slices,
    int kt_per) {
    __shared__ XLds lds;
    const int tiles_n = N / BN;
    const int grid = gridDim.x;
    int bid = blockIdx.x;
    if ((grid & 7) == 0) bid = (bid & 7) * (grid >> 3) + (bid >> 3);
    // split K: the slices of one tile are consecutive (one XCD), as in the
    // bf16 split kernel
    const int slice = part ? bid % slices : 0;
    if (part) bid /= slices;
    const int kt0 = slice * kt_per;
    const int ktiles = !part ? K / BK : (slice == slices - 1 ? K / BK - kt0 : kt_per);
    gemm_tile_f32x3(lds, a, codes, scales, zeros, out, (bid / tiles_n) * XBM, M,
                    (bid % tiles_n) * BN, K, N, ep, part ? part + (size_t)slice * M * N : nullptr,
                    kt0, ktiles);
}

// The grouped product of f32 rows (the reference API's grouped dtype,
// tensor/grouped.go:138-212) on the matrix cores: the f32 tiles above walking
// the (expert, 128-row block, column tile) list of the segments given by
// `seg` ([E+1]: expert e's rows are [seg[e], min(seg[e+1], T))), each block
// against its expert's planes, as int4_grouped_bf16_kernel does for bf16
// rows.  The list is dealt to the XCDs in contiguous eighths so a block's
// column tiles share its rows in one L2.  Rows past every segment are not
// written here.
__global__ __launch_bounds__(kThreads, 1) void int4_grouped_f32x3_kernel(
    const float* __restrict__ x, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    const uint32_t* __restrict__ seg, float* __restrict__ out, int E, int T, int K, int N) {
    __shared__ XLds lds;
    const int tiles_n = N / BN;
    auto rows_of = [&](int e, uint32_t& first, uint32_t& last) {
        first = seg[e];
        last = seg[e + 1];
        if (last > (uint32_t)T) last = (uint32_t)T;
        return last > first ? (int)(last - first) : 0;
    };
    int blocks_all = 0;
    for (int e = 0; e < E; e++) {
        uint32_t f, l;
        blocks_all += (rows_of(e, f, l) + XBM - 1) / XBM;
    }
    const int work = blocks_all * tiles_n;
    const int per_xcd = (work + 7) / 8;
    const int slot = blockIdx.x >> 3;
    if (slot >= per_xcd) return;
    const int li = (blockIdx.x & 7) * per_xcd + slot;
    if (li >= work) return;
    int idx = li / tiles_n;
    const int n0 = (li % tiles_n) * BN;
    int e = 0, m0 = 0, m_end = 0;
    bool found = false;
    for (; e < E; e++) {
        uint32_t first, last;
        const int blocks = (rows_of(e, first, last) + XBM - 1) / XBM;
        if (idx < blocks) {
            m0 = (int)first + idx * XBM;
            m_end = (int)last;
            found = true;
            break;
        }
        idx -= blocks;
    }
    if (!found) return;
    const size_t per_expert = (size_t)K * N;
    gemm_tile_f32x3(lds, x, codes + e * (per_expert >> 3), scales + e * (per_expert >> 7),
                    zeros + e * (per_expert >> 7), out, m0, m_end, n0, K, N, Epilogue{},
                    nullptr, 0, K / BK);
}

// ---- f32 activations, fp32 VALU tiles -------------------------------------

constexpr int FM = 64, FN = 64, FK = 32;

__global__ __launch_bounds__(256) void int4_gemm_f32_kernel(
    const float* __restrict__ a, const uint32_t* __restrict__ codes,
    const uint16_t* __restrict__ scales, const uint16_t* __restrict__ zeros,
    void* __restrict__ out, int M, int K, int N, Epilogue ep) {
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
            if (col < N) store_out(out, (size_t)row * N + col, col, acc[i][j], ep);
        }
    }
}

}  // namespace

bool int4_gemm_bf16_supported(int M, int K, int N) {
    // per-lane load offsets within a tile stay below 2^31 (gemm_tile_bf16)
    return M >= 1 && K >= BK && K % BK == 0 && N >= BN && N % BN == 0 &&
           K < (1 << 22) && N < (1 << 26);
}

template <int MT>
void launch_band(hipStream_t st, const uint16_t* a, Int4Planes w, uint16_t* out, int m_first,
                 int bands, int M, int K, int N, const float* bias) {
    const dim3 grid(bands * (N / BN));
    if (bias)
        ACCEL_LAUNCH(tname("int4_gemm_bf16_kernel", MT, true) + grid_note(bands * (N / BN), 1),
                     (int4_gemm_bf16_kernel<MT, true>), grid, dim3(kThreads), 0, st, a,
                           w.codes, w.scales, w.zeros, out, m_first, M, K, N, bias);
    else
        ACCEL_LAUNCH(tname("int4_gemm_bf16_kernel", MT, false) + grid_note(bands * (N / BN), 1),
                     (int4_gemm_bf16_kernel<MT, false>), grid, dim3(kThreads), 0, st, a,
                           w.codes, w.scales, w.zeros, out, m_first, M, K, N, bias);
}

template <int MT>
void launch_band_splitk(hipStream_t st, const uint16_t* a, Int4Planes w, float* part,
                        int m_first, int bands, int M, int K, int N, int slices, int kt_per) {
    const dim3 grid(bands * (N / BN) * slices);
    ACCEL_LAUNCH(tname("int4_gemm_bf16_splitk_kernel", MT) + grid_note(bands * (N / BN), slices),
                 (int4_gemm_bf16_splitk_kernel<MT>), grid, dim3(kThreads), 0, st, a,
                       w.codes, w.scales, w.zeros, part, m_first, M, K, N, slices, kt_per);
}

// K slices for a product whose tiles leave CUs idle: as many as fill the
// chip once, each of at least four stages.
static int gemm_slices(const Device* d, int M, int K, int N) {
    const int tiles = (M + BM - 1) / BM * (N / BN);
    const int ktiles = K / BK;
    if (tiles * 2 > d->cu_count) return 1;
    return std::max(1, std::min(d->cu_count / tiles, ktiles / 4));
}

hipError_t launch_int4_gemm_bf16(Device* d, hipStream_t st, const uint16_t* a, Int4Planes w,
                                 uint16_t* out, int M, int K, int N, const float* bias,
                                 int* status) {
    *status = ACCEL_OK;
    const int slices = gemm_slices(d, M, K, N);
    if (slices > 1) {
        // Split K: each slice's f32 sums to the workspace, then one pass adds
        // them in slice order and rounds.
        const size_t stride = (size_t)M * N;
        void* ws = workspace(d, st, (size_t)slices * stride * sizeof(float), status);
        if (!ws) return hipSuccess;
        float* part = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
        const int kt_per = (K / BK) / slices;
        const int full = M / BM;
        if (full > 0) launch_band_splitk<8>(st, a, w, part, 0, full, M, K, N, slices, kt_per);
        const int rest = M - full * BM;
        if (rest > 0) {
            const int mf = full * BM;
            switch ((rest + 31) / 32) {
                case 1: launch_band_splitk<1>(st, a, w, part, mf, 1, M, K, N, slices, kt_per); break;
                case 2: launch_band_splitk<2>(st, a, w, part, mf, 1, M, K, N, slices, kt_per); break;
                case 3: launch_band_splitk<3>(st, a, w, part, mf, 1, M, K, N, slices, kt_per); break;
                case 4: launch_band_splitk<4>(st, a, w, part, mf, 1, M, K, N, slices, kt_per); break;
                case 5: launch_band_splitk<5>(st, a, w, part, mf, 1, M, K, N, slices, kt_per); break;
                case 6: launch_band_splitk<6>(st, a, w, part, mf, 1, M, K, N, slices, kt_per); break;
                case 7: launch_band_splitk<7>(st, a, w, part, mf, 1, M, K, N, slices, kt_per); break;
                default: launch_band_splitk<8>(st, a, w, part, mf, 1, M, K, N, slices, kt_per); break;
            }
        }
        const long long quads = (long long)stride / 4;
        ACCEL_LAUNCH(std::string("int4_gemm_reduce_kernel"), int4_gemm_reduce_kernel,
                     dim3((unsigned)((quads + 255) / 256)),
                           dim3(256), 0, st, part, (void*)out, quads, N, slices,
                           (long long)stride, bias, true);
        return launch_status();
    }
    // full 256-row bands in one launch, a partial last band in another with
    // only its own m-tiles
    const int full = M / BM;
    if (full > 0) launch_band<8>(st, a, w, out, 0, full, M, K, N, bias);
    const int rest = M - full * BM;
    if (rest > 0) {
        const int m_first = full * BM;
        switch ((rest + 31) / 32) {
            case 1: launch_band<1>(st, a, w, out, m_first, 1, M, K, N, bias); break;
            case 2: launch_band<2>(st, a, w, out, m_first, 1, M, K, N, bias); break;
            case 3: launch_band<3>(st, a, w, out, m_first, 1, M, K, N, bias); break;
            case 4: launch_band<4>(st, a, w, out, m_first, 1, M, K, N, bias); break;
            case 5: launch_band<5>(st, a, w, out, m_first, 1, M, K, N, bias); break;
            case 6: launch_band<6>(st, a, w, out, m_first, 1, M, K, N, bias); break;
            case 7: launch_band<7>(st, a, w, out, m_first, 1, M, K, N, bias); break;
            default: launch_band<8>(st, a, w, out, m_first, 1, M, K, N, bias); break;
        }
    }
    return launch_status();
}

hipError_t launch_int4_grouped_bf16(Device*, hipStream_t st, const uint16_t* x,
                                    Int4Planes w, const uint32_t* off, uint16_t* out, int E,
                                    int T, int K, int N, bool) {
    // Upper bound on (expert, row block) pairs: every expert can add one
    // partial block.
    const long long max_blocks = (T + BM - 1) / BM + (long long)E;
    const long long wgs = (max_blocks * (N / BN) + 7) / 8 * 8;
    if (wgs > (1ll << 31) - 8) return hipErrorInvalidConfiguration;
    dim3 grid((unsigned)wgs);
    ACCEL_LAUNCH(std::string("int4_grouped_bf16_kernel"), int4_grouped_bf16_kernel, grid, dim3(kThreads), 0, st, x, w.codes,
                       w.scales, w.zeros, off, out, E, T, K, N);
    return launch_status();
}

hipError_t launch_int4_grouped_f32x3(hipStream_t st, const float* x, Int4Planes w,
                                     const uint32_t* seg, float* out, int E, int T, int K,
                                     int N) {
    // upper bound on (expert, row block) pairs: every expert can add one
    // partial block
    const long long max_blocks = (T + XBM - 1) / XBM + (long long)E;
    const long long wgs = (max_blocks * (N / BN) + 7) / 8 * 8;
    if (wgs > (1ll << 31) - 8) return hipErrorInvalidConfiguration;
    ACCEL_LAUNCH(std::string("int4_grouped_f32x3_kernel") + grid_note(wgs, 0),
                 int4_grouped_f32x3_kernel, dim3((unsigned)wgs), dim3(kThreads), 0, st, x,
                 w.codes, w.scales, w.zeros, seg, out, E, T, K, N);
    return launch_status();
}

bool int4_gemm_f32x3_supported(int K, int N) {
    return K >= BK && K % BK == 0 && N >= BN && N % BN == 0 && K < (1 << 30) && N < (1 << 30);
}

hipError_t launch_int4_gemm_f32x3(Device* d, hipStream_t st, const float* a, Int4Planes w,
                                  void* out, int M, int K, int N, Epilogue ep, int* status) {
    *status = ACCEL_OK;
    const int tiles = (M + XBM - 1) / XBM * (N / BN);
    const int ktiles = K / BK;
    // K slices when the tiles leave CUs idle, as for the bf16 tiles
    const int slices =
        tiles * 2 > d->cu_count ? 1 : std::max(1, std::min(d->cu_count / tiles, ktiles / 4));
    if (slices == 1) {
        ACCEL_LAUNCH(std::string("int4_gemm_f32x3_kernel") + grid_note(tiles, 1),
                     int4_gemm_f32x3_kernel, dim3(tiles), dim3(kThreads), 0, st, a,
                           w.codes, w.scales, w.zeros, out, M, K, N, ep, (float*)nullptr, 1, 0);
        return launch_status();
    }
    const size_t stride = (size_t)M * N;
    void* ws = workspace(d, st, (size_t)slices * stride * sizeof(float), status);
    if (!ws) return hipSuccess;
    float* part = reinterpret_cast<float*>(static_cast<char*>(ws) + kWorkspaceCounterBytes);
    ACCEL_LAUNCH(std::string("int4_gemm_f32x3_kernel") + grid_note(tiles, slices),
                 int4_gemm_f32x3_kernel, dim3(tiles * slices), dim3(kThreads), 0, st, a,
                       w.codes, w.scales, w.zeros, out, M, K, N, ep, part, slices,
                       ktiles / slices);
    const long long quads = (long long)stride / 4;
    ACCEL_LAUNCH(std::string("int4_gemm_reduce_kernel"), int4_gemm_reduce_kernel,
                 dim3((unsigned)((quads + 255) / 256)), dim3(256),
                       0, st, part, out, quads, N, slices, (long long)stride, ep.bias, ep.bf16);
    return launch_status();
}

hipError_t launch_int4_gemm_f32(Device*, hipStream_t st, const float* a, Int4Planes w,
                                void* out, int M, int K, int N, Epilogue ep) {
    dim3 grid((N + FN - 1) / FN, (M + FM - 1) / FM);
    ACCEL_LAUNCH(std::string("int4_gemm_f32_kernel"), int4_gemm_f32_kernel, grid, dim3(256), 0, st, a, w.codes, w.scales,
                       w.zeros, out, M, K, N, ep);
    return launch_status();
}

}  // namespace accel
