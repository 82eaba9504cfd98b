// Internal declarations shared by the translation units of libaccel_hip.so.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/accel_hip.h"

namespace accel {

// Records a message for accel_hip_last_error() on this thread and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Bits of the device fault word: what a kernel reports when it gives up
// instead of producing its result.
constexpr uint32_t kFaultWaitGaveUp = 1u;     // a split-K hand-off's bounded wait ran out

// Per-device state: the open flag, sticky loss, fault injection, the
// library-owned workspace and the fault word.
struct Device {
    int ordinal = -1;
    bool open = false;
    std::atomic<int> lost{0};
    std::mutex mu;
    int64_t submissions = 0;
    int64_t lose_at = 0;
    void* ws = nullptr;        // workspace (device memory)
    size_t ws_bytes = 0;
    uint64_t ws_gen = 0;       // bumped each time the workspace is reallocated
    // Workspaces replaced by a larger one while a live executable still
    // names them (its kernels carry the old addresses): freed when the last
    // such executable is destroyed, or at close.
    struct Retired {
        void* ptr;
        uint64_t gen;
    };
    std::vector<Retired> retired;
    std::unordered_map<void*, uint64_t> exec_gen;   // live executable -> workspace generation
    // Fault word: host memory the kernels write (system scope) when a bounded
    // wait gives up; read after every wait.
    uint32_t* fault_host = nullptr;
    uint32_t* fault_dev = nullptr;
    int32_t wait_limit = 1 << 22;   // spins of a hand-off's bounded wait
    // This device's copy of the no-allocation entry point's static scratch
    // (its device address, from hipGetSymbolAddress at open).
    void* scratch = nullptr;
    int cu_count = 256;
    size_t lds_per_block = 65536;
    // The last int4 product's selection (accel_hip_last_selection), under mu.
    bool sel_valid = false;
    std::string sel_op, sel_kernel, sel_reason, sel_rejected;
};

// The open device `dev`, made current on this thread, or nullptr with the
// error recorded.
Device* device(int dev);

// Counts an accepted submission and applies fault injection; returns
// ACCEL_OK or ACCEL_E_DEVICE_LOST (cpu.go:179-191's beginSubmission).
int begin_submission(Device* d);

// Classifies a HIP status after a launch or a wait.  Errors that leave the
// device's memory undefined mark it lost for good; an allocation failure
// does not.  Returns the ACCEL_* code.
int classify(Device* d, hipError_t e, const char* what);

// The workspace, at least `bytes` long beyond its counters.  The first
// kWorkspaceCounterBytes are kept zero between launches by the kernels that
// use them (a counter is reset by the workgroup that consumes it).  It grows
// only outside graph capture: a call that needs more on a capturing stream
// is refused (ACCEL_E_INVALID).  A workspace that a live executable names is
// retired, not freed, when it grows.
constexpr size_t kWorkspaceCounterBytes = 1 << 16;
void* workspace(Device* d, hipStream_t st, size_t bytes, int* status);

// After a wait on the device: ACCEL_OK, or ACCEL_E_HIP with the message
// naming what a kernel reported in the fault word (which is then cleared,
// together with the workspaces' counters, so later calls start clean).
int take_fault(Device* d);

// ---- the selection report: which kernels a product became -----------------
//
// Every launch site of the int4 products names its kernel, template
// arguments included, the way a profiler's kernel trace shows it.  While the
// calling thread records (LaunchRecord), the names collect in order; while it
// plans without running (dry), nothing is launched and workspace() hands out
// a placeholder address without allocating, so a selection can be asked for
// on a host with no GPU.
struct LaunchRecord {
    explicit LaunchRecord(bool dry);
    ~LaunchRecord();
    std::vector<std::string> names;
    std::string joined() const;   // the launches in order, " + " between them
    LaunchRecord* outer;
    bool dry;
};
// The calling thread's innermost record, or nullptr.
LaunchRecord* launch_record();
inline bool dry_run() {
    const LaunchRecord* r = launch_record();
    return r && r->dry;
}

inline void targ(std::string& s, int v) { s += std::to_string(v); }
inline void targ(std::string& s, bool v) { s += v ? "true" : "false"; }
inline void targ(std::string& s, const char* v) { s += v; }
// "base<a, b, ...>" as a profiler names a template kernel.
template <typename... A>
std::string tname(const char* base, A... args) {
    std::string s = base;
    if constexpr (sizeof...(A) > 0) {
        s += '<';
        bool first = true;
        ((s += first ? "" : ", ", first = false, targ(s, args)), ...);
        s += '>';
    }
    return s;
}
// The grid beside a kernel's name: " [T tiles x S K slices]", " [T tiles]"
// with one slice, " [W workgroups]" with slices 0.
inline std::string grid_note(long long tiles, int slices) {
    if (slices == 0) return " [" + std::to_string(tiles) + " workgroups]";
    std::string s = " [" + std::to_string(tiles) + (tiles == 1 ? " tile" : " tiles");
    if (slices > 1) s += " x " + std::to_string(slices) + " K slices";
    return s + "]";
}
// A template type argument's name as the profiler prints it.
template <typename T> constexpr const char* type_name();
template <> constexpr const char* type_name<float>() { return "float"; }
template <> constexpr const char* type_name<uint16_t>() { return "unsigned short"; }

// A launcher's result: the launch error, or success while planning dry.
inline hipError_t launch_status() { return dry_run() ? hipSuccess : hipGetLastError(); }

// Launch `...` (hipLaunchKernelGGL's arguments) and note NAME in the
// thread's record; under a dry record only the name is noted.  NAME is
// evaluated only while recording.
#define ACCEL_LAUNCH(NAME, ...)                                              \
    do {                                                                     \
        if (::accel::LaunchRecord* rec_ = ::accel::launch_record())          \
            rec_->names.push_back(NAME);                                     \
        if (!::accel::dry_run()) hipLaunchKernelGGL(__VA_ARGS__);            \
    } while (0)

// ---- kernel launchers (defined in the .hip files) ------------------------

struct Int4Planes {
    const uint32_t* codes;
    const uint16_t* scales;
    const uint16_t* zeros;
    // prepared grouped weights: each expert's side copy of its scales and
    // zeros for the matrix-core decode (int4_side_bytes(K, N) apart), or null
    const uint16_t* side = nullptr;
    // or each expert's panel-layout copy (int4_panel_bytes(K, N) rounded up
    // to 256 bytes apart) for the few-rows panel kernel, or null
    const void* panels = nullptr;
    size_t panel_stride = 0;
};

// What the last store of a product does: add bias[col] (f32, one value per
// output column, broadcast over rows) when `bias` is set, then write f32 or,
// with `bf16`, the sum rounded once to bf16 (nearest, ties to even).  The
// default stores the plain f32 sum.
struct Epilogue {
    const float* bias = nullptr;
    bool bf16 = false;
};

// The no-allocation Int4MatVec's static scratch: split-K tickets (the first
// kWorkspaceCounterBytes), then partial sums.  init_scratch resolves this
// device's copy (call with the device current, once per open).
constexpr size_t kScratchBytes = kWorkspaceCounterBytes + (size_t(4) << 20);
int init_scratch(Device* d);
// Int4MatVec (a f32 [K] -> out f32 [N]) with any cross-workgroup buffer
// taken from the static scratch instead of the workspace; refuses
// (ACCEL_E_INVALID) a shape whose split-K sums exceed it.  Allocates nothing.
hipError_t launch_int4_matvec_noalloc(Device* d, hipStream_t st, const float* a, Int4Planes w,
                                      float* out, int K, int N, int* status);

// Decode product, M <= 16 rows of f32 activations -> out (f32, or bf16 with
// ep.bf16).
hipError_t launch_int4_decode_f32(Device* d, hipStream_t st, const float* a,
                                  Int4Planes w, void* out, int M, int K, int N,
                                  int* status, Epilogue ep = Epilogue{});
// One row of bf16 activations (a [1, K] or [K]) -> bf16 out [N] on the VALU
// decode kernel (f32 arithmetic, one rounding); int4_decode_f32_supported(1,
// K, N, codes) limits.
hipError_t launch_int4_decode_bf16_row(Device* d, hipStream_t st, const uint16_t* a,
                                       Int4Planes w, uint16_t* out, int K, int N, int* status,
                                       const float* bias);
// 2..16 rows of bf16 activations (16-byte aligned, K % 32 == 0) -> bf16 out
// [M, N] on the matrix-core decode kernel (f32 arithmetic, one rounding).
bool int4_decode_bf16_rows_supported(int M, int K, int N, const void* a, const void* codes);
hipError_t launch_int4_decode_bf16_rows(Device* d, hipStream_t st, const uint16_t* a,
                                        Int4Planes w, uint16_t* out, int M, int K, int N,
                                        int* status, const float* bias);
// Any shape, f32 activations: one thread per output element (small or ragged
// shapes).
hipError_t launch_int4_generic_f32(hipStream_t st, const float* a, Int4Planes w,
                                   void* out, int M, int K, int N, Epilogue ep = Epilogue{});
// Any shape, bf16 activations and output (ep.bf16 is implied).
hipError_t launch_int4_generic_bf16(hipStream_t st, const uint16_t* a, Int4Planes w,
                                    uint16_t* out, int M, int K, int N,
                                    const float* bias = nullptr);
// Prefill product on MFMA: bf16 activations [M,K] -> bf16 out [M,N].  Products
// with too few tiles to fill the chip split K (f32 sums in the workspace,
// then one reduction pass); *status reports a workspace that cannot grow.
hipError_t launch_int4_gemm_bf16(Device* d, hipStream_t st, const uint16_t* a,
                                 Int4Planes w, uint16_t* out, int M, int K, int N,
                                 const float* bias, int* status);
bool int4_gemm_bf16_supported(int M, int K, int N);
// f32 activations with M > 16 on the bf16 matrix cores to f32 accuracy
// (three-term split of x * 512 s against the exact codes); K % 64 == 0,
// N % 128 == 0 and 16-byte aligned activations.
// Too few tiles to fill the chip split K as the bf16 tiles do.
hipError_t launch_int4_gemm_f32x3(Device* d, hipStream_t st, const float* a,
                                  Int4Planes w, void* out, int M, int K, int N,
                                  Epilogue ep, int* status);
bool int4_gemm_f32x3_supported(int K, int N);
// f32 activations with M > 16, fp32 arithmetic: the other shapes.
hipError_t launch_int4_gemm_f32(Device* d, hipStream_t st, const float* a,
                                Int4Planes w, void* out, int M, int K, int N,
                                Epilogue ep = Epilogue{});
bool int4_decode_f32_supported(int M, int K, int N, const void* codes);
// Int4MatVec of up to four matrices against one f32 vector [K] in one launch
// (all must take the decode kernel: int4_matvec_set_supported).
bool int4_matvec_set_supported(const Int4Planes* w, const int* N, int count, int K);
hipError_t launch_int4_matvec_set(Device* d, hipStream_t st, const float* a, const Int4Planes* w,
                                  float* const* out, const int* N, int count, int K,
                                  int* status);
// The same for M = 2..16 rows of f32 activations on the matrix-core decode
// kernel, each matrix with its own launch's plan.
bool int4_matmul_set_supported(const float* a, const Int4Planes* w, const int* N, int count,
                               int M, int K);
hipError_t launch_int4_matmul_set(Device* d, hipStream_t st, const float* a, const Int4Planes* w,
                                  float* const* out, const int* N, int count, int M, int K,
                                  int* status);

// Grouped products over offsets [E+1] already on the device.
hipError_t launch_segment_offsets(hipStream_t st, const uint32_t* counts,
                                  uint32_t* offsets, int rows);
hipError_t launch_grouped_f32(hipStream_t st, const float* x, const float* w,
                              const uint32_t* off, float* out, int E, int T, int K,
                              int N, bool write_padding);
hipError_t launch_int4_grouped_f32(hipStream_t st, const float* x, Int4Planes w,
                                   const uint32_t* off, float* out, int E, int T,
                                   int K, int N, bool write_padding);
// BASELINE config 1's literal format (32-row groups along K, f32 scale, no
// zero): f32 x [K] -> f32 out [N]; K % 32 == 0, N % 256 == 0.
bool int4_g32_matvec_supported(int K, int N);
hipError_t launch_int4_g32_matvec(Device* d, hipStream_t st, const float* a,
                                  const uint32_t* codes, const float* scales, float* out, int K,
                                  int N, int* status);
// Ragged int4 GEMV (decode MoE): f32 or bf16 x [T, K] (out in the same type),
// T <= kGroupedDecodeRows, each
// row against its expert's [K, N] matrix with the decode kernels (an
// expert's rows in blocks of up to 16 on the matrix cores, in a second launch); the
// matvec form (write_padding) writes 0 to rows past every segment.
constexpr int kGroupedDecodeRows = 64;
// f32 rows take the decode kernels up to this many: past it (and past 64 bf16
// rows, which have the grouped tiles) they run one lane per element.  Measured
// (us, decode kernels / one lane per element), 8 experts of 4096 x 14336, top-2
// routing: 128 rows 173 / 6543, 256 rows 288 / 11139, 512 rows 484 / 20581.
// K is split only while the rows' fewest blocks (ceil(T / 16)) times the
// column tiles leave CUs idle, so the split-K sums stay small: at N = 14336
// (56 tiles of 256 columns) rows past 64 run one slice and take none.
constexpr int kGroupedDecodeRowsF32 = 1024;
// The grouped decode launches take the workspace's counters (`tickets`) and an
// area past the offsets for their split-K sums, of the size
// int4_grouped_decode_area gives for the same x, dtype, w and shape (the
// workspace is sized once, before the offsets are computed, so it cannot grow
// and move them); both plan with the same routing rules.
bool int4_grouped_decode_supported(int T, int K, int N, const void* codes, bool bf16);
size_t int4_grouped_decode_area(const Device* d, const void* x, bool bf16, Int4Planes w, int E,
                                int T, int K, int N);
hipError_t launch_int4_grouped_decode(Device* d, hipStream_t st, const void* x, bool bf16,
                                      Int4Planes w, const uint32_t* off, void* out, int E, int T,
                                      int K, int N, bool write_padding, int* status,
                                      uint32_t* tickets, float* area);
// f32 rows of a grouped int4 product on the matrix cores (the f32 tiles, to
// f32 accuracy) over segment bounds `seg` [E+1] on the device: expert e's
// rows are [seg[e], min(seg[e+1], T)); other rows are not written.  Shape
// limits: int4_gemm_f32x3_supported(K, N) and 16-byte aligned x.  Used past
// the decode kernels' kGroupedDecodeRowsF32 rows: measured at config 4's
// experts (8 x [4096, 14336], top-2), tiles / decode kernels: 256 rows 462 /
// 216 us, 512 rows 471 / 343, 1024 rows 637 / 636 -- a tile's 64 stages cost
// the same for 30 rows as for 128, and an expert of 129..256 rows takes two.
hipError_t launch_int4_grouped_f32x3(hipStream_t st, const float* x, Int4Planes w,
                                     const uint32_t* seg, float* out, int E, int T, int K,
                                     int N);
// The matvec form's segment bounds from the offsets (grouped.hip): bounds[e]
// .. bounds[e+1] are expert e's rows under e(t) = #{r : off[r+1] <= t}; the
// offsets themselves when their sum did not wrap.
hipError_t launch_segment_bounds(hipStream_t st, const uint32_t* off, uint32_t* bounds, int E);
hipError_t launch_zero_tail_f32(hipStream_t st, const uint32_t* off, float* out, int E, int T,
                                int N);
hipError_t launch_int4_grouped_bf16(Device* d, hipStream_t st, const uint16_t* x,
                                    Int4Planes w, const uint32_t* off, uint16_t* out,
                                    int E, int T, int K, int N, bool write_padding);

// Prepared (bind-time) weights for one-row products: the planes copied into
// 16-column K-major panels and per-group scale/zero rows (panel.hip).
bool int4_panel_supported(int64_t K, int64_t N);
size_t int4_panel_bytes(int K, int N, size_t* sz_offset);
hipError_t launch_int4_panel_prepare(hipStream_t st, Int4Planes w, void* dst, int K, int N);
// a f32 [K] -> out[i] [N[i]] (f32, or bf16 with ep.bf16) over `count` (1..4)
// prepared matrices of K rows, in one launch.
constexpr int kMaxPreparedSet = 4;
// Prepared weights for the matrix-core decode: the codes in the reference
// order and a side copy of the scales and zeros, one contiguous block per
// (group, 32-row step).  K % 32 == 0 and N % 128 == 0.
bool int4_side_supported(int64_t K, int64_t N);
size_t int4_side_bytes(int K, int N);
hipError_t launch_int4_side_prepare(hipStream_t st, Int4Planes w, uint16_t* side, int K, int N);
bool int4_decode_side_rows_supported(int M, const float* a);
hipError_t launch_int4_decode_side(Device* d, hipStream_t st, const float* a,
                                   const uint32_t* const* codes, const uint16_t* const* side,
                                   float* const* out, const int* N, int count, int M, int K,
                                   int* status);
// M rows of a ([M, K], K even, rows 8-byte aligned) against count (1..4)
// prepared matrices of K rows, out[i] [M, N[i]], in passes of up to eight
// rows.
bool int4_panel_rows_supported(int M, int K, const float* a);
hipError_t launch_int4_panel_rows(hipStream_t st, const float* a, int M,
                                  const void* const* prepared, void* const* out, const int* N,
                                  int count, int K, Epilogue ep);
hipError_t launch_int4_panel_matvec(hipStream_t st, const float* a, const void* const* prepared,
                                    void* const* out, const int* N, int count, int K,
                                    Epilogue ep);
// out [N] = SwiGLU(a . gate, a . up) (internal/kernels/elementwise.go:85-91)
// for two prepared [K, N] matrices, one launch.
hipError_t launch_int4_panel_swiglu(hipStream_t st, const float* a, const void* gate,
                                    const void* up, float* out, int N, int K);
// The ragged GEMV on experts prepared into the panel layout, stride bytes
// apart: x f32 [T, K], K even, x 8-byte aligned, sorted offsets.
hipError_t launch_int4_grouped_panel_rows(hipStream_t st, const float* x, const void* panels_base,
                                          size_t stride, const uint32_t* off, float* out, int E,
                                          int T, int K, int N);
// Whether the grouped decode product takes the panel kernel for these rows
// (w.panels set, f32 rows, 3 <= T < 2E and T <= 64, K even, x 8-byte
// aligned).
bool grouped_panel_route(const void* x, Int4Planes w, bool bf16, int E, int T, int K);

// Decode-step neighbours: MatVecF32F16 (f32 a [K], f16 w [K,N] -> f32 [N]),
// SwiGLU over n elements, RMSNorm over `rows` rows of `width`.
hipError_t launch_matvec_f32_f16(Device* d, hipStream_t st, const float* a, const uint16_t* w,
                                 float* out, int K, int N, int* status);
hipError_t launch_swiglu(hipStream_t st, const float* a, const float* b, float* out, int64_t n);
hipError_t launch_rmsnorm(hipStream_t st, const float* x, const float* w, float* out, int rows,
                          int width, float eps);

// int8 weights (one f16 scale per 32 flat weights): a [M,K] f32 or f16 bits
// -> f32 [M,N].
hipError_t launch_int8_product(Device* d, hipStream_t st, const void* a, bool f16_act,
                               const int8_t* quants, const uint16_t* scales, float* out, int M,
                               int K, int N, int* status);

// Device quantizer.
hipError_t launch_int4_quantize(hipStream_t st, const float* w, int64_t n,
                                uint32_t* packed, uint16_t* scales, uint16_t* zeros);

// Host quantizer shared by the C entry point.
void int4_quantize_host(const float* w, int64_t n, uint32_t* packed, uint16_t* scales,
                        uint16_t* zeros);
void int4_dequantize_host(const uint32_t* packed, const uint16_t* scales,
                          const uint16_t* zeros, int64_t n, float* out);

}  // namespace accel
