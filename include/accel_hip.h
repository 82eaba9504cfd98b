/*
 * accel_hip.h -- C ABI of libaccel_hip.so, the MI355X (gfx950) backend for
 * golang-design/accel's int4 weight-only linear path.
 *
 * Two layers are exported.
 *
 *  1. The backend seam.  What the reference's internal/driver interfaces ask
 *     of a backend (Adapter, Device, Block, Executable, Fence, Timer,
 *     KernelSupport), as plain functions over opaque handles, so a Go
 *     internal/hip package can bind them with purego the way
 *     internal/metal binds Metal.  A dispatch names a reference kernel record
 *     (e.g. "QuantMatVecInt4") and passes its bindings in record order plus
 *     the std140 uniform bytes; the library picks the gfx950 kernel.
 *
 *  2. The operator layer.  The tensor-package entry points of the path
 *     (tensor.Int4MatVec, Int4MatMul, GroupedMatVec, GroupedMatMul, the
 *     SegmentOffsets node and quant.Int4Quantize), with the reference's
 *     validation and refusal messages, over device pointers.
 *
 * Conventions.  Every function returns an int status: ACCEL_OK (0) or a
 * negative ACCEL_E_* code, with a message for the calling thread in
 * accel_hip_last_error().  No C++ exception crosses this boundary.  Device
 * pointers are those returned by accel_hip_alloc (or any hipMalloc'd
 * memory of the same device).  A stream argument may be NULL for the
 * device's null stream.  Dtype codes: ACCEL_F32, ACCEL_F16, ACCEL_BF16,
 * ACCEL_U32.  Half-precision values cross the ABI as uint16_t bit patterns,
 * as the reference moves them ("The host slice for an f16 buffer is
 * []uint16", internal/kernels/differential_darwin_test.go:242-244).
 *
 * Workspace.  Kernels that reduce across workgroups (the decode product's
 * K split) and the grouped products (segment offsets, tile lists) use a
 * per-device workspace owned by the library.  Two operator calls that run
 * concurrently on different streams of one device race on it; serialize
 * them or use one stream per device.  The workspace grows on demand outside
 * graph capture; a call that would need it to grow on a capturing stream is
 * refused (ACCEL_E_INVALID).  When it grows, a workspace that a live
 * executable still names is kept until that executable is destroyed, so an
 * executable stays valid across later, larger eager calls.
 *
 * Faults.  A kernel that gives up instead of producing its result (a
 * split-K hand-off whose bounded wait runs out) records it in the device's
 * fault word; the next
 * stream_sync, event_sync or event_query that completes reports it as
 * ACCEL_E_HIP with a message, and clears it (the analogue of the
 * reference's per-node fault words read back by Fence.Wait,
 * internal/metal/exec_darwin.go:46-53,822-826).
 */
#ifndef ACCEL_HIP_H
#define ACCEL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define ACCEL_OK 0
#define ACCEL_E_INVALID (-1)     /* refused by validation (tensor layer b.fail) */
#define ACCEL_E_NO_DEVICE (-2)   /* no such device, or device not open */
#define ACCEL_E_DEVICE_LOST (-3) /* sticky: driver.ErrDeviceLost */
#define ACCEL_E_OOM (-4)         /* allocation failed; not loss */
#define ACCEL_E_UNSUPPORTED (-5) /* kernel record with no gfx950 artifact */
#define ACCEL_E_HIP (-6)         /* other HIP runtime error */

/* ---- dtypes (the reference's accel.DType subset on this path) ----------- */
#define ACCEL_F32 1
#define ACCEL_F16 2
#define ACCEL_BF16 3
#define ACCEL_U32 4
#define ACCEL_I8 5

/* Message for the last failing call on this thread ("" if none). */
const char* accel_hip_last_error(void);

/* ABI version: bumped on any incompatible change of this header. */
int accel_hip_abi_version(void);

/* ===================================================================== */
/* 1. Backend seam                                                       */
/* ===================================================================== */

/* Adapter.Info (internal/driver/driver.go:149-160) plus the figures the
 * roofline needs. */
typedef struct accel_hip_info {
    char name[128];          /* marketing name */
    char arch[64];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int32_t compute_units;
    int32_t wavefront;       /* 64 on CDNA */
    int32_t lds_per_block;   /* bytes of LDS a workgroup may use */
    int32_t clock_khz;       /* peak shader clock */
    int32_t mem_clock_khz;
    int32_t mem_bus_bits;
    uint64_t hbm_bytes;
    int32_t l2_bytes;
    int32_t pci_bus;
} accel_hip_info_t;

/* Number of HIP devices; 0 (and ACCEL_OK) where there is no GPU.  Replaces
 * platformAdapters' enumeration (adapters_other.go:18, device.go:48-52). */
int accel_hip_probe(int* count);
int accel_hip_info(int dev, accel_hip_info_t* out);

/* Adapter.Open / Device.Close (driver.go:149-190).  open sets the device
 * current for the calling thread and creates the per-device state;
 * close frees the workspace.  Both are idempotent. */
int accel_hip_open(int dev);
int accel_hip_close(int dev);

/* Device.Lost (driver.go:178-186): 1 once the device is lost, for good
 * (internal/driver/plan.go:385-391), else 0. */
int accel_hip_lost(int dev);

/* Fault injection, the analogue of CPUOptions.LoseAtSubmission
 * (accel.go:306-314; internal/cpu/cpu.go:179-191): the device is marked lost
 * when the n-th accepted submission (counting from 1, from now) begins, and
 * that submission launches nothing.  0 disables. */
int accel_hip_inject_loss(int dev, int64_t at_submission);

/* Device.Alloc / Block.Free / Block.Write / Block.Read
 * (driver.go:163-238).  write and read are synchronous with the device. */
int accel_hip_alloc(int dev, size_t bytes, void** ptr);
int accel_hip_free(int dev, void* ptr);
int accel_hip_write(int dev, void* dst, size_t offset, const void* src, size_t bytes);
int accel_hip_read(int dev, const void* src, size_t offset, void* dst, size_t bytes);
/* Plan copy node (internal/driver/plan.go:112-140), stream-ordered. */
int accel_hip_copy(int dev, void* stream, void* dst, const void* src, size_t bytes);

/* Streams: one per in-flight submission (Executable.Submit must not wait,
 * plan.go:360-371). */
int accel_hip_stream_create(int dev, void** stream);
int accel_hip_stream_destroy(int dev, void* stream);
int accel_hip_stream_sync(int dev, void* stream);

/* Fence (plan.go:374-383) and Timer (plan.go:349-353) as HIP events. */
int accel_hip_event_create(int dev, void** event);
int accel_hip_event_destroy(int dev, void* event);
int accel_hip_event_record(int dev, void* event, void* stream);
/* 1 = done (a lost device is done), 0 = pending, <0 = error (including a
 * fault a kernel reported; see Faults above). */
int accel_hip_event_query(int dev, void* event);
int accel_hip_event_sync(int dev, void* event);
int accel_hip_event_elapsed(int dev, void* start, void* end, float* ms);

/* Executable (plan.go:360-371) as a HIP graph.  Operator calls and
 * dispatches issued on `stream` between capture_begin and capture_end are
 * recorded, not run; exec_launch replays them as one submission (the
 * reference's resubmittable compiled plan, GraphCompiler.Compile,
 * plan.go:398-400).  Issue every captured call once eagerly before capturing,
 * so the workspace it needs is already allocated (a call that would grow it
 * inside the capture is refused).  An executable records the workspace it
 * was captured against; that workspace lives until the executable is
 * destroyed. */
int accel_hip_capture_begin(int dev, void* stream);
int accel_hip_capture_end(int dev, void* stream, void** exec);
int accel_hip_exec_launch(int dev, void* exec, void* stream);
int accel_hip_exec_destroy(int dev, void* exec);

/* Test and diagnostic hooks; no reference counterpart.
 *  set_wait_limit: the spins a split-K hand-off's bounded wait may take
 *    before it gives up and reports kFault "wait gave up" (default 1 << 22;
 *    0 makes every such wait give up at once, so a test can force the fault
 *    from the host while every kernel still exits normally).
 *  workspace_generation: how many times the workspace has been allocated,
 *    and how many replaced workspaces live executables still hold. */
int accel_hip_set_wait_limit(int dev, int32_t spins);
/* Launch-floor probes for the roofline's ceiling, with the M = 1 decode
 * kernel's launch shape (256 workgroups of 512 lanes): kind 0 launches an
 * empty kernel; kind 1 reads `bytes` (a multiple of 16, at most 16 MiB) from
 * the 16-byte aligned device pointer `src` with 16-byte loads, all of a
 * lane's issued before any is used; kind 2 reads `bytes` (a multiple of 16,
 * any size) from `src` with a grid-stride loop, which evicts the device's
 * caches with clean lines (a copy would leave dirty lines whose writeback
 * lands in the work after it).  `sink` is a device buffer of at least 1 KiB
 * the read kernels may write.  Diagnostics for the benchmark. */
int accel_hip_floor(int dev, void* stream, int kind, const void* src, size_t bytes, void* sink);
int accel_hip_workspace_generation(int dev, uint64_t* gen, int32_t* retired);

/* KernelSupport.SupportsKernel (plan.go:424-428): 1 if the named reference
 * kernel record has a gfx950 implementation here, else 0.  Records without
 * one are refused; nothing falls back to another implementation
 * (the rule at internal/metal/exec_darwin.go:140-149). */
int accel_hip_supports_kernel(const char* kernel);

/* One PlanNode{Op: OpDispatch} (plan.go:112-201): the kernel record's name,
 * its bindings as device pointers in record order with their element counts
 * (the `_lens` words, internal/metal/exec_darwin.go:494-528), and its std140
 * uniform block.  count is Dispatch.Count, advisory: the library chooses
 * its own grid.  Supported records and their binding orders:
 *   QuantMatVecInt4  a f32, bq u32, bs f16, bz f16, out f32; GEMMDims
 *   QuantMatMulInt4  a f32, bq u32, bs f16, bz f16, out f32; GEMMDims
 *   GroupedMatVec    x f32, w f32, offsets u32, out f32;      GroupedDims
 *   GroupedMatMul    x f32, w f32, offsets u32, out f32;      GroupedTiledDims
 *   SegmentOffsets   counts u32, offsets u32;                 SegmentDims
 *   SwiGLU           a f32, b f32, out f32;                   (no uniform)
 *   RMSNorm          x f32, w f32, out f32;                   RowDims
 *   MatVecF32F16     a f32, b f16, out f32;                   GEMMDims
 *   QuantMatVecF32   a f32, bq i8, bs f16, out f32;           GEMMDims (M = 1)
 *   QuantMatVec      a f16, bq i8, bs f16, out f32;           GEMMDims (M = 1)
 *   QuantMatMulTiledF32  a f32, bq i8, bs f16, out f32;       GEMMDims
 *   QuantMatMulTiled     a f16, bq i8, bs f16, out f32;       GEMMDims
 * (internal/kernels/accel_kernels.go:6799-6808,7052-7061; GEMMDims is
 * {M@0,N@4,K@8}, GroupedDims {Experts@0,K@4,N@8}, GroupedTiledDims
 * {Experts@0,Tokens@4,K@8,N@12}, SegmentDims {Rows@0}, :173-231; RowDims
 * {Rows@0,Width@4,Eps@8 f32}, internal/kernels/norm.go:13-22; SwiGLU's length
 * is out's, elementwise.go:85-91). */
int accel_hip_dispatch(int dev, void* stream, const char* kernel,
                       const void* const* bindings, const uint64_t* lens,
                       int32_t nbindings, const void* uniform, size_t uniform_bytes,
                       const uint32_t count[3]);

/* ===================================================================== */
/* 2. Operator layer                                                     */
/* ===================================================================== */

/* A device tensor: data pointer, dtype and row-major shape. */
typedef struct accel_tensor {
    void* data;
    int32_t dtype;
    int32_t rank;
    int64_t shape[4];
} accel_tensor_t;

/* tensor.Int4 (tensor/int4.go:25-38): packed u32 codes (eight weights per
 * word, low nibble first), f16 scales and zeros (one each per 128 weights of
 * the flattened [K,N] matrix), and the weight count.  Element counts, not
 * bytes. */
typedef struct accel_int4 {
    const uint32_t* codes;
    int64_t codes_len;
    const uint16_t* scales;
    int64_t scales_len;
    const uint16_t* zeros;
    int64_t zeros_len;
    int64_t weights;
} accel_int4_t;

/* A published 4-bit checkpoint layer (specs/048-int4.md:126-131,167 name
 * reading these files as the unbuilt next step of the int4 format).  Both
 * families keep one f16 scale and one 4-bit zero per output column per group
 * of `group_size` input rows, w(k,n) = (q(k,n) - z(g,n)) * s(g,n), where the
 * reference format keeps one scale and zero per 128 consecutive weights of the
 * flat [K,N] array; a repack therefore re-quantizes.
 *   ACCEL_QFMT_AWQ      AutoAWQ "gemm" packing: qweight u32 [K, N/8], eight
 *                       columns a word with column 8j+c in nibble
 *                       {0,4,1,5,2,6,3,7}[c]; qzeros u32 [groups, N/8] packed
 *                       the same way; scales f16 [groups, N]; g = k / group.
 *   ACCEL_QFMT_GPTQ     GPTQ ("gptq" checkpoint format): qweight u32 [K/8, N],
 *                       row 8i+j in nibble j of word (i, n); qzeros u32
 *                       [groups, N/8], column 8j+c in nibble c, holding z - 1;
 *                       scales f16 [groups, N]; g = g_idx[k] when g_idx is
 *                       given (act-order), else k / group.
 *   ACCEL_QFMT_GPTQ_V2  as GPTQ, with qzeros holding z itself ("gptq_v2"). */
#define ACCEL_QFMT_AWQ 1
#define ACCEL_QFMT_GPTQ 2
#define ACCEL_QFMT_GPTQ_V2 3
typedef struct {
    int32_t format;
    int32_t group_size;      /* input rows a group spans; K for a single group */
    int64_t K, N;            /* in_features, out_features */
    int64_t groups;          /* rows of scales and qzeros */
    const uint32_t* qweight;
    const uint32_t* qzeros;
    const uint16_t* scales;
    const int32_t* g_idx;    /* GPTQ only: [K] group of each input row, or NULL */
} accel_foreign_int4_t;

/* Repacks a published 4-bit layer into the reference int4 format
 * (quant/int4.go:71-138 applied to the layer's dequantized [K,N] weights):
 * every weight is dequantized exactly in f32, (q - z) * s, and each group of
 * 128 consecutive flat weights is quantized by the reference's Int4Quantize.
 * Where a reference group's weights share one published (scale, zero) and use
 * the full code range the repack is lossless (codes, scale and zero come back
 * exactly); elsewhere the second rounding is bounded by Int4ErrorBound.
 * Host memory: codes [ceil(K*N/8)], scales and zeros [ceil(K*N/128)].
 * Refused: an unknown format, N % 8 != 0, GPTQ with K % 8 != 0, AWQ with K
 * not a multiple of group_size, groups that do not cover K, or a g_idx entry
 * outside [0, groups). */
int accel_int4_repack_host(const accel_foreign_int4_t* src, uint32_t* codes,
                           uint16_t* scales, uint16_t* zeros);

/* The same repack on the device, bit-identical to the host's: src's planes
 * and dst's (weights = K*N) are device memory.  One wave per reference group,
 * dequantizing its 128 weights from the published planes in registers and
 * quantizing them with the device Int4Quantize.  A g_idx entry outside
 * [0, groups) is reported as ACCEL_E_INVALID after the stream is synchronized
 * (the call waits for the repack, a load-time operation). */
int accel_int4_repack(int dev, void* stream, const accel_foreign_int4_t* src,
                      accel_int4_t* dst);

/* tensor.Int4MatVec (tensor/int4.go:99-147): out[n] = sum_k a[k] * w(k,n),
 * w = s==0 ? z : (code-z)*s.  a is f32 [K]; out is f32 [N], N = weights/K. */
int accel_int4_matvec(int dev, void* stream, const accel_tensor_t* a,
                      const accel_int4_t* w, accel_tensor_t* out);

/* BASELINE config 1's literal weight format, an additive variant with no
 * counterpart in the reference (whose groups are 128 flat weights with an f16
 * scale and an f16 zero, quant/int4.go:29,71-138): groups of 32 rows of one
 * column along K, one f32 scale per group, no zero point.  codes are packed
 * as quant/int4 packs them (element k*N + n is nibble (k*N+n) % 8 of word
 * (k*N+n) / 8, low nibble first, quant/int4.go:141-153); scales is [K/32, N];
 * w = (q - 8) * s.  Reported separately from the reference format. */
typedef struct accel_int4_g32 {
    const uint32_t* codes;   /* K*N/8 words */
    const float* scales;     /* K/32 * N */
    int64_t K, N;
} accel_int4_g32_t;

/* Host packer of that format: s = f32(amax / 7) over the group (0 for a
 * group of zeros), q = clamp(rne(f32(w / s)), -8, 7) + 8.  w is [K, N] f32,
 * finite; K % 32 == 0, K*N % 8 == 0. */
int accel_int4_g32_quantize(const float* w, int64_t K, int64_t N, uint32_t* packed,
                            float* scales);

/* out[N] = a[K] @ w for the format above, f32 activations and result
 * (Int4MatVec's shape and checks on a and out); K % 32 == 0, N % 256 == 0. */
int accel_int4_g32_matvec(int dev, void* stream, const accel_tensor_t* a,
                          const accel_int4_g32_t* w, accel_tensor_t* out);

/* Int4MatVec that allocates nothing: the same checks, kernels and results
 * (bit for bit) as accel_int4_matvec, with the K-split's tickets and partial
 * sums in a static device array of 4 MiB + 64 KiB that every GPU the library
 * runs on holds until the process ends, instead of the workspace (which may
 * call hipMalloc to grow).  No counterpart in the reference: it is for
 * callers that cannot allocate (code under graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Refused (ACCEL_E_INVALID) when the
 * shape's split-K sums exceed 4 MiB: slices * N * 4 > 4 MiB, where the
 * column tile is 512 for N >= 8192 with N % 512 == 0 (slices =
 * min(64, ceil(K / 128))), else 256 for N % 256 == 0 (slices =
 * min(64, ceil(K / 256))), else 128 (slices = min(64, ceil(K / 512))).
 * So N <= 16384 passes at any K, and a 4096 x 128256 LM head (256-
 * column tiles, 16 slices, 8.2 MB of sums) is refused; accel_int4_select
 * answers the same question without running anything.  Calls that overlap
 * on one GPU share the array and race; serialize them. */
int accel_int4_matvec_noalloc(int dev, void* stream, const accel_tensor_t* a,
                              const accel_int4_t* w, accel_tensor_t* out);

/* Int4MatVec over `count` (1..4) matrices w[i] that share one f32 vector a
 * [K], out[i] f32 [N_i], in one launch per tile width (N_i a multiple of 256,
 * or of 128 only) where every matrix takes the decode kernel (N_i a multiple
 * of 128, 16-byte aligned codes), else one launch each.
 * Each out[i] is exactly Int4MatVec(a, w[i]).  No reference counterpart as
 * one call: it is the plan-level merge of the reference's separate
 * Int4MatVec dispatches that read the same activations (a decode step's q, k,
 * v and gate, up), with Int4MatVec's checks and wording per matrix. */
int accel_int4_matvec_set(int dev, void* stream, const accel_tensor_t* a,
                          const accel_int4_t* w, accel_tensor_t* out, int count);

/* The same for f32 rows a [M,K] and out[i] f32 [M,N_i] (Int4MatMul's checks
 * per matrix): M = 1 as above; 2 <= M <= 16 with K % 32 == 0 and 16-byte
 * aligned a on the matrix-core decode kernel, one launch per tile width, each
 * matrix with the plan its own launch takes, so out[i] is exactly
 * Int4MatMul(a, w[i]); other shapes one Int4MatMul each. */
int accel_int4_matmul_set(int dev, void* stream, const accel_tensor_t* a,
                          const accel_int4_t* w, accel_tensor_t* out, int count);

/* tensor.Int4MatMul (tensor/int4.go:168-212): a [M,K] -> out [M,N].  The
 * reference takes f32 a and gives f32 out; this also accepts bf16 a with bf16
 * out (fp32 accumulation), the additive dtype selection QuantMatMul makes by
 * activation dtype (tensor/quantized.go:87-113).  M <= 16 runs the decode
 * kernels; larger M the MFMA kernels. */
int accel_int4_matmul(int dev, void* stream, const accel_tensor_t* a,
                      const accel_int4_t* w, accel_tensor_t* out);

/* The int4 analogue of tensor.Linear (tensor/matmul.go:184-225, kernel
 * LinearTiled, internal/kernels/matvec.go:232-293): x [K] or [M,K] times the
 * int4 matrix, plus bias[n] (f32 [N], broadcast over rows) added once to each
 * f32 sum in the product's own epilogue, in place of Int4MatMul followed by
 * an Add (and a cast) node.  x is f32 or bf16; out is f32 or bf16 for f32 x
 * (a bf16 out is the f32 sum plus bias rounded once), bf16 for bf16 x.  bias
 * may be NULL: the epilogue then only narrows.  Refusals follow Linear's:
 * a non-f32 bias, or one that is not [N]. */
int accel_int4_linear(int dev, void* stream, const accel_tensor_t* x,
                      const accel_int4_t* w, const accel_tensor_t* bias,
                      accel_tensor_t* out);

/* A weight bound for one-row products (opaque; owned by the caller).  The
 * reference binds a tensor.Int4's planes to a plan once
 * (tensor/int4.go:82-127: Int4 is a Weight of the graph) and runs them many
 * times; a backend may keep its own copy of a bound weight in the layout its
 * kernels read best.  This one is K-major panels of 16 columns (each row's
 * 8 code bytes, rows in pairs) with each group's f16 scale and zero side by
 * side per row: one workgroup then owns a column strip over all of K, and
 * the decode kernel's K split and its hand-off are gone.  The reference
 * planes are not changed and stay the format everything else reads. */
typedef struct accel_int4_prepared accel_int4_prepared_t;

/* Copies w ([K, N] in the reference format: N % 128 == 0, 8-byte aligned
 * codes) into a new device allocation in the panel layout, on `stream`, and
 * waits for the copy.  The same bytes as the planes (plus one padding row
 * for odd K).  No reference counterpart as one call: it is what a backend's
 * GraphCompiler.Compile (internal/driver/plan.go:398-400) would do for an
 * Int4 weight operand of a QuantMatVecInt4 node. */
int accel_int4_prepare(int dev, void* stream, const accel_int4_t* w, int64_t K, int64_t N,
                       accel_int4_prepared_t** out);
/* The same for the matrix-core decode (2..16 rows, and one): the code plane
 * copied as it is and a side copy of the scales and zeros, one contiguous
 * block per (128-column group, 32-row step), so a step's scales and zeros are
 * one load, not a piece of each of its 32 rows of the planes.  K % 32 == 0,
 * N % 128 == 0.  The same bytes as the planes.  A weight prepared this way
 * serves accel_int4_matmul_prepared[_set] (passes of 16 rows past 16) and
 * accel_int4_matvec_prepared[_set] through the matrix-core decode kernel,
 * which then takes 16-byte aligned activations; past one row its results
 * are accel_int4_matmul's on the planes bit for bit. */
int accel_int4_prepare_tiles(int dev, void* stream, const accel_int4_t* w, int64_t K,
                             int64_t N, accel_int4_prepared_t** out);
int accel_int4_prepared_free(int dev, accel_int4_prepared_t* w);
/* Device bytes the prepared copy holds. */
int accel_int4_prepared_bytes(const accel_int4_prepared_t* w, uint64_t* bytes);

/* tensor.Int4MatVec (tensor/int4.go:99-147) over a prepared weight: a f32
 * [K] -> out f32 [N], the same arithmetic per weight as accel_int4_matvec
 * (within f32 rounding of it: the sums are added in another order).  One
 * launch; allocates nothing. */
int accel_int4_matvec_prepared(int dev, void* stream, const accel_tensor_t* a,
                               const accel_int4_prepared_t* w, accel_tensor_t* out);

/* The same over `count` (1..4) prepared weights of K rows that share one f32
 * vector a [K], out[i] f32 [N_i], in one launch; each out[i] is exactly
 * accel_int4_matvec_prepared(a, w[i]).  No reference counterpart as one
 * call: the plan-level merge of Int4MatVec dispatches that read the same
 * activations (a decode step's q, k, v and gate, up). */
int accel_int4_matvec_prepared_set(int dev, void* stream, const accel_tensor_t* a,
                                   const accel_int4_prepared_t* const* w, accel_tensor_t* out,
                                   int count);

/* SwiGLU of two one-row products that share a [K] (a decode step's gate and
 * up projections), out f32 [N] = SwiGLU(a . gate, a . up) with tensor.SwiGLU
 * (tensor/elementwise.go:161-188; kernel internal/kernels/elementwise.go:
 * 85-91), gate and up [K, N] prepared by accel_int4_prepare.  Equal bit for
 * bit to accel_int4_matvec_prepared_set(a, {gate, up}) followed by
 * accel_swiglu, in one launch: the two products' results never reach memory.
 * No reference counterpart as one call: the plan-level fusion of the two
 * QuantMatVecInt4 dispatches with the SwiGLU dispatch that reads them. */
int accel_int4_matvec_prepared_swiglu(int dev, void* stream, const accel_tensor_t* a,
                                      const accel_int4_prepared_t* gate,
                                      const accel_int4_prepared_t* up, accel_tensor_t* out);

/* tensor.Int4MatMul (tensor/int4.go:168-212) over a prepared weight: a f32
 * [M, K] -> out f32 [M, N], within f32 rounding of accel_int4_matmul (the
 * sums are added in another order).  One row is accel_int4_matvec_prepared
 * bit for bit; 2..8 rows are one launch of the rows kernel (every row against
 * each panel, no K split), more rows passes of eight.  Past one row, K must be
 * even and a's rows 8-byte aligned.  Allocates nothing.  Faster than
 * accel_int4_matmul on the planes at two rows (4096 x 14336: 11.9 against
 * 16.4 us), about even at four, slower at eight (37.2 against 16.9): a panel
 * re-reads every row's activations. */
int accel_int4_matmul_prepared(int dev, void* stream, const accel_tensor_t* a,
                               const accel_int4_prepared_t* w, accel_tensor_t* out);

/* The same over `count` (1..4) prepared weights of K rows that share a
 * [M, K], out[i] f32 [M, N_i], in one launch a pass; each out[i] is exactly
 * accel_int4_matmul_prepared(a, w[i]).  No reference counterpart as one
 * call: the plan-level merge of Int4MatMul dispatches that read the same
 * activations (a decode step's q, k, v and gate, up at batch M). */
int accel_int4_matmul_prepared_set(int dev, void* stream, const accel_tensor_t* a,
                                   const accel_int4_prepared_t* const* w, accel_tensor_t* out,
                                   int count);

/* Which kernel an operator became, and why: KernelSelection{Op, Kernel,
 * Reason, Rejected} (tensor/compile.go:36-42), as Plan.Selections reports it
 * (tensor/plan.go:36-41), for the int4 products.  kernel lists the launches
 * in order, " + " between them, each named as a profiler's kernel trace
 * names it (template arguments included) with its grid in brackets;
 * rejected lists the routes turned down, each with its reason, "; " between
 * them.  Strings are NUL-terminated and cut to fit. */
typedef struct accel_selection {
    char op[32];
    char kernel[320];
    char reason[320];
    char rejected[1024];
} accel_selection_t;

#define ACCEL_SELECT_BIAS 1       /* the product adds a bias (Int4Linear) */
#define ACCEL_SELECT_BF16_OUT 2   /* f32 rows with a bf16 result (Int4Linear) */

/* The selection an int4 product of [M, K] x [K, N] with activations of
 * `dtype` (ACCEL_F32 or ACCEL_BF16) at `a` over the planes of `w` would
 * make on device dev, planned without launching or allocating anything (the
 * addresses matter only for their alignment; NULL a or w: 256-byte aligned).
 * dev < 0 plans for an MI355X as this library models it (256 CUs), so the
 * question can be asked on a host without a GPU.  op is "Int4MatVec",
 * "Int4MatMul", "Int4Linear", "Int4MatVecPrepared", "Int4MatMulPrepared",
 * "Int4MatMulPreparedTiles" or "Int4MatVecNoAlloc"
 * (NULL: Int4MatVec for
 * M = 1, else Int4MatMul); flags are ACCEL_SELECT_*.  For Int4MatVecNoAlloc
 * it returns that entry point's refusal (ACCEL_E_INVALID) for a shape whose
 * split-K sums exceed its static scratch, so a caller can ask before it
 * captures.  No reference counterpart as one call: the reference reports a
 * selection only from a compiled plan. */
int accel_int4_select(int dev, const char* op, int32_t dtype, int64_t M, int64_t K, int64_t N,
                      const void* a, const accel_int4_t* w, int32_t flags,
                      accel_selection_t* sel);

/* The selection the last int4 product on device dev made (Int4MatVec,
 * Int4MatMul, Int4Linear, the sets, the prepared products, the grouped
 * products and Int4MatVecNoAlloc), as launched; ACCEL_E_INVALID before the
 * first. */
int accel_hip_last_selection(int dev, accel_selection_t* sel);

/* The SegmentOffsets node (tensor/segment.go:31-50;
 * internal/kernels/segment.go:40-50): offsets[r] = sum of counts[<r],
 * offsets[rows] = total.  counts u32 [rows], offsets u32 [rows+1]. */
int accel_segment_offsets(int dev, void* stream, const accel_tensor_t* counts,
                          accel_tensor_t* offsets);

/* tensor.GroupedMatVec (tensor/grouped.go:48-115): x f32 [T,K], w f32
 * [E,K,N], counts u32 [E] -> out f32 [T,N]; token t uses expert
 * e(t) = #{r : off[r+1] <= t}; a token past the last segment is written 0. */
int accel_grouped_matvec(int dev, void* stream, const accel_tensor_t* x,
                         const accel_tensor_t* w, const accel_tensor_t* counts,
                         accel_tensor_t* out);

/* tensor.GroupedMatMul (tensor/grouped.go:138-212): same operands; rows
 * [off[e], min(off[e+1], T)) use expert e and rows outside every segment are
 * left as they were. */
int accel_grouped_matmul(int dev, void* stream, const accel_tensor_t* x,
                         const accel_tensor_t* w, const accel_tensor_t* counts,
                         accel_tensor_t* out);

/* The int4 composition of the two grouped operators: the weight is
 * `experts` stacked [K,N] int4 matrices quantized as one flat [E,K,N] array
 * (groups never straddle experts when K*N % 128 == 0, which is required).
 * x is f32 or bf16 [T,K]; out matches x's dtype, [T,N].  The matvec form
 * writes 0 past the last segment (grouped.go:66-77); the matmul form leaves
 * such rows unwritten (groupedtiled.go:87-132). */
int accel_int4_grouped_matvec(int dev, void* stream, const accel_tensor_t* x,
                              const accel_int4_t* w, int64_t experts,
                              const accel_tensor_t* counts, accel_tensor_t* out);
int accel_int4_grouped_matmul(int dev, void* stream, const accel_tensor_t* x,
                              const accel_int4_t* w, int64_t experts,
                              const accel_tensor_t* counts, accel_tensor_t* out);

/* The grouped int4 weight bound once for routed decode rows: the three
 * planes copied as they are and, after them, each expert's side copy of its
 * scales and zeros (the layout of accel_int4_prepare_tiles, one expert after
 * another), so a matrix-core decode step reads its scales and zeros as one
 * load.  `experts` stacked [K,N]; K % 32 == 0, N % 128 == 0, N < 2^27.  The
 * copy holds the planes' bytes twice over the scales and zeros (about 1.06x
 * the planes).  No reference counterpart as one call: what a backend's
 * GraphCompiler.Compile (internal/driver/plan.go:398-400) would do for the
 * Int4 weight operand of a grouped node.  Freed with
 * accel_int4_prepared_free; the single-matrix prepared operators refuse it. */
int accel_int4_prepare_grouped(int dev, void* stream, const accel_int4_t* w, int64_t experts,
                               int64_t K, int64_t N, accel_int4_prepared_t** out);
/* The same experts bound for the decode MoE's few routed rows: the three
 * planes copied as they are and, after them, each expert's copy in
 * accel_int4_prepare's panel layout (2x the planes' bytes).  The grouped
 * products then take f32 rows, three or more and fewer than two an expert
 * on average (K even, rows 8-byte aligned), on the few-rows panel kernel: one
 * workgroup an (expert, 16-column panel), K whole, no hand-off; within the
 * f32 tolerance of the planes' products (the sums run in another order),
 * not bit for bit.  Other rows take the planes' routes.  N % 128 == 0,
 * 8-byte aligned codes.  No reference counterpart as one call (as
 * accel_int4_prepare_grouped). */
int accel_int4_prepare_grouped_panels(int dev, void* stream, const accel_int4_t* w,
                                      int64_t experts, int64_t K, int64_t N,
                                      accel_int4_prepared_t** out);

/* accel_int4_grouped_matvec / accel_int4_grouped_matmul over experts
 * prepared by accel_int4_prepare_grouped (the same results bit for bit;
 * routed rows on the matrix-core decode read the side copies) or by
 * accel_int4_prepare_grouped_panels (few f32 rows on the panel kernel, as
 * above): the same operands otherwise, and the same checks. */
int accel_int4_grouped_matvec_prepared(int dev, void* stream, const accel_tensor_t* x,
                                       const accel_int4_prepared_t* w,
                                       const accel_tensor_t* counts, accel_tensor_t* out);
int accel_int4_grouped_matmul_prepared(int dev, void* stream, const accel_tensor_t* x,
                                       const accel_int4_prepared_t* w,
                                       const accel_tensor_t* counts, accel_tensor_t* out);

/* ---- decode-step neighbours of the int4 products ---------------------- */

/* tensor.SwiGLU (tensor/elementwise.go:161-188; kernel
 * internal/kernels/elementwise.go:85-91): out = gate / (1 + Exp(-gate)) *
 * value, f32, one shape for all three; Exp is the f64 exponential rounded to
 * f32 (kmath/kmath.go:55).  Bit-identical to the reference CPU backend. */
int accel_swiglu(int dev, void* stream, const accel_tensor_t* gate,
                 const accel_tensor_t* value, accel_tensor_t* out);

/* tensor.RMSNorm (tensor/ops.go:105-135; kernel internal/kernels/norm.go:
 * 47-80): each row of x (f32, any rank >= 1) times RSqrt(mean(x^2) + eps),
 * times gain (f32 [width]); eps > 0 and finite.  The reference's reduction
 * order, so bit-identical to the reference CPU backend. */
int accel_rmsnorm(int dev, void* stream, const accel_tensor_t* x,
                  const accel_tensor_t* gain, float eps, accel_tensor_t* out);

/* tensor.MatMul's M = 1 selection for f32 activations and f16 weights
 * (tensor/matmul.go:113-121; kernel MatVecF32F16, internal/kernels/
 * matvec.go:79-105): x f32 [K] or [1,K], w f16 [K,N] -> out f32 [N] or
 * [1,N].  Other M are ACCEL_E_UNSUPPORTED. */
int accel_matvec_f32_f16(int dev, void* stream, const accel_tensor_t* x,
                         const accel_tensor_t* w, accel_tensor_t* out);

/* ---- int8 weights ------------------------------------------------------ */

/* tensor.QuantMatMul (tensor/quantized.go:72-163): x f32 or f16 [M,K] times
 * the int8 weight {quants i8 [K,N], scales f16 [ceil(K*N/32)]} -> out f32
 * [M,N], w(k,n) = q[kN+n] * s[(kN+n)/32].  M = 1 is the reference's
 * QuantMatVec(F32) selection, larger M its tiled kernel; both run here. */
int accel_quant_matmul(int dev, void* stream, const accel_tensor_t* x,
                       const accel_tensor_t* quants, const accel_tensor_t* scales,
                       accel_tensor_t* out);

/* quant.Int8Quantize / Int8Dequantize (quant/quant.go:60-135) on host memory:
 * quants one per weight, scales ceil(n/32) f16. */
int accel_int8_quantize(const float* w, int64_t n, int8_t* quants, uint16_t* scales);
int accel_int8_dequantize(const int8_t* quants, const uint16_t* scales, int64_t n,
                          float* out);

/* quant.Int4Quantize (quant/int4.go:71-138) on host memory: packed holds
 * ceil(n/8) words, scales and zeros ceil(n/128) f16 each. */
int accel_int4_quantize(const float* w, int64_t n, uint32_t* packed,
                        uint16_t* scales, uint16_t* zeros);

/* quant.Int4Dequantize (quant/int4.go:160-175) on host memory. */
int accel_int4_dequantize(const uint32_t* packed, const uint16_t* scales,
                          const uint16_t* zeros, int64_t n, float* out);

/* quant.Int4Quantize on the device, bit-identical to the host form: the
 * same f32 range arithmetic, f16 narrowing and f64 divide-and-round.
 * Pointers are device memory. */
int accel_int4_quantize_device(int dev, void* stream, const float* w, int64_t n,
                               uint32_t* packed, uint16_t* scales, uint16_t* zeros);

#ifdef __cplusplus
}
#endif

#endif /* ACCEL_HIP_H */
