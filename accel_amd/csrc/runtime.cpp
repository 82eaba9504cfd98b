// The backend seam of the C ABI: adapters, devices, blocks, streams, fences,
// timers and kernel-record dispatch.  Mirrors what internal/driver asks of a
// backend (internal/driver/driver.go:149-238, plan.go:31-428) as functions a
// purego binding can call.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <string>

#include "internal.hpp"

namespace accel {

namespace {
// The calling thread's last message.  A fixed buffer: recording an error
// allocates nothing.
thread_local char g_last_error[1024];
constexpr int kMaxDevices = 64;
Device g_devices[kMaxDevices];
std::mutex g_open_mu;
}  // namespace

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error[0] = '\0'; }

namespace {
thread_local LaunchRecord* g_record = nullptr;
}  // namespace

LaunchRecord::LaunchRecord(bool dry_) : outer(g_record), dry(dry_ || (g_record && g_record->dry)) {
    g_record = this;
}
LaunchRecord::~LaunchRecord() { g_record = outer; }
LaunchRecord* launch_record() { return g_record; }
std::string LaunchRecord::joined() const {
    std::string s;
    for (size_t i = 0; i < names.size(); i++) {
        if (i) s += " + ";
        s += names[i];
    }
    return s;
}

Device* device(int dev) {
    if (dev < 0 || dev >= kMaxDevices) {
        fail(ACCEL_E_NO_DEVICE, "accel_hip: device %d does not exist", dev);
        return nullptr;
    }
    Device* d = &g_devices[dev];
    if (!d->open) {
        fail(ACCEL_E_NO_DEVICE, "accel_hip: device %d is not open", dev);
        return nullptr;
    }
    if (hipSetDevice(dev) != hipSuccess) {
        fail(ACCEL_E_NO_DEVICE, "accel_hip: hipSetDevice(%d) failed", dev);
        return nullptr;
    }
    return d;
}

int begin_submission(Device* d) {
    std::lock_guard<std::mutex> lk(d->mu);
    if (d->lost.load()) return fail(ACCEL_E_DEVICE_LOST, "accel: device lost");
    d->submissions++;
    if (d->lose_at > 0 && d->submissions >= d->lose_at) {
        d->lost.store(1);
        return fail(ACCEL_E_DEVICE_LOST, "accel: device lost (injected at submission %lld)",
                    (long long)d->submissions);
    }
    return ACCEL_OK;
}

int classify(Device* d, hipError_t e, const char* what) {
    if (e == hipSuccess) return ACCEL_OK;
    switch (e) {
        case hipErrorOutOfMemory:
            return fail(ACCEL_E_OOM, "accel_hip: %s: %s", what, hipGetErrorString(e));
        case hipErrorIllegalAddress:
        case hipErrorLaunchFailure:
        case hipErrorECCNotCorrectable:
        case hipErrorAssert:
        case hipErrorLaunchTimeOut:
            if (d) d->lost.store(1);
            return fail(ACCEL_E_DEVICE_LOST, "accel: device lost (%s: %s)", what,
                        hipGetErrorString(e));
        default:
            return fail(ACCEL_E_HIP, "accel_hip: %s: %s", what, hipGetErrorString(e));
    }
}

namespace {

// Frees the retired workspaces that no live executable names any more.  The
// caller holds d->mu.
void free_unreferenced(Device* d) {
    bool waited = false;
    for (size_t i = 0; i < d->retired.size();) {
        bool named = false;
        for (const auto& kv : d->exec_gen)
            if (kv.second == d->retired[i].gen) named = true;
        if (named) {
            i++;
            continue;
        }
        if (!waited) {
            (void)hipDeviceSynchronize();
            waited = true;
        }
        (void)hipFree(d->retired[i].ptr);
        d->retired.erase(d->retired.begin() + (ptrdiff_t)i);
    }
}

bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

}  // namespace

void* workspace(Device* d, hipStream_t st, size_t bytes, int* status) {
    *status = ACCEL_OK;
    const size_t need = kWorkspaceCounterBytes + bytes;
    // planning a selection: an address to compute offsets from, never used
    if (dry_run()) return reinterpret_cast<void*>(uintptr_t(1) << 40);
    std::lock_guard<std::mutex> lk(d->mu);
    if (d->ws && d->ws_bytes >= need) return d->ws;
    if (capturing(st)) {
        *status = fail(ACCEL_E_INVALID,
                       "accel_hip: this call needs a workspace of %zu bytes and the device has "
                       "%zu; a workspace cannot grow inside a graph capture: issue the call "
                       "once outside the capture first",
                       need, d->ws_bytes);
        return nullptr;
    }
    // Growing.  Queued eager work may still use the old buffer, so wait for
    // it; an executable captured against it keeps its address, so a named
    // buffer is retired rather than freed.
    if (d->ws) {
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            *status = classify(d, e, "workspace growth");
            return nullptr;
        }
        bool named = false;
        for (const auto& kv : d->exec_gen)
            if (kv.second == d->ws_gen) named = true;
        if (named)
            d->retired.push_back({d->ws, d->ws_gen});
        else
            (void)hipFree(d->ws);
        d->ws = nullptr;
        d->ws_bytes = 0;
    }
    const size_t sz = need < (size_t(8) << 20) ? (size_t(8) << 20) : need;
    hipError_t e = hipMalloc(&d->ws, sz);
    if (e != hipSuccess) {
        d->ws = nullptr;
        *status = classify(d, e, "workspace allocation");
        return nullptr;
    }
    e = hipMemset(d->ws, 0, kWorkspaceCounterBytes);
    if (e != hipSuccess) {
        (void)hipFree(d->ws);
        d->ws = nullptr;
        *status = classify(d, e, "workspace clear");
        return nullptr;
    }
    d->ws_bytes = sz;
    d->ws_gen++;
    return d->ws;
}

int take_fault(Device* d) {
    if (!d->fault_host) return ACCEL_OK;
    const uint32_t f = __atomic_exchange_n(d->fault_host, 0u, __ATOMIC_ACQ_REL);
    if (!f) return ACCEL_OK;
    // A kernel that gave up left its hand-off counters mid-way: wait for the
    // device, then clear the counters of every workspace.
    (void)hipDeviceSynchronize();
    {
        std::lock_guard<std::mutex> lk(d->mu);
        if (d->ws) (void)hipMemset(d->ws, 0, kWorkspaceCounterBytes);
        for (const auto& r : d->retired) (void)hipMemset(r.ptr, 0, kWorkspaceCounterBytes);
        if (d->scratch) (void)hipMemset(d->scratch, 0, kWorkspaceCounterBytes);
    }
    const char* what = f == kFaultWaitGaveUp ? "a split-K hand-off's bounded wait gave up"
                                              : "unknown fault bits";
    return fail(ACCEL_E_HIP,
                "accel_hip: device fault word 0x%x (%s): the results of the work waited on "
                "are undefined",
                f, what);
}

}  // namespace accel

using namespace accel;

#define ACCEL_API extern "C" __attribute__((visibility("default")))

ACCEL_API const char* accel_hip_last_error(void) { return g_last_error; }

ACCEL_API int accel_hip_abi_version(void) { return 1; }

ACCEL_API int accel_hip_probe(int* count) {
    clear_error();
    if (!count) return fail(ACCEL_E_INVALID, "accel_hip_probe: count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) n = 0;
    else if (e != hipSuccess) {
        *count = 0;
        return fail(ACCEL_OK, "accel_hip_probe: %s", hipGetErrorString(e));
    }
    *count = n;
    return ACCEL_OK;
}

ACCEL_API int accel_hip_info(int dev, accel_hip_info_t* out) {
    clear_error();
    if (!out) return fail(ACCEL_E_INVALID, "accel_hip_info: out is NULL");
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess)
        return fail(ACCEL_E_NO_DEVICE, "accel_hip_info(%d): %s", dev, hipGetErrorString(e));
    memset(out, 0, sizeof *out);
    snprintf(out->name, sizeof out->name, "%s", p.name);
    snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
    out->compute_units = p.multiProcessorCount;
    out->wavefront = p.warpSize;
    out->lds_per_block = (int32_t)p.sharedMemPerBlock;
    out->clock_khz = p.clockRate;
    out->mem_clock_khz = p.memoryClockRate;
    out->mem_bus_bits = p.memoryBusWidth;
    out->hbm_bytes = p.totalGlobalMem;
    out->l2_bytes = p.l2CacheSize;
    out->pci_bus = p.pciBusID;
    return ACCEL_OK;
}

ACCEL_API int accel_hip_open(int dev) {
    clear_error();
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || dev < 0 || dev >= n || dev >= kMaxDevices)
        return fail(ACCEL_E_NO_DEVICE, "accel_hip_open: no HIP device %d", dev);
    std::lock_guard<std::mutex> lk(g_open_mu);
    Device* d = &g_devices[dev];
    if (d->open) return ACCEL_OK;
    hipError_t e = hipSetDevice(dev);
    if (e != hipSuccess) return classify(nullptr, e, "hipSetDevice");
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return classify(nullptr, e, "hipGetDeviceProperties");
    std::string arch = p.gcnArchName;
    if (arch.rfind("gfx950", 0) != 0)
        return fail(ACCEL_E_UNSUPPORTED,
                    "accel_hip_open: device %d is %s; this library carries gfx950 code only",
                    dev, p.gcnArchName);
    if (!d->fault_host) {
        void* h = nullptr;
        // mapped and coherent (fine-grained): the kernels' system-scope
        // atomics must reach the host whatever HIP_HOST_COHERENT says
        e = hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocCoherent);
        if (e != hipSuccess) return classify(nullptr, e, "fault word allocation");
        void* dp = nullptr;
        e = hipHostGetDevicePointer(&dp, h, 0);
        if (e != hipSuccess) {
            (void)hipHostFree(h);
            return classify(nullptr, e, "fault word mapping");
        }
        d->fault_host = static_cast<uint32_t*>(h);
        d->fault_dev = static_cast<uint32_t*>(dp);
    }
    *d->fault_host = 0;
    if (!d->scratch) {
        const int rc = init_scratch(d);
        if (rc != ACCEL_OK) return rc;
    }
    d->wait_limit = 1 << 22;
    d->ordinal = dev;
    d->cu_count = p.multiProcessorCount;
    d->lds_per_block = p.sharedMemPerBlock;
    d->lost.store(0);
    d->submissions = 0;
    d->lose_at = 0;
    d->sel_valid = false;
    d->open = true;
    return ACCEL_OK;
}

ACCEL_API int accel_hip_close(int dev) {
    clear_error();
    if (dev < 0 || dev >= kMaxDevices) return ACCEL_OK;
    std::lock_guard<std::mutex> lk(g_open_mu);
    Device* d = &g_devices[dev];
    if (!d->open) return ACCEL_OK;
    (void)hipSetDevice(dev);
    (void)hipDeviceSynchronize();
    if (d->ws) (void)hipFree(d->ws);
    for (const auto& r : d->retired) (void)hipFree(r.ptr);
    d->retired.clear();
    d->exec_gen.clear();
    d->ws = nullptr;
    d->ws_bytes = 0;
    if (d->fault_host) *d->fault_host = 0;
    d->open = false;
    return ACCEL_OK;
}

ACCEL_API int accel_hip_lost(int dev) {
    if (dev < 0 || dev >= kMaxDevices) return 0;
    return g_devices[dev].lost.load() ? 1 : 0;
}

ACCEL_API int accel_hip_inject_loss(int dev, int64_t at_submission) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    std::lock_guard<std::mutex> lk(d->mu);
    d->submissions = 0;
    d->lose_at = at_submission;
    return ACCEL_OK;
}

ACCEL_API int accel_hip_alloc(int dev, size_t bytes, void** ptr) {
    clear_error();
    if (!ptr) return fail(ACCEL_E_INVALID, "accel_hip_alloc: ptr is NULL");
    *ptr = nullptr;
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (d->lost.load()) return fail(ACCEL_E_DEVICE_LOST, "accel: device lost");
    if (bytes == 0) bytes = 1;
    return classify(d, hipMalloc(ptr, bytes), "hipMalloc");
}

ACCEL_API int accel_hip_free(int dev, void* ptr) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!ptr) return ACCEL_OK;
    return classify(d, hipFree(ptr), "hipFree");
}

ACCEL_API int accel_hip_write(int dev, void* dst, size_t offset, const void* src,
                              size_t bytes) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (d->lost.load()) return fail(ACCEL_E_DEVICE_LOST, "accel: device lost");
    if (bytes == 0) return ACCEL_OK;
    if (!dst || !src) return fail(ACCEL_E_INVALID, "accel_hip_write: NULL pointer");
    return classify(d, hipMemcpy((char*)dst + offset, src, bytes, hipMemcpyHostToDevice),
                    "hipMemcpy(HtoD)");
}

ACCEL_API int accel_hip_read(int dev, const void* src, size_t offset, void* dst,
                             size_t bytes) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (d->lost.load()) return fail(ACCEL_E_DEVICE_LOST, "accel: device lost");
    if (bytes == 0) return ACCEL_OK;
    if (!dst || !src) return fail(ACCEL_E_INVALID, "accel_hip_read: NULL pointer");
    return classify(d,
                    hipMemcpy(dst, (const char*)src + offset, bytes, hipMemcpyDeviceToHost),
                    "hipMemcpy(DtoH)");
}

ACCEL_API int accel_hip_copy(int dev, void* stream, void* dst, const void* src,
                             size_t bytes) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    int st = begin_submission(d);
    if (st != ACCEL_OK) return st;
    if (bytes == 0) return ACCEL_OK;
    return classify(d, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                                      (hipStream_t)stream),
                    "hipMemcpyAsync(DtoD)");
}

ACCEL_API int accel_hip_stream_create(int dev, void** stream) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!stream) return fail(ACCEL_E_INVALID, "accel_hip_stream_create: NULL out");
    hipStream_t s = nullptr;
    // Default priority only: every stream of this library is created the same way.
    int rc = classify(d, hipStreamCreateWithFlags(&s, hipStreamNonBlocking),
                      "hipStreamCreate");
    *stream = s;
    return rc;
}

ACCEL_API int accel_hip_stream_destroy(int dev, void* stream) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!stream) return ACCEL_OK;
    return classify(d, hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
}

ACCEL_API int accel_hip_stream_sync(int dev, void* stream) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (d->lost.load()) return fail(ACCEL_E_DEVICE_LOST, "accel: device lost");
    const int rc = classify(d, hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
    return rc != ACCEL_OK ? rc : take_fault(d);
}

ACCEL_API int accel_hip_event_create(int dev, void** event) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!event) return fail(ACCEL_E_INVALID, "accel_hip_event_create: NULL out");
    hipEvent_t ev = nullptr;
    int rc = classify(d, hipEventCreate(&ev), "hipEventCreate");
    *event = ev;
    return rc;
}

ACCEL_API int accel_hip_event_destroy(int dev, void* event) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!event) return ACCEL_OK;
    return classify(d, hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
}

ACCEL_API int accel_hip_event_record(int dev, void* event, void* stream) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (d->lost.load()) return fail(ACCEL_E_DEVICE_LOST, "accel: device lost");
    return classify(d, hipEventRecord((hipEvent_t)event, (hipStream_t)stream),
                    "hipEventRecord");
}

ACCEL_API int accel_hip_event_query(int dev, void* event) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (d->lost.load()) return 1;  // a lost device is done (plan.go:380-382)
    hipError_t e = hipEventQuery((hipEvent_t)event);
    if (e == hipSuccess) {
        const int rc = take_fault(d);
        return rc != ACCEL_OK ? rc : 1;
    }
    if (e == hipErrorNotReady) return 0;
    return classify(d, e, "hipEventQuery");
}

ACCEL_API int accel_hip_event_sync(int dev, void* event) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (d->lost.load()) return fail(ACCEL_E_DEVICE_LOST, "accel: device lost");
    const int rc = classify(d, hipEventSynchronize((hipEvent_t)event), "hipEventSynchronize");
    return rc != ACCEL_OK ? rc : take_fault(d);
}

ACCEL_API int accel_hip_event_elapsed(int dev, void* start, void* end, float* ms) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!ms) return fail(ACCEL_E_INVALID, "accel_hip_event_elapsed: NULL out");
    return classify(d, hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end),
                    "hipEventElapsedTime");
}

ACCEL_API int accel_hip_capture_begin(int dev, void* stream) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (d->lost.load()) return fail(ACCEL_E_DEVICE_LOST, "accel: device lost");
    if (!stream)
        return fail(ACCEL_E_INVALID, "accel_hip_capture_begin: the null stream cannot capture");
    return classify(d,
                    hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal),
                    "hipStreamBeginCapture");
}

ACCEL_API int accel_hip_capture_end(int dev, void* stream, void** exec) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!exec) return fail(ACCEL_E_INVALID, "accel_hip_capture_end: NULL out");
    *exec = nullptr;
    hipGraph_t g = nullptr;
    int rc = classify(d, hipStreamEndCapture((hipStream_t)stream, &g), "hipStreamEndCapture");
    if (rc != ACCEL_OK) return rc;
    hipGraphExec_t ge = nullptr;
    rc = classify(d, hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (rc != ACCEL_OK) return rc;
    {
        // the executable's kernels carry this workspace's addresses
        std::lock_guard<std::mutex> lk(d->mu);
        d->exec_gen[ge] = d->ws_gen;
    }
    *exec = ge;
    return ACCEL_OK;
}

ACCEL_API int accel_hip_exec_launch(int dev, void* exec, void* stream) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!exec) return fail(ACCEL_E_INVALID, "accel_hip_exec_launch: NULL executable");
    int st = begin_submission(d);
    if (st != ACCEL_OK) return st;
    return classify(d, hipGraphLaunch((hipGraphExec_t)exec, (hipStream_t)stream),
                    "hipGraphLaunch");
}

ACCEL_API int accel_hip_exec_destroy(int dev, void* exec) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!exec) return ACCEL_OK;
    const int rc = classify(d, hipGraphExecDestroy((hipGraphExec_t)exec), "hipGraphExecDestroy");
    std::lock_guard<std::mutex> lk(d->mu);
    d->exec_gen.erase(exec);
    free_unreferenced(d);
    return rc;
}

ACCEL_API int accel_hip_set_wait_limit(int dev, int32_t spins) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (spins < 0) return fail(ACCEL_E_INVALID, "accel_hip_set_wait_limit: %d spins", spins);
    std::lock_guard<std::mutex> lk(d->mu);
    d->wait_limit = spins;
    return ACCEL_OK;
}

// ---- launch-floor probes ----------------------------------------------------
//
// The ceilings a decode product's roofline sits under, measured with the
// M = 1 decode kernel's launch shape (256 workgroups of 512 lanes): an empty
// kernel (what a launch costs before any work), and a pure read of `bytes`
// with 16-byte loads, every lane's loads issued before any is used (what
// moving the bytes costs without the product's arithmetic or hand-off).
// Diagnostics for bench.py; no reference counterpart.
namespace {
constexpr int kFloorBlocks = 256, kFloorThreads = 512, kFloorLoads = 8;
typedef uint32_t floor_u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kFloorThreads) void floor_empty_kernel(uint32_t* sink) {
    if (threadIdx.x == 0 && blockIdx.x == 0xffffff) sink[0] = 1;
}

// L 16-byte loads a lane, issued together (a lane past the end re-reads
// chunk 0, which the caches serve, and leaves it out).
template <int L>
__global__ __launch_bounds__(kFloorThreads) void floor_read_kernel(const floor_u32x4* src,
                                                                   size_t chunks, uint32_t* sink) {
    const size_t grid = (size_t)gridDim.x * blockDim.x;
    const size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    floor_u32x4 v[L];
#pragma unroll
    for (int k = 0; k < L; k++) {
        const size_t i = g + k * grid;
        v[k] = __builtin_nontemporal_load(src + (i < chunks ? i : 0));
    }
    uint32_t x = 0;
#pragma unroll
    for (int k = 0; k < L; k++)
        if (g + k * grid < chunks) x ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    if (x == 0x9e3779b9u) sink[blockIdx.x] = x;   // keeps the loads; almost never stores
}

// Reads `chunks` 16-byte chunks with a grid-stride loop and writes (almost)
// nothing: evicts the device's caches with clean lines, so no writeback of
// the eviction lands in the work timed after it (a copy would leave up to the
// Infinity Cache's size of dirty lines behind).
__global__ __launch_bounds__(256) void floor_evict_kernel(const floor_u32x4* src, size_t chunks,
                                                          uint32_t* sink) {
    uint32_t x = 0;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < chunks;
         i += (size_t)gridDim.x * blockDim.x) {
        const floor_u32x4 v = __builtin_nontemporal_load(src + i);
        x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (x == 0x9e3779b9u) sink[blockIdx.x & 255] = x;
}

template <int L>
void launch_floor_read(hipStream_t st, const void* src, size_t chunks, void* sink) {
    hipLaunchKernelGGL(floor_read_kernel<L>, dim3(kFloorBlocks), dim3(kFloorThreads), 0, st,
                       static_cast<const floor_u32x4*>(src), chunks,
                       static_cast<uint32_t*>(sink));
}
}  // namespace

ACCEL_API int accel_hip_floor(int dev, void* stream, int kind, const void* src, size_t bytes,
                              void* sink) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    if (!sink) return fail(ACCEL_E_INVALID, "accel_hip_floor: sink is NULL");
    hipStream_t st = (hipStream_t)stream;
    if (kind == 0) {
        hipLaunchKernelGGL(floor_empty_kernel, dim3(kFloorBlocks), dim3(kFloorThreads), 0, st,
                           static_cast<uint32_t*>(sink));
    } else if (kind == 1) {
        const size_t chunks = bytes / 16;
        if (!src || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16 || chunks == 0 ||
            chunks > (size_t)kFloorBlocks * kFloorThreads * kFloorLoads)
            return fail(ACCEL_E_INVALID,
                        "accel_hip_floor: a read of %zu bytes needs a 16-byte aligned source, "
                        "a multiple of 16 bytes and at most %zu bytes",
                        bytes, (size_t)kFloorBlocks * kFloorThreads * kFloorLoads * 16);
        const size_t lanes = (size_t)kFloorBlocks * kFloorThreads;
        switch ((chunks + lanes - 1) / lanes) {
            case 1: launch_floor_read<1>(st, src, chunks, sink); break;
            case 2: launch_floor_read<2>(st, src, chunks, sink); break;
            case 3: launch_floor_read<3>(st, src, chunks, sink); break;
            case 4: launch_floor_read<4>(st, src, chunks, sink); break;
            case 5: launch_floor_read<5>(st, src, chunks, sink); break;
            case 6: launch_floor_read<6>(st, src, chunks, sink); break;
            case 7: launch_floor_read<7>(st, src, chunks, sink); break;
            default: launch_floor_read<8>(st, src, chunks, sink); break;
        }
    } else if (kind == 2) {
        if (!src || bytes % 16 || reinterpret_cast<uintptr_t>(src) % 16 || bytes == 0)
            return fail(ACCEL_E_INVALID,
                        "accel_hip_floor: an eviction of %zu bytes needs a 16-byte aligned "
                        "source and a multiple of 16 bytes",
                        bytes);
        hipLaunchKernelGGL(floor_evict_kernel, dim3(4096), dim3(256), 0, st,
                           static_cast<const floor_u32x4*>(src), bytes / 16,
                           static_cast<uint32_t*>(sink));
    } else {
        return fail(ACCEL_E_INVALID,
                    "accel_hip_floor: kind %d is not 0 (empty), 1 (read) or 2 (evict)", kind);
    }
    return classify(d, hipGetLastError(), "accel_hip_floor launch");
}

ACCEL_API int accel_hip_workspace_generation(int dev, uint64_t* gen, int32_t* retired) {
    clear_error();
    Device* d = device(dev);
    if (!d) return ACCEL_E_NO_DEVICE;
    std::lock_guard<std::mutex> lk(d->mu);
    if (gen) *gen = d->ws_gen;
    if (retired) *retired = (int32_t)d->retired.size();
    return ACCEL_OK;
}
