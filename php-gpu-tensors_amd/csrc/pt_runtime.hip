// Runtime half of the C-ABI: status strings, device queries, streams,
// events, the stream-ordered memory pool, transfers, hipRTC modules and
// graph capture.  Replaces src/cuda_wrapper.cpp, src/backends/cuda/
// memory_pool.c and the driver-API calls of src/fusion_*.c /
// src/compiler_ce.c in the reference.
#include "pt_common.h"

#include <hip/hiprtc.h>

#include <algorithm>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <string>
#include <vector>

namespace pt {

static thread_local char g_error[1024];
static std::once_flag g_init_once;
static pt_status g_init_status = PT_OK;
static hipStream_t g_stream = nullptr;
static hipMemPool_t g_pool = nullptr;
static pt_backend_info g_info;

void set_error(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

pt_status fail(pt_status status, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return status;
}

pt_status check_hip(hipError_t err, const char *what)
{
    if (err == hipSuccess) return PT_OK;
    set_error("%s: %s", what, hipGetErrorString(err));
    return err == hipErrorOutOfMemory ? PT_ERR_NOMEM : PT_ERR_RUNTIME;
}

pt_backend_info &counters() { return g_info; }

static void init_once()
{
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count < 1) {
        g_init_status = fail(PT_ERR_NO_DEVICE, "no HIP device is visible");
        return;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) {
        g_init_status = fail(PT_ERR_RUNTIME, "hipGetDeviceProperties failed");
        return;
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        g_init_status = fail(PT_ERR_NO_DEVICE,
                             "device 0 is %s; this backend is built for gfx950 only",
                             prop.gcnArchName);
        return;
    }
    if (hipSetDevice(0) != hipSuccess ||
        hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) {
        g_init_status = fail(PT_ERR_RUNTIME, "could not create the default stream");
        return;
    }
    if (hipDeviceGetDefaultMemPool(&g_pool, 0) != hipSuccess) {
        g_init_status = fail(PT_ERR_RUNTIME, "device has no default memory pool");
        return;
    }
    // Keep freed blocks cached in the pool (the reference's pool never returns
    // memory to the driver either, memory_pool.c:350-381).
    uint64_t threshold = UINT64_MAX;
    if (hipMemPoolSetAttribute(g_pool, hipMemPoolAttrReleaseThreshold, &threshold) != hipSuccess) {
        g_init_status = fail(PT_ERR_RUNTIME, "could not set the memory pool's release threshold");
        return;
    }
    snprintf(g_info.last_matmul, sizeof(g_info.last_matmul), "none");
}

pt_status ensure_init()
{
    std::call_once(g_init_once, init_once);
    return g_init_status;
}

// Stream that calls without an explicit stream use on this thread: the
// runtime stream unless pt_stream_set_current chose another.
static thread_local hipStream_t t_current = nullptr;

hipStream_t stream_of(pt_stream_t s)
{
    return s ? (hipStream_t)s : (t_current ? t_current : g_stream);
}

// Static scratch of the no-allocation entry points (pt_reduce_noalloc): a
// file-scope device array that every GPU the library runs on holds for the
// life of the process.  Host code never uses the array's name as an
// address: its device address is looked up per device with
// hipGetSymbolAddress (with that device current) the first time an entry
// point runs there.
//
// Calls that overlap on one device (other threads, other streams) are
// ordered on the GPU instead of racing on the array: each device keeps the
// event the last call recorded on its stream after its kernels, and a call
// makes its own stream wait for that event before its first kernel.  The
// wait, the kernels and the record happen under one host lock, so the
// hand-off order is the order in which the calls take the lock.  The event
// is created with the device's address, once, at the first call there; a
// call allocates nothing.  Under stream capture the hand-off is skipped
// (the graph orders its own nodes), so a graph holding such a call must not
// run while another call on that device does.
static __device__ __align__(256) unsigned char scratch[PT_STATIC_SCRATCH_BYTES];
static std::mutex g_static_mu;       // set-up of the per-device entries
static std::mutex g_static_call_mu;  // held from static_scratch_begin to static_scratch_end
static void *g_static_ptr[64];
static hipEvent_t g_static_last[64];
static bool g_static_recorded[64];
static thread_local int t_static_dev = -1;
static thread_local bool t_static_capturing = false;

static pt_status static_scratch_setup(int *dev_out, void **ptr)
{
    int dev = 0;
    PT_TRY(check_hip(hipGetDevice(&dev), "hipGetDevice"));
    if (dev < 0 || dev >= 64) return fail(PT_ERR_RUNTIME, "device %d outside the static scratch table", dev);
    std::lock_guard<std::mutex> lock(g_static_mu);
    if (!g_static_ptr[dev]) {
        void *p = nullptr;
        PT_TRY(check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "static scratch address"));
        if (!p) return fail(PT_ERR_RUNTIME, "static scratch has no device address");
        PT_TRY(check_hip(hipEventCreateWithFlags(&g_static_last[dev], hipEventDisableTiming),
                         "static scratch event"));
        g_static_ptr[dev] = p;
    }
    *dev_out = dev;
    *ptr = g_static_ptr[dev];
    return PT_OK;
}

// Scratch of the multi-kernel operations (split-K partials, column and
// global reduction partials).  By default it comes from the stream-ordered
// pool.  Between pt_workspace_begin and pt_workspace_end it is carved from
// a caller-owned arena instead (a stack: each operation frees what it took
// before it returns), so that a captured HIP graph holds no allocation; in
// measuring mode (no arena) it still comes from the pool and the peak is
// recorded, which sizes the arena.
// Between static_scratch_begin and static_scratch_end the arena is the
// device's static scratch (`fixed`: never the pool).
struct Workspace {
    bool active = false, measure = false, fixed = false;
    char *base = nullptr;
    size_t bytes = 0, top = 0, peak = 0;
    std::vector<std::pair<void *, size_t>> stack;
};
static thread_local Workspace t_ws;

static size_t ws_round(size_t n) { return (n + 255) & ~(size_t)255; }

pt_status scratch_alloc(void **ptr, size_t bytes, hipStream_t stream)
{
    if (!t_ws.active) return check_hip(hipMallocAsync(ptr, bytes ? bytes : 1, stream), "scratch allocation");
    const size_t need = ws_round(bytes ? bytes : 1);
    if (t_ws.fixed) {
        // static scratch: a bump pointer, nothing allocated (not even host memory)
        if (t_ws.top + need > t_ws.bytes)
            return fail(PT_ERR_INVALID, "operation needs %zu bytes of scratch; the static scratch holds %zu",
                        t_ws.top + need, t_ws.bytes);
        *ptr = t_ws.base + t_ws.top;
        t_ws.top += need;
        return PT_OK;
    }
    if (t_ws.measure) {
        PT_TRY(check_hip(hipMallocAsync(ptr, need, stream), "scratch allocation"));
    } else {
        if (t_ws.top + need > t_ws.bytes)
            return fail(PT_ERR_NOMEM, "workspace of %zu bytes cannot hold %zu more scratch bytes", t_ws.bytes, need);
        *ptr = t_ws.base + t_ws.top;
    }
    t_ws.top += need;
    if (t_ws.top > t_ws.peak) t_ws.peak = t_ws.top;
    t_ws.stack.push_back({*ptr, need});
    return PT_OK;
}

void scratch_free(void *ptr, hipStream_t stream)
{
    if (!ptr) return;
    if (!t_ws.active) {
        (void)hipFreeAsync(ptr, stream);
        return;
    }
    if (t_ws.fixed) return;  // static scratch: released by static_scratch_end
    for (size_t i = t_ws.stack.size(); i-- > 0;) {
        if (t_ws.stack[i].first != ptr) continue;
        if (t_ws.measure) (void)hipFreeAsync(ptr, stream);
        // the region is not handed out again before pt_workspace_end, so
        // operations that run concurrently (branches of a captured graph)
        // never share scratch
        t_ws.stack.erase(t_ws.stack.begin() + (long)i);
        return;
    }
}

// Scratch of the calls between static_scratch_begin and static_scratch_end
// comes from the device's static scratch array (a stack, as a workspace);
// a request beyond it fails with PT_ERR_INVALID instead of allocating.
pt_status static_scratch_begin(hipStream_t stream)
{
    if (t_ws.active) return fail(PT_ERR_INVALID, "a workspace is already active on this thread");
    void *p = nullptr;
    int dev = 0;
    PT_TRY(static_scratch_setup(&dev, &p));
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    PT_TRY(check_hip(hipStreamIsCapturing(stream, &cap), "hipStreamIsCapturing"));
    g_static_call_mu.lock();
    if (cap == hipStreamCaptureStatusNone && g_static_recorded[dev]) {
        const pt_status st = check_hip(hipStreamWaitEvent(stream, g_static_last[dev], 0), "static scratch hand-off");
        if (st != PT_OK) {
            g_static_call_mu.unlock();
            return st;
        }
    }
    t_static_dev = dev;
    t_static_capturing = cap != hipStreamCaptureStatusNone;
    t_ws = Workspace();
    t_ws.active = true;
    t_ws.fixed = true;
    t_ws.base = (char *)p;
    t_ws.bytes = PT_STATIC_SCRATCH_BYTES;
    return PT_OK;
}

pt_status static_scratch_end(hipStream_t stream)
{
    t_ws = Workspace();
    pt_status st = PT_OK;
    const int dev = t_static_dev;
    if (!t_static_capturing) {
        st = check_hip(hipEventRecord(g_static_last[dev], stream), "static scratch hand-off record");
        if (st == PT_OK) g_static_recorded[dev] = true;
    }
    t_static_dev = -1;
    g_static_call_mu.unlock();
    return st;
}

}  // namespace pt

using namespace pt;

extern "C" {

pt_status pt_init(void) { return ensure_init(); }

const char *pt_status_string(pt_status status)
{
    switch (status) {
    case PT_OK: return "success";
    case PT_ERR_INVALID: return "invalid argument";
    case PT_ERR_RUNTIME: return "HIP runtime failure";
    case PT_ERR_UNSUPPORTED: return "unsupported dtype or operation";
    case PT_ERR_NOMEM: return "out of device memory";
    case PT_ERR_COMPILE: return "runtime compilation failed";
    case PT_ERR_NO_DEVICE: return "no gfx950 device";
    default: return "unknown status";
    }
}

const char *pt_last_error(void) { return g_error; }

pt_status pt_version(int *major, int *minor)
{
    if (major) *major = 0;
    if (minor) *minor = 1;
    return PT_OK;
}

pt_status pt_device_count(int *count)
{
    int n = 0;
    hipError_t err = hipGetDeviceCount(&n);
    if (err != hipSuccess) n = 0;
    *count = n;
    return PT_OK;
}

pt_status pt_device_set(int device)
{
    PT_TRY(ensure_init());
    if (device != 0)
        return fail(PT_ERR_INVALID, "one owning device per process: only device 0 is supported");
    return check_hip(hipSetDevice(device), "hipSetDevice");
}

pt_status pt_device_get(int *device)
{
    PT_TRY(ensure_init());
    return check_hip(hipGetDevice(device), "hipGetDevice");
}

pt_status pt_device_info_get(int device, pt_device_info *info)
{
    hipDeviceProp_t prop;
    PT_TRY(check_hip(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties"));
    memset(info, 0, sizeof(*info));
    snprintf(info->name, sizeof(info->name), "%s", prop.name);
    snprintf(info->arch, sizeof(info->arch), "%s", prop.gcnArchName);
    info->compute_units = prop.multiProcessorCount;
    info->clock_khz = prop.clockRate;
    info->memory_clock_khz = prop.memoryClockRate;
    info->memory_bus_width = prop.memoryBusWidth;
    info->total_memory = prop.totalGlobalMem;
    info->lds_per_block = prop.sharedMemPerBlock;
    info->warp_size = prop.warpSize;
    info->max_threads_per_block = prop.maxThreadsPerBlock;
    info->l2_cache_bytes = prop.l2CacheSize;
    return PT_OK;
}

pt_status pt_device_synchronize(void)
{
    PT_TRY(ensure_init());
    return check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

// ------------------------------------------------------------- streams
pt_stream_t pt_default_stream(void)
{
    if (ensure_init() != PT_OK) return nullptr;
    return (pt_stream_t)g_stream;
}

pt_status pt_stream_create(pt_stream_t *stream)
{
    PT_TRY(ensure_init());
    hipStream_t s;
    PT_TRY(check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate"));
    *stream = (pt_stream_t)s;
    return PT_OK;
}

pt_status pt_stream_destroy(pt_stream_t stream)
{
    if (!stream) return PT_OK;
    return check_hip(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
}

pt_status pt_stream_synchronize(pt_stream_t stream)
{
    PT_TRY(ensure_init());
    return check_hip(hipStreamSynchronize(stream_of(stream)), "hipStreamSynchronize");
}

pt_status pt_stream_query(pt_stream_t stream, int *finished)
{
    PT_TRY(ensure_init());
    hipError_t err = hipStreamQuery(stream_of(stream));
    if (err == hipErrorNotReady) {
        *finished = 0;
        return PT_OK;
    }
    *finished = 1;
    return check_hip(err, "hipStreamQuery");
}

pt_status pt_stream_wait_event(pt_stream_t stream, pt_event_t event)
{
    PT_TRY(ensure_init());
    return check_hip(hipStreamWaitEvent(stream_of(stream), (hipEvent_t)event, 0),
                     "hipStreamWaitEvent");
}

pt_status pt_event_create(pt_event_t *event)
{
    PT_TRY(ensure_init());
    hipEvent_t e;
    PT_TRY(check_hip(hipEventCreate(&e), "hipEventCreate"));
    *event = (pt_event_t)e;
    return PT_OK;
}

pt_status pt_event_destroy(pt_event_t event)
{
    if (!event) return PT_OK;
    return check_hip(hipEventDestroy((hipEvent_t)event), "hipEventDestroy");
}

pt_status pt_event_record(pt_event_t event, pt_stream_t stream)
{
    return check_hip(hipEventRecord((hipEvent_t)event, stream_of(stream)), "hipEventRecord");
}

pt_status pt_event_synchronize(pt_event_t event)
{
    return check_hip(hipEventSynchronize((hipEvent_t)event), "hipEventSynchronize");
}

pt_status pt_event_query(pt_event_t event, int *finished)
{
    hipError_t err = hipEventQuery((hipEvent_t)event);
    if (err == hipErrorNotReady) {
        *finished = 0;
        return PT_OK;
    }
    *finished = 1;
    return check_hip(err, "hipEventQuery");
}

pt_status pt_event_elapsed_ms(pt_event_t start, pt_event_t stop, float *ms)
{
    return check_hip(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop),
                     "hipEventElapsedTime");
}

// -------------------------------------------------------------- memory
pt_status pt_mem_init(size_t pool_bytes)
{
    PT_TRY(ensure_init());
    uint64_t threshold = pool_bytes ? (uint64_t)pool_bytes : UINT64_MAX;
    return check_hip(hipMemPoolSetAttribute(g_pool, hipMemPoolAttrReleaseThreshold, &threshold),
                     "hipMemPoolSetAttribute");
}

pt_status pt_alloc(void **ptr, size_t bytes, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    *ptr = nullptr;
    hipError_t err = hipMallocAsync(ptr, bytes ? bytes : 1, stream_of(stream));
    if (err != hipSuccess)
        return fail(err == hipErrorOutOfMemory ? PT_ERR_NOMEM : PT_ERR_RUNTIME,
                    "device allocation of %zu bytes failed: %s", bytes, hipGetErrorString(err));
    return PT_OK;
}

pt_status pt_free(void *ptr, pt_stream_t stream)
{
    if (!ptr) return PT_OK;
    PT_TRY(ensure_init());
    return check_hip(hipFreeAsync(ptr, stream_of(stream)), "hipFreeAsync");
}

pt_status pt_mem_info(size_t *free_bytes, size_t *total_bytes, size_t *pool_reserved)
{
    PT_TRY(ensure_init());
    size_t f = 0, t = 0;
    PT_TRY(check_hip(hipMemGetInfo(&f, &t), "hipMemGetInfo"));
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    if (pool_reserved) {
        uint64_t reserved = 0;
        PT_TRY(check_hip(hipMemPoolGetAttribute(g_pool, hipMemPoolAttrReservedMemCurrent, &reserved),
                         "hipMemPoolGetAttribute"));
        *pool_reserved = (size_t)reserved;
    }
    return PT_OK;
}

// pt_memcpy_h2d / pt_memcpy_d2h: pt_transfer.hip

pt_status pt_memcpy_d2d(void *dst, const void *src, size_t bytes, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!bytes) return PT_OK;
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, stream_of(stream)),
                     "device to device copy");
}

// Byte fill through a kernel rather than hipMemsetAsync, so that the call
// records a kernel node when a caller captures it into a graph (memset
// nodes have replayed wrongly after the first replay on this platform).
__global__ __launch_bounds__(256) void k_memset_bytes(unsigned char *dst, unsigned char v, size_t n)
{
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = v;
}

pt_status pt_memset(void *dst, int value, size_t bytes, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!bytes) return PT_OK;
    size_t blocks = (bytes + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    k_memset_bytes<<<(unsigned)blocks, 256, 0, stream_of(stream)>>>((unsigned char *)dst, (unsigned char)value,
                                                                     bytes);
    return check_hip(hipGetLastError(), "memset kernel launch");
}

pt_status pt_host_alloc_pinned(void **ptr, size_t bytes)
{
    PT_TRY(ensure_init());
    return check_hip(hipHostMalloc(ptr, bytes ? bytes : 1, hipHostMallocDefault), "hipHostMalloc");
}

pt_status pt_host_free_pinned(void *ptr)
{
    if (!ptr) return PT_OK;
    return check_hip(hipHostFree(ptr), "hipHostFree");
}

// ------------------------------------------------------------ counters
pt_status pt_backend_info_get(pt_backend_info *info)
{
    *info = g_info;
    return PT_OK;
}

pt_status pt_backend_info_reset(void)
{
    char last[32];
    memcpy(last, g_info.last_matmul, sizeof(last));
    memset(&g_info, 0, sizeof(g_info));
    memcpy(g_info.last_matmul, last, sizeof(last));
    return PT_OK;
}

// --------------------------------------------------------------- hipRTC
pt_status pt_rtc_compile(const char *source, const char *program_name,
                         pt_module_t *module, char *log, size_t log_bytes)
{
    PT_TRY(ensure_init());
    if (log && log_bytes) log[0] = 0;
    hiprtcProgram prog;
    if (hiprtcCreateProgram(&prog, source, program_name ? program_name : "fusion.hip",
                            0, nullptr, nullptr) != HIPRTC_SUCCESS)
        return fail(PT_ERR_COMPILE, "hiprtcCreateProgram failed");
    // No contraction: a fused a+b*c must round like the eager kernels
    // (fusion_precision.phpt:15-16); packed fp32 VALU ops stay disabled.
    const char *opts[] = {"--offload-arch=gfx950", "-O3",      "-ffp-contract=off", "-std=c++17",
                          "-Xclang",               "-target-feature", "-Xclang",           "-packed-fp32-ops"};
    hiprtcResult rc = hiprtcCompileProgram(prog, (int)(sizeof(opts) / sizeof(opts[0])), opts);
    if (rc != HIPRTC_SUCCESS) {
        size_t n = 0;
        hiprtcGetProgramLogSize(prog, &n);
        std::string text(n + 1, '\0');
        if (n) hiprtcGetProgramLog(prog, &text[0]);
        if (log && log_bytes) snprintf(log, log_bytes, "%s", text.c_str());
        hiprtcDestroyProgram(&prog);
        return fail(PT_ERR_COMPILE, "hipRTC compilation failed: %.900s", text.c_str());
    }
    size_t code_size = 0;
    hiprtcGetCodeSize(prog, &code_size);
    std::vector<char> code(code_size);
    hiprtcGetCode(prog, code.data());
    hiprtcDestroyProgram(&prog);
    hipModule_t mod;
    PT_TRY(check_hip(hipModuleLoadData(&mod, code.data()), "hipModuleLoadData"));
    *module = (pt_module_t)mod;
    g_info.rtc_compiles++;
    return PT_OK;
}

pt_status pt_module_function(pt_module_t module, const char *name, pt_function_t *function)
{
    hipFunction_t fn;
    PT_TRY(check_hip(hipModuleGetFunction(&fn, (hipModule_t)module, name), "hipModuleGetFunction"));
    *function = (pt_function_t)fn;
    return PT_OK;
}

pt_status pt_module_unload(pt_module_t module)
{
    if (!module) return PT_OK;
    return check_hip(hipModuleUnload((hipModule_t)module), "hipModuleUnload");
}

pt_status pt_launch(pt_function_t function, unsigned grid_x, unsigned block_x,
                    void **params, pt_stream_t stream)
{
    if (!grid_x) return PT_OK;
    return check_hip(hipModuleLaunchKernel((hipFunction_t)function, grid_x, 1, 1, block_x, 1, 1,
                                           0, stream_of(stream), params, nullptr),
                     "hipModuleLaunchKernel");
}

// --------------------------------------------------------------- graphs
struct GraphHandle {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

pt_status pt_workspace_begin(void *base, size_t bytes)
{
    if (t_ws.active) return fail(PT_ERR_INVALID, "a workspace is already active on this thread");
    if ((base == nullptr) != (bytes == 0)) return fail(PT_ERR_INVALID, "workspace needs a base and a size");
    if (((uintptr_t)base & 255) != 0) return fail(PT_ERR_INVALID, "workspace base must be 256-byte aligned");
    t_ws = Workspace();
    t_ws.active = true;
    t_ws.measure = base == nullptr;
    t_ws.base = (char *)base;
    t_ws.bytes = bytes;
    return PT_OK;
}

pt_status pt_workspace_end(size_t *peak_bytes)
{
    if (!t_ws.active) return fail(PT_ERR_INVALID, "no workspace is active on this thread");
    if (peak_bytes) *peak_bytes = t_ws.peak;
    const bool leaked = !t_ws.stack.empty();
    t_ws = Workspace();
    if (leaked) return fail(PT_ERR_RUNTIME, "scratch still held at the end of the workspace");
    return PT_OK;
}

pt_status pt_stream_set_current(pt_stream_t stream)
{
    t_current = (hipStream_t)stream;
    return PT_OK;
}

pt_status pt_graph_begin_capture(pt_stream_t stream)
{
    PT_TRY(ensure_init());
    hipStream_t s = stream_of(stream);
    return check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal),
                     "hipStreamBeginCapture");
}

pt_status pt_graph_end_capture(pt_stream_t stream, pt_graph_t *graph)
{
    hipGraph_t g = nullptr;
    PT_TRY(check_hip(hipStreamEndCapture(stream_of(stream), &g), "hipStreamEndCapture"));
    GraphHandle *h = new GraphHandle;
    h->graph = g;
    hipError_t err = hipGraphInstantiate(&h->exec, g, nullptr, nullptr, 0);
    if (err != hipSuccess) {
        (void)hipGraphDestroy(g);
        delete h;
        return check_hip(err, "hipGraphInstantiate");
    }
    *graph = (pt_graph_t)h;
    return PT_OK;
}

pt_status pt_graph_end_capture_update(pt_stream_t stream, pt_graph_t graph)
{
    GraphHandle *h = (GraphHandle *)graph;
    hipGraph_t g = nullptr;
    PT_TRY(check_hip(hipStreamEndCapture(stream_of(stream), &g), "hipStreamEndCapture"));
    hipGraphExecUpdateResult result;
    hipGraphNode_t error_node = nullptr;
    hipError_t err = hipGraphExecUpdate(h->exec, g, &error_node, &result);
    if (err != hipSuccess || result != hipGraphExecUpdateSuccess) {
        (void)hipGetLastError();
        hipGraphExec_t fresh;
        hipError_t e2 = hipGraphInstantiate(&fresh, g, nullptr, nullptr, 0);
        if (e2 != hipSuccess) {
            (void)hipGraphDestroy(g);
            return check_hip(e2, "hipGraphInstantiate");
        }
        (void)hipGraphExecDestroy(h->exec);
        h->exec = fresh;
    }
    if (h->graph) (void)hipGraphDestroy(h->graph);
    h->graph = g;
    return PT_OK;
}

pt_status pt_graph_launch(pt_graph_t graph, pt_stream_t stream)
{
    GraphHandle *h = (GraphHandle *)graph;
    g_info.graph_launches++;
    return check_hip(hipGraphLaunch(h->exec, stream_of(stream)), "hipGraphLaunch");
}

pt_status pt_graph_destroy(pt_graph_t graph)
{
    GraphHandle *h = (GraphHandle *)graph;
    if (!h) return PT_OK;
    if (h->exec) (void)hipGraphExecDestroy(h->exec);
    if (h->graph) (void)hipGraphDestroy(h->graph);
    delete h;
    return PT_OK;
}

pt_status pt_graph_node_count(pt_graph_t graph, size_t *nodes)
{
    GraphHandle *h = (GraphHandle *)graph;
    size_t n = 0;
    PT_TRY(check_hip(hipGraphGetNodes(h->graph, nullptr, &n), "hipGraphGetNodes"));
    *nodes = n;
    return PT_OK;
}

}  // extern "C"
