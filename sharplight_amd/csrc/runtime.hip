// Device, memory, stream and event entry points of libsharplight_hip, and the shared error plumbing.
//
// These are what the managed provider needs around the kernels: CheckAvailability / GetDevices /
// OpenDevice (src/Sharplight.Core/Runtime/IExecutionProvider.cs:25-40), the memory a compiled segment
// owns (IComputeDevice.Compile, IComputeDevice.cs:33-38) and SetInput / Execute / GetOutput
// (ICompiledSegment.cs:6-25), which the Vulkan provider implements with its own device, buffer and
// fence calls (src/Sharplight.Vulkan/VulkanDevice.cs, VulkanSegment.cs:374-479).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "common.hpp"

namespace slhip {

static thread_local char t_last_error[512] = "";

int fail(int status, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_last_error, sizeof t_last_error, fmt, ap);
    va_end(ap);
    return status;
}

int hip_fail(hipError_t e, const char* what)
{
    if (e == hipSuccess) return SLHIP_OK;
    return fail(SLHIP_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
}

int check_launch(const char* kernel)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(SLHIP_ERR_HIP, "launch of %s failed: %s", kernel, hipGetErrorString(e));
    return SLHIP_OK;
}

static constexpr int kMaxDevices = 64;
static std::mutex g_err_mu;
static uint32_t* g_err_word[kMaxDevices] = {};

// The device error record (see error_word): a file-scope device variable (zero at load), so that no
// call -- including a first one under graph capture -- allocates; each device holds its own copy, whose
// address is looked up once per device. In host code only that address is used: the variable's name
// there is a host-side stand-in.
__device__ __align__(32) uint32_t g_device_error[8];

int error_word(uint32_t** word)
{
    int dev = 0;
    SLHIP_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return fail(SLHIP_ERR_INVALID, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_err_mu);
    if (!g_err_word[dev]) {
        void* p = nullptr;
        SLHIP_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(g_device_error)));
        g_err_word[dev] = static_cast<uint32_t*>(p);
    }
    *word = g_err_word[dev];
    return SLHIP_OK;
}

int make_cache_rows(const slhip_cache_rows* in, int64_t T, CacheRowsDev* out)
{
    if (!in) return fail(SLHIP_ERR_INVALID, "cache rows are null");
    CacheRowsDev r{};
    r.mode = in->mode;
    r.ctx = in->ctx;
    if (in->ctx < 0) return fail(SLHIP_ERR_INVALID, "cache rows: negative context");
    switch (in->mode) {
    case SLHIP_ROWS_PAST:
        // CacheWriteOp.Run (src/Sharplight.Cpu/CacheWriteOp.cs:118-121)
        if (in->n_past < 0 || in->n_past + T > in->ctx)
            return fail(SLHIP_ERR_CACHE, "KV cache overflow: n_past %lld + T %lld > context %lld.",
                        static_cast<long long>(in->n_past), static_cast<long long>(T), static_cast<long long>(in->ctx));
        r.n_past = in->n_past;
        break;
    case SLHIP_ROWS_SEQ:
        if (!in->seq || in->slots < 1) return fail(SLHIP_ERR_INVALID, "cache rows: SEQ needs seq and slots >= 1");
        r.seq = in->seq;
        r.slots = in->slots;
        r.slot_ctx = in->ctx / in->slots;
        break;
    case SLHIP_ROWS_PAGED:
        if (!in->seq || !in->pages || in->block_size < 1 || in->page_slots < 0 || in->blocks_per_slot < 0)
            return fail(SLHIP_ERR_INVALID, "cache rows: PAGED needs seq, pages and block_size >= 1");
        r.seq = in->seq;
        r.pages = in->pages;
        r.page_slots = in->page_slots;
        r.bps = in->blocks_per_slot;
        r.bs = in->block_size;
        break;
    default: return fail(SLHIP_ERR_INVALID, "cache rows: bad mode %d", in->mode);
    }
    *out = r;
    return SLHIP_OK;
}

// Reads and clears the current device's error record after the stream drained; reports it as the
// reference reports the same condition (GatherOp.cs:60-63, CacheWriteOp.cs:103-117, KvPages.cs:38-49).
static int take_device_error()
{
    int dev = 0;
    SLHIP_CHECK_HIP(hipGetDevice(&dev));
    uint32_t* w = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_err_mu);
        if (dev >= 0 && dev < kMaxDevices) w = g_err_word[dev];
    }
    if (!w) return SLHIP_OK;
    uint32_t h[8] = {};
    SLHIP_CHECK_HIP(hipMemcpy(h, w, sizeof h, hipMemcpyDeviceToHost));
    if (!h[0]) return SLHIP_OK;
    SLHIP_CHECK_HIP(hipMemset(w, 0, sizeof h));
    const long long v1 = static_cast<long long>(static_cast<uint64_t>(h[4]) | (static_cast<uint64_t>(h[5]) << 32));
    const int slot = static_cast<int>(h[2]), pos = static_cast<int>(h[3]);
    switch (h[0]) {
    case kErrGatherIndex: {
        const long long id = static_cast<long long>(static_cast<uint64_t>(h[1]) | (static_cast<uint64_t>(h[2]) << 32));
        return fail(SLHIP_ERR_INDEX, "Gather index %lld out of range [0,%u).", id, h[3]);
    }
    case kErrCacheSeq:
        return fail(SLHIP_ERR_CACHE, "KV cache overflow: sequence row %u slot %d position %d (slot context %lld).",
                    h[1], slot, pos, v1);
    case kErrCachePageTable:
        return fail(SLHIP_ERR_CACHE, "Sequence slot %d / position %d outside the block table [%lld, %u].", slot, pos,
                    v1, h[6]);
    case kErrCacheBlock:
        return fail(SLHIP_ERR_CACHE, "Block %lld of slot %d (position %d) is outside the KV cache of %u rows.", v1,
                    slot, pos, h[6]);
    default: return fail(SLHIP_ERR_HIP, "device error record holds unknown code %u", h[0]);
    }
}

}  // namespace slhip

using namespace slhip;

extern "C" {

SLHIP_API const char* slhip_last_error(void) { return t_last_error; }

SLHIP_API int slhip_abi_version(void) { return SLHIP_ABI_VERSION; }

SLHIP_API int slhip_device_count(int* count)
{
    if (!count) return fail(SLHIP_ERR_INVALID, "count is null");
    *count = 0;
    hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) {
        *count = 0;
        return SLHIP_OK;
    }
    if (e != hipSuccess) {
        *count = 0;
        return fail(SLHIP_ERR_NO_DEVICE, "HIP runtime unavailable: %s", hipGetErrorString(e));
    }
    return SLHIP_OK;
}

SLHIP_API int slhip_device_props_get(int device, slhip_device_props* props)
{
    if (!props) return fail(SLHIP_ERR_INVALID, "props is null");
    int n = 0;
    int st = slhip_device_count(&n);
    if (st) return st;
    if (device < 0 || device >= n) return fail(SLHIP_ERR_INVALID, "device %d out of range [0,%d)", device, n);
    hipDeviceProp_t p;
    SLHIP_CHECK_HIP(hipGetDeviceProperties(&p, device));
    memset(props, 0, sizeof *props);
    snprintf(props->name, sizeof props->name, "%s", p.name);
    snprintf(props->arch, sizeof props->arch, "%s", p.gcnArchName);
    props->total_memory = static_cast<int64_t>(p.totalGlobalMem);
    props->compute_units = p.multiProcessorCount;
    props->wavefront_size = p.warpSize;
    props->pci_domain = p.pciDomainID;
    props->pci_bus = p.pciBusID;
    props->pci_device = p.pciDeviceID;
    props->clock_khz = p.clockRate;
    props->l2_bytes = p.l2CacheSize;
    props->max_threads_per_block = p.maxThreadsPerBlock;
    props->lds_bytes_per_block = static_cast<int32_t>(p.sharedMemPerBlock);
    return SLHIP_OK;
}

SLHIP_API int slhip_set_device(int device)
{
    SLHIP_CHECK_HIP(hipSetDevice(device));
    // The device's index-error word is allocated here, at open time, so that no later op call (possibly
    // under graph capture) allocates.
    uint32_t* w = nullptr;
    return error_word(&w);
}

SLHIP_API int slhip_get_device(int* device)
{
    if (!device) return fail(SLHIP_ERR_INVALID, "device is null");
    SLHIP_CHECK_HIP(hipGetDevice(device));
    return SLHIP_OK;
}

SLHIP_API int slhip_mem_info(size_t* free_bytes, size_t* total_bytes)
{
    size_t f = 0, t = 0;
    SLHIP_CHECK_HIP(hipMemGetInfo(&f, &t));
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return SLHIP_OK;
}

SLHIP_API int slhip_malloc(void** ptr, size_t bytes)
{
    if (!ptr) return fail(SLHIP_ERR_INVALID, "ptr is null");
    *ptr = nullptr;
    if (bytes == 0) return SLHIP_OK;
    SLHIP_CHECK_HIP(hipMalloc(ptr, bytes));
    return SLHIP_OK;
}

SLHIP_API int slhip_free(void* ptr)
{
    if (!ptr) return SLHIP_OK;
    SLHIP_CHECK_HIP(hipFree(ptr));
    return SLHIP_OK;
}

SLHIP_API int slhip_host_malloc(void** ptr, size_t bytes)
{
    if (!ptr) return fail(SLHIP_ERR_INVALID, "ptr is null");
    *ptr = nullptr;
    if (bytes == 0) return SLHIP_OK;
    SLHIP_CHECK_HIP(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
    return SLHIP_OK;
}

SLHIP_API int slhip_host_free(void* ptr)
{
    if (!ptr) return SLHIP_OK;
    SLHIP_CHECK_HIP(hipHostFree(ptr));
    return SLHIP_OK;
}

static int copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, slhip_stream stream)
{
    if (bytes == 0) return SLHIP_OK;
    if (!dst || !src) return fail(SLHIP_ERR_INVALID, "memcpy with a null pointer");
    SLHIP_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, kind, to_stream(stream)));
    return SLHIP_OK;
}

SLHIP_API int slhip_memcpy_h2d(void* dst, const void* src, size_t bytes, slhip_stream stream)
{
    return copy(dst, src, bytes, hipMemcpyHostToDevice, stream);
}

SLHIP_API int slhip_memcpy_d2h(void* dst, const void* src, size_t bytes, slhip_stream stream)
{
    return copy(dst, src, bytes, hipMemcpyDeviceToHost, stream);
}

SLHIP_API int slhip_memcpy_d2d(void* dst, const void* src, size_t bytes, slhip_stream stream)
{
    return copy(dst, src, bytes, hipMemcpyDeviceToDevice, stream);
}

SLHIP_API int slhip_memset(void* dst, int value, size_t bytes, slhip_stream stream)
{
    if (bytes == 0) return SLHIP_OK;
    if (!dst) return fail(SLHIP_ERR_INVALID, "memset of a null pointer");
    SLHIP_CHECK_HIP(hipMemsetAsync(dst, value, bytes, to_stream(stream)));
    return SLHIP_OK;
}

SLHIP_API int slhip_stream_create(slhip_stream* stream)
{
    if (!stream) return fail(SLHIP_ERR_INVALID, "stream is null");
    hipStream_t s = nullptr;
    SLHIP_CHECK_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return SLHIP_OK;
}

SLHIP_API int slhip_stream_destroy(slhip_stream stream)
{
    if (!stream) return SLHIP_OK;
    SLHIP_CHECK_HIP(hipStreamDestroy(to_stream(stream)));
    return SLHIP_OK;
}

SLHIP_API int slhip_stream_sync(slhip_stream stream)
{
    SLHIP_CHECK_HIP(hipStreamSynchronize(to_stream(stream)));
    return take_device_error();
}

SLHIP_API int slhip_event_create(slhip_event* event)
{
    if (!event) return fail(SLHIP_ERR_INVALID, "event is null");
    hipEvent_t e = nullptr;
    SLHIP_CHECK_HIP(hipEventCreate(&e));
    *event = e;
    return SLHIP_OK;
}

SLHIP_API int slhip_event_destroy(slhip_event event)
{
    if (!event) return SLHIP_OK;
    SLHIP_CHECK_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
    return SLHIP_OK;
}

SLHIP_API int slhip_event_record(slhip_event event, slhip_stream stream)
{
    if (!event) return fail(SLHIP_ERR_INVALID, "event is null");
    SLHIP_CHECK_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(event), to_stream(stream)));
    return SLHIP_OK;
}

SLHIP_API int slhip_event_synchronize(slhip_event event)
{
    if (!event) return fail(SLHIP_ERR_INVALID, "event is null");
    SLHIP_CHECK_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)));
    return SLHIP_OK;
}

SLHIP_API int slhip_event_elapsed_ms(float* ms, slhip_event start, slhip_event stop)
{
    if (!ms || !start || !stop) return fail(SLHIP_ERR_INVALID, "null argument");
    SLHIP_CHECK_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
    return SLHIP_OK;
}

SLHIP_API int slhip_graph_begin(slhip_stream stream)
{
    if (!stream) return fail(SLHIP_ERR_INVALID, "graph capture needs a created stream, not the null stream");
    SLHIP_CHECK_HIP(hipStreamBeginCapture(to_stream(stream), hipStreamCaptureModeThreadLocal));
    return SLHIP_OK;
}

SLHIP_API int slhip_graph_end(slhip_stream stream, slhip_graph* graph)
{
    if (!stream || !graph) return fail(SLHIP_ERR_INVALID, "null argument");
    *graph = nullptr;
    hipGraph_t g = nullptr;
    SLHIP_CHECK_HIP(hipStreamEndCapture(to_stream(stream), &g));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *graph = exec;
    return SLHIP_OK;
}

SLHIP_API int slhip_graph_launch(slhip_graph graph, slhip_stream stream)
{
    if (!graph) return fail(SLHIP_ERR_INVALID, "graph is null");
    SLHIP_CHECK_HIP(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph), to_stream(stream)));
    return SLHIP_OK;
}

SLHIP_API int slhip_graph_destroy(slhip_graph graph)
{
    if (!graph) return SLHIP_OK;
    SLHIP_CHECK_HIP(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph)));
    return SLHIP_OK;
}

}  // extern "C"
