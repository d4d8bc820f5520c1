// Host-only stand-in for the HIP runtime (libamdhip64.so.7), for CPU tests of
// the library's host code: model loading, step building, schedule choices,
// tuning, graph capture and the C ABI run without a GPU.
//
// Device memory is host memory (zero-filled), copies and fills are memcpy and
// memset, kernel launches are counted and do nothing, events measure elapsed
// "time" as 5 ns per kernel launch between them (so timed choices are
// deterministic), streams, graphs and events are small host objects.  The
// device looks like one MI355X: 256 CUs, gfx950, 160 KiB of LDS per CU.
// Only the entry points libaexrt_hip.so imports are provided, under the
// symbol versions it was linked against (hip_stub.map).  Test infrastructure:
// nothing of the product loads it; a test puts its directory first on
// LD_LIBRARY_PATH in a child process.
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <set>

namespace {

std::atomic<uint64_t> g_launches{0};
std::mutex g_mu;
std::set<void*> g_device_allocs;  // live hipMalloc blocks (double frees are reported)

struct StubEvent {
    uint64_t launches = 0;
};
struct StubStream {
    bool capturing = false;
};
struct StubGraph {
    int id = 0;
};

thread_local dim3 t_grid, t_block;
thread_local size_t t_shm = 0;
thread_local hipStream_t t_stream = nullptr;

void* alloc_zeroed(size_t size) {
    void* p = nullptr;
    if (posix_memalign(&p, 256, size ? size : 1) != 0) return nullptr;
    std::memset(p, 0, size);
    return p;
}

}  // namespace

extern "C" {

void** __hipRegisterFatBinary(const void* data) {
    static void* handle[2] = {nullptr, nullptr};
    handle[0] = const_cast<void*>(data);
    return handle;
}
void __hipRegisterFunction(void**, const void*, char*, const char*, unsigned int, uint3*, uint3*, dim3*, dim3*, int*) {}
void __hipRegisterVar(void**, void*, char*, char*, int, size_t, int, int) {}
void __hipUnregisterFatBinary(void**) {}

hipError_t __hipPushCallConfiguration(dim3 gridDim, dim3 blockDim, size_t sharedMem, hipStream_t stream) {
    t_grid = gridDim;
    t_block = blockDim;
    t_shm = sharedMem;
    t_stream = stream;
    return hipSuccess;
}
hipError_t __hipPopCallConfiguration(dim3* gridDim, dim3* blockDim, size_t* sharedMem, hipStream_t* stream) {
    *gridDim = t_grid;
    *blockDim = t_block;
    *sharedMem = t_shm;
    *stream = t_stream;
    return hipSuccess;
}

hipError_t hipLaunchKernel(const void* f, dim3 grid, dim3 block, void** args, size_t shm, hipStream_t stream) {
    (void)args, (void)stream;
    if (!f || grid.x == 0 || grid.y == 0 || grid.z == 0 || block.x * block.y * block.z == 0 ||
        block.x * block.y * block.z > 1024 || shm > 160 * 1024)
        return hipErrorInvalidConfiguration;
    g_launches.fetch_add(1);
    return hipSuccess;
}

hipError_t hipDeviceGetAttribute(int* pi, hipDeviceAttribute_t attr, int) {
    switch (attr) {
        case hipDeviceAttributeMultiprocessorCount: *pi = 256; break;
        case hipDeviceAttributeMaxSharedMemoryPerBlock: *pi = 160 * 1024; break;
        case hipDeviceAttributeWarpSize: *pi = 64; break;
        default: *pi = 0; break;
    }
    return hipSuccess;
}
hipError_t hipDeviceSynchronize(void) { return hipSuccess; }

hipError_t hipEventCreate(hipEvent_t* event) {
    *event = reinterpret_cast<hipEvent_t>(new StubEvent());
    return hipSuccess;
}
hipError_t hipEventCreateWithFlags(hipEvent_t* event, unsigned) { return hipEventCreate(event); }
hipError_t hipEventDestroy(hipEvent_t event) {
    delete reinterpret_cast<StubEvent*>(event);
    return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t event, hipStream_t) {
    if (!event) return hipErrorInvalidHandle;
    reinterpret_cast<StubEvent*>(event)->launches = g_launches.load();
    return hipSuccess;
}
hipError_t hipEventSynchronize(hipEvent_t event) { return event ? hipSuccess : hipErrorInvalidHandle; }
hipError_t hipEventElapsedTime(float* ms, hipEvent_t start, hipEvent_t stop) {
    if (!start || !stop) return hipErrorInvalidHandle;
    const uint64_t a = reinterpret_cast<StubEvent*>(start)->launches, b = reinterpret_cast<StubEvent*>(stop)->launches;
    *ms = 1e-3f + 5e-6f * (float)(b > a ? b - a : 0);
    return hipSuccess;
}

hipError_t hipMalloc(void** ptr, size_t size) {
    *ptr = alloc_zeroed(size);
    if (!*ptr) return hipErrorOutOfMemory;
    std::lock_guard<std::mutex> lock(g_mu);
    g_device_allocs.insert(*ptr);
    return hipSuccess;
}
hipError_t hipFree(void* ptr) {
    if (!ptr) return hipSuccess;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if (g_device_allocs.erase(ptr) != 1) {
            std::fprintf(stderr, "hip stub: hipFree of %p, which hipMalloc did not return or was freed\n", ptr);
            std::abort();
        }
    }
    std::free(ptr);
    return hipSuccess;
}
hipError_t hipHostMalloc(void** ptr, size_t size, unsigned int) {
    *ptr = alloc_zeroed(size);
    return *ptr ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipHostFree(void* ptr) {
    std::free(ptr);
    return hipSuccess;
}
hipError_t hipMemcpy(void* dst, const void* src, size_t n, hipMemcpyKind) {
    if (n && (!dst || !src)) return hipErrorInvalidValue;
    std::memmove(dst, src, n);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind kind, hipStream_t) {
    return hipMemcpy(dst, src, n, kind);
}
hipError_t hipMemset(void* dst, int value, size_t n) {
    if (n && !dst) return hipErrorInvalidValue;
    std::memset(dst, value, n);
    return hipSuccess;
}
hipError_t hipMemsetAsync(void* dst, int value, size_t n, hipStream_t) { return hipMemset(dst, value, n); }

hipError_t hipGetDevice(int* id) {
    *id = 0;
    return hipSuccess;
}
hipError_t hipSetDevice(int id) { return id == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDeviceCount(int* count) {
    *count = 1;
    return hipSuccess;
}
hipError_t hipGetDevicePropertiesR0600(hipDeviceProp_tR0600* prop, int id) {
    if (id != 0) return hipErrorInvalidDevice;
    std::memset(prop, 0, sizeof(*prop));
    std::snprintf(prop->name, sizeof(prop->name), "host stub of an MI355X");
    std::snprintf(prop->gcnArchName, sizeof(prop->gcnArchName), "gfx950:sramecc+:xnack-");
    prop->multiProcessorCount = 256;
    prop->warpSize = 64;
    prop->sharedMemPerBlock = 160 * 1024;
    prop->maxThreadsPerBlock = 1024;
    prop->totalGlobalMem = (size_t)288 << 30;
    return hipSuccess;
}
const char* hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "hip stub error"; }
hipError_t hipGetLastError(void) { return hipSuccess; }
hipError_t hipGetSymbolAddress(void** devPtr, const void* symbol) {
    // the host shadow of a __device__ variable has the variable's size
    *devPtr = const_cast<void*>(symbol);
    return symbol ? hipSuccess : hipErrorInvalidSymbol;
}

hipError_t hipOccupancyMaxActiveBlocksPerMultiprocessor(int* numBlocks, const void* f, int blockSize, size_t dyn) {
    if (!f || blockSize <= 0) return hipErrorInvalidValue;
    int by_waves = 32 * 64 / blockSize;  // 8 waves per SIMD, 4 SIMDs
    int by_lds = dyn ? (int)((160 * 1024) / (dyn + 4096)) : 8;
    *numBlocks = by_waves < by_lds ? by_waves : by_lds;
    return hipSuccess;
}

hipError_t hipStreamCreateWithFlags(hipStream_t* stream, unsigned int) {
    *stream = reinterpret_cast<hipStream_t>(new StubStream());
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t stream) {
    delete reinterpret_cast<StubStream*>(stream);
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipStreamWaitEvent(hipStream_t, hipEvent_t event, unsigned int) {
    return event ? hipSuccess : hipErrorInvalidHandle;
}
hipError_t hipStreamBeginCapture(hipStream_t stream, hipStreamCaptureMode) {
    if (!stream) return hipErrorInvalidValue;
    StubStream* s = reinterpret_cast<StubStream*>(stream);
    if (s->capturing) return hipErrorIllegalState;
    s->capturing = true;
    return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t stream, hipGraph_t* pGraph) {
    StubStream* s = reinterpret_cast<StubStream*>(stream);
    if (!s || !s->capturing) return hipErrorIllegalState;
    s->capturing = false;
    *pGraph = reinterpret_cast<hipGraph_t>(new StubGraph());
    return hipSuccess;
}
hipError_t hipGraphInstantiate(hipGraphExec_t* exec, hipGraph_t graph, hipGraphNode_t*, char*, size_t) {
    if (!graph) return hipErrorInvalidValue;
    *exec = reinterpret_cast<hipGraphExec_t>(new StubGraph());
    return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t exec, hipStream_t) { return exec ? hipSuccess : hipErrorInvalidValue; }
hipError_t hipGraphExecDestroy(hipGraphExec_t exec) {
    delete reinterpret_cast<StubGraph*>(exec);
    return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t graph) {
    delete reinterpret_cast<StubGraph*>(graph);
    return hipSuccess;
}

}  // extern "C"
