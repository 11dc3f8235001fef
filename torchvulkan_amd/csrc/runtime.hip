// Runtime half of the C ABI: devices, one library stream per device, a
// hipMalloc-backed caching allocator and stream-ordered copies.
//
// Replaces, for the dense-contraction path, the reference's Vulkan runtime:
// VulkanContext device enumeration (src/vulkan/vulkan_context.cpp:251-357),
// DeviceContext memory counters (src/vulkan/device_context.h:64-68), the
// VulkanAllocator (src/vulkan/allocator.cpp:59-200) and its LRU buffer pools
// (src/vulkan/cache.cpp:78-89). The reference records work and flushes it with
// one blocking submit; here every call is enqueued on an in-order HIP stream,
// so hazards between kernels are ordered by the stream itself.
#include "tvk_common.h"
#include "scratch_pool.h"

#include <atomic>
#include <cstdlib>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>
#include <cstring>
#include <algorithm>

namespace tvk {

static thread_local std::string g_last_error;
void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

namespace {

constexpr int kMaxDevices = 64;

struct DeviceState {
    hipStream_t stream = nullptr;
    // size class -> cached free blocks
    std::map<size_t, std::vector<void*>> free_blocks;
    size_t allocated = 0;   // bytes in live blocks (size-class rounded)
    size_t peak = 0;
    size_t reserved = 0;    // bytes obtained from hipMalloc and not yet released
    size_t limit = 0;       // 0 = none
};

struct Block {
    size_t size;
    int device;
    bool host;   // served from pinned host memory (past the device's memory, strict allocation off)
};

std::mutex g_mu;
DeviceState g_dev[kMaxDevices];
std::unordered_map<void*, Block> g_live;

// Size classes: 512 B granules below 1 MiB, 2 MiB granules above, so cached
// blocks are reused across nearby request sizes without unbounded waste.
size_t size_class(size_t bytes) {
    if (bytes < (1u << 20)) return (bytes + 511) & ~size_t(511);
    const size_t g = size_t(2) << 20;
    return (bytes + g - 1) / g * g;
}

// TORCHVULKAN_STRICT_ALLOCATION, read when the library loads; tvk_set_strict_allocation changes it
std::atomic<int> g_strict_alloc{[] {
    const char* e = std::getenv("TORCHVULKAN_STRICT_ALLOCATION");
    return (e && e[0] && std::strcmp(e, "0") != 0) ? 1 : 0;
}()};
thread_local int g_last_spilled = 0;

// Pinned host blocks of tvk_host_malloc: start -> bytes
std::mutex g_host_mu;
std::map<uintptr_t, size_t> g_host_blocks;

bool valid_device(int d) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return false;
    return d >= 0 && d < n && d < kMaxDevices;
}

// Releases all cached blocks of one device (caller holds g_mu).
void release_cached_locked(int device) {
    DeviceState& st = g_dev[device];
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(device);
    if (st.stream) (void)hipStreamSynchronize(st.stream);
    for (auto& kv : st.free_blocks) {
        for (void* p : kv.second) {
            (void)hipFree(p);
            st.reserved -= kv.first;
        }
    }
    st.free_blocks.clear();
    (void)hipSetDevice(prev);
}

// The scratch pool's operations on one device: hipMalloc'd buffers and a
// device-wide drain before any free (every call makes the device current for
// its duration).
struct HipScratchBackend {
    typedef hipStream_t Stream;
    int device = 0;

    struct On {
        int prev = 0;
        explicit On(int d) { (void)hipGetDevice(&prev); (void)hipSetDevice(d); }
        ~On() { (void)hipSetDevice(prev); }
    };
    void* alloc(size_t bytes) {
        On on(device);
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
        return p;
    }
    void free(void* p) { On on(device); (void)hipFree(p); }
    void sync_device() { On on(device); (void)hipDeviceSynchronize(); }
};

struct DeviceScratch {
    HipScratchBackend backend;
    ScratchPool<HipScratchBackend> pool;
    explicit DeviceScratch(int d) : pool(backend) { backend.device = d; }
};

std::mutex g_scratch_mu;
DeviceScratch* g_scratch[kMaxDevices] = {};

DeviceScratch* device_scratch(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[device]) g_scratch[device] = new DeviceScratch(device);   // lives until the process ends
    return g_scratch[device];
}

}  // namespace

void* Scratch::get(size_t bytes, hipStream_t stream) {
    release();
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    auto* buf = device_scratch(dev)->pool.acquire(bytes, stream);
    if (!buf) return nullptr;
    lease_ = buf;
    device_ = dev;
    stream_ = stream;
    return buf->ptr;
}

void Scratch::release() {
    if (!lease_) return;
    device_scratch(device_)->pool.release(static_cast<ScratchPool<HipScratchBackend>::Buffer*>(lease_));
    lease_ = nullptr;
}

namespace {
constexpr int64_t kSplitCounters = 16384;   // 64 KB a stream: 16384 output tiles
// Counter arrays are never freed (a launch may hold one it looked up before a
// free could run); instead at most this many streams a device get one, 2 MB in
// all. Launches on further streams take the two-launch reduction.
constexpr int kMaxCounterStreams = 32;
std::mutex g_counter_mu;
std::map<std::pair<int, hipStream_t>, unsigned*> g_counters;
int g_counter_streams[kMaxDevices] = {};
}  // namespace

unsigned* split_counters(hipStream_t stream, int64_t count) {
    if (count <= 0 || count > kSplitCounters) return nullptr;
    // One handle that stands for every thread's own stream: launches from two
    // threads could overlap on one counter array.
    if (stream == hipStreamPerThread) return nullptr;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    // Under capture the graph could be replayed on another stream, concurrently
    // with launches on this one, so captured launches never take the array
    // (checked before the lookup: the stream may have used it before capture).
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_counter_mu);
    auto it = g_counters.find({dev, stream});
    if (it != g_counters.end()) return it->second;
    if (g_counter_streams[dev] >= kMaxCounterStreams) return nullptr;
    unsigned* p = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&p), kSplitCounters * sizeof(unsigned)) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    if (hipMemsetAsync(p, 0, kSplitCounters * sizeof(unsigned), stream) != hipSuccess) {
        (void)hipGetLastError();
        (void)hipFree(p);
        return nullptr;
    }
    g_counters[{dev, stream}] = p;
    ++g_counter_streams[dev];
    return p;
}

hipStream_t device_stream(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState& st = g_dev[device];
    if (!st.stream) {
        int prev = 0;
        (void)hipGetDevice(&prev);
        (void)hipSetDevice(device);
        // default priority: the library never creates prioritised streams
        (void)hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking);
        (void)hipSetDevice(prev);
    }
    return st.stream;
}

}  // namespace tvk

using namespace tvk;

extern "C" {

const char* tvk_last_error(void) { return g_last_error.c_str(); }

tvk_status tvk_device_count(int* count) {
    if (!count) return fail(TVK_ERR_INVALID, "tvk_device_count: count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;  // no runtime/GPU: zero devices, not an error
    *count = n;
    clear_error();
    return TVK_OK;
}

tvk_status tvk_set_device(int device) {
    if (!valid_device(device)) return fail(TVK_ERR_INVALID, "tvk_set_device: invalid device index " + std::to_string(device));
    TVK_HIP_CHECK(hipSetDevice(device));
    return TVK_OK;
}

tvk_status tvk_get_device(int* device) {
    if (!device) return fail(TVK_ERR_INVALID, "tvk_get_device: device is NULL");
    TVK_HIP_CHECK(hipGetDevice(device));
    return TVK_OK;
}

tvk_status tvk_get_stream(int device, void** stream) {
    if (!stream) return fail(TVK_ERR_INVALID, "tvk_get_stream: stream is NULL");
    if (!valid_device(device)) return fail(TVK_ERR_INVALID, "tvk_get_stream: invalid device index " + std::to_string(device));
    hipStream_t s = device_stream(device);
    if (!s) return fail(TVK_ERR_DEVICE, "tvk_get_stream: could not create the device stream");
    *stream = s;
    return TVK_OK;
}

tvk_status tvk_synchronize(int device) {
    if (!valid_device(device)) return fail(TVK_ERR_INVALID, "tvk_synchronize: invalid device index " + std::to_string(device));
    int prev = 0;
    TVK_HIP_CHECK(hipGetDevice(&prev));
    TVK_HIP_CHECK(hipSetDevice(device));
    hipError_t e = hipStreamSynchronize(device_stream(device));
    (void)hipSetDevice(prev);
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_synchronize: ") + hipGetErrorString(e));
    return TVK_OK;
}

tvk_status tvk_event_create(int device, int timing, void** event) {
    if (!event) return fail(TVK_ERR_INVALID, "tvk_event_create: event is NULL");
    *event = nullptr;
    if (!valid_device(device)) return fail(TVK_ERR_INVALID, "tvk_event_create: invalid device index " + std::to_string(device));
    int prev = 0;
    TVK_HIP_CHECK(hipGetDevice(&prev));
    TVK_HIP_CHECK(hipSetDevice(device));
    hipEvent_t e = nullptr;
    const hipError_t r = hipEventCreateWithFlags(&e, timing ? hipEventDefault : hipEventDisableTiming);
    (void)hipSetDevice(prev);
    if (r != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_event_create: ") + hipGetErrorString(r));
    *event = e;
    return TVK_OK;
}

tvk_status tvk_event_destroy(void* event) {
    if (event) TVK_HIP_CHECK(hipEventDestroy(static_cast<hipEvent_t>(event)));
    return TVK_OK;
}

tvk_status tvk_event_record(void* event, void* stream) {
    if (!event) return fail(TVK_ERR_INVALID, "tvk_event_record: event is NULL");
    TVK_HIP_CHECK(hipEventRecord(static_cast<hipEvent_t>(event), resolve_stream(stream)));
    return TVK_OK;
}

tvk_status tvk_event_query(void* event, int* done) {
    if (!event || !done) return fail(TVK_ERR_INVALID, "tvk_event_query: NULL argument");
    const hipError_t r = hipEventQuery(static_cast<hipEvent_t>(event));
    if (r == hipErrorNotReady) {
        *done = 0;
        return TVK_OK;
    }
    if (r != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_event_query: ") + hipGetErrorString(r));
    *done = 1;
    return TVK_OK;
}

tvk_status tvk_event_synchronize(void* event) {
    if (!event) return fail(TVK_ERR_INVALID, "tvk_event_synchronize: event is NULL");
    TVK_HIP_CHECK(hipEventSynchronize(static_cast<hipEvent_t>(event)));
    return TVK_OK;
}

tvk_status tvk_event_elapsed(void* start, void* end, float* ms) {
    if (!start || !end || !ms) return fail(TVK_ERR_INVALID, "tvk_event_elapsed: NULL argument");
    TVK_HIP_CHECK(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)));
    return TVK_OK;
}

tvk_status tvk_stream_wait_event(void* stream, void* event) {
    if (!event) return fail(TVK_ERR_INVALID, "tvk_stream_wait_event: event is NULL");
    TVK_HIP_CHECK(hipStreamWaitEvent(resolve_stream(stream), static_cast<hipEvent_t>(event), 0));
    return TVK_OK;
}

tvk_status tvk_stream_query(void* stream, int* done) {
    if (!done) return fail(TVK_ERR_INVALID, "tvk_stream_query: done is NULL");
    const hipError_t r = hipStreamQuery(resolve_stream(stream));
    if (r == hipErrorNotReady) {
        *done = 0;
        return TVK_OK;
    }
    if (r != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_stream_query: ") + hipGetErrorString(r));
    *done = 1;
    return TVK_OK;
}

tvk_status tvk_device_properties(int device, tvk_device_props* out) {
    if (!out) return fail(TVK_ERR_INVALID, "tvk_device_properties: out is NULL");
    if (!valid_device(device)) return fail(TVK_ERR_INVALID, "tvk_device_properties: invalid device index " + std::to_string(device));
    hipDeviceProp_t p;
    TVK_HIP_CHECK(hipGetDeviceProperties(&p, device));
    memset(out, 0, sizeof(*out));
    strncpy(out->name, p.name, sizeof(out->name) - 1);
    strncpy(out->arch, p.gcnArchName, sizeof(out->arch) - 1);
    out->total_memory = p.totalGlobalMem;
    out->compute_units = p.multiProcessorCount;
    out->clock_khz = p.clockRate;
    out->wavefront_size = p.warpSize;
    out->lds_per_block = p.sharedMemPerBlock;
    out->pci_bus_id = p.pciBusID;
    out->has_fp64 = 1;
    out->has_fp16 = 1;
    out->has_bf16 = 1;
    return TVK_OK;
}

tvk_status tvk_malloc(int device, size_t bytes, void** out) {
    if (!out) return fail(TVK_ERR_INVALID, "tvk_malloc: out is NULL");
    *out = nullptr;
    g_last_spilled = 0;
    if (!valid_device(device)) return fail(TVK_ERR_INVALID, "tvk_malloc: invalid device index " + std::to_string(device));
    if (bytes == 0) return TVK_OK;
    const size_t sz = size_class(bytes);
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState& st = g_dev[device];
    void* p = nullptr;
    bool host = false;
    hipError_t e = hipSuccess;
    if (st.limit && st.allocated + sz > st.limit) {
        e = hipErrorOutOfMemory;   // past the budget: spill or fail, as when the device is full
    } else {
        auto it = st.free_blocks.find(sz);
        if (it != st.free_blocks.end() && !it->second.empty()) {
            p = it->second.back();
            it->second.pop_back();
        } else {
            int prev = 0;
            (void)hipGetDevice(&prev);
            (void)hipSetDevice(device);
            e = hipMalloc(&p, sz);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                // give the cache back and retry once
                release_cached_locked(device);
                (void)hipSetDevice(device);
                e = hipMalloc(&p, sz);
            }
            (void)hipSetDevice(prev);
            if (e == hipSuccess) st.reserved += sz;
            else (void)hipGetLastError();
        }
    }
    if (!p) {
        // The reference's allocateBuffer (src/vulkan/allocator.cpp:171-200): past
        // the budget it allocates anyway unless strict allocation is on. Here the
        // memory then comes from pinned host memory, which kernels reach over the
        // host link.
        const std::string what = "tvk_malloc: out of memory on device " + std::to_string(device) + ". Tried to allocate " +
                                 std::to_string(bytes) + " bytes with " + std::to_string(st.allocated) + " bytes in use" +
                                 (st.limit ? " (limit " + std::to_string(st.limit) + ")" : std::string());
        if (g_strict_alloc.load()) return fail(TVK_ERR_OOM, what + ".");
        int prev = 0;
        (void)hipGetDevice(&prev);
        (void)hipSetDevice(device);
        e = hipHostMalloc(&p, sz, hipHostMallocMapped | hipHostMallocPortable);
        if (e == hipSuccess) {
            // kernels take the pointer as a device address: only a block the
            // device sees at the same address is handed out
            void* dp = nullptr;
            if (hipHostGetDevicePointer(&dp, p, 0) != hipSuccess || dp != p) {
                (void)hipGetLastError();
                (void)hipHostFree(p);
                p = nullptr;
                e = hipErrorOutOfMemory;
            }
        }
        (void)hipSetDevice(prev);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return fail(TVK_ERR_OOM, what + ", and pinned host memory could not hold it either.");
        }
        host = true;
        g_last_spilled = 1;
    }
    g_live[p] = Block{sz, device, host};
    st.allocated += sz;
    if (st.allocated > st.peak) st.peak = st.allocated;
    *out = p;
    return TVK_OK;
}

tvk_status tvk_free(void* ptr) {
    if (!ptr) return TVK_OK;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_live.find(ptr);
    if (it == g_live.end()) return fail(TVK_ERR_INVALID, "tvk_free: pointer was not allocated by tvk_malloc");
    DeviceState& st = g_dev[it->second.device];
    st.allocated -= it->second.size;
    if (it->second.host) {
        // spilled blocks are not cached: freed once the device has drained the
        // work that may still read or write them
        int prev = 0;
        (void)hipGetDevice(&prev);
        (void)hipSetDevice(it->second.device);
        (void)hipDeviceSynchronize();
        (void)hipHostFree(ptr);
        (void)hipSetDevice(prev);
    } else {
        st.free_blocks[it->second.size].push_back(ptr);
    }
    g_live.erase(it);
    return TVK_OK;
}

tvk_status tvk_set_strict_allocation(int strict) {
    g_strict_alloc.store(strict ? 1 : 0);
    return TVK_OK;
}

tvk_status tvk_get_strict_allocation(int* strict) {
    if (!strict) return fail(TVK_ERR_INVALID, "tvk_get_strict_allocation: strict is NULL");
    *strict = g_strict_alloc.load();
    return TVK_OK;
}

tvk_status tvk_last_malloc_spilled(int* spilled) {
    if (!spilled) return fail(TVK_ERR_INVALID, "tvk_last_malloc_spilled: spilled is NULL");
    *spilled = g_last_spilled;
    return TVK_OK;
}

tvk_status tvk_host_malloc(size_t bytes, void** out) {
    if (!out) return fail(TVK_ERR_INVALID, "tvk_host_malloc: out is NULL");
    *out = nullptr;
    if (bytes == 0) return TVK_OK;
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return fail(TVK_ERR_OOM, "tvk_host_malloc: could not pin " + std::to_string(bytes) + " bytes of host memory");
    }
    std::lock_guard<std::mutex> lk(g_host_mu);
    g_host_blocks[reinterpret_cast<uintptr_t>(p)] = bytes;
    *out = p;
    return TVK_OK;
}

tvk_status tvk_host_free(void* ptr) {
    if (!ptr) return TVK_OK;
    {
        std::lock_guard<std::mutex> lk(g_host_mu);
        auto it = g_host_blocks.find(reinterpret_cast<uintptr_t>(ptr));
        if (it == g_host_blocks.end()) return fail(TVK_ERR_INVALID, "tvk_host_free: pointer was not allocated by tvk_host_malloc");
        g_host_blocks.erase(it);
    }
    TVK_HIP_CHECK(hipHostFree(ptr));
    return TVK_OK;
}

tvk_status tvk_host_pointer_pinned(const void* ptr, int* pinned) {
    if (!pinned) return fail(TVK_ERR_INVALID, "tvk_host_pointer_pinned: pinned is NULL");
    *pinned = 0;
    const uintptr_t a = reinterpret_cast<uintptr_t>(ptr);
    std::lock_guard<std::mutex> lk(g_host_mu);
    auto it = g_host_blocks.upper_bound(a);
    if (it == g_host_blocks.begin()) return TVK_OK;
    --it;
    *pinned = a < it->first + std::max<size_t>(it->second, 1) ? 1 : 0;
    return TVK_OK;
}

tvk_status tvk_empty_cache(int device) {
    if (!valid_device(device)) return fail(TVK_ERR_INVALID, "tvk_empty_cache: invalid device index " + std::to_string(device));
    {
        std::lock_guard<std::mutex> lk(g_mu);
        release_cached_locked(device);
    }
    device_scratch(device)->pool.trim();   // idle scratch buffers, after the device has drained
    return TVK_OK;
}

tvk_status tvk_pointer_device(const void* ptr, int* device) {
    if (!device) return fail(TVK_ERR_INVALID, "tvk_pointer_device: device is NULL");
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_live.find(const_cast<void*>(ptr));
    *device = it == g_live.end() ? -1 : it->second.device;
    return TVK_OK;
}

tvk_status tvk_set_memory_limit(int device, size_t bytes) {
    if (device < 0 || device >= kMaxDevices) return fail(TVK_ERR_INVALID, "tvk_set_memory_limit: invalid device index");
    std::lock_guard<std::mutex> lk(g_mu);
    g_dev[device].limit = bytes;
    return TVK_OK;
}

#define TVK_STAT_GETTER(fn, field)                                                          \
    tvk_status fn(int device, size_t* bytes) {                                              \
        if (!bytes) return fail(TVK_ERR_INVALID, #fn ": bytes is NULL");                    \
        if (device < 0 || device >= kMaxDevices) return fail(TVK_ERR_INVALID, #fn ": invalid device index"); \
        std::lock_guard<std::mutex> lk(g_mu);                                               \
        *bytes = g_dev[device].field;                                                       \
        return TVK_OK;                                                                      \
    }
TVK_STAT_GETTER(tvk_memory_allocated, allocated)
TVK_STAT_GETTER(tvk_max_memory_allocated, peak)

// The caching allocator's blocks plus the scratch pool's buffers.
tvk_status tvk_memory_reserved(int device, size_t* bytes) {
    if (!bytes) return fail(TVK_ERR_INVALID, "tvk_memory_reserved: bytes is NULL");
    if (device < 0 || device >= kMaxDevices) return fail(TVK_ERR_INVALID, "tvk_memory_reserved: invalid device index");
    size_t pool = 0;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        if (g_scratch[device]) pool = g_scratch[device]->pool.total_bytes();
    }
    std::lock_guard<std::mutex> lk(g_mu);
    *bytes = g_dev[device].reserved + pool;
    return TVK_OK;
}

tvk_status tvk_reset_peak_memory_stats(int device) {
    if (device < 0 || device >= kMaxDevices) return fail(TVK_ERR_INVALID, "tvk_reset_peak_memory_stats: invalid device index");
    std::lock_guard<std::mutex> lk(g_mu);
    g_dev[device].peak = g_dev[device].allocated;
    return TVK_OK;
}

tvk_status tvk_mem_get_info(int device, size_t* free_bytes, size_t* total_bytes) {
    if (!free_bytes || !total_bytes) return fail(TVK_ERR_INVALID, "tvk_mem_get_info: NULL output");
    if (!valid_device(device)) return fail(TVK_ERR_INVALID, "tvk_mem_get_info: invalid device index " + std::to_string(device));
    int prev = 0;
    TVK_HIP_CHECK(hipGetDevice(&prev));
    TVK_HIP_CHECK(hipSetDevice(device));
    hipError_t e = hipMemGetInfo(free_bytes, total_bytes);
    (void)hipSetDevice(prev);
    if (e != hipSuccess) return fail(TVK_ERR_DEVICE, std::string("tvk_mem_get_info: ") + hipGetErrorString(e));
    return TVK_OK;
}

tvk_status tvk_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream, int blocking) {
    if (bytes == 0) return TVK_OK;
    if (!dst || !src) return fail(TVK_ERR_INVALID, "tvk_memcpy_h2d: NULL pointer");
    hipStream_t s = resolve_stream(stream);
    TVK_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
    if (blocking) TVK_HIP_CHECK(hipStreamSynchronize(s));
    return TVK_OK;
}

tvk_status tvk_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream, int blocking) {
    if (bytes == 0) return TVK_OK;
    if (!dst || !src) return fail(TVK_ERR_INVALID, "tvk_memcpy_d2h: NULL pointer");
    hipStream_t s = resolve_stream(stream);
    TVK_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
    if (blocking) TVK_HIP_CHECK(hipStreamSynchronize(s));
    return TVK_OK;
}

tvk_status tvk_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return TVK_OK;
    if (!dst || !src) return fail(TVK_ERR_INVALID, "tvk_memcpy_d2d: NULL pointer");
    TVK_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, resolve_stream(stream)));
    return TVK_OK;
}

}  // extern "C"
