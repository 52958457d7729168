// Runtime of libwm_hip: device/stream state, error reporting, the caching
// device allocator, host<->device copies and measurement helpers.
//
// The reference keeps every tensor in a std::vector<float> (core/tensor.h:35-36)
// and allocates a fresh, zero-filled one per op output (core/tensor.cpp:408-414).
// On the GPU that allocation pattern would call hipMalloc/hipFree per op, and
// hipFree synchronises the device; the pool below keeps freed blocks and hands
// them back stream-ordered instead.
#include "wm_common.hpp"

#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <map>
#include <unordered_map>
#include <vector>

namespace wm {

namespace {

struct DeviceState {
    int device = -1;
    hipStream_t stream = nullptr;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    int cus = 0;
};

// An open kernel span (wm_span_begin .. wm_span_end): one (start, stop)
// event pair per launch, passed to hipExtLaunchKernelGGL with that launch.
// Used from one host thread (span_events does not lock).
constexpr int kSpanMax = 64;
struct Span {
    bool open = false;
    int launches = 0;
    hipEvent_t start[kSpanMax] = {}, stop[kSpanMax] = {};
    float kernel_ms[kSpanMax] = {};  // of the last closed span
    int closed = 0;                  // kernels timed in the last closed span
};

std::mutex g_mu;
DeviceState g_dev;
Span g_span;
thread_local std::string g_err;

// Size classes: 512 B granularity below 1 MiB, 2 MiB granularity above.
size_t size_class(size_t bytes) {
    if (bytes == 0) bytes = 1;
    const size_t small = 512, large = size_t(2) << 20;
    if (bytes < (size_t(1) << 20)) return (bytes + small - 1) / small * small;
    return (bytes + large - 1) / large * large;
}

struct Pool {
    std::multimap<size_t, void*> free_blocks;       // size class -> block
    std::unordered_map<void*, size_t> live;         // block -> size class
    size_t cached_bytes = 0;

    void release_all() {
        for (auto& kv : free_blocks) (void)hipFree(kv.second);
        free_blocks.clear();
        cached_bytes = 0;
    }
};
Pool g_pool;

int init_locked(int device) {
    if (g_dev.device == device && g_dev.stream) return WM_OK;
    if (g_dev.stream) {
        return set_error(WM_ERR_INVALID,
                         "wm_init: library already initialised on device " +
                             std::to_string(g_dev.device));
    }
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return set_error(WM_ERR_HIP, std::string("wm_init: no HIP device: ") +
                                         hipGetErrorString(e));
    if (device < 0 || device >= count)
        return set_error(WM_ERR_INVALID, "wm_init: device index out of range");
    if ((e = hipSetDevice(device)) != hipSuccess)
        return set_error(WM_ERR_HIP, std::string("hipSetDevice: ") + hipGetErrorString(e));
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
        return set_error(WM_ERR_HIP, std::string("hipGetDeviceProperties: ") +
                                         hipGetErrorString(e));
    // Default-priority, non-blocking stream: every library call is ordered on it.
    if ((e = hipStreamCreateWithFlags(&g_dev.stream, hipStreamNonBlocking)) != hipSuccess)
        return set_error(WM_ERR_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(e));
    if ((e = hipEventCreate(&g_dev.ev_start)) != hipSuccess ||
        (e = hipEventCreate(&g_dev.ev_stop)) != hipSuccess)
        return set_error(WM_ERR_HIP, std::string("hipEventCreate: ") + hipGetErrorString(e));
    g_dev.device = device;
    g_dev.cus = prop.multiProcessorCount;
    return WM_OK;
}

}  // namespace

int set_error(int status, const std::string& msg) {
    g_err = msg;
    return status;
}

int ensure_init() {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_dev.stream) return WM_OK;
    return init_locked(0);
}

hipStream_t stream() { return g_dev.stream; }
int device() { return g_dev.device >= 0 ? g_dev.device : 0; }
int num_cus() { return g_dev.cus > 0 ? g_dev.cus : 256; }

// Blocks the pool has handed out (wm_alloc and workspace), for tests that
// check an entry point allocates nothing.
static int64_t g_handouts = 0;

static void* pool_alloc(size_t bytes) {
    std::lock_guard<std::mutex> lk(g_mu);
    ++g_handouts;
    size_t cls = size_class(bytes);
    auto it = g_pool.free_blocks.find(cls);
    if (it != g_pool.free_blocks.end()) {
        void* p = it->second;
        g_pool.free_blocks.erase(it);
        g_pool.cached_bytes -= cls;
        g_pool.live[p] = cls;
        return p;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, cls);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        // Give cached blocks back to the driver and retry once.
        (void)hipStreamSynchronize(g_dev.stream);
        g_pool.release_all();
        e = hipMalloc(&p, cls);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    g_pool.live[p] = cls;
    return p;
}

static bool pool_free(void* p) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_pool.live.find(p);
    if (it == g_pool.live.end()) return false;
    g_pool.free_blocks.emplace(it->second, p);
    g_pool.cached_bytes += it->second;
    g_pool.live.erase(it);
    return true;
}

void* ws_alloc(size_t bytes) { return pool_alloc(bytes); }
void ws_free(void* p) { (void)pool_free(p); }


std::atomic<int64_t> g_launches{0};

void span_events(hipEvent_t* start, hipEvent_t* stop) {
    g_launches.fetch_add(1, std::memory_order_relaxed);
    if (!g_span.open) {
        *start = *stop = nullptr;
        return;
    }
    if (g_span.launches >= kSpanMax) {  // counted, not timed; wm_span_end reports it
        *start = *stop = nullptr;
        ++g_span.launches;
        return;
    }
    *start = g_span.start[g_span.launches];
    *stop = g_span.stop[g_span.launches];
    ++g_span.launches;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(WM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return WM_OK;
}

// Stream-ordered upload of a small host table (kernel launch descriptors)
// without waiting for the stream: the bytes go through a pinned staging
// buffer; before the buffer is rewritten the host waits for the event of the
// previous upload's copy, which has normally long completed.
namespace {
void* g_stage = nullptr;
size_t g_stage_bytes = 0;
hipEvent_t g_stage_ev = nullptr;
bool g_stage_pending = false;
}  // namespace

int upload_async(void* dev_dst, const void* host_src, size_t bytes) {
    if (bytes == 0) return WM_OK;
    WM_CHECK_INIT();
    std::lock_guard<std::mutex> lk(g_mu);
    hipError_t e = hipSuccess;
    if (g_stage_pending) {
        if ((e = hipEventSynchronize(g_stage_ev)) != hipSuccess)
            return set_error(WM_ERR_HIP, std::string("upload: ") + hipGetErrorString(e));
        g_stage_pending = false;
    }
    if (bytes > g_stage_bytes) {
        if (g_stage) (void)hipHostFree(g_stage);
        g_stage = nullptr;
        g_stage_bytes = 0;
        const size_t want = std::max<size_t>(bytes, size_t(64) << 10);
        if ((e = hipHostMalloc(&g_stage, want, hipHostMallocDefault)) != hipSuccess)
            return set_error(WM_ERR_NOMEM, std::string("upload: pinned staging: ") + hipGetErrorString(e));
        g_stage_bytes = want;
    }
    if (!g_stage_ev && (e = hipEventCreateWithFlags(&g_stage_ev, hipEventDisableTiming)) != hipSuccess)
        return set_error(WM_ERR_HIP, std::string("upload: ") + hipGetErrorString(e));
    std::memcpy(g_stage, host_src, bytes);
    if ((e = hipMemcpyAsync(dev_dst, g_stage, bytes, hipMemcpyHostToDevice, g_dev.stream)) != hipSuccess ||
        (e = hipEventRecord(g_stage_ev, g_dev.stream)) != hipSuccess)
        return set_error(WM_ERR_HIP, std::string("upload: ") + hipGetErrorString(e));
    g_stage_pending = true;
    return WM_OK;
}

}  // namespace wm

using namespace wm;

extern "C" {

int wm_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    return init_locked(device);
}

const char* wm_last_error(void) { return g_err.c_str(); }

int wm_alloc(void** ptr, size_t bytes) {
    if (!ptr) return set_error(WM_ERR_INVALID, "wm_alloc: null out pointer");
    WM_CHECK_INIT();
    void* p = pool_alloc(bytes);
    if (!p) {
        *ptr = nullptr;
        return set_error(WM_ERR_NOMEM, "wm_alloc: out of device memory for " +
                                           std::to_string(bytes) + " bytes");
    }
    *ptr = p;
    return WM_OK;
}

int wm_free(void* ptr) {
    if (!ptr) return WM_OK;
    if (!pool_free(ptr))
        return set_error(WM_ERR_INVALID, "wm_free: pointer was not allocated by wm_alloc");
    return WM_OK;
}

int wm_empty_cache(void) {
    WM_CHECK_INIT();
    hipError_t e = hipStreamSynchronize(g_dev.stream);
    std::lock_guard<std::mutex> lk(g_mu);
    g_pool.release_all();
    if (e != hipSuccess) return set_error(WM_ERR_HIP, hipGetErrorString(e));
    return WM_OK;
}

static int copy_sync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind,
                     const char* what) {
    if (bytes == 0) return WM_OK;
    if (!dst || !src) return set_error(WM_ERR_INVALID, std::string(what) + ": null pointer");
    WM_CHECK_INIT();
    // Enqueue on the library stream so the copy is ordered after every kernel
    // that produced or still reads the buffer.
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, g_dev.stream);
    if (e == hipSuccess) e = hipStreamSynchronize(g_dev.stream);
    if (e != hipSuccess) return set_error(WM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return WM_OK;
}

int wm_h2d(void* dst, const void* src, size_t bytes) {
    return copy_sync(dst, src, bytes, hipMemcpyHostToDevice, "wm_h2d");
}

int wm_d2h(void* dst, const void* src, size_t bytes) {
    return copy_sync(dst, src, bytes, hipMemcpyDeviceToHost, "wm_d2h");
}

int wm_d2d(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return WM_OK;
    if (!dst || !src) return set_error(WM_ERR_INVALID, "wm_d2d: null pointer");
    WM_CHECK_INIT();
    // Whole 16-byte aligned runs go through the streaming copy kernel (a
    // read and a write stream at the copy roofline, timed like every other
    // kernel); what is left (< 16 bytes, or misaligned buffers) through the
    // runtime's copy.
    size_t head = 0;
    if (aligned16(dst) && aligned16(src)) {
        head = bytes / 16 * 16;
        if (head) WM_TRY(wm_copy_kernel(static_cast<float*>(dst), static_cast<const float*>(src),
                                        (int64_t)(head / sizeof(float))));
    }
    if (head == bytes) return WM_OK;
    hipError_t e = hipMemcpyAsync(static_cast<char*>(dst) + head, static_cast<const char*>(src) + head, bytes - head,
                                  hipMemcpyDeviceToDevice, g_dev.stream);
    if (e != hipSuccess) return set_error(WM_ERR_HIP, std::string("wm_d2d: ") + hipGetErrorString(e));
    return WM_OK;
}

int wm_sync(void) {
    WM_CHECK_INIT();
    hipError_t e = hipStreamSynchronize(g_dev.stream);
    if (e != hipSuccess) return set_error(WM_ERR_HIP, std::string("wm_sync: ") + hipGetErrorString(e));
    return WM_OK;
}

int wm_device_cus(int* cus) {
    if (!cus) return set_error(WM_ERR_INVALID, "wm_device_cus: null pointer");
    WM_CHECK_INIT();
    *cus = num_cus();
    return WM_OK;
}

int wm_timer_start(void) {
    WM_CHECK_INIT();
    hipError_t e = hipEventRecord(g_dev.ev_start, g_dev.stream);
    if (e != hipSuccess) return set_error(WM_ERR_HIP, std::string("wm_timer_start: ") + hipGetErrorString(e));
    return WM_OK;
}

int wm_timer_stop(float* elapsed_ms) {
    if (!elapsed_ms) return set_error(WM_ERR_INVALID, "wm_timer_stop: null pointer");
    WM_CHECK_INIT();
    hipError_t e = hipEventRecord(g_dev.ev_stop, g_dev.stream);
    if (e == hipSuccess) e = hipEventSynchronize(g_dev.ev_stop);
    if (e == hipSuccess) e = hipEventElapsedTime(elapsed_ms, g_dev.ev_start, g_dev.ev_stop);
    if (e != hipSuccess) return set_error(WM_ERR_HIP, std::string("wm_timer_stop: ") + hipGetErrorString(e));
    return WM_OK;
}

int wm_pool_handouts(int64_t* count) {
    if (!count) return set_error(WM_ERR_INVALID, "wm_pool_handouts: null pointer");
    std::lock_guard<std::mutex> lk(g_mu);
    *count = g_handouts;
    return WM_OK;
}

int wm_span_begin(void) {
    WM_CHECK_INIT();
    hipError_t e = hipSuccess;
    for (int i = 0; i < kSpanMax && e == hipSuccess; ++i) {
        if (!g_span.start[i]) e = hipEventCreate(&g_span.start[i]);
        if (e == hipSuccess && !g_span.stop[i]) e = hipEventCreate(&g_span.stop[i]);
    }
    if (e != hipSuccess) return set_error(WM_ERR_HIP, std::string("wm_span_begin: ") + hipGetErrorString(e));
    g_span.open = true;
    g_span.launches = 0;
    return WM_OK;
}

int wm_span_end(float* kernel_ms, float* span_ms, int* kernels) {
    if (!kernel_ms) return set_error(WM_ERR_INVALID, "wm_span_end: null pointer");
    if (!g_span.open) return set_error(WM_ERR_INVALID, "wm_span_end: no open span");
    g_span.open = false;
    const int n = g_span.launches;
    if (kernels) *kernels = n;
    if (n == 0) return set_error(WM_ERR_INVALID, "wm_span_end: no kernel ran in the span");
    if (n > kSpanMax) return set_error(WM_ERR_INVALID, "wm_span_end: more launches than the span times");
    hipError_t e = hipEventSynchronize(g_span.stop[n - 1]);
    float total = 0.f;
    g_span.closed = 0;
    for (int i = 0; i < n && e == hipSuccess; ++i) {
        float ms = 0.f;
        e = hipEventElapsedTime(&ms, g_span.start[i], g_span.stop[i]);
        g_span.kernel_ms[i] = ms;
        total += ms;
    }
    if (e == hipSuccess) g_span.closed = n;
    if (e == hipSuccess && span_ms) e = hipEventElapsedTime(span_ms, g_span.start[0], g_span.stop[n - 1]);
    if (e != hipSuccess) return set_error(WM_ERR_HIP, std::string("wm_span_end: ") + hipGetErrorString(e));
    *kernel_ms = total;
    return WM_OK;
}

int wm_launch_count(int64_t* count) {
    if (!count) return set_error(WM_ERR_INVALID, "wm_launch_count: null pointer");
    *count = g_launches.load(std::memory_order_relaxed);
    return WM_OK;
}

int wm_span_kernel(int i, float* ms) {
    if (!ms) return set_error(WM_ERR_INVALID, "wm_span_kernel: null pointer");
    if (i < 0 || i >= g_span.closed) return set_error(WM_ERR_INVALID, "wm_span_kernel: no such kernel in the last span");
    *ms = g_span.kernel_ms[i];
    return WM_OK;
}

}  // extern "C"
