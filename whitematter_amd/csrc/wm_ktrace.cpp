// libwm_ktrace: in-process kernel-dispatch timing for bench.py.
//
// The durations a rocprofv3 kernel trace reports are the dispatch packets'
// own start / end timestamps, which rocprofiler-sdk reads from the
// completion signal of every dispatch.  Event pairs recorded around a
// dispatch (hipExtLaunchKernelGGL's start / stop events) measure marker
// packets as well and read about 4 us longer per dispatch on MI355X.  This
// library registers itself as a rocprofiler-sdk tool inside the benchmark
// process (rocprofiler_force_configure, before the HIP runtime starts) and
// traces kernel dispatches with callbacks: the dispatches enqueued while a
// window is open (wm_ktrace_begin .. wm_ktrace_end) are tagged at enqueue
// time, on the launching thread, and their start / end timestamps are kept
// when they complete -- the same numbers a trace of the same run shows,
// for exactly the op's own dispatches (a cache-flush fill launched before
// the window is not among them).
//
// Measurement only: nothing in libwm_hip or the Tensor library uses it.  It
// is host code (no kernels) linked against librocprofiler-sdk.
//
// Use from one host thread:
//   wm_ktrace_init()             once, before the first HIP call of the process
//   wm_ktrace_begin()            open a window
//   ... launch the op's kernels ...
//   wm_ktrace_end(&n)            close it: n dispatches were enqueued in it
//   wm_ktrace_take(timeout, ms)  wait for the n to complete; their durations
#include <rocprofiler-sdk/registration.h>
#include <rocprofiler-sdk/rocprofiler.h>

#include <cxxabi.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

struct Dispatch {
    uint64_t id;         // dispatch id: issue order
    uint64_t kernel_id;  // key into g_names
    uint64_t start_ns, end_ns;
};

// Window tag carried from a dispatch's enqueue to its completion in the
// record's user data: 0 = not timed, otherwise the window's number.
std::atomic<uint64_t> g_window{0};     // the open window's number (0: none open)
uint64_t g_last_window = 0;            // the last window opened
std::atomic<int> g_enqueued{0};        // dispatches enqueued in the last window

std::mutex g_mu;
std::vector<Dispatch> g_done;                       // completed dispatches of the last window
std::vector<Dispatch> g_taken;                      // the last wm_ktrace_take's records, issue order
std::unordered_map<uint64_t, std::string> g_names;  // kernel id -> demangled name

rocprofiler_context_id_t g_ctx{0};
int g_state = 0;  // 0 not configured, 1 tracing, -1 failed
std::string g_err;

void on_dispatch(rocprofiler_callback_tracing_record_t rec, rocprofiler_user_data_t* user, void*) {
    if (rec.kind != ROCPROFILER_CALLBACK_TRACING_KERNEL_DISPATCH) return;
    if (rec.operation == ROCPROFILER_KERNEL_DISPATCH_ENQUEUE) {
        if (rec.phase == ROCPROFILER_CALLBACK_PHASE_ENTER) {
            const uint64_t w = g_window.load(std::memory_order_acquire);
            user->value = w;
            if (w) g_enqueued.fetch_add(1, std::memory_order_acq_rel);
        }
        return;
    }
    if (rec.operation != ROCPROFILER_KERNEL_DISPATCH_COMPLETE || user->value == 0) return;
    const auto* d = static_cast<const rocprofiler_callback_tracing_kernel_dispatch_data_t*>(rec.payload);
    std::lock_guard<std::mutex> lk(g_mu);
    if (user->value != g_last_window) return;  // a window that was already given up on
    g_done.push_back({d->dispatch_info.dispatch_id, d->dispatch_info.kernel_id, d->start_timestamp,
                      d->end_timestamp});
}

void on_code_object(rocprofiler_callback_tracing_record_t rec, rocprofiler_user_data_t*, void*) {
    if (rec.kind != ROCPROFILER_CALLBACK_TRACING_CODE_OBJECT ||
        rec.operation != ROCPROFILER_CODE_OBJECT_DEVICE_KERNEL_SYMBOL_REGISTER ||
        rec.phase != ROCPROFILER_CALLBACK_PHASE_LOAD)
        return;
    const auto* d =
        static_cast<const rocprofiler_callback_tracing_code_object_kernel_symbol_register_data_t*>(rec.payload);
    std::string name = d->kernel_name ? d->kernel_name : "";
    int status = 0;
    char* dem = abi::__cxa_demangle(name.c_str(), nullptr, nullptr, &status);
    if (status == 0 && dem) name = dem;
    std::free(dem);
    std::lock_guard<std::mutex> lk(g_mu);
    g_names[d->kernel_id] = name;
}

#define KT_TRY(call, what)                                                        \
    do {                                                                           \
        rocprofiler_status_t s_ = (call);                                          \
        if (s_ != ROCPROFILER_STATUS_SUCCESS) {                                    \
            g_err = std::string(what) + ": " + rocprofiler_get_status_string(s_); \
            return -1;                                                             \
        }                                                                          \
    } while (0)

int tool_init(rocprofiler_client_finalize_t, void*) {
    KT_TRY(rocprofiler_create_context(&g_ctx), "create_context");
    KT_TRY(rocprofiler_configure_callback_tracing_service(g_ctx, ROCPROFILER_CALLBACK_TRACING_CODE_OBJECT, nullptr,
                                                          0, on_code_object, nullptr),
           "code object tracing");
    KT_TRY(rocprofiler_configure_callback_tracing_service(g_ctx, ROCPROFILER_CALLBACK_TRACING_KERNEL_DISPATCH,
                                                          nullptr, 0, on_dispatch, nullptr),
           "kernel dispatch tracing");
    int valid = 0;
    if (rocprofiler_context_is_valid(g_ctx, &valid) != ROCPROFILER_STATUS_SUCCESS || !valid) {
        g_err = "context is not valid";
        return -1;
    }
    KT_TRY(rocprofiler_start_context(g_ctx), "start_context");
    g_state = 1;
    return 0;
}

void tool_fini(void*) {}

rocprofiler_tool_configure_result_t* configure(uint32_t, const char*, uint32_t, rocprofiler_client_id_t* id) {
    id->name = "wm_ktrace";
    static rocprofiler_tool_configure_result_t cfg{sizeof(rocprofiler_tool_configure_result_t), &tool_init,
                                                   &tool_fini, nullptr};
    return &cfg;
}

}  // namespace

extern "C" {

// Register the tracer.  Must run before the process's first HIP / HSA call.
// Returns 0 when dispatches are being traced; otherwise -1 and
// wm_ktrace_error() says why (another tool such as rocprofv3 already holds
// the configuration, or the runtime started first).
int wm_ktrace_init(void) {
    if (g_state == 1) return 0;
    if (g_state == -1) return -1;
    int inited = 0;
    rocprofiler_is_initialized(&inited);
    if (inited != 0) {
        g_state = -1;
        g_err = "rocprofiler is already configured in this process (another tool, or the runtime started first)";
        return -1;
    }
    rocprofiler_status_t s = rocprofiler_force_configure(&configure);
    if (s != ROCPROFILER_STATUS_SUCCESS) {
        g_state = -1;
        g_err = std::string("rocprofiler_force_configure: ") + rocprofiler_get_status_string(s);
        return -1;
    }
    if (g_state != 1) {  // force_configure runs tool_init before it returns; it failed
        if (g_err.empty()) g_err = "tool initialisation did not run";
        g_state = -1;
        return -1;
    }
    return 0;
}

const char* wm_ktrace_error(void) { return g_err.c_str(); }

// Open a timing window: every dispatch enqueued from now until
// wm_ktrace_end is recorded when it completes.
int wm_ktrace_begin(void) {
    if (g_state != 1) return -1;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_done.clear();
        ++g_last_window;
    }
    g_enqueued.store(0, std::memory_order_release);
    g_window.store(g_last_window, std::memory_order_release);
    return 0;
}

// Close the window; *enqueued = the dispatches enqueued while it was open.
int wm_ktrace_end(int* enqueued) {
    if (g_state != 1) return -1;
    g_window.store(0, std::memory_order_release);
    if (enqueued) *enqueued = g_enqueued.load(std::memory_order_acquire);
    return 0;
}

// Wait (up to timeout_ms) until every dispatch of the last window has
// completed, then write their durations in ms, in issue order, into
// ms[0 .. n-1] (n = the window's dispatch count; at most max are written).
// The records stay available to wm_ktrace_name until the next take.
// Returns the number of dispatches, or -1 if they did not all complete in
// time (wm_ktrace_error).
int wm_ktrace_take(int timeout_ms, double* ms, int max) {
    if (g_state != 1) return -1;
    const int n = g_enqueued.load(std::memory_order_acquire);
    const auto t_end = std::chrono::steady_clock::now() + std::chrono::milliseconds(timeout_ms);
    for (;;) {
        {
            std::lock_guard<std::mutex> lk(g_mu);
            if ((int)g_done.size() >= n) {
                std::sort(g_done.begin(), g_done.end(),
                          [](const Dispatch& a, const Dispatch& b) { return a.id < b.id; });
                g_taken = g_done;
                g_done.clear();
                if (ms)
                    for (int i = 0; i < n && i < max; ++i)
                        ms[i] = (double)(g_taken[i].end_ns - g_taken[i].start_ns) * 1e-6;
                return n;
            }
        }
        if (std::chrono::steady_clock::now() > t_end) {
            g_err = "not every dispatch of the window completed in time";
            return -1;
        }
        std::this_thread::sleep_for(std::chrono::microseconds(100));
    }
}

// The demangled kernel name of dispatch i of the last take (empty if unknown).
int wm_ktrace_name(int i, char* buf, int len) {
    if (!buf || len <= 0) return -1;
    std::lock_guard<std::mutex> lk(g_mu);
    if (i < 0 || i >= (int)g_taken.size()) return -1;
    auto it = g_names.find(g_taken[i].kernel_id);
    const std::string s = it == g_names.end() ? std::string() : it->second;
    std::strncpy(buf, s.c_str(), (size_t)len - 1);
    buf[len - 1] = '\0';
    return 0;
}

}  // extern "C"
