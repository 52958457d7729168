// wm_io.hip -- device-direct byte streams (include/wm_io.h): two pinned
// staging buffers alternate between the caller's byte source / sink and
// async copies on the library stream.  Host code only.
#include "wm_common.hpp"

#include "../../include/wm_io.h"

#include <algorithm>
#include <mutex>
#include <string>

namespace wm {
namespace {

struct Staging {
    std::mutex mu;
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};  // the last copy that used buf[i]
    bool pending[2] = {false, false};
};

Staging& staging() {
    static Staging s;
    return s;
}

int hip_fail(const char* who, hipError_t e) {
    return set_error(WM_ERR_HIP, std::string(who) + ": " + hipGetErrorString(e));
}

// Allocate the buffers and events once; wait for nothing.
int ready(Staging& s, const char* who) {
    for (int i = 0; i < 2; ++i) {
        hipError_t e;
        if (!s.buf[i] && (e = hipHostMalloc(&s.buf[i], WM_IO_CHUNK, hipHostMallocDefault)) != hipSuccess) {
            s.buf[i] = nullptr;
            return set_error(WM_ERR_NOMEM, std::string(who) + ": pinned staging: " + hipGetErrorString(e));
        }
        if (!s.done[i] && (e = hipEventCreateWithFlags(&s.done[i], hipEventDisableTiming)) != hipSuccess)
            return hip_fail(who, e);
    }
    return WM_OK;
}

// Wait until buf[i] is free (its last copy has finished).
int drain(Staging& s, int i, const char* who) {
    if (!s.pending[i]) return WM_OK;
    const hipError_t e = hipEventSynchronize(s.done[i]);
    s.pending[i] = false;
    return e == hipSuccess ? WM_OK : hip_fail(who, e);
}

}  // namespace
}  // namespace wm

using namespace wm;

int wm_read_into_device(wm_read_fn read, void* ctx, void* dst, int64_t bytes) {
    static const char* who = "wm_read_into_device";
    if (bytes < 0) return set_error(WM_ERR_INVALID, "wm_read_into_device: negative size");
    if (bytes == 0) return WM_OK;
    if (!read || !dst) return set_error(WM_ERR_INVALID, "wm_read_into_device: null pointer");
    WM_CHECK_INIT();
    Staging& s = staging();
    std::lock_guard<std::mutex> lk(s.mu);
    WM_TRY(ready(s, who));
    char* out = static_cast<char*>(dst);
    int64_t off = 0;
    for (int i = 0; off < bytes; i ^= 1) {
        const int64_t n = std::min<int64_t>(WM_IO_CHUNK, bytes - off);
        WM_TRY(drain(s, i, who));
        const int64_t got = read(ctx, s.buf[i], n);
        if (got > 0) {
            hipError_t e = hipMemcpyAsync(out + off, s.buf[i], (size_t)got, hipMemcpyHostToDevice, stream());
            if (e == hipSuccess) e = hipEventRecord(s.done[i], stream());
            if (e != hipSuccess) return hip_fail(who, e);
            s.pending[i] = true;
            off += got;
        }
        if (got != n)
            return set_error(WM_ERR_IO, "wm_read_into_device: source ended after " + std::to_string(off) + " of " +
                                            std::to_string(bytes) + " bytes");
    }
    return WM_OK;
}

int wm_write_from_device(wm_write_fn write, void* ctx, const void* src, int64_t bytes) {
    static const char* who = "wm_write_from_device";
    if (bytes < 0) return set_error(WM_ERR_INVALID, "wm_write_from_device: negative size");
    if (bytes == 0) return WM_OK;
    if (!write || !src) return set_error(WM_ERR_INVALID, "wm_write_from_device: null pointer");
    WM_CHECK_INIT();
    Staging& s = staging();
    std::lock_guard<std::mutex> lk(s.mu);
    WM_TRY(ready(s, who));
    const char* in = static_cast<const char*>(src);
    const int64_t nchunks = (bytes + WM_IO_CHUNK - 1) / WM_IO_CHUNK;
    auto issue = [&](int64_t c) -> int {
        const int i = (int)(c & 1);
        WM_TRY(drain(s, i, who));
        const int64_t off = c * WM_IO_CHUNK, n = std::min<int64_t>(WM_IO_CHUNK, bytes - off);
        hipError_t e = hipMemcpyAsync(s.buf[i], in + off, (size_t)n, hipMemcpyDeviceToHost, stream());
        if (e == hipSuccess) e = hipEventRecord(s.done[i], stream());
        if (e != hipSuccess) return hip_fail(who, e);
        s.pending[i] = true;
        return WM_OK;
    };
    WM_TRY(issue(0));
    for (int64_t c = 0; c < nchunks; ++c) {
        // The copy of chunk c+1 runs while chunk c is written.
        if (c + 1 < nchunks) WM_TRY(issue(c + 1));
        const int i = (int)(c & 1);
        WM_TRY(drain(s, i, who));
        const int64_t n = std::min<int64_t>(WM_IO_CHUNK, bytes - c * WM_IO_CHUNK);
        if (write(ctx, s.buf[i], n) != n) {
            // leave no copy in flight into a buffer the next call will reuse
            (void)drain(s, i ^ 1, who);
            return set_error(WM_ERR_IO, "wm_write_from_device: sink refused bytes after " +
                                            std::to_string(c * (int64_t)WM_IO_CHUNK) + " of " + std::to_string(bytes));
        }
    }
    return WM_OK;
}
