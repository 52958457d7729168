// Shared host/device helpers for libwm_hip (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <cstdint>
#include <cstddef>
#include <cmath>
#include <string>

#include "../../include/wm_hip.h"

namespace wm {

// ---------------------------------------------------------------------------
// Host-side runtime state (defined in wm_runtime.hip)
// ---------------------------------------------------------------------------

// Record a failure message for wm_last_error() and return the status code.
int set_error(int status, const std::string& msg);
// Initialise device 0 if nothing is initialised yet.  Returns WM_OK or error.
int ensure_init();
hipStream_t stream();
int num_cus();
// The device the library runs on (wm_init's, or 0).
int device();

// Stream-ordered workspace from the caching allocator.  Freed blocks go back
// to the pool immediately: every kernel runs on the one library stream, so a
// later allocation can only be used by work enqueued after the earlier work.
void* ws_alloc(size_t bytes);
void ws_free(void* p);

struct Workspace {
    void* p = nullptr;
    explicit Workspace(size_t bytes) : p(bytes ? ws_alloc(bytes) : nullptr) {}
    ~Workspace() { if (p) ws_free(p); }
    Workspace(const Workspace&) = delete;
    Workspace& operator=(const Workspace&) = delete;
    template <class T> T* as() const { return static_cast<T*>(p); }
};

// Enqueue a copy of a small host table to device memory on the library
// stream without synchronising (pinned staging; see wm_runtime.hip).
int upload_async(void* dev_dst, const void* host_src, size_t bytes);

// Check the launch that was just enqueued.
int check_launch(const char* what);

// Called once per launch: counts it, and gives the events for it -- both
// null unless a kernel span is open (wm_span_begin); then each launch of
// the span gets its own (start, stop) pair.  Spans are single-threaded.
void span_events(hipEvent_t* start, hipEvent_t* stop);

// Every kernel of the library is launched through here: a plain launch, or
// one whose dispatch carries the open kernel span's events.
template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t st,
                          Args... args) {
    hipEvent_t e0, e1;
    span_events(&e0, &e1);
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, st, e0, e1, 0u, args...);
}

#define WM_TRY(expr)                 \
    do {                             \
        int wm_rc_ = (expr);         \
        if (wm_rc_ != WM_OK) return wm_rc_; \
    } while (0)

#define WM_CHECK_INIT() WM_TRY(::wm::ensure_init())

// Number of workgroups for a grid-stride launch over `items` work items of
// `per_block` items each: enough to fill every CU several times over, never
// more than the work needs.
inline unsigned grid_for(int64_t items, int64_t per_block, int waves_per_cu = 8) {
    if (items <= 0) return 1;
    int64_t need = (items + per_block - 1) / per_block;
    int64_t cap = (int64_t)num_cus() * waves_per_cu;
    if (cap < 1) cap = 1;
    return (unsigned)(need < cap ? need : cap);
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

// Streaming (non-temporal) 128-bit and 32-bit global accesses for data that is
// touched once per kernel: inputs read once, outputs written once, gradient
// read-modify-writes.  Measured on MI355X: a read-only sweep reaches ~6.8 TB/s
// with non-temporal loads against ~4.4 TB/s with cached loads when the
// caches hold dirty lines from earlier work.  Data that is reused across
// threads (broadcast vectors, partial sums) keeps ordinary cached loads.
typedef float wm_v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 ld_stream(const float* p) {
    wm_v4f v = __builtin_nontemporal_load(reinterpret_cast<const wm_v4f*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void st_stream(float* p, float4 v) {
    wm_v4f w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<wm_v4f*>(p));
}

__device__ __forceinline__ float ld_stream1(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream1(float* p, float v) { __builtin_nontemporal_store(v, p); }

// fp16 storage conversions with the reference's semantics (core/amp.h:15-72).
// half -> float is exact, subnormals included; the hardware conversion is
// exact with fp16 denormals enabled (the default mode for HIP kernels).
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;
}

// float -> half truncating toward zero, as float_to_half does: convert with
// the hardware's round-to-nearest-even, then step one ulp back toward zero if
// that rounded up in magnitude.  float_to_half sends |x| >= 65536 to Inf and
// keeps the top NaN payload bits, so those two cases take its bit formula.
// (Checked against float_to_half on every exponent x every 10-bit mantissa x
// the low-bit patterns at each truncation point, plus 42M random bit
// patterns.)
__device__ __forceinline__ uint32_t float_to_half_bits_rtz(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    if (__builtin_isnan(f)) return sign | 0x7C00u | ((x & 0x7FFFFFu) >> 13);
    if (fabsf(f) >= 65536.0f) return sign | 0x7C00u;
    const _Float16 h = (_Float16)f;
    uint32_t b = __builtin_bit_cast(uint16_t, h);
    if (fabsf((float)h) > fabsf(f)) b -= 1;
    return b;
}

// e^d within ~2 ulp, for the softmax family (whose arguments are x - max <= 0
// or a log-probability).  d log2(e) = n + r with n = rint(d * L_hi) and
// r = (d * L_hi - n) + d * L_lo (two fmas: L_hi + L_lo is log2(e) to ~2^-50),
// so |r| <= 0.5 + 2^-20; 2^r comes from the hardware exp2 and the exponent
// shift by n is exact (it rounds once for a subnormal result and overflows to
// inf past the float range).  d < -200 is clamped, since e^d underflows to
// 0 either way; NaN stays NaN.  Nine vector instructions against thirteen for
// the device expf, which adds range checks this argument range never needs.
__device__ __forceinline__ float exp_rr(float d) {
    d = d < -200.0f ? -200.0f : d;
    const float n = rintf(d * 1.44269502f);
    const float r = fmaf(d, 1.92596303e-08f, fmaf(d, 1.44269502f, -n));
    return ldexpf(__builtin_amdgcn_exp2f(r), (int)n);
}

// tanh within 2 ulp of the exact value for every float (the unary contract),
// in about half the instructions of the device library's tanhf:
//   |x| < 1   x + x^3 P(x^2), P of degree 6 fitted here for relative error
//             on [0, 1] (checked on every float below 1 in this exact
//             evaluation order: at most 1.13 ulp);
//   |x| >= 1  1 - 2 / (2^(2|x| log2 e) + 1) with the hardware exp2 and
//             reciprocal; with each of those off by a full ulp the result is
//             still within 1.83 ulp (checked on every float in [1, 10];
//             above that it is 1).
// The sign comes from x, so tanh(-0) = -0; NaN stays NaN; +-inf give +-1.
__device__ __forceinline__ float tanh_fast(float x) {
    const float a = fabsf(x);
    const float s = a * a;
    float p = fmaf(s, -0.000359800237f, 0.00230526947f);
    p = fmaf(s, p, -0.0079500787f);
    p = fmaf(s, p, 0.0214881711f);
    p = fmaf(s, p, -0.0538798086f);
    p = fmaf(s, p, 0.133323342f);
    p = fmaf(s, p, -0.333332956f);
    const float near0 = fmaf(a * s, p, a);
    const float e = __builtin_amdgcn_exp2f(a * 2.88539008f);  // 2 log2(e)
    const float far = fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);
    return copysignf(a < 1.0f ? near0 : far, x);
}

// Two floats -> two truncated halves packed low/high, as two
// float_to_half_bits_rtz calls.  The hardware's packed round-toward-zero
// conversion is exactly the truncation for every finite |x| < 65536 (normal
// and subnormal halves alike); NaN, infinities and |x| >= 65536 take the
// reference's bit formula in a branch a wave skips when none of its lanes
// holds one.
__device__ __forceinline__ uint32_t float2_to_half2_bits_rtz(float a, float b) {
    typedef __fp16 wm_h2 __attribute__((ext_vector_type(2)));
    uint32_t bits = __builtin_bit_cast(uint32_t, (wm_h2)__builtin_amdgcn_cvt_pkrtz(a, b));
    if (!(fabsf(a) < 65536.0f) || !(fabsf(b) < 65536.0f))
        bits = float_to_half_bits_rtz(a) | (float_to_half_bits_rtz(b) << 16);
    return bits;
}

// DPP lane moves inside a 16-lane row (deterministic, no LDS traffic).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 64 lanes of a wave; every lane gets the total.  Fixed
// combination order, so the result is deterministic.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x124>(v);  // row_ror:4
    v += dpp_mov<0x128>(v);  // row_ror:8
    float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));
    v = fmaxf(v, dpp_mov<0x4E>(v));
    v = fmaxf(v, dpp_mov<0x124>(v));
    v = fmaxf(v, dpp_mov<0x128>(v));
    float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Block-wide sum for blockDim.x == NT (multiple of 64).  `lds` must hold
// NT/64 floats.  Every thread gets the total; order is fixed.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* lds) {
    constexpr int NW = NT / 64;
    v = wave_sum(v);
    if (NW == 1) return v;
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += lds[i];
    return t;
}

}  // namespace wm
