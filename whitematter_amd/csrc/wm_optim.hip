// Parameter-update kernels: optimizer steps (SGD, Adam, AdamW, RMSprop),
// gradient clipping and gradient unscaling (reference core/optimizer.cpp,
// core/amp.h:125-147).
//
// Every update is one streaming pass over the parameter's arrays: each
// element's state is read once and written once, 128-bit non-temporal
// accesses when every array is 16-byte aligned and n % 4 == 0.  The
// arithmetic is the reference loop body's float expression in its source
// order, with contraction into fused multiply-adds switched off and IEEE
// division and square root (hipcc's defaults for float), so the results
// equal a strict IEEE evaluation of the reference source bit for bit.
//
// The two reductions (sum of squares for the gradient norm, first non-finite
// position for unscaling) are fixed-partition two-pass reductions: per-block
// partials, then one block combining them in order, so they are
// deterministic.
#include "wm_common.hpp"
#include "../../include/wm_optim.h"

#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <vector>

namespace wm {

constexpr int kBlock = 256;

// ---------------------------------------------------------------------------
// Per-element updates (the reference loop bodies)
// ---------------------------------------------------------------------------

struct SgdArgs {
    float lr, momentum;
};

// core/optimizer.cpp:26-33
template <bool MOM>
__device__ __forceinline__ void sgd_elem(float& p, float g, float& vel, const SgdArgs& a) {
#pragma clang fp contract(off)
    if constexpr (MOM) {
        vel = a.momentum * vel + g;
        p = p - a.lr * vel;
    } else {
        p = p - a.lr * g;
    }
}

struct AdamArgs {
    float lr, beta1, beta2, omb1, omb2, eps, bc1, bc2, wd;
};

// core/optimizer.cpp:55-64 (Adam), :85-98 (AdamW, DECOUPLED)
template <bool DECOUPLED>
__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v, const AdamArgs& a) {
#pragma clang fp contract(off)
    m = a.beta1 * m + a.omb1 * g;
    v = a.beta2 * v + a.omb2 * g * g;
    const float m_hat = m / a.bc1;
    const float v_hat = v / a.bc2;
    if constexpr (DECOUPLED) p = p - a.lr * (m_hat / (sqrtf(v_hat) + a.eps) + a.wd * p);
    else p = p - a.lr * m_hat / (sqrtf(v_hat) + a.eps);
}

struct RmsArgs {
    float lr, alpha, oma, eps, momentum, wd;
};

// core/optimizer.cpp:116-136
template <bool WD, bool MOM>
__device__ __forceinline__ void rms_elem(float& p, float g, float& v, float& buf, const RmsArgs& a) {
#pragma clang fp contract(off)
    if constexpr (WD) g = g + a.wd * p;
    v = a.alpha * v + a.oma * g * g;
    const float avg = sqrtf(v) + a.eps;
    if constexpr (MOM) {
        buf = a.momentum * buf + g / avg;
        p = p - a.lr * buf;
    } else {
        p = p - a.lr * g / avg;
    }
}

// ---------------------------------------------------------------------------
// One streaming kernel for all updates: p and g, plus up to two state arrays
// (s1, s2), updated by UPD::apply(p, g, s1, s2).
// ---------------------------------------------------------------------------

template <int KIND, bool A, bool B>
struct Upd;  // KIND 0: SGD (A = momentum); 1: Adam (A = decoupled); 2: RMSprop (A = wd, B = momentum)

template <bool A, bool B>
struct Upd<0, A, B> {
    SgdArgs a;
    static constexpr int NS = A ? 1 : 0;
    __device__ __forceinline__ void operator()(float& p, float g, float& s1, float&) const { sgd_elem<A>(p, g, s1, a); }
};
template <bool A, bool B>
struct Upd<1, A, B> {
    AdamArgs a;
    static constexpr int NS = 2;
    __device__ __forceinline__ void operator()(float& p, float g, float& s1, float& s2) const {
        adam_elem<A>(p, g, s1, s2, a);
    }
};
template <bool A, bool B>
struct Upd<2, A, B> {
    RmsArgs a;
    static constexpr int NS = B ? 2 : 1;
    __device__ __forceinline__ void operator()(float& p, float g, float& s1, float& s2) const {
        rms_elem<A, B>(p, g, s1, s2, a);
    }
};

template <class U>
__global__ void __launch_bounds__(kBlock) update_vec_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                             float* __restrict__ s1, float* __restrict__ s2,
                                                             int64_t n4, U upd) {
    constexpr int NS = U::NS;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
        const int64_t e = 4 * i;
        float4 vp = ld_stream(p + e);
        const float4 vg = ld_stream(g + e);
        float4 v1 = NS > 0 ? ld_stream(s1 + e) : make_float4(0.f, 0.f, 0.f, 0.f);
        float4 v2 = NS > 1 ? ld_stream(s2 + e) : make_float4(0.f, 0.f, 0.f, 0.f);
        upd(vp.x, vg.x, v1.x, v2.x);
        upd(vp.y, vg.y, v1.y, v2.y);
        upd(vp.z, vg.z, v1.z, v2.z);
        upd(vp.w, vg.w, v1.w, v2.w);
        st_stream(p + e, vp);
        if (NS > 0) st_stream(s1 + e, v1);
        if (NS > 1) st_stream(s2 + e, v2);
    }
}

template <class U>
__global__ void __launch_bounds__(kBlock) update_scalar_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                                float* __restrict__ s1, float* __restrict__ s2,
                                                                int64_t n, U upd) {
    constexpr int NS = U::NS;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        float vp = p[i];
        float v1 = NS > 0 ? s1[i] : 0.f;
        float v2 = NS > 1 ? s2[i] : 0.f;
        upd(vp, g[i], v1, v2);
        p[i] = vp;
        if (NS > 0) s1[i] = v1;
        if (NS > 1) s2[i] = v2;
    }
}

template <class U>
int launch_update(float* p, const float* g, float* s1, float* s2, int64_t n, const U& upd, const char* what) {
    if (n == 0) return WM_OK;
    constexpr int NS = U::NS;
    const bool vec = n % 4 == 0 && aligned16(p) && aligned16(g) && (NS < 1 || aligned16(s1)) &&
                     (NS < 2 || aligned16(s2));
    if (vec)
        launch_kernel(update_vec_kernel<U>, dim3(grid_for(n / 4, kBlock, 16)), dim3(kBlock), 0, stream(), p, g,
                           s1, s2, n / 4, upd);
    else
        launch_kernel(update_scalar_kernel<U>, dim3(grid_for(n, kBlock, 16)), dim3(kBlock), 0, stream(), p, g,
                           s1, s2, n, upd);
    return check_launch(what);
}

// ---------------------------------------------------------------------------
// Sum of squares (gradient norm) and clipping
// ---------------------------------------------------------------------------

constexpr int kMaxPart = 1024;

__global__ void __launch_bounds__(kBlock) sumsq_partial_kernel(const float* __restrict__ g, int64_t n,
                                                                float* __restrict__ part) {
    __shared__ float lds[kBlock / 64];
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    float s = 0.f;
    const bool vec = ((uintptr_t)g & 15u) == 0;
    const int64_t n4 = vec ? n / 4 : 0;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
        const float4 v = ld_stream(g + 4 * i);
        s += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) s += g[i] * g[i];
    s = block_sum<kBlock>(s, lds);
    if (threadIdx.x == 0) part[blockIdx.x] = s;
}

// *total += sum(part[0..nb)), one block, fixed order.
__global__ void __launch_bounds__(kBlock) sumsq_finalize_kernel(const float* __restrict__ part, int nb,
                                                                 float* __restrict__ total) {
    __shared__ float lds[kBlock / 64];
    float s = 0.f;
    for (int i = threadIdx.x; i < nb; i += kBlock) s += part[i];
    s = block_sum<kBlock>(s, lds);
    if (threadIdx.x == 0) *total = *total + s;
}

__global__ void __launch_bounds__(kBlock) clip_norm_kernel(float* __restrict__ g, int64_t n,
                                                            const float* __restrict__ total, float max_norm) {
    const float clip_coef = max_norm / (sqrtf(*total) + 1e-6f);
    if (!(clip_coef < 1.0f)) return;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) g[i] = g[i] * clip_coef;
}

__global__ void __launch_bounds__(kBlock) clip_value_kernel(float* __restrict__ g, int64_t n, float c) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        const float v = g[i];
        g[i] = v > c ? c : (v < -c ? -c : v);
    }
}

// ---------------------------------------------------------------------------
// Unscaling: first position whose scaled value is not finite, then a prefix
// scale.
// ---------------------------------------------------------------------------

__device__ __forceinline__ int64_t min_i64(int64_t a, int64_t b) { return a < b ? a : b; }

// part[block] = smallest i of the block's stride set with !isfinite(g[i] * s),
// or n.
__global__ void __launch_bounds__(kBlock) first_bad_partial_kernel(const float* __restrict__ g, int64_t n, float s,
                                                                    int64_t* __restrict__ part) {
    __shared__ int64_t lds[kBlock];
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    int64_t first = n;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        if (!__builtin_isfinite(g[i] * s)) { first = i; break; }  // later i of this thread are larger
    }
    lds[threadIdx.x] = first;
    __syncthreads();
    for (int w = kBlock / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) lds[threadIdx.x] = min_i64(lds[threadIdx.x], lds[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = lds[0];
}

__global__ void __launch_bounds__(kBlock) first_bad_finalize_kernel(const int64_t* __restrict__ part, int nb,
                                                                     int64_t n, int64_t* __restrict__ out) {
    __shared__ int64_t lds[kBlock];
    int64_t first = n;
    for (int i = threadIdx.x; i < nb; i += kBlock) first = min_i64(first, part[i]);
    lds[threadIdx.x] = first;
    __syncthreads();
    for (int w = kBlock / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) lds[threadIdx.x] = min_i64(lds[threadIdx.x], lds[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = lds[0];
}

__global__ void __launch_bounds__(kBlock) scale_prefix_kernel(float* __restrict__ g, int64_t count, float s) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < count; i += stride) g[i] = g[i] * s;
}

// ---------------------------------------------------------------------------
// Multi-tensor launches: one kernel over every tensor of a parameter list.
// The list is cut into chunks (a tensor's last chunk may be shorter); a
// descriptor table in device memory gives each tensor's arrays, size and
// first chunk, and each workgroup finds its chunk's tensor by binary search.
// One launch per optimizer step instead of one per parameter tensor: a
// model's many small bias and norm vectors otherwise cost a kernel launch
// each, longer than their memory traffic.
//
// Two chunkings share the table.  The element-wise passes (updates, maps)
// take kChunkS = one float4 per thread, one chunk per workgroup, on a grid
// that covers the list: short-lived workgroups reading adjacent chunks
// measured 63 -> 72 % of the HBM peak for AdamW against 64K-element chunks
// (GPT-2-small list).  The reductions (sum of squares, first non-finite)
// keep kChunk elements per chunk, so their second pass folds few partials.
// ---------------------------------------------------------------------------

constexpr int64_t kChunk = 65536;              // reductions: elements per chunk
constexpr int kUpdU = 4;                         // float4 per thread per element-wise chunk
constexpr int64_t kChunkS = 4 * (int64_t)kBlock * kUpdU;  // element-wise passes
// The reductions' sweep issues kRedU float4 loads per thread before using
// any: one load in flight per wave left the sum of squares at 80 % and the
// finiteness search at 60 % of the HBM peak (GPT-2-small list).
constexpr int kRedU = 4;
constexpr int64_t kRedStride = 4 * (int64_t)kBlock;

struct MultiEntry {
    float* p;          // updated array (params; gradients for clipping / unscaling)
    const float* g;    // gradient (updates only)
    float* s1;         // state arrays (may be null)
    float* s2;
    int64_t n;
    int64_t chunk0;    // global index of the tensor's first kChunk chunk
    int64_t chunk0s;   // ... of its first kChunkS chunk
    int vec;           // every array of the tensor is 16-byte aligned
    float gs_unscale;  // the gradient's deferred scaling (wm_grad_scale): elements
    int64_t gs_count;  //   [0, gs_count) times gs_unscale, then every element times
    const float* gs_sumsq;  // clip_grad_norm_'s coefficient from *gs_sumsq when < 1
    float gs_max_norm;
    int pad;
};

// The deferred scaling of an entry's gradient (the g array of an update, the
// p array of the gradient passes), as the eager passes would have left it in
// memory: the unscale's product, then the clip's, each rounded to fp32
// (__fmul_rn: never fused into a neighbouring add).  coef() is read once per
// chunk.
struct GradScaleApply {
    float unscale, coef;
    int64_t count;
    bool clip;
    __device__ __forceinline__ explicit GradScaleApply(const MultiEntry& e)
        : unscale(e.gs_unscale), coef(1.0f), count(e.gs_count), clip(false) {
        if (e.gs_sumsq) {
#pragma clang fp contract(off)
            const float c = e.gs_max_norm / (sqrtf(*e.gs_sumsq) + 1e-6f);  // core/optimizer.cpp:157
            clip = c < 1.0f;
            coef = c;
        }
    }
    __device__ __forceinline__ float operator()(float g, int64_t i) const {
        if (i < count) g = __fmul_rn(g, unscale);
        if (clip) g = __fmul_rn(g, coef);
        return g;
    }
};

// Largest k with tab[k].chunk0 <= c.
__device__ __forceinline__ int find_entry(const MultiEntry* tab, int count, int64_t c) {
    int lo = 0, hi = count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tab[mid].chunk0 <= c) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// The kChunkS chunks are many (one per workgroup), so their lookup starts
// from a coarse index stored after the entries: coarse[j] is the entry that
// holds chunk j * kCoarse.  The entry of chunk c lies between coarse[j] and
// coarse[j + 1] (j = c / kCoarse), which for a tensor of kCoarse chunks or
// more is one entry: the search then takes two loads instead of log2(count).
constexpr int64_t kCoarse = 256;

__device__ __forceinline__ int find_entry_s(const MultiEntry* tab, int count, int64_t chunks, int64_t c) {
    const int* coarse = reinterpret_cast<const int*>(tab + count);
    const int64_t j = c / kCoarse;
    int lo = coarse[j];
    int hi = (j + 1) * kCoarse < chunks ? coarse[j + 1] : count - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tab[mid].chunk0s <= c) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

template <class U>
__global__ void __launch_bounds__(kBlock) multi_update_kernel(const MultiEntry* __restrict__ tab, int count,
                                                               int64_t chunks, U upd) {
    constexpr int NS = U::NS;
    for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const MultiEntry e = tab[find_entry_s(tab, count, chunks, c)];
        const GradScaleApply gs(e);
        const int64_t start = (c - e.chunk0s) * kChunkS;
        const int64_t end = min(e.n, start + kChunkS);
        if (e.vec && end - start == kChunkS) {
            // a whole chunk: every load issued before the first update
            float4 vp[kUpdU], vg[kUpdU], v1[kUpdU], v2[kUpdU];
#pragma unroll
            for (int u = 0; u < kUpdU; ++u) {
                const int64_t i = start + 4 * (int64_t)threadIdx.x + u * kRedStride;
                vp[u] = ld_stream(e.p + i);
                vg[u] = ld_stream(e.g + i);
                v1[u] = NS > 0 ? ld_stream(e.s1 + i) : make_float4(0.f, 0.f, 0.f, 0.f);
                v2[u] = NS > 1 ? ld_stream(e.s2 + i) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int u = 0; u < kUpdU; ++u) {
                const int64_t i = start + 4 * (int64_t)threadIdx.x + u * kRedStride;
                upd(vp[u].x, gs(vg[u].x, i), v1[u].x, v2[u].x);
                upd(vp[u].y, gs(vg[u].y, i + 1), v1[u].y, v2[u].y);
                upd(vp[u].z, gs(vg[u].z, i + 2), v1[u].z, v2[u].z);
                upd(vp[u].w, gs(vg[u].w, i + 3), v1[u].w, v2[u].w);
                st_stream(e.p + i, vp[u]);
                if (NS > 0) st_stream(e.s1 + i, v1[u]);
                if (NS > 1) st_stream(e.s2 + i, v2[u]);
            }
            continue;
        }
        int64_t tail = start;
        if (e.vec) {
            const int64_t end4 = start + ((end - start) & ~int64_t(3));
            for (int64_t i = start + 4 * (int64_t)threadIdx.x; i < end4; i += 4 * kBlock) {
                float4 vp = ld_stream(e.p + i);
                const float4 vg = ld_stream(e.g + i);
                float4 v1 = NS > 0 ? ld_stream(e.s1 + i) : make_float4(0.f, 0.f, 0.f, 0.f);
                float4 v2 = NS > 1 ? ld_stream(e.s2 + i) : make_float4(0.f, 0.f, 0.f, 0.f);
                upd(vp.x, gs(vg.x, i), v1.x, v2.x);
                upd(vp.y, gs(vg.y, i + 1), v1.y, v2.y);
                upd(vp.z, gs(vg.z, i + 2), v1.z, v2.z);
                upd(vp.w, gs(vg.w, i + 3), v1.w, v2.w);
                st_stream(e.p + i, vp);
                if (NS > 0) st_stream(e.s1 + i, v1);
                if (NS > 1) st_stream(e.s2 + i, v2);
            }
            tail = end4;
        }
        for (int64_t i = tail + threadIdx.x; i < end; i += kBlock) {
            float vp = e.p[i];
            float v1 = NS > 0 ? e.s1[i] : 0.f;
            float v2 = NS > 1 ? e.s2[i] : 0.f;
            upd(vp, gs(e.g[i], i), v1, v2);
            e.p[i] = vp;
            if (NS > 0) e.s1[i] = v1;
            if (NS > 1) e.s2[i] = v2;
        }
    }
}

// In-place per-element maps on the p arrays, each element first taken through
// its entry's deferred scaling: kind 0 scales by clip_grad_norm_'s
// coefficient when it is < 1 (read from *total on the device), kind 1 clips to
// [-a, a], kind 2 multiplies by a every element before the cutoff (table row
// cut_tensor, element cut_index) in parameter order, kind 3 only writes the
// deferred scaling into the array.
__global__ void __launch_bounds__(kBlock) multi_map_kernel(const MultiEntry* __restrict__ tab, int count,
                                                            int64_t chunks, int kind, const float* __restrict__ total,
                                                            float a, int cut_tensor, int64_t cut_index) {
    float coef = 1.0f;
    if (kind == 0) {
        coef = a / (sqrtf(*total) + 1e-6f);
        if (!(coef < 1.0f)) return;
    }
    for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const int k = find_entry_s(tab, count, chunks, c);
        const MultiEntry e = tab[k];
        const GradScaleApply gs(e);
        const int64_t start = (c - e.chunk0s) * kChunkS;
        int64_t end = min(e.n, start + kChunkS);
        if (kind == 2) {
            if (k > cut_tensor) continue;
            if (k == cut_tensor) end = min(end, cut_index);
        }
        auto map1 = [&](float v, int64_t i) {
            v = gs(v, i);
            if (kind == 0) return v * coef;
            if (kind == 1) return v > a ? a : (v < -a ? -a : v);
            if (kind == 2) return v * a;
            return v;
        };
        int64_t tail = start;
        if (e.vec && end > start) {
            const int64_t end4 = start + ((end - start) & ~int64_t(3));
            for (int64_t i = start + 4 * (int64_t)threadIdx.x; i < end4; i += 4 * kBlock) {
                float4 v = ld_stream(e.p + i);
                v.x = map1(v.x, i); v.y = map1(v.y, i + 1); v.z = map1(v.z, i + 2); v.w = map1(v.w, i + 3);
                st_stream(e.p + i, v);
            }
            tail = end4;
        }
        for (int64_t i = tail + threadIdx.x; i < end; i += kBlock) e.p[i] = map1(e.p[i], i);
    }
}

// part[c] = sum of (x * mul)^2 over chunk c (mul = 1 is exact: the plain
// sum of squares).
__global__ void __launch_bounds__(kBlock) multi_sumsq_kernel(const MultiEntry* __restrict__ tab, int count,
                                                              int64_t chunks, float mul, float* __restrict__ part) {
    __shared__ float lds[kBlock / 64];
    for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const MultiEntry e = tab[find_entry(tab, count, c)];
        const GradScaleApply gs(e);
        const int64_t start = (c - e.chunk0) * kChunk;
        const int64_t end = min(e.n, start + kChunk);
        float s = 0.f;
        int64_t tail = start;
        if (e.vec) {
            const int64_t end4 = start + ((end - start) & ~int64_t(3));
            auto acc = [&](const float4 v, int64_t i) {
                const float a = gs(v.x, i) * mul, b = gs(v.y, i + 1) * mul, c2 = gs(v.z, i + 2) * mul,
                            d = gs(v.w, i + 3) * mul;
                s += a * a + b * b + c2 * c2 + d * d;
            };
            int64_t i = start + 4 * (int64_t)threadIdx.x;
            for (; i + (kRedU - 1) * kRedStride < end4; i += kRedU * kRedStride) {
                float4 v[kRedU];
#pragma unroll
                for (int u = 0; u < kRedU; ++u) v[u] = ld_stream(e.p + i + u * kRedStride);
#pragma unroll
                for (int u = 0; u < kRedU; ++u) acc(v[u], i + u * kRedStride);
            }
            for (; i < end4; i += kRedStride) acc(ld_stream(e.p + i), i);
            tail = end4;
        }
        for (int64_t i = tail + threadIdx.x; i < end; i += kBlock) {
            const float a = gs(e.p[i], i) * mul;
            s += a * a;
        }
        s = block_sum<kBlock>(s, lds);
        if (threadIdx.x == 0) part[c] = s;
        __syncthreads();
    }
}

// *total = (accumulate ? *total : 0) + sum(part[0..chunks)), one block, fixed order.
__global__ void __launch_bounds__(kBlock) multi_sum_finalize_kernel(const float* __restrict__ part, int64_t chunks,
                                                                     float* __restrict__ total, int accumulate) {
    __shared__ float lds[kBlock / 64];
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < chunks; i += kBlock) s += part[i];
    s = block_sum<kBlock>(s, lds);
    if (threadIdx.x == 0) *total = accumulate ? *total + s : s;
}

// first[c] = smallest in-tensor index of chunk c whose scaled value is not
// finite, or -1.  The scan has no early exit (each thread keeps its first
// non-finite index), so its loads pipeline like the sum of squares'; the
// block's minimum is only formed when some thread found one.
__global__ void __launch_bounds__(kBlock) multi_first_bad_kernel(const MultiEntry* __restrict__ tab, int count,
                                                                  int64_t chunks, float scale,
                                                                  int64_t* __restrict__ first) {
    __shared__ int64_t lds[kBlock];
    for (int64_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        const MultiEntry e = tab[find_entry(tab, count, c)];
        const GradScaleApply gs(e);
        const int64_t start = (c - e.chunk0) * kChunk;
        const int64_t end = min(e.n, start + kChunk);
        int64_t f = e.n;
        int64_t tail = start;
        if (e.vec) {
            const int64_t end4 = start + ((end - start) & ~int64_t(3));
            auto scan = [&](const float4 v, int64_t i) {
                const bool b0 = !__builtin_isfinite(gs(v.x, i) * scale), b1 = !__builtin_isfinite(gs(v.y, i + 1) * scale),
                           b2 = !__builtin_isfinite(gs(v.z, i + 2) * scale),
                           b3 = !__builtin_isfinite(gs(v.w, i + 3) * scale);
                if ((b0 || b1 || b2 || b3) && f == e.n) f = i + (b0 ? 0 : b1 ? 1 : b2 ? 2 : 3);
            };
            int64_t i = start + 4 * (int64_t)threadIdx.x;
            for (; i + (kRedU - 1) * kRedStride < end4; i += kRedU * kRedStride) {
                float4 v[kRedU];
#pragma unroll
                for (int u = 0; u < kRedU; ++u) v[u] = ld_stream(e.p + i + u * kRedStride);
#pragma unroll
                for (int u = 0; u < kRedU; ++u) scan(v[u], i + u * kRedStride);
            }
            for (; i < end4; i += kRedStride) scan(ld_stream(e.p + i), i);
            tail = end4;
        }
        for (int64_t i = tail + threadIdx.x; i < end; i += kBlock)
            if (!__builtin_isfinite(gs(e.p[i], i) * scale) && f == e.n) f = i;
        if (__syncthreads_or(f < e.n)) {
            lds[threadIdx.x] = f;
            __syncthreads();
            for (int w = kBlock / 2; w > 0; w >>= 1) {
                if ((int)threadIdx.x < w) lds[threadIdx.x] = min_i64(lds[threadIdx.x], lds[threadIdx.x + w]);
                __syncthreads();
            }
            if (threadIdx.x == 0) first[c] = lds[0];
            __syncthreads();
        } else if (threadIdx.x == 0) {
            first[c] = -1;
        }
    }
}

// out[0], out[1] = (entry, index) of the first non-finite position in chunk
// order (= parameter order), or (count, 0).  One block.
__global__ void __launch_bounds__(kBlock) multi_first_bad_finalize_kernel(const MultiEntry* __restrict__ tab,
                                                                           int count, int64_t chunks,
                                                                           const int64_t* __restrict__ first,
                                                                           int64_t* __restrict__ out) {
    __shared__ int64_t lds[kBlock];
    int64_t best = chunks;  // first chunk holding a non-finite value
    for (int64_t c = threadIdx.x; c < chunks; c += kBlock) {
        if (first[c] >= 0) { best = c; break; }
    }
    lds[threadIdx.x] = best;
    __syncthreads();
    for (int w = kBlock / 2; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) lds[threadIdx.x] = min_i64(lds[threadIdx.x], lds[threadIdx.x + w]);
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int64_t c = lds[0];
        if (c < chunks) {
            out[0] = find_entry(tab, count, c);
            out[1] = first[c];
        } else {
            out[0] = count;
            out[1] = 0;
        }
    }
}

// A descriptor table's device copy; returned to the pool when the last
// holder lets go (the pool's reuse is ordered on the library stream, after
// the launches that read it).
struct DevTable {
    void* p = nullptr;
    explicit DevTable(size_t bytes) : p(ws_alloc(bytes)) {}
    ~DevTable() { if (p) ws_free(p); }
    DevTable(const DevTable&) = delete;
    DevTable& operator=(const DevTable&) = delete;
};

// Device copies of the last kTableSlots descriptor tables.  A training loop
// passes the same lists every step, so a table equal byte for byte to a
// cached one is used again instead of uploaded: the upload is a copy
// dispatch on the stream (~4 us) and may wait for the staging buffer.
// Tables are read-only on the device; each launch holds its table until the
// launch is enqueued, so an eviction by another thread cannot recycle it
// under a pending launch.
class TableCache {
    static constexpr size_t kTableSlots = 16;
    struct Slot {
        std::vector<unsigned char> bytes;
        std::shared_ptr<DevTable> dev;
        uint64_t used = 0;
    };
    std::mutex mu_;
    std::vector<Slot> slots_;
    uint64_t clock_ = 0;

public:
    int get(const std::vector<unsigned char>& bytes, std::shared_ptr<DevTable>* out, const char* what) {
        std::lock_guard<std::mutex> lk(mu_);
        for (auto& s : slots_)
            if (s.bytes == bytes) {
                s.used = ++clock_;
                *out = s.dev;
                return WM_OK;
            }
        auto dev = std::make_shared<DevTable>(bytes.size());
        if (!dev->p) return set_error(WM_ERR_NOMEM, std::string(what) + ": descriptor table");
        WM_TRY(upload_async(dev->p, bytes.data(), bytes.size()));
        Slot* s = nullptr;
        if (slots_.size() < kTableSlots) {
            slots_.emplace_back();
            s = &slots_.back();
        } else {
            s = &*std::min_element(slots_.begin(), slots_.end(),
                                   [](const Slot& a, const Slot& b) { return a.used < b.used; });
        }
        s->bytes = bytes;
        s->dev = dev;
        s->used = ++clock_;
        *out = std::move(dev);
        return WM_OK;
    }
};
// Never destroyed: a static destructor could run after the pool's.
TableCache& tables() {
    static TableCache* t = new TableCache;
    return *t;
}

// Descriptor table of a parameter list on the device (entries with n == 0 or
// a null array are dropped; `index` maps table rows back to list positions).
struct MultiTable {
    std::vector<MultiEntry> host;
    std::vector<int> index;
    int64_t chunks = 0;    // kChunk chunks (reductions)
    int64_t chunks_s = 0;  // kChunkS chunks (element-wise passes)
    std::shared_ptr<DevTable> dev;

    int build(int count, float* const* p, const float* const* g, float* const* s1, float* const* s2,
              const int64_t* n, int ns, const char* what, const wm_grad_scale* gscale = nullptr) {
        for (int k = 0; k < count; ++k) {
            if (n[k] < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative size");
            if (n[k] == 0) continue;
            MultiEntry e;
            std::memset(&e, 0, sizeof e);  // padding included: tables are compared byte for byte
            e.p = p[k];
            e.g = g ? g[k] : nullptr;
            e.s1 = ns > 0 && s1 ? s1[k] : nullptr;
            e.s2 = ns > 1 && s2 ? s2[k] : nullptr;
            if (!e.p || (g && !e.g) || (ns > 0 && !e.s1) || (ns > 1 && !e.s2))
                return set_error(WM_ERR_INVALID, std::string(what) + ": null pointer");
            e.n = n[k];
            e.chunk0 = chunks;
            e.chunk0s = chunks_s;
            e.vec = aligned16(e.p) && (!e.g || aligned16(e.g)) && (!e.s1 || aligned16(e.s1)) &&
                    (!e.s2 || aligned16(e.s2));
            e.gs_unscale = 1.0f;
            if (gscale) {
                const wm_grad_scale& q = gscale[k];
                if (q.unscale_count < 0 || q.unscale_count > n[k])
                    return set_error(WM_ERR_INVALID, std::string(what) + ": unscale_count outside the tensor");
                e.gs_unscale = q.unscale;
                e.gs_count = q.unscale_count;
                e.gs_sumsq = q.clip_sumsq;
                e.gs_max_norm = q.clip_max_norm;
            }
            chunks += (n[k] + kChunk - 1) / kChunk;
            chunks_s += (n[k] + kChunkS - 1) / kChunkS;
            host.push_back(e);
            index.push_back(k);
        }
        if (host.empty()) return WM_OK;
        // entries, then the coarse index of the kChunkS chunks (find_entry_s)
        const size_t ncoarse = (size_t)((chunks_s + kCoarse - 1) / kCoarse);
        const size_t eb = host.size() * sizeof(MultiEntry);
        std::vector<unsigned char> buf(eb + ncoarse * sizeof(int));
        std::memcpy(buf.data(), host.data(), eb);
        int* coarse = reinterpret_cast<int*>(buf.data() + eb);
        size_t k = 0;
        for (size_t j = 0; j < ncoarse; ++j) {
            const int64_t c = (int64_t)j * kCoarse;
            while (k + 1 < host.size() && host[k + 1].chunk0s <= c) ++k;
            coarse[j] = (int)k;
        }
        return tables().get(buf, &dev, what);
    }
    const MultiEntry* table() const { return static_cast<const MultiEntry*>(dev->p); }
    int count() const { return (int)host.size(); }
    unsigned grid() const { return grid_for(chunks, 1, 8); }
    unsigned grid_s() const { return grid_for(chunks_s, 1, 1 << 12); }
};

// Consecutive runs of list positions in which no array written by one
// tensor overlaps an array of another (a parameter listed twice, state
// buffers shared between entries).  Each run is one launch and the runs go
// in list order, so such a tensor is updated once per listing, one update
// after the other, as the reference's loop over the list does; read-only
// arrays (gradients of an update) may overlap each other freely.
std::vector<std::pair<int, int>> independent_runs(int count, float* const* p, const float* const* g,
                                                  float* const* s1, float* const* s2, const int64_t* n, int ns) {
    struct Range {
        uintptr_t lo, hi;
        int pos;
        bool written;
    };
    std::vector<Range> r;
    r.reserve((size_t)count * 4);
    auto add = [&](const void* a, int k, bool w) {
        if (a) r.push_back({(uintptr_t)a, (uintptr_t)a + (uintptr_t)n[k] * sizeof(float), k, w});
    };
    for (int k = 0; k < count; ++k) {
        if (n[k] <= 0) continue;
        add(p[k], k, true);
        if (g) add(g[k], k, false);
        if (ns > 0 && s1) add(s1[k], k, true);
        if (ns > 1 && s2) add(s2[k], k, true);
    }
    std::sort(r.begin(), r.end(), [](const Range& a, const Range& b) { return a.lo < b.lo; });
    // last[j]: the latest earlier list position whose arrays conflict with j's
    std::vector<int> last(count, -1);
    std::vector<const Range*> open;
    for (const Range& x : r) {
        size_t keep = 0;
        for (const Range* o : open) {
            if (o->hi <= x.lo) continue;  // ended before x starts
            open[keep++] = o;
            if (o->pos != x.pos && (o->written || x.written)) {
                const int a = std::min(o->pos, x.pos), b = std::max(o->pos, x.pos);
                last[b] = std::max(last[b], a);
            }
        }
        open.resize(keep);
        open.push_back(&x);
    }
    std::vector<std::pair<int, int>> runs;
    int start = 0;
    for (int j = 1; j < count; ++j)
        if (last[j] >= start) {
            runs.emplace_back(start, j);
            start = j;
        }
    runs.emplace_back(start, count);
    return runs;
}

template <class U>
int launch_multi(int count, float* const* p, const float* const* g, float* const* s1, float* const* s2,
                 const int64_t* n, const U& upd, const char* what, const wm_grad_scale* gs = nullptr) {
    if (count < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative count");
    if (count == 0) return WM_OK;
    if (!p || !g || !n || (U::NS > 0 && !s1) || (U::NS > 1 && !s2))
        return set_error(WM_ERR_INVALID, std::string(what) + ": null array");
    WM_CHECK_INIT();
    for (const auto& run : independent_runs(count, p, g, s1, s2, n, U::NS)) {
        const int b = run.first;
        MultiTable t;
        WM_TRY(t.build(run.second - b, p + b, g + b, s1 ? s1 + b : nullptr, s2 ? s2 + b : nullptr, n + b, U::NS,
                       what, gs ? gs + b : nullptr));
        if (t.chunks == 0) continue;
        launch_kernel(multi_update_kernel<U>, dim3(t.grid_s()), dim3(kBlock), 0, stream(), t.table(), t.count(),
                      t.chunks_s, upd);
        WM_TRY(check_launch(what));
    }
    return WM_OK;
}

static int check_n(int64_t n, const char* what) {
    if (n < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative size");
    return WM_OK;
}

}  // namespace wm

using namespace wm;

extern "C" {

int wm_sgd_step(float* p, const float* g, float* velocity, int64_t n, float lr, float momentum) {
    WM_TRY(check_n(n, "wm_sgd_step"));
    if (n == 0) return WM_OK;
    if (!p || !g) return set_error(WM_ERR_INVALID, "wm_sgd_step: null pointer");
    WM_CHECK_INIT();
    const SgdArgs a{lr, momentum};
    if (momentum > 0.0f) {
        if (!velocity) return set_error(WM_ERR_INVALID, "wm_sgd_step: momentum > 0 needs a velocity buffer");
        return launch_update(p, g, velocity, nullptr, n, Upd<0, true, false>{a}, "wm_sgd_step");
    }
    return launch_update(p, g, nullptr, nullptr, n, Upd<0, false, false>{a}, "wm_sgd_step");
}

static int adam_common(bool decoupled, float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1,
                       float beta2, float eps, float bc1, float bc2, float wd, const char* what) {
    WM_TRY(check_n(n, what));
    if (n == 0) return WM_OK;
    if (!p || !g || !m || !v) return set_error(WM_ERR_INVALID, std::string(what) + ": null pointer");
    WM_CHECK_INIT();
    const AdamArgs a{lr, beta1, beta2, 1.0f - beta1, 1.0f - beta2, eps, bc1, bc2, wd};
    if (decoupled) return launch_update(p, g, m, v, n, Upd<1, true, false>{a}, what);
    return launch_update(p, g, m, v, n, Upd<1, false, false>{a}, what);
}

int wm_adam_step(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                 float eps, float bias_correction1, float bias_correction2) {
    return adam_common(false, p, g, m, v, n, lr, beta1, beta2, eps, bias_correction1, bias_correction2, 0.0f,
                       "wm_adam_step");
}

int wm_adamw_step(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                  float eps, float bias_correction1, float bias_correction2, float weight_decay) {
    return adam_common(true, p, g, m, v, n, lr, beta1, beta2, eps, bias_correction1, bias_correction2, weight_decay,
                       "wm_adamw_step");
}

int wm_rmsprop_step(float* p, const float* g, float* v, float* buffer, int64_t n, float lr, float alpha, float eps,
                    float momentum, float weight_decay) {
    WM_TRY(check_n(n, "wm_rmsprop_step"));
    if (n == 0) return WM_OK;
    if (!p || !g || !v) return set_error(WM_ERR_INVALID, "wm_rmsprop_step: null pointer");
    const bool mom = momentum > 0.0f, wd = weight_decay != 0.0f;
    if (mom && !buffer) return set_error(WM_ERR_INVALID, "wm_rmsprop_step: momentum > 0 needs a momentum buffer");
    WM_CHECK_INIT();
    const RmsArgs a{lr, alpha, 1.0f - alpha, eps, momentum, weight_decay};
    if (wd && mom) return launch_update(p, g, v, buffer, n, Upd<2, true, true>{a}, "wm_rmsprop_step");
    if (wd) return launch_update(p, g, v, nullptr, n, Upd<2, true, false>{a}, "wm_rmsprop_step");
    if (mom) return launch_update(p, g, v, buffer, n, Upd<2, false, true>{a}, "wm_rmsprop_step");
    return launch_update(p, g, v, nullptr, n, Upd<2, false, false>{a}, "wm_rmsprop_step");
}

int wm_grad_sumsq_accumulate(const float* g, int64_t n, float* total) {
    WM_TRY(check_n(n, "wm_grad_sumsq_accumulate"));
    if (!total) return set_error(WM_ERR_INVALID, "wm_grad_sumsq_accumulate: null total");
    if (n == 0) return WM_OK;
    if (!g) return set_error(WM_ERR_INVALID, "wm_grad_sumsq_accumulate: null pointer");
    WM_CHECK_INIT();
    const int nb = (int)std::min<int64_t>(grid_for(n / 4 + 1, kBlock, 4), kMaxPart);
    Workspace ws((size_t)nb * sizeof(float));
    if (!ws.p) return set_error(WM_ERR_NOMEM, "wm_grad_sumsq_accumulate: workspace");
    launch_kernel(sumsq_partial_kernel, dim3(nb), dim3(kBlock), 0, stream(), g, n, ws.as<float>());
    WM_TRY(check_launch("wm_grad_sumsq_accumulate"));
    launch_kernel(sumsq_finalize_kernel, dim3(1), dim3(kBlock), 0, stream(), ws.as<float>(), nb, total);
    return check_launch("wm_grad_sumsq_accumulate(finalize)");
}

int wm_clip_grad_norm_scale(float* g, int64_t n, const float* total_sumsq, float max_norm) {
    WM_TRY(check_n(n, "wm_clip_grad_norm_scale"));
    if (n == 0) return WM_OK;
    if (!g || !total_sumsq) return set_error(WM_ERR_INVALID, "wm_clip_grad_norm_scale: null pointer");
    WM_CHECK_INIT();
    launch_kernel(clip_norm_kernel, dim3(grid_for(n, kBlock, 16)), dim3(kBlock), 0, stream(), g, n, total_sumsq,
                       max_norm);
    return check_launch("wm_clip_grad_norm_scale");
}

int wm_clip_grad_value(float* g, int64_t n, float clip_value) {
    WM_TRY(check_n(n, "wm_clip_grad_value"));
    if (n == 0) return WM_OK;
    if (!g) return set_error(WM_ERR_INVALID, "wm_clip_grad_value: null pointer");
    WM_CHECK_INIT();
    launch_kernel(clip_value_kernel, dim3(grid_for(n, kBlock, 16)), dim3(kBlock), 0, stream(), g, n,
                       clip_value);
    return check_launch("wm_clip_grad_value");
}

int wm_grad_unscale(int count, float* const* grads, const int64_t* sizes, float inv_scale, int* found_inf) {
    if (count < 0) return set_error(WM_ERR_INVALID, "wm_grad_unscale: negative count");
    if (!found_inf) return set_error(WM_ERR_INVALID, "wm_grad_unscale: null found_inf");
    *found_inf = 0;
    if (count == 0) return WM_OK;
    if (!grads || !sizes) return set_error(WM_ERR_INVALID, "wm_grad_unscale: null pointer");
    std::vector<float*> gl(grads, grads + count);
    std::vector<int64_t> nl(sizes, sizes + count);
    for (int k = 0; k < count; ++k)
        if (!gl[k]) nl[k] = 0;  // a missing gradient is skipped like an empty one
    WM_CHECK_INIT();
    // Runs of gradients that do not overlap, in list order: a gradient listed
    // twice is scaled (and searched) twice, one pass after the other.
    for (const auto& run : independent_runs(count, gl.data(), nullptr, nullptr, nullptr, nl.data(), 0)) {
        const int b = run.first;
        MultiTable t;
        WM_TRY(t.build(run.second - b, gl.data() + b, nullptr, nullptr, nullptr, nl.data() + b, 0,
                       "wm_grad_unscale"));
        if (t.chunks == 0) continue;
        // 1. the first non-finite scaled position in parameter order
        Workspace first((size_t)t.chunks * sizeof(int64_t)), where(2 * sizeof(int64_t));
        if (!first.p || !where.p) return set_error(WM_ERR_NOMEM, "wm_grad_unscale: workspace");
        launch_kernel(multi_first_bad_kernel, dim3(t.grid()), dim3(kBlock), 0, stream(), t.table(), t.count(),
                      t.chunks, inv_scale, first.as<int64_t>());
        WM_TRY(check_launch("wm_grad_unscale(find)"));
        launch_kernel(multi_first_bad_finalize_kernel, dim3(1), dim3(kBlock), 0, stream(), t.table(), t.count(),
                      t.chunks, first.as<int64_t>(), where.as<int64_t>());
        WM_TRY(check_launch("wm_grad_unscale(find finalize)"));
        int64_t cut[2] = {0, 0};
        WM_TRY(wm_d2h(cut, where.p, sizeof(cut)));
        // 2. scale everything before it (everything when there is none)
        launch_kernel(multi_map_kernel, dim3(t.grid_s()), dim3(kBlock), 0, stream(), t.table(), t.count(),
                      t.chunks_s, 2, nullptr, inv_scale, (int)cut[0], cut[1]);
        WM_TRY(check_launch("wm_grad_unscale(scale)"));
        if (cut[0] < t.count()) {
            *found_inf = 1;
            return WM_OK;
        }
    }
    return WM_OK;
}

// ---- multi-tensor variants ---------------------------------------------------

static int sgd_multi(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                     float* const* velocity, const int64_t* n, float lr, float momentum, const char* what) {
    const SgdArgs a{lr, momentum};
    if (momentum > 0.0f) return launch_multi(count, p, g, velocity, nullptr, n, Upd<0, true, false>{a}, what, gs);
    return launch_multi(count, p, g, nullptr, nullptr, n, Upd<0, false, false>{a}, what, gs);
}

static int adam_multi(bool decoupled, int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                      float* const* m, float* const* v, const int64_t* n, float lr, float beta1, float beta2,
                      float eps, float bc1, float bc2, float wd, const char* what) {
    const AdamArgs a{lr, beta1, beta2, 1.0f - beta1, 1.0f - beta2, eps, bc1, bc2, wd};
    if (decoupled) return launch_multi(count, p, g, m, v, n, Upd<1, true, false>{a}, what, gs);
    return launch_multi(count, p, g, m, v, n, Upd<1, false, false>{a}, what, gs);
}

static int rmsprop_multi(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                         float* const* v, float* const* buffer, const int64_t* n, float lr, float alpha, float eps,
                         float momentum, float weight_decay, const char* what) {
    const RmsArgs a{lr, alpha, 1.0f - alpha, eps, momentum, weight_decay};
    const bool mom = momentum > 0.0f, wd = weight_decay != 0.0f;
    if (wd && mom) return launch_multi(count, p, g, v, buffer, n, Upd<2, true, true>{a}, what, gs);
    if (wd) return launch_multi(count, p, g, v, nullptr, n, Upd<2, true, false>{a}, what, gs);
    if (mom) return launch_multi(count, p, g, v, buffer, n, Upd<2, false, true>{a}, what, gs);
    return launch_multi(count, p, g, v, nullptr, n, Upd<2, false, false>{a}, what, gs);
}

int wm_sgd_step_multi(int count, float* const* p, const float* const* g, float* const* velocity, const int64_t* n,
                      float lr, float momentum) {
    return sgd_multi(count, p, g, nullptr, velocity, n, lr, momentum, "wm_sgd_step_multi");
}

int wm_adam_step_multi(int count, float* const* p, const float* const* g, float* const* m, float* const* v,
                       const int64_t* n, float lr, float beta1, float beta2, float eps, float bias_correction1,
                       float bias_correction2) {
    return adam_multi(false, count, p, g, nullptr, m, v, n, lr, beta1, beta2, eps, bias_correction1,
                      bias_correction2, 0.0f, "wm_adam_step_multi");
}

int wm_adamw_step_multi(int count, float* const* p, const float* const* g, float* const* m, float* const* v,
                        const int64_t* n, float lr, float beta1, float beta2, float eps, float bias_correction1,
                        float bias_correction2, float weight_decay) {
    return adam_multi(true, count, p, g, nullptr, m, v, n, lr, beta1, beta2, eps, bias_correction1, bias_correction2,
                      weight_decay, "wm_adamw_step_multi");
}

int wm_rmsprop_step_multi(int count, float* const* p, const float* const* g, float* const* v, float* const* buffer,
                          const int64_t* n, float lr, float alpha, float eps, float momentum, float weight_decay) {
    return rmsprop_multi(count, p, g, nullptr, v, buffer, n, lr, alpha, eps, momentum, weight_decay,
                         "wm_rmsprop_step_multi");
}

int wm_sgd_step_multi_gs(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                         float* const* velocity, const int64_t* n, float lr, float momentum) {
    return sgd_multi(count, p, g, gs, velocity, n, lr, momentum, "wm_sgd_step_multi_gs");
}

int wm_adam_step_multi_gs(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                          float* const* m, float* const* v, const int64_t* n, float lr, float beta1, float beta2,
                          float eps, float bias_correction1, float bias_correction2) {
    return adam_multi(false, count, p, g, gs, m, v, n, lr, beta1, beta2, eps, bias_correction1, bias_correction2,
                      0.0f, "wm_adam_step_multi_gs");
}

int wm_adamw_step_multi_gs(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                           float* const* m, float* const* v, const int64_t* n, float lr, float beta1, float beta2,
                           float eps, float bias_correction1, float bias_correction2, float weight_decay) {
    return adam_multi(true, count, p, g, gs, m, v, n, lr, beta1, beta2, eps, bias_correction1, bias_correction2,
                      weight_decay, "wm_adamw_step_multi_gs");
}

int wm_rmsprop_step_multi_gs(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                             float* const* v, float* const* buffer, const int64_t* n, float lr, float alpha,
                             float eps, float momentum, float weight_decay) {
    return rmsprop_multi(count, p, g, gs, v, buffer, n, lr, alpha, eps, momentum, weight_decay,
                         "wm_rmsprop_step_multi_gs");
}

static int multi_grads(int count, const float* const* g, const int64_t* n, MultiTable& t, const char* what,
                       const wm_grad_scale* gs = nullptr) {
    if (count < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative count");
    if (count > 0 && (!g || !n)) return set_error(WM_ERR_INVALID, std::string(what) + ": null array");
    WM_CHECK_INIT();
    return t.build(count, const_cast<float* const*>(g), nullptr, nullptr, nullptr, n, 0, what, gs);
}

static int sumsq_multi(int count, const float* const* g, const int64_t* n, float mul, float* total, const char* what,
                       const wm_grad_scale* gs = nullptr) {
    if (!total) return set_error(WM_ERR_INVALID, std::string(what) + ": null total");
    MultiTable t;
    WM_TRY(multi_grads(count, g, n, t, what, gs));
    if (t.chunks == 0) return wm_fill(total, 0.0f, 1);
    Workspace part((size_t)t.chunks * sizeof(float));
    if (!part.p) return set_error(WM_ERR_NOMEM, std::string(what) + ": workspace");
    launch_kernel(multi_sumsq_kernel, dim3(t.grid()), dim3(kBlock), 0, stream(), t.table(), t.count(), t.chunks, mul,
                  part.as<float>());
    WM_TRY(check_launch(what));
    launch_kernel(multi_sum_finalize_kernel, dim3(1), dim3(kBlock), 0, stream(), part.as<float>(), t.chunks, total, 0);
    return check_launch(what);
}

int wm_grad_sumsq_multi(int count, const float* const* g, const int64_t* n, float* total) {
    return sumsq_multi(count, g, n, 1.0f, total, "wm_grad_sumsq_multi");
}

int wm_grad_sumsq_scaled_multi(int count, const float* const* g, const int64_t* n, float mul, float* total) {
    return sumsq_multi(count, g, n, mul, total, "wm_grad_sumsq_scaled_multi");
}

// (list position, element) of the first element whose value times `scale`
// is not finite, in list order, or (count, 0); one search launch and its
// finalize, then one synchronisation for the answer.
static int first_bad_multi(int count, const float* const* g, const wm_grad_scale* gs, const int64_t* n, float scale,
                           int64_t* where_out, const char* what) {
    where_out[0] = count;
    where_out[1] = 0;
    MultiTable t;
    WM_TRY(multi_grads(count, g, n, t, what, gs));
    if (t.chunks == 0) return WM_OK;
    Workspace first((size_t)t.chunks * sizeof(int64_t));
    if (!first.p) return set_error(WM_ERR_NOMEM, std::string(what) + ": workspace");
    // The answer goes straight to pinned host memory (no copy dispatch after
    // the finalize kernel); one buffer per process, held across the wait.
    static std::mutex mu;
    static int64_t* host_where = nullptr;
    static int64_t* dev_where = nullptr;
    std::lock_guard<std::mutex> lk(mu);
    if (!host_where) {
        void* h = nullptr;
        void* d = nullptr;
        hipError_t e = hipHostMalloc(&h, 2 * sizeof(int64_t), hipHostMallocMapped | hipHostMallocCoherent);
        if (e == hipSuccess) e = hipHostGetDevicePointer(&d, h, 0);
        if (e != hipSuccess) {
            if (h) (void)hipHostFree(h);
            return set_error(WM_ERR_HIP, std::string(what) + ": pinned result: " + hipGetErrorString(e));
        }
        host_where = static_cast<int64_t*>(h);
        dev_where = static_cast<int64_t*>(d);
    }
    launch_kernel(multi_first_bad_kernel, dim3(t.grid()), dim3(kBlock), 0, stream(), t.table(), t.count(), t.chunks,
                  scale, first.as<int64_t>());
    WM_TRY(check_launch(what));
    launch_kernel(multi_first_bad_finalize_kernel, dim3(1), dim3(kBlock), 0, stream(), t.table(), t.count(),
                  t.chunks, first.as<int64_t>(), dev_where);
    WM_TRY(check_launch(what));
    const hipError_t e = hipStreamSynchronize(stream());
    if (e != hipSuccess) return set_error(WM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    const int64_t cut[2] = {host_where[0], host_where[1]};
    if (cut[0] < t.count()) {  // table row -> list position
        where_out[0] = t.index[(size_t)cut[0]];
        where_out[1] = cut[1];
    }
    return WM_OK;
}

int wm_grads_finite_multi(int count, const float* const* g, const int64_t* n, int* all_finite) {
    if (!all_finite) return set_error(WM_ERR_INVALID, "wm_grads_finite_multi: null all_finite");
    *all_finite = 1;
    int64_t where[2];
    WM_TRY(first_bad_multi(count, g, nullptr, n, 1.0f, where, "wm_grads_finite_multi"));
    *all_finite = where[0] < count ? 0 : 1;
    return WM_OK;
}

int wm_grad_first_bad_multi_gs(int count, const float* const* g, const wm_grad_scale* gs, const int64_t* n,
                               float scale, int64_t* where) {
    if (!where) return set_error(WM_ERR_INVALID, "wm_grad_first_bad_multi_gs: null where");
    return first_bad_multi(count, g, gs, n, scale, where, "wm_grad_first_bad_multi_gs");
}

int wm_grad_sumsq_multi_gs(int count, const float* const* g, const wm_grad_scale* gs, const int64_t* n, float mul,
                           float* total) {
    return sumsq_multi(count, g, n, mul, total, "wm_grad_sumsq_multi_gs", gs);
}

// An in-place map over a gradient list, one launch per run of gradients that
// do not overlap (a gradient listed twice is mapped twice, in list order).
static int map_grads(int count, float* const* g, const int64_t* n, int mode, const float* total, float arg,
                     const char* what, const wm_grad_scale* gs = nullptr) {
    if (count < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative count");
    if (count > 0 && (!g || !n)) return set_error(WM_ERR_INVALID, std::string(what) + ": null array");
    if (count == 0) return WM_OK;
    WM_CHECK_INIT();
    for (const auto& run : independent_runs(count, g, nullptr, nullptr, nullptr, n, 0)) {
        const int b = run.first;
        MultiTable t;
        WM_TRY(t.build(run.second - b, g + b, nullptr, nullptr, nullptr, n + b, 0, what, gs ? gs + b : nullptr));
        if (t.chunks == 0) continue;
        launch_kernel(multi_map_kernel, dim3(t.grid_s()), dim3(kBlock), 0, stream(), t.table(), t.count(),
                      t.chunks_s, mode, total, arg, 0, (int64_t)0);
        WM_TRY(check_launch(what));
    }
    return WM_OK;
}

int wm_clip_grad_norm_scale_multi(int count, float* const* g, const int64_t* n, const float* total_sumsq,
                                  float max_norm) {
    if (!total_sumsq) return set_error(WM_ERR_INVALID, "wm_clip_grad_norm_scale_multi: null total");
    return map_grads(count, g, n, 0, total_sumsq, max_norm, "wm_clip_grad_norm_scale_multi");
}

int wm_clip_grad_value_multi(int count, float* const* g, const int64_t* n, float clip_value) {
    return map_grads(count, g, n, 1, nullptr, clip_value, "wm_clip_grad_value_multi");
}

int wm_grad_scale_apply_multi(int count, float* const* g, const wm_grad_scale* gs, const int64_t* n) {
    if (count > 0 && !gs) return set_error(WM_ERR_INVALID, "wm_grad_scale_apply_multi: null scales");
    return map_grads(count, g, n, 3, nullptr, 0.0f, "wm_grad_scale_apply_multi", gs);
}

}  // extern "C"
