// Row softmax / log_softmax forward and backward, one row per workgroup.
//
// Reference: softmax core/tensor.cpp:1548-1591, log_softmax :1593-1635.  Both
// take a 2-D tensor and always work along the last axis (the dim argument is
// normalised and then ignored).  The reference walks each row three times
// (max; exp + sum into the output; scale by 1/sum) and its softmax backward is
// the explicit O(C^2) Jacobian loop (:1577-1588).  Here a row is loaded once
// into registers (up to 1024 threads x ITEMS float4), the max and the sum of
// exp(x - max) are combined across the workgroup through LDS, and the row is
// written once; the backward uses the closed form
//   dx_j += y_j * (g_j - sum_k g_k y_k)
// which is that Jacobian contracted with g.  Rows longer than the register
// tile stream through three passes instead.
#include "wm_common.hpp"

#include <algorithm>

namespace wm {

template <int NT>
__device__ __forceinline__ float block_max(float v, float* lds) {
    constexpr int NW = NT / 64;
    v = wave_max(v);
    if (NW == 1) return v;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = lds[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) m = fmaxf(m, lds[i]);
    return m;
}

// Registers of one thread: ITEMS float4 slots.  Element e of slot t lives at
// column (t * NT + tid) * 4 + e (VEC) or t * NT * 4 + e * NT + tid (scalar),
// so each load instruction of a wave is contiguous either way.
template <int NT, int ITEMS, bool VEC>
struct RowTile {
    float v[ITEMS][4];

    __device__ __forceinline__ static int64_t col(int t, int e) {
        return VEC ? ((int64_t)(t * NT + (int)threadIdx.x) * 4 + e) : ((int64_t)t * NT * 4 + (int64_t)e * NT + threadIdx.x);
    }

    __device__ __forceinline__ void load(const float* row, int64_t cols, float fill) {
#pragma unroll
        for (int t = 0; t < ITEMS; ++t) {
            if constexpr (VEC) {
                int64_t c = col(t, 0);
                if (c < cols) {
                    float4 q = ld_stream(row + c);
                    v[t][0] = q.x; v[t][1] = q.y; v[t][2] = q.z; v[t][3] = q.w;
                } else {
                    v[t][0] = v[t][1] = v[t][2] = v[t][3] = fill;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    int64_t c = col(t, e);
                    v[t][e] = c < cols ? ld_stream1(row + c) : fill;
                }
            }
        }
    }

    __device__ __forceinline__ void store(float* row, int64_t cols) const {
#pragma unroll
        for (int t = 0; t < ITEMS; ++t) {
            if constexpr (VEC) {
                int64_t c = col(t, 0);
                if (c < cols) st_stream(row + c, make_float4(v[t][0], v[t][1], v[t][2], v[t][3]));
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    int64_t c = col(t, e);
                    if (c < cols) st_stream1(row + c, v[t][e]);
                }
            }
        }
    }
};

// One-barrier block reductions for the forward kernel, which gives the max
// and the sum separate LDS arrays: a thread can only write a row's partial to
// one array after every thread has passed the barrier of the other array's
// reduction for that row, i.e. after all reads of the previous row's values.
template <int NT>
__device__ __forceinline__ float block_max_1(float v, float* lds) {
    constexpr int NW = NT / 64;
    v = wave_max(v);
    if (NW == 1) return v;
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = lds[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) m = fmaxf(m, lds[i]);
    return m;
}

template <int NT>
__device__ __forceinline__ float block_sum_1(float v, float* lds) {
    constexpr int NW = NT / 64;
    v = wave_sum(v);
    if (NW == 1) return v;
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) t += lds[i];
    return t;
}

// LOG = false: softmax, true: log_softmax.
// Each thread first takes the max m_t of its own slots and the sum
// s_t = sum exp(x - m_t) (keeping exp(x - m_t) for softmax), so the
// exponentials are computed while the rest of the workgroup's loads are
// still arriving; the row max M and the sum S = sum_t s_t exp(m_t - M) then
// take one barrier each.  softmax writes exp(x - m_t) * exp(m_t - M) / S and
// log_softmax x - (M + log S): the reference's x - max, exp, sum and scale
// (core/tensor.cpp:1548-1591, :1593-1635) regrouped, within a few ulp.
// Padding slots hold -inf and contribute exp(-inf) = 0.  A thread whose slots
// are all -inf uses 0 in place of m_t and contributes nothing.  NaN and
// infinite inputs turn the whole row to NaN, as in the reference.
template <int NT, int ITEMS, bool VEC, bool LOG>
__global__ void __launch_bounds__(NT) softmax_fwd_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                          int64_t rows, int64_t cols) {
    __shared__ float lds_m[NT / 64], lds_s[NT / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        RowTile<NT, ITEMS, VEC> tile;
        tile.load(x + r * cols, cols, -INFINITY);
        float mt = -INFINITY;
#pragma unroll
        for (int t = 0; t < ITEMS; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) mt = fmaxf(mt, tile.v[t][e]);
        const float base = mt == -INFINITY ? 0.f : mt;
        float st = 0.f;
#pragma unroll
        for (int t = 0; t < ITEMS; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ex = exp_rr(tile.v[t][e] - base);
                st += ex;
                if (!LOG) tile.v[t][e] = ex;
            }
        const float m = block_max_1<NT>(mt, lds_m);
        const float ct = mt == -INFINITY ? 0.f : exp_rr(mt - m);
        const float s = block_sum_1<NT>(st * ct, lds_s);
        if (LOG) {
            const float log_sum = m + logf(s);
#pragma unroll
            for (int t = 0; t < ITEMS; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) tile.v[t][e] = tile.v[t][e] - log_sum;
        } else {
            const float k = ct * (1.0f / s);
#pragma unroll
            for (int t = 0; t < ITEMS; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) tile.v[t][e] *= k;
        }
        tile.store(out + r * cols, cols);
    }
}

// softmax:     gx (+)= y * (g - sum(g*y)),  y = out
// log_softmax: gx (+)= g - exp(out) * sum(g)
// For softmax the dot product is split into the dominant element (y > 0.5;
// at most one per row) and the rest: for the dominant j,
//   g_j - sum(g*y) = g_j * (1 - y_j) - sum_{k != j} g_k y_k,
// which avoids the cancellation of g_j - g_j y_j when y_j is close to 1 (a
// spike in the logits), matching what the reference's explicit Jacobian
// (y_j (1 - y_j) on the diagonal) computes.
__device__ __forceinline__ float softmax_dx(float g, float y, float s_dom, float s_rest) {
    return y > 0.5f ? y * (g * (1.0f - y) - s_rest) : y * (g - (s_dom + s_rest));
}

template <int NT, int ITEMS, bool VEC, bool LOG>
__global__ void __launch_bounds__(NT) softmax_bwd_kernel(const float* __restrict__ g, const float* __restrict__ out,
                                                          float* __restrict__ gx, int acc, int64_t rows, int64_t cols) {
    __shared__ float lds[NT / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        RowTile<NT, ITEMS, VEC> tg, ty;
        tg.load(g + r * cols, cols, 0.f);
        ty.load(out + r * cols, cols, 0.f);
        float s = 0.f, sd = 0.f;
#pragma unroll
        for (int t = 0; t < ITEMS; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (LOG) s += tg.v[t][e];
                else {
                    const float p = tg.v[t][e] * ty.v[t][e];
                    if (ty.v[t][e] > 0.5f) sd += p;
                    else s += p;
                }
            }
        s = block_sum<NT>(s, lds);
        if (!LOG) sd = block_sum<NT>(sd, lds);
#pragma unroll
        for (int t = 0; t < ITEMS; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (LOG) tg.v[t][e] = tg.v[t][e] - exp_rr(ty.v[t][e]) * s;
                else tg.v[t][e] = softmax_dx(tg.v[t][e], ty.v[t][e], sd, s);
            }
        if (acc) {
            RowTile<NT, ITEMS, VEC> old;
            old.load(gx + r * cols, cols, 0.f);
#pragma unroll
            for (int t = 0; t < ITEMS; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) tg.v[t][e] = old.v[t][e] + tg.v[t][e];
        }
        tg.store(gx + r * cols, cols);
    }
}

// Rows too long for the register tile: three streaming passes per row.
template <bool LOG>
__global__ void __launch_bounds__(1024) softmax_fwd_long_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                                 int64_t rows, int64_t cols) {
    __shared__ float lds[16];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * cols;
        float* orow = out + r * cols;
        float m = -INFINITY;
        for (int64_t c = threadIdx.x; c < cols; c += 1024) m = fmaxf(m, xr[c]);
        m = block_max<1024>(m, lds);
        float s = 0.f;
        for (int64_t c = threadIdx.x; c < cols; c += 1024) s += exp_rr(xr[c] - m);
        s = block_sum<1024>(s, lds);
        if (LOG) {
            const float log_sum = m + logf(s);
            for (int64_t c = threadIdx.x; c < cols; c += 1024) orow[c] = xr[c] - log_sum;
        } else {
            const float inv = 1.0f / s;
            for (int64_t c = threadIdx.x; c < cols; c += 1024) orow[c] = exp_rr(xr[c] - m) * inv;
        }
        __syncthreads();
    }
}

template <bool LOG>
__global__ void __launch_bounds__(1024) softmax_bwd_long_kernel(const float* __restrict__ g,
                                                                 const float* __restrict__ out, float* __restrict__ gx,
                                                                 int acc, int64_t rows, int64_t cols) {
    __shared__ float lds[16];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* gr = g + r * cols;
        const float* yr = out + r * cols;
        float* dr = gx + r * cols;
        float s = 0.f, sd = 0.f;
        for (int64_t c = threadIdx.x; c < cols; c += 1024) {
            if (LOG) s += gr[c];
            else if (yr[c] > 0.5f) sd += gr[c] * yr[c];
            else s += gr[c] * yr[c];
        }
        s = block_sum<1024>(s, lds);
        if (!LOG) sd = block_sum<1024>(sd, lds);
        for (int64_t c = threadIdx.x; c < cols; c += 1024) {
            float d = LOG ? gr[c] - exp_rr(yr[c]) * s : softmax_dx(gr[c], yr[c], sd, s);
            dr[c] = acc ? dr[c] + d : d;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------

// Pick the register tile: NT = 64 for rows up to 2048 columns, else 1024;
// ITEMS the smallest power of two (<= 8) covering the row.
struct TileChoice {
    int nt = 0, items = 0;  // nt == 0: long-row path
};

static TileChoice choose_tile(int64_t cols) {
    TileChoice t;
    const int nts[2] = {64, 1024};
    for (int nt : nts) {
        for (int items = 1; items <= 8; items *= 2) {
            if (cols <= (int64_t)nt * 4 * items) { t.nt = nt; t.items = items; return t; }
        }
    }
    return t;
}

template <bool LOG>
int launch_softmax_fwd(float* out, const float* x, int64_t rows, int64_t cols) {
    hipStream_t st = stream();
    TileChoice tc = choose_tile(cols);
    const bool vec = cols % 4 == 0 && aligned16(out) && aligned16(x);
    // Several rows per CU in flight; the grid-stride loop covers the rest.
    dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * (tc.nt == 64 ? 32 : 4)));
    if (tc.nt == 0) {
        hipLaunchKernelGGL(softmax_fwd_long_kernel<LOG>, grid, dim3(1024), 0, st, out, x, rows, cols);
        return check_launch("wm_softmax_fwd(long)");
    }
#define WM_SF(NTv, IT)                                                                                        \
    if (tc.nt == NTv && tc.items == IT) {                                                                     \
        if (vec) hipLaunchKernelGGL((softmax_fwd_kernel<NTv, IT, true, LOG>), grid, dim3(NTv), 0, st, out, x, rows, cols); \
        else hipLaunchKernelGGL((softmax_fwd_kernel<NTv, IT, false, LOG>), grid, dim3(NTv), 0, st, out, x, rows, cols); \
        return check_launch("wm_softmax_fwd");                                                                \
    }
    WM_SF(64, 1) WM_SF(64, 2) WM_SF(64, 4) WM_SF(64, 8)
    WM_SF(1024, 1) WM_SF(1024, 2) WM_SF(1024, 4) WM_SF(1024, 8)
#undef WM_SF
    return set_error(WM_ERR_INVALID, "wm_softmax_fwd: no tile");
}

template <bool LOG>
int launch_softmax_bwd(const float* g, const float* out, float* gx, int acc, int64_t rows, int64_t cols) {
    hipStream_t st = stream();
    TileChoice tc = choose_tile(cols);
    const bool vec = cols % 4 == 0 && aligned16(g) && aligned16(out) && aligned16(gx);
    dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * (tc.nt == 64 ? 32 : 4)));
    if (tc.nt == 0) {
        hipLaunchKernelGGL(softmax_bwd_long_kernel<LOG>, grid, dim3(1024), 0, st, g, out, gx, acc, rows, cols);
        return check_launch("wm_softmax_bwd(long)");
    }
#define WM_SB(NTv, IT)                                                                                              \
    if (tc.nt == NTv && tc.items == IT) {                                                                           \
        if (vec) hipLaunchKernelGGL((softmax_bwd_kernel<NTv, IT, true, LOG>), grid, dim3(NTv), 0, st, g, out, gx, acc, rows, cols); \
        else hipLaunchKernelGGL((softmax_bwd_kernel<NTv, IT, false, LOG>), grid, dim3(NTv), 0, st, g, out, gx, acc, rows, cols); \
        return check_launch("wm_softmax_bwd");                                                                      \
    }
    WM_SB(64, 1) WM_SB(64, 2) WM_SB(64, 4) WM_SB(64, 8)
    WM_SB(1024, 1) WM_SB(1024, 2) WM_SB(1024, 4) WM_SB(1024, 8)
#undef WM_SB
    return set_error(WM_ERR_INVALID, "wm_softmax_bwd: no tile");
}

static int check_rc(int64_t rows, int64_t cols, const void* a, const void* b, const char* what) {
    if (rows < 0 || cols < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative extent");
    if (rows > 0 && cols > 0 && (!a || !b)) return set_error(WM_ERR_INVALID, std::string(what) + ": null pointer");
    return WM_OK;
}

}  // namespace wm

using namespace wm;

extern "C" {

int wm_softmax_fwd(float* out, const float* x, int64_t rows, int64_t cols) {
    WM_TRY(check_rc(rows, cols, out, x, "wm_softmax_fwd"));
    if (rows == 0 || cols == 0) return WM_OK;
    WM_CHECK_INIT();
    return launch_softmax_fwd<false>(out, x, rows, cols);
}

int wm_log_softmax_fwd(float* out, const float* x, int64_t rows, int64_t cols) {
    WM_TRY(check_rc(rows, cols, out, x, "wm_log_softmax_fwd"));
    if (rows == 0 || cols == 0) return WM_OK;
    WM_CHECK_INIT();
    return launch_softmax_fwd<true>(out, x, rows, cols);
}

int wm_softmax_bwd(const float* g, const float* out, float* gx, int accumulate, int64_t rows, int64_t cols) {
    WM_TRY(check_rc(rows, cols, g, out, "wm_softmax_bwd"));
    if (rows == 0 || cols == 0) return WM_OK;
    if (!gx) return set_error(WM_ERR_INVALID, "wm_softmax_bwd: null gx");
    WM_CHECK_INIT();
    return launch_softmax_bwd<false>(g, out, gx, accumulate, rows, cols);
}

int wm_log_softmax_bwd(const float* g, const float* out, float* gx, int accumulate, int64_t rows, int64_t cols) {
    WM_TRY(check_rc(rows, cols, g, out, "wm_log_softmax_bwd"));
    if (rows == 0 || cols == 0) return WM_OK;
    if (!gx) return set_error(WM_ERR_INVALID, "wm_log_softmax_bwd: null gx");
    WM_CHECK_INIT();
    return launch_softmax_bwd<true>(g, out, gx, accumulate, rows, cols);
}

}  // extern "C"
