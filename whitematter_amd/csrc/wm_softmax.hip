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
#include "wm_rows.hpp"

#include <algorithm>

namespace wm {

// LOG = false: softmax, true: log_softmax.  row_max_sum (wm_rows.hpp) gives
// the row max M, the sum S = sum exp(x - M) (regrouped per thread) and each
// thread's exp(x - m_t) for softmax; softmax writes exp(x - m_t) *
// exp(m_t - M) / S and log_softmax x - (M + log S): the reference's x - max,
// exp, sum and scale (core/tensor.cpp:1548-1591, :1593-1635) regrouped,
// within a few ulp.  NaN and infinite inputs turn the whole row to NaN, as in
// the reference.
template <int NT, int ITEMS, bool VEC, bool LOG>
__global__ void __launch_bounds__(NT) softmax_fwd_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                          int64_t rows, int64_t cols) {
    __shared__ float lds_m[NT / 64], lds_s[NT / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        RowTile<NT, ITEMS, VEC> tile;
        tile.load(x + r * cols, cols, -INFINITY);
        const RowMaxSum ms = row_max_sum<NT, ITEMS, VEC, !LOG>(tile, lds_m, lds_s);
        if (LOG) {
            const float log_sum = ms.m + logf(ms.s);
#pragma unroll
            for (int t = 0; t < ITEMS; ++t)
#pragma unroll
                for (int e = 0; e < 4; ++e) tile.v[t][e] = tile.v[t][e] - log_sum;
        } else {
            const float k = ms.ct * (1.0f / ms.s);
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

template <bool LOG>
int launch_softmax_fwd(float* out, const float* x, int64_t rows, int64_t cols) {
    hipStream_t st = stream();
    TileChoice tc = choose_tile(cols);
    const bool vec = cols % 4 == 0 && aligned16(out) && aligned16(x);
    // One workgroup per row (a wave for rows of up to 2048 columns) on a grid
    // that covers every row: 70.3 -> 74.5 % of the HBM peak at [8192, 32000]
    // (backward 75 -> 76.5 %) against 4 workgroups per CU each looping over
    // rows; the one-wave tile, in the attention softmax at 1024 columns,
    // 68.4 -> 75.7 % against 32 workgroups per CU.
    dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * (1 << 12)));
    if (tc.nt == 0) {
        launch_kernel(softmax_fwd_long_kernel<LOG>, grid, dim3(1024), 0, st, out, x, rows, cols);
        return check_launch("wm_softmax_fwd(long)");
    }
#define WM_SF(NTv, IT)                                                                                        \
    if (tc.nt == NTv && tc.items == IT) {                                                                     \
        if (vec) launch_kernel((softmax_fwd_kernel<NTv, IT, true, LOG>), grid, dim3(NTv), 0, st, out, x, rows, cols); \
        else launch_kernel((softmax_fwd_kernel<NTv, IT, false, LOG>), grid, dim3(NTv), 0, st, out, x, rows, cols); \
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
    dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * (1 << 12)));  // as in the forward
    if (tc.nt == 0) {
        launch_kernel(softmax_bwd_long_kernel<LOG>, grid, dim3(1024), 0, st, g, out, gx, acc, rows, cols);
        return check_launch("wm_softmax_bwd(long)");
    }
#define WM_SB(NTv, IT)                                                                                              \
    if (tc.nt == NTv && tc.items == IT) {                                                                           \
        if (vec) launch_kernel((softmax_bwd_kernel<NTv, IT, true, LOG>), grid, dim3(NTv), 0, st, g, out, gx, acc, rows, cols); \
        else launch_kernel((softmax_bwd_kernel<NTv, IT, false, LOG>), grid, dim3(NTv), 0, st, g, out, gx, acc, rows, cols); \
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
