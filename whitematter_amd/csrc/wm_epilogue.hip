// Fused fp16-storage epilogue: out = tanh(clamp((h + res) * g, lo, hi)) and
// its row mean, forward and backward, for [rows, cols] activations stored as
// fp16 with fp32 compute (the AMP storage scheme of the reference's
// HalfTensor, core/amp.h:256-286).
//
// In the reference this is a chain of Tensor ops on fp32 tensors converted
// from fp16 storage (half_to_float, core/amp.h:40-72): add (core/tensor.cpp
// :897), mul by a broadcast [cols] vector (:1063), clamp (:1524), tanh_
// (:1302), then reshape + mean(1, keepdim) (:2250, :1709).  Each op makes a
// full pass over HBM; here the forward reads h and res once (2 bytes each)
// and writes out (2 bytes) and the row means, and the backward recomputes the
// chain from h, res and g instead of reading saved intermediates.
//
// Backward of the chain, as the reference closures compose it (mean reuses
// sum's closure, so its gradient is not divided by cols):
//   dw = dm[row]                      (mean -> sum closure, :1697-1703)
//   dv = dw * (1 - w*w)               (tanh_, :1316-1317; w recomputed)
//   du = lo < u < hi ? dv : 0         (clamp, :1538-1540)
//   dt = du * g[col],  dg[col] += du * t   (mul, broadcast, :1122-1142)
//   dh += dt,  dres += dt             (add, :911-920)
#include "wm_common.hpp"

#include <algorithm>

namespace wm {

constexpr int kBlock = 256;

__device__ __forceinline__ float h2f(uint32_t h) { return half_bits_to_float(h); }
__device__ __forceinline__ uint32_t f2h(float f) { return float_to_half_bits_rtz(f); }

struct Chain {
    float t, u, w;
};

// FC: lo and hi are neither zero nor NaN.  Then the hardware min / max give
// the reference's clamp bit for bit: fminf(u, hi) is u below hi, hi above
// it, hi for a NaN u (as (u < hi) ? u : hi is), and a tie returns the same
// bits either way since hi is not a signed zero; likewise fmaxf(lo, m).
template <bool FC>
__device__ __forceinline__ Chain chain(float h, float r, float g, float lo, float hi) {
    Chain c;
    c.t = h + r;
    c.u = c.t * g;
    float v;
    if constexpr (FC) {
        v = fmaxf(lo, fminf(c.u, hi));
    } else {
        const float m = (c.u < hi) ? c.u : hi;  // std::min(hi, u)
        v = (lo < m) ? m : lo;                  // std::max(lo, .)
    }
    c.w = tanh_fast(v);
    return c;
}

// Forward: one wave per row.  With 128-bit accesses lane l takes 8
// consecutive columns at 512 j + 8 l for j = 0, 1, ..., so every load and
// store instruction of a wave covers 1 KB of one fp16 row; U steps of loads
// are issued before any is used.  The row mean is a DPP / shuffle wave sum:
// no barrier anywhere.  VEC: cols % 8 == 0 and 16-byte aligned.
template <bool VEC, bool FC>
__global__ void __launch_bounds__(kBlock) epilogue_fwd_kernel(uint16_t* __restrict__ out, float* __restrict__ mean,
                                                               const uint16_t* __restrict__ h,
                                                               const uint16_t* __restrict__ res,
                                                               const float* __restrict__ g, int64_t rows,
                                                               int64_t cols, float lo, float hi) {
    constexpr int U = 4;
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * kBlock) >> 6;
    for (int64_t r = wave; r < rows; r += nwaves) {
        const uint16_t* hr = h + r * cols;
        const uint16_t* rr = res + r * cols;
        uint16_t* orow = out ? out + r * cols : nullptr;
        float s = 0.f;
        if constexpr (VEC) {
            // one step: 8 columns at c from each input, 8 outputs
            auto step = [&](float4 hq, float4 rq, int64_t c) {
                const float4 g0 = *reinterpret_cast<const float4*>(g + c);
                const float4 g1 = *reinterpret_cast<const float4*>(g + c + 4);
                const uint32_t hw[4] = {__float_as_uint(hq.x), __float_as_uint(hq.y), __float_as_uint(hq.z),
                                        __float_as_uint(hq.w)};
                const uint32_t rw[4] = {__float_as_uint(rq.x), __float_as_uint(rq.y), __float_as_uint(rq.z),
                                        __float_as_uint(rq.w)};
                const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
                float wv[8];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    wv[2 * k] = chain<FC>(h2f(hw[k] & 0xFFFFu), h2f(rw[k] & 0xFFFFu), gv[2 * k], lo, hi).w;
                    wv[2 * k + 1] = chain<FC>(h2f(hw[k] >> 16), h2f(rw[k] >> 16), gv[2 * k + 1], lo, hi).w;
                }
                const float t = ((wv[0] + wv[1]) + (wv[2] + wv[3])) + ((wv[4] + wv[5]) + (wv[6] + wv[7]));
                s += t;
                // tanh gives [-1, 1] or NaN, and the hardware's packed
                // truncating conversion is the reference's float_to_half for
                // every finite |x| < 65536: only a NaN (t is NaN iff some w
                // is) takes the bit formula
                uint32_t ow[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    typedef __fp16 wm_h2 __attribute__((ext_vector_type(2)));
                    ow[k] = __builtin_bit_cast(uint32_t, (wm_h2)__builtin_amdgcn_cvt_pkrtz(wv[2 * k], wv[2 * k + 1]));
                }
                if (__builtin_isnan(t)) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) ow[k] = float2_to_half2_bits_rtz(wv[2 * k], wv[2 * k + 1]);
                }
                if (orow)
                    st_stream(reinterpret_cast<float*>(orow + c),
                              make_float4(__uint_as_float(ow[0]), __uint_as_float(ow[1]), __uint_as_float(ow[2]),
                                          __uint_as_float(ow[3])));
            };
            int64_t c = (int64_t)lane * 8;
            for (; c + (U - 1) * 512 < cols; c += U * 512) {
                float4 hq[U], rq[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    hq[u] = ld_stream(reinterpret_cast<const float*>(hr + c + u * 512));
                    rq[u] = ld_stream(reinterpret_cast<const float*>(rr + c + u * 512));
                }
#pragma unroll
                for (int u = 0; u < U; ++u) step(hq[u], rq[u], c + u * 512);
            }
            for (; c < cols; c += 512)
                step(ld_stream(reinterpret_cast<const float*>(hr + c)), ld_stream(reinterpret_cast<const float*>(rr + c)),
                     c);
        } else {
            for (int64_t c = lane; c < cols; c += 64) {
                const Chain ch = chain<FC>(h2f(hr[c]), h2f(rr[c]), g[c], lo, hi);
                s += ch.w;
                if (orow) orow[c] = (uint16_t)f2h(ch.w);
            }
        }
        s = wave_sum(s);
        if (lane == 0) mean[r] = s / (float)cols;
    }
}

// Forward for rows of 1024 to 8192 columns (VEC): one workgroup of NT
// threads per row, thread t taking the 8 columns at 8 (u NT + t) for u < S.
// All of a row's loads are issued before any math and the row mean is one
// fixed-order block sum.  A short-lived workgroup reading one contiguous row
// measured 67.8 -> 73.1 % of the HBM peak against a wave walking each row
// (config 5, [32768, 4096], 256 threads x 2 steps).
template <int NT, int S, bool FC>
__global__ void __launch_bounds__(NT) epilogue_fwd_wg_kernel(uint16_t* __restrict__ out, float* __restrict__ mean,
                                                              const uint16_t* __restrict__ h,
                                                              const uint16_t* __restrict__ res,
                                                              const float* __restrict__ g, int64_t rows,
                                                              int64_t cols, float lo, float hi) {
    __shared__ float lds[NT / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const uint16_t* hr = h + r * cols;
        const uint16_t* rr = res + r * cols;
        uint16_t* orow = out ? out + r * cols : nullptr;
        float4 hq[S], rq[S];
#pragma unroll
        for (int u = 0; u < S; ++u) {
            const int64_t c = ((int64_t)u * NT + threadIdx.x) * 8;
            hq[u] = c < cols ? ld_stream(reinterpret_cast<const float*>(hr + c)) : make_float4(0.f, 0.f, 0.f, 0.f);
            rq[u] = c < cols ? ld_stream(reinterpret_cast<const float*>(rr + c)) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        float s = 0.f;
#pragma unroll
        for (int u = 0; u < S; ++u) {
            const int64_t c = ((int64_t)u * NT + threadIdx.x) * 8;
            if (c >= cols) continue;
            const float4 g0 = *reinterpret_cast<const float4*>(g + c);
            const float4 g1 = *reinterpret_cast<const float4*>(g + c + 4);
            const uint32_t hw[4] = {__float_as_uint(hq[u].x), __float_as_uint(hq[u].y), __float_as_uint(hq[u].z),
                                    __float_as_uint(hq[u].w)};
            const uint32_t rw[4] = {__float_as_uint(rq[u].x), __float_as_uint(rq[u].y), __float_as_uint(rq[u].z),
                                    __float_as_uint(rq[u].w)};
            const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
            float wv[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                wv[2 * k] = chain<FC>(h2f(hw[k] & 0xFFFFu), h2f(rw[k] & 0xFFFFu), gv[2 * k], lo, hi).w;
                wv[2 * k + 1] = chain<FC>(h2f(hw[k] >> 16), h2f(rw[k] >> 16), gv[2 * k + 1], lo, hi).w;
            }
            const float t = ((wv[0] + wv[1]) + (wv[2] + wv[3])) + ((wv[4] + wv[5]) + (wv[6] + wv[7]));
            s += t;
            uint32_t ow[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                typedef __fp16 wm_h2 __attribute__((ext_vector_type(2)));
                ow[k] = __builtin_bit_cast(uint32_t, (wm_h2)__builtin_amdgcn_cvt_pkrtz(wv[2 * k], wv[2 * k + 1]));
            }
            if (__builtin_isnan(t)) {
#pragma unroll
                for (int k = 0; k < 4; ++k) ow[k] = float2_to_half2_bits_rtz(wv[2 * k], wv[2 * k + 1]);
            }
            if (orow)
                st_stream(reinterpret_cast<float*>(orow + c),
                          make_float4(__uint_as_float(ow[0]), __uint_as_float(ow[1]), __uint_as_float(ow[2]),
                                      __uint_as_float(ow[3])));
        }
        s = block_sum<NT>(s, lds);
        if (threadIdx.x == 0) mean[r] = s / (float)cols;
    }
}

// Backward: a workgroup owns 8*kBlock adjacent columns and row group k
// (blockIdx.y of K = gridDim.y), the rows k, k + K, k + 2K, ...: the resident
// workgroups then read one narrow band of rows that advances down the
// matrix (67.6 -> 73.4 % of the HBM peak at config 5 against contiguous
// blocks of rows / K rows).  With 128-bit accesses lane i of wave w handles
// the two 4-column groups at tile + 512 w + 4 i and 256 columns further on,
// so every load and store instruction of a wave covers one contiguous span
// (512 B of fp16 input, 1 KB of fp32 gradient).  Each thread keeps its 8
// column partials of dg in registers over its rows (fixed order) and writes
// them to part[k, col] for a fixed-order second pass.
typedef unsigned int wm_v2u __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void load_half4(const uint16_t* p, float* out) {
    const wm_v2u q = __builtin_nontemporal_load(reinterpret_cast<const wm_v2u*>(p));
    out[0] = half_bits_to_float(q.x & 0xFFFFu);
    out[1] = half_bits_to_float(q.x >> 16);
    out[2] = half_bits_to_float(q.y & 0xFFFFu);
    out[3] = half_bits_to_float(q.y >> 16);
}

template <bool VEC, bool FC>
__global__ void __launch_bounds__(kBlock) epilogue_bwd_kernel(const float* __restrict__ dm,
                                                               const uint16_t* __restrict__ h,
                                                               const uint16_t* __restrict__ res,
                                                               const float* __restrict__ g, float* __restrict__ gh,
                                                               int acc_h, float* __restrict__ gres, int acc_res,
                                                               float* __restrict__ part, int64_t rows, int64_t cols,
                                                               float lo, float hi) {
    constexpr int W = VEC ? 8 : 1;
    int64_t cg[2];  // first column of each 4-column group (VEC), or the one column
    if constexpr (VEC) {
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        cg[0] = (int64_t)blockIdx.x * (kBlock * 8) + w * 512 + lane * 4;
        cg[1] = cg[0] + 256;
        if (cg[0] >= cols) return;  // cols % 512 == 0 on this path: both groups are in range
    } else {
        cg[0] = (int64_t)blockIdx.x * kBlock + threadIdx.x;
        if (cg[0] >= cols) return;
    }
    float gv[W], acc[W];
#pragma unroll
    for (int j = 0; j < W; ++j) {
        gv[j] = VEC ? g[cg[j / 4] + (j % 4)] : g[cg[0]];
        acc[j] = 0.f;
    }
#pragma unroll 2
    for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
        const float dw = dm[r];
        const int64_t roff = r * cols;
        float hv[W], rv[W];
        if constexpr (VEC) {
            load_half4(h + roff + cg[0], hv);
            load_half4(h + roff + cg[1], hv + 4);
            load_half4(res + roff + cg[0], rv);
            load_half4(res + roff + cg[1], rv + 4);
        } else {
            hv[0] = half_bits_to_float(h[roff + cg[0]]);
            rv[0] = half_bits_to_float(res[roff + cg[0]]);
        }
        float dt[W];
#pragma unroll
        for (int j = 0; j < W; ++j) {
            Chain ch = chain<FC>(hv[j], rv[j], gv[j], lo, hi);
            const float dv = dw * (1.0f - ch.w * ch.w);
            const float du = (ch.u > lo && ch.u < hi) ? dv : 0.0f;
            dt[j] = du * gv[j];
            acc[j] += du * ch.t;
        }
        if constexpr (VEC) {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int64_t off = roff + cg[q];
                const float4 d = make_float4(dt[4 * q], dt[4 * q + 1], dt[4 * q + 2], dt[4 * q + 3]);
                if (gh) {
                    float4 o = d;
                    if (acc_h) {
                        const float4 p = ld_stream(gh + off);
                        o.x += p.x; o.y += p.y; o.z += p.z; o.w += p.w;
                    }
                    st_stream(gh + off, o);
                }
                if (gres) {
                    float4 o = d;
                    if (acc_res) {
                        const float4 p = ld_stream(gres + off);
                        o.x += p.x; o.y += p.y; o.z += p.z; o.w += p.w;
                    }
                    st_stream(gres + off, o);
                }
            }
        } else {
            const int64_t off = roff + cg[0];
            if (gh) gh[off] = acc_h ? gh[off] + dt[0] : dt[0];
            if (gres) gres[off] = acc_res ? gres[off] + dt[0] : dt[0];
        }
    }
    if (part) {
        float* pr = part + (int64_t)blockIdx.y * cols;
        if constexpr (VEC) {
            *reinterpret_cast<float4*>(pr + cg[0]) = make_float4(acc[0], acc[1], acc[2], acc[3]);
            *reinterpret_cast<float4*>(pr + cg[1]) = make_float4(acc[4], acc[5], acc[6], acc[7]);
        } else {
            pr[cg[0]] = acc[0];
        }
    }
}

// gg[c] (+)= sum_k part[k, c]: 64 columns per workgroup of 16 waves; wave
// w folds k = w, w + 16, ... (four loads in flight per lane), and the 16
// wave sums are added in wave order through LDS (a fixed order).
constexpr int kSumBlock = 1024;
__global__ void __launch_bounds__(kSumBlock) epilogue_gsum_kernel(const float* __restrict__ part,
                                                                   float* __restrict__ gg, int acc, int64_t K,
                                                                   int64_t C) {
    constexpr int NW = kSumBlock / 64;
    __shared__ float lds[NW][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int64_t c0 = (int64_t)blockIdx.x * 64; c0 < C; c0 += (int64_t)gridDim.x * 64) {
        const int64_t c = c0 + lane;
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        if (c < C) {
            int64_t k = w;
            for (; k + 3 * NW < K; k += 4 * NW) {
#pragma unroll
                for (int j = 0; j < 4; ++j) s[j] += part[(k + j * NW) * C + c];
            }
            for (int j = 0; k < K; k += NW, ++j) s[j & 3] += part[k * C + c];
        }
        lds[w][lane] = (s[0] + s[1]) + (s[2] + s[3]);
        __syncthreads();
        if (w == 0 && c < C) {
            float t = lds[0][lane];
#pragma unroll
            for (int ww = 1; ww < NW; ++ww) t += lds[ww][lane];
            gg[c] = acc ? gg[c] + t : t;
        }
        __syncthreads();
    }
}

// The clamp bounds for which the hardware min / max reproduce the
// reference's compare-and-select clamp (see chain).
inline bool clamp_is_minmax(float lo, float hi) {
    return lo != 0.f && hi != 0.f && !std::isnan(lo) && !std::isnan(hi);
}

}  // namespace wm

using namespace wm;

extern "C" {

int wm_epilogue_f16_fwd(uint16_t* out, float* mean, const uint16_t* h, const uint16_t* res, const float* g,
                        int64_t rows, int64_t cols, float lo, float hi) {
    if (rows < 0 || cols < 0) return set_error(WM_ERR_INVALID, "wm_epilogue_f16_fwd: negative extent");
    if (rows == 0 || cols == 0) return WM_OK;
    if (!mean || !h || !res || !g) return set_error(WM_ERR_INVALID, "wm_epilogue_f16_fwd: null pointer");
    WM_CHECK_INIT();
    const bool vec = cols % 8 == 0 && aligned16(h) && aligned16(res) && aligned16(g) && (!out || aligned16(out));
    dim3 grid(grid_for(rows, kBlock / 64, 16));
    const bool fc = clamp_is_minmax(lo, hi);
#define WM_EPI_FWD(V, F)                                                                                       \
    launch_kernel(epilogue_fwd_kernel<V, F>, grid, dim3(kBlock), 0, stream(), out, mean, h, res, g, rows, cols, lo, \
                  hi)
    if (vec && cols >= 1024 && cols <= 8192) {
        const dim3 g1(grid_for(rows, 1, 1 << 12));
#define WM_EPI_WG(S, F)                                                                                       \
    launch_kernel(epilogue_fwd_wg_kernel<kBlock, S, F>, g1, dim3(kBlock), 0, stream(), out, mean, h, res, g, rows, \
                  cols, lo, hi)
        if (cols <= 2048) { if (fc) WM_EPI_WG(1, true); else WM_EPI_WG(1, false); }
        else if (cols <= 4096) { if (fc) WM_EPI_WG(2, true); else WM_EPI_WG(2, false); }
        else { if (fc) WM_EPI_WG(4, true); else WM_EPI_WG(4, false); }
#undef WM_EPI_WG
        return check_launch("wm_epilogue_f16_fwd");
    }
    if (vec) { if (fc) WM_EPI_FWD(true, true); else WM_EPI_FWD(true, false); }
    else { if (fc) WM_EPI_FWD(false, true); else WM_EPI_FWD(false, false); }
#undef WM_EPI_FWD
    return check_launch("wm_epilogue_f16_fwd");
}

int wm_epilogue_f16_bwd(const float* dm, const uint16_t* h, const uint16_t* res, const float* g, float* gh,
                        int acc_h, float* gres, int acc_res, float* gg, int acc_g, int64_t rows, int64_t cols,
                        float lo, float hi) {
    if (rows < 0 || cols < 0) return set_error(WM_ERR_INVALID, "wm_epilogue_f16_bwd: negative extent");
    if (cols == 0) return WM_OK;
    if (rows == 0) {
        if (gg && !acc_g) return wm_fill(gg, 0.f, cols);
        return WM_OK;
    }
    if (!dm || !h || !res || !g) return set_error(WM_ERR_INVALID, "wm_epilogue_f16_bwd: null pointer");
    if (!gh && !gres && !gg) return WM_OK;
    WM_CHECK_INIT();
    const bool vec = cols % 512 == 0 && aligned16(h) && aligned16(res) && aligned16(g) && (!gh || aligned16(gh)) &&
                     (!gres || aligned16(gres));
    const int64_t W = vec ? 8 : 1;
    const int64_t col_tiles = (cols + kBlock * W - 1) / (kBlock * W);
    // ~4 workgroups per CU, each row group of at least 16 rows: each thread
    // folds its columns' dg partials over rows / K rows, and the second pass
    // reads K partials per column
    int64_t K = std::min<int64_t>(((int64_t)num_cus() * 4 + col_tiles - 1) / col_tiles, (rows + 15) / 16);
    K = std::max<int64_t>(1, std::min<int64_t>(K, 65535));
    Workspace ws(gg ? (size_t)(K * cols) * sizeof(float) : 0);
    if (gg && !ws.p) return set_error(WM_ERR_NOMEM, "wm_epilogue_f16_bwd: workspace");
    dim3 grid((unsigned)col_tiles, (unsigned)K);
    const bool fc = clamp_is_minmax(lo, hi);
#define WM_EPI_BWD(V, F)                                                                                     \
    launch_kernel(epilogue_bwd_kernel<V, F>, grid, dim3(kBlock), 0, stream(), dm, h, res, g, gh, acc_h, gres, \
                  acc_res, ws.as<float>(), rows, cols, lo, hi)
    if (vec) { if (fc) WM_EPI_BWD(true, true); else WM_EPI_BWD(true, false); }
    else { if (fc) WM_EPI_BWD(false, true); else WM_EPI_BWD(false, false); }
#undef WM_EPI_BWD
    WM_TRY(check_launch("wm_epilogue_f16_bwd"));
    if (gg) {
        launch_kernel(epilogue_gsum_kernel, dim3(grid_for(cols, 64, 8)), dim3(kSumBlock), 0, stream(),
                      ws.as<float>(), gg, acc_g, K, cols);
        WM_TRY(check_launch("wm_epilogue_f16_bwd(gsum)"));
    }
    return WM_OK;
}

}  // extern "C"
