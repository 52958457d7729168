// Reductions over the middle axis of an [outer, n, inner] view, and their
// backward passes.
//
// The reference has three shapes of reduction loop: full (core/tensor.cpp
// :1638-1656, :1727-1748), over rows of a 2-D tensor (dim 0, :1662-1683,
// strided j-outer/i-inner) and over columns (dim 1, :1684-1706), plus the
// N-d argmax/argmin slices (:2096-2142).  All of them are the same
// [outer, n, inner] reduction here:
//   inner == 1  contiguous rows: one wave per (row, chunk), 128-bit loads,
//               DPP/shuffle wave combine; rows that are too few to fill the
//               chip are split into chunks and finished by a second pass;
//   inner  > 1  strided columns: threads own adjacent inner positions
//               (coalesced 128-bit loads), walk a chunk of n, and a second
//               pass combines the chunks in order.
// (value, index) reductions keep the reference's strict-compare scan: the
// first element starts the scan, a later element wins only if strictly
// greater (max) / smaller (min), so ties go to the lowest position and a NaN
// only wins when it is the first element.  The partition and the combine
// order are fixed, so every result is deterministic.
#include "wm_common.hpp"

#include <algorithm>

namespace wm {

constexpr int kBlock = 256;
constexpr int64_t kEmpty = -1;

// ---------------------------------------------------------------------------
// (value, position) state and its combine
// ---------------------------------------------------------------------------

template <bool MAXOP>
__device__ __forceinline__ bool strictly_better(float x, float v) {
    return MAXOP ? (x > v) : (x < v);
}

// Fold element x at position k into (v, i); positions arrive in increasing
// order within one thread.
// Branch-free: an empty state takes any non-NaN element (or a NaN at
// position 0); a non-empty one only a strictly better element.
template <bool MAXOP, class I>
__device__ __forceinline__ void scan_push(float& v, I& i, float x, I k) {
    const bool take = strictly_better<MAXOP>(x, v) || (i == kEmpty && (!__builtin_isnan(x) || k == 0));
    v = take ? x : v;
    i = take ? k : i;
}

// Combine two states over disjoint position sets (any order).
template <bool MAXOP, class I>
__device__ __forceinline__ void combine(float& v, I& i, float v2, I i2) {
    if (i2 == kEmpty) return;
    if (i == 0 && __builtin_isnan(v)) return;                 // NaN first element wins
    if (i2 == 0 && __builtin_isnan(v2)) { v = v2; i = i2; return; }
    if (i == kEmpty || strictly_better<MAXOP>(v2, v) || (!strictly_better<MAXOP>(v, v2) && i2 < i)) {
        v = v2; i = i2;
    }
}

template <bool MAXOP>
__device__ __forceinline__ void wave_combine(float& v, int64_t& i) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        float v2 = __shfl_xor(v, off, 64);
        int64_t i2 = __shfl_xor(i, off, 64);
        combine<MAXOP>(v, i, v2, i2);
    }
}

// Reduction kinds: 0 = sum/mean, 1 = max family, 2 = min family.
__host__ __device__ constexpr int kind_of(int op) {
    return (op == WM_R_SUM || op == WM_R_MEAN) ? 0 : ((op == WM_R_MAX || op == WM_R_ARGMAX) ? 1 : 2);
}

// Write the final result of one output slot.
template <int OP>
__device__ __forceinline__ void write_result(float* val, int64_t* idx, int64_t slot, float v, int64_t i, int64_t n) {
    if constexpr (OP == WM_R_SUM) { val[slot] = v; }
    else if constexpr (OP == WM_R_MEAN) { val[slot] = v / (float)n; }
    else if constexpr (OP == WM_R_MAX || OP == WM_R_MIN) {
        if (val) val[slot] = v;
        if (idx) idx[slot] = i;
    } else {
        if (val) val[slot] = (float)i;
        if (idx) idx[slot] = i;
    }
}

// ---------------------------------------------------------------------------
// inner == 1: rows
// ---------------------------------------------------------------------------

// One wave per (row, chunk).  Partials (value, position) go to pv/pi when the
// row is split (K > 1), else the result is written directly.  Each lane keeps
// four 128-bit loads in flight and folds them in increasing position order.
template <int OP, bool VEC>
__global__ void __launch_bounds__(kBlock) reduce_rows_kernel(const float* __restrict__ x, int64_t rows, int64_t n,
                                                              int64_t chunk, int64_t K, float* __restrict__ val,
                                                              int64_t* __restrict__ idx, float* __restrict__ pv,
                                                              int64_t* __restrict__ pi) {
    constexpr int KIND = kind_of(OP);
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * kBlock) >> 6;
    for (int64_t item = wave; item < rows * K; item += nwaves) {
        const int64_t r = item / K;
        const int64_t k = item - r * K;
        const int64_t c0 = k * chunk;
        const int64_t c1 = min(n, c0 + chunk);
        const float* xr = x + r * n;
        float v = 0.f;
        int64_t pos = kEmpty;
        float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (VEC) {
            int64_t c = c0 + lane * 4;
            for (; c + 3 * 256 < c1; c += 4 * 256) {
                float4 a[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) a[u] = ld_stream(xr + c + u * 256);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if constexpr (KIND == 0) {
                        s.x += a[u].x; s.y += a[u].y; s.z += a[u].z; s.w += a[u].w;
                    } else {
                        const int64_t p = c + u * 256;
                        scan_push<KIND == 1>(v, pos, a[u].x, p);
                        scan_push<KIND == 1>(v, pos, a[u].y, p + 1);
                        scan_push<KIND == 1>(v, pos, a[u].z, p + 2);
                        scan_push<KIND == 1>(v, pos, a[u].w, p + 3);
                    }
                }
            }
            for (; c < c1; c += 256) {
                float4 a0 = ld_stream(xr + c);
                if constexpr (KIND == 0) {
                    s.x += a0.x; s.y += a0.y; s.z += a0.z; s.w += a0.w;
                } else {
                    scan_push<KIND == 1>(v, pos, a0.x, c);
                    scan_push<KIND == 1>(v, pos, a0.y, c + 1);
                    scan_push<KIND == 1>(v, pos, a0.z, c + 2);
                    scan_push<KIND == 1>(v, pos, a0.w, c + 3);
                }
            }
        } else {
            for (int64_t c = c0 + lane; c < c1; c += 64) {
                float a0 = ld_stream1(xr + c);
                if constexpr (KIND == 0) s.x += a0;
                else scan_push<KIND == 1>(v, pos, a0, c);
            }
        }
        if constexpr (KIND == 0) v = wave_sum((s.x + s.y) + (s.z + s.w));
        else wave_combine<KIND == 1>(v, pos);
        if (lane == 0) {
            if (K == 1) write_result<OP>(val, idx, r, v, pos, n);
            else {
                pv[r * K + k] = v;
                if (KIND != 0) pi[r * K + k] = pos;
            }
        }
    }
}

// Second pass for split rows: one block per row, chunks combined in a fixed
// tree (block_sum or the (value, position) combine).
template <int OP>
__global__ void __launch_bounds__(kBlock) reduce_rows_finalize_kernel(const float* __restrict__ pv,
                                                                       const int64_t* __restrict__ pi, int64_t rows,
                                                                       int64_t K, int64_t n, float* __restrict__ val,
                                                                       int64_t* __restrict__ idx) {
    constexpr int KIND = kind_of(OP);
    __shared__ float lv[kBlock / 64];
    __shared__ int64_t li[kBlock / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        if constexpr (KIND == 0) {
            float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            int64_t k = threadIdx.x;
            for (; k + 7 * kBlock < K; k += 8 * kBlock) {
#pragma unroll
                for (int j = 0; j < 8; ++j) a[j] += pv[r * K + k + j * kBlock];
            }
            for (int j = 0; k < K; k += kBlock, ++j) a[j & 7] += pv[r * K + k];
            float s = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
            s = block_sum<kBlock>(s, lv);
            if (threadIdx.x == 0) write_result<OP>(val, idx, r, s, 0, n);
        } else {
            float v = 0.f;
            int64_t pos = kEmpty;
            int64_t k = threadIdx.x;
            for (; k + 7 * kBlock < K; k += 8 * kBlock) {
                float bv[8];
                int64_t bi[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) { bv[j] = pv[r * K + k + j * kBlock]; bi[j] = pi[r * K + k + j * kBlock]; }
#pragma unroll
                for (int j = 0; j < 8; ++j) combine<KIND == 1>(v, pos, bv[j], bi[j]);
            }
            for (; k < K; k += kBlock) combine<KIND == 1>(v, pos, pv[r * K + k], pi[r * K + k]);
            wave_combine<KIND == 1>(v, pos);
            if ((threadIdx.x & 63) == 0) { lv[threadIdx.x >> 6] = v; li[threadIdx.x >> 6] = pos; }
            __syncthreads();
            if (threadIdx.x == 0) {
                float bv = lv[0];
                int64_t bi = li[0];
                for (int w = 1; w < kBlock / 64; ++w) combine<KIND == 1>(bv, bi, lv[w], li[w]);
                write_result<OP>(val, idx, r, bv, bi, n);
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// inner > 1: columns
// ---------------------------------------------------------------------------

// Lane l of each wave owns W adjacent inner positions (W = 4 with 128-bit
// loads) of output row o, so a wave reads 64*W contiguous floats per position
// of n.  The workgroup's 4 waves take four contiguous quarters of the chunk
// [k0, k1) of n, each walking its quarter in increasing order with four loads
// in flight; the four wave results are combined in wave order through LDS.
// Splitting the chunk inside the workgroup (rather than over more
// workgroups) keeps the number of partial results, and so the second pass,
// four times smaller for the same parallelism.  Items are (o, chunk, inner
// tile) triples, tile fastest; every thread of a workgroup walks the same
// items, so the barriers are uniform.
// IdxT: the positions a thread tracks (int32_t whenever n fits, which
// halves the compare-and-select work of the max family); partials and
// results are int64_t.
template <int OP, bool VEC, class IdxT>
__global__ void __launch_bounds__(kBlock) reduce_cols_kernel(const float* __restrict__ x, int64_t outer, int64_t n,
                                                              int64_t inner, int64_t chunk, int64_t K,
                                                              float* __restrict__ val, int64_t* __restrict__ idx,
                                                              float* __restrict__ pv, int64_t* __restrict__ pi) {
    constexpr int KIND = kind_of(OP);
    constexpr int W = VEC ? 4 : 1;
    constexpr int NW = kBlock / 64;
    __shared__ float lv[NW][64 * W];
    __shared__ IdxT li[KIND != 0 ? NW : 1][KIND != 0 ? 64 * W : 1];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t tile_elems = (int64_t)64 * W;
    const int64_t tiles = (inner + tile_elems - 1) / tile_elems;
    const int64_t items = outer * K * tiles;
    for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
        const int64_t t = item % tiles;
        const int64_t ok = item / tiles;
        const int64_t k = ok % K;
        const int64_t o = ok / K;
        const int64_t i0 = t * tile_elems + (int64_t)lane * W;
        const int64_t k0 = k * chunk, k1 = min(n, k0 + chunk);
        const int64_t q = (k1 - k0 + NW - 1) / NW;
        const int64_t r0 = min(k1, k0 + w * q), r1 = min(k1, r0 + q);
        const float* xp = x + o * n * inner + i0;
        float v[W];
        IdxT pos[W];
#pragma unroll
        for (int j = 0; j < W; ++j) { v[j] = 0.f; pos[j] = (IdxT)kEmpty; }
        if (i0 < inner) {
            int64_t p = r0;
            for (; p + 3 < r1; p += 4) {
                float a[4][W];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if constexpr (VEC) {
                        float4 qv = ld_stream(xp + (p + u) * inner);
                        a[u][0] = qv.x; a[u][1] = qv.y; a[u][2] = qv.z; a[u][3] = qv.w;
                    } else {
                        a[u][0] = ld_stream1(xp + (p + u) * inner);
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int j = 0; j < W; ++j) {
                        if constexpr (KIND == 0) v[j] += a[u][j];
                        else scan_push<KIND == 1>(v[j], pos[j], a[u][j], (IdxT)(p + u));
                    }
            }
            for (; p < r1; ++p) {
                float a[W];
                if constexpr (VEC) {
                    float4 qv = ld_stream(xp + p * inner);
                    a[0] = qv.x; a[1] = qv.y; a[2] = qv.z; a[3] = qv.w;
                } else {
                    a[0] = ld_stream1(xp + p * inner);
                }
#pragma unroll
                for (int j = 0; j < W; ++j) {
                    if constexpr (KIND == 0) v[j] += a[j];
                    else scan_push<KIND == 1>(v[j], pos[j], a[j], (IdxT)p);
                }
            }
        }
        __syncthreads();  // the previous item's LDS reads are done
#pragma unroll
        for (int j = 0; j < W; ++j) {
            lv[w][lane * W + j] = v[j];
            if constexpr (KIND != 0) li[w][lane * W + j] = pos[j];
        }
        __syncthreads();
        if (w == 0) {
#pragma unroll
            for (int j = 0; j < W; ++j) {
                const int64_t i = i0 + j;
                if (i >= inner) break;
                float tv = lv[0][lane * W + j];
                IdxT ti = (IdxT)kEmpty;
                if constexpr (KIND == 0) {
                    tv = (tv + lv[1][lane * W + j]) + (lv[2][lane * W + j] + lv[3][lane * W + j]);
                } else {
                    ti = li[0][lane * W + j];
#pragma unroll
                    for (int ww = 1; ww < NW; ++ww) combine<KIND == 1>(tv, ti, lv[ww][lane * W + j], li[ww][lane * W + j]);
                }
                if (K == 1) write_result<OP>(val, idx, o * inner + i, tv, ti, n);
                else {
                    pv[(o * K + k) * inner + i] = tv;
                    if (KIND != 0) pi[(o * K + k) * inner + i] = ti;
                }
            }
        }
    }
}

// Second pass for split columns.  A workgroup owns 16 adjacent output slots
// and its 256 threads form 16 groups of 16 lanes: group g combines chunks
// k = g, g + 16, g + 32, ... of its lane's slot in increasing k, and the 16
// group results are combined in group order through LDS.  Small slot tiles
// spread the pass over many workgroups; it is latency-bound otherwise.
template <int OP>
__global__ void __launch_bounds__(kBlock) reduce_cols_finalize_kernel(const float* __restrict__ pv,
                                                                       const int64_t* __restrict__ pi, int64_t outer,
                                                                       int64_t K, int64_t inner, int64_t n,
                                                                       float* __restrict__ val,
                                                                       int64_t* __restrict__ idx) {
    constexpr int KIND = kind_of(OP);
    constexpr int S = 16;          // slots per workgroup
    constexpr int G = kBlock / S;  // groups
    __shared__ float lv[G][S];
    __shared__ int64_t li[KIND != 0 ? G : 1][S];
    const int c = threadIdx.x & (S - 1), g = threadIdx.x / S;
    const int64_t total = outer * inner;
    for (int64_t s0 = (int64_t)blockIdx.x * S; s0 < total; s0 += (int64_t)gridDim.x * S) {
        const int64_t s = s0 + c;
        float rv = 0.f;
        int64_t ri = kEmpty;
        if (s < total) {
            const int64_t o = s / inner, i = s - o * inner;
            const float* pvs = pv + o * K * inner + i;
            if constexpr (KIND == 0) {
                int64_t k = g;
                for (; k + 3 * G < K; k += 4 * G) {
                    float b[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) b[u] = pvs[(k + u * G) * inner];
                    rv = ((rv + b[0]) + b[1]) + (b[2] + b[3]);
                }
                for (; k < K; k += G) rv += pvs[k * inner];
            } else {
                const int64_t* pis = pi + o * K * inner + i;
                int64_t k = g;
                for (; k + 3 * G < K; k += 4 * G) {
                    float bv[4];
                    int64_t bi[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) { bv[u] = pvs[(k + u * G) * inner]; bi[u] = pis[(k + u * G) * inner]; }
#pragma unroll
                    for (int u = 0; u < 4; ++u) combine<KIND == 1>(rv, ri, bv[u], bi[u]);
                }
                for (; k < K; k += G) combine<KIND == 1>(rv, ri, pvs[k * inner], pis[k * inner]);
            }
        }
        lv[g][c] = rv;
        if constexpr (KIND != 0) li[g][c] = ri;
        __syncthreads();
        if (g == 0 && s < total) {
            float tv = lv[0][c];
            int64_t ti = kEmpty;
            if constexpr (KIND == 0) {
#pragma unroll
                for (int gg = 1; gg < G; ++gg) tv += lv[gg][c];
            } else {
                ti = li[0][c];
#pragma unroll
                for (int gg = 1; gg < G; ++gg) combine<KIND == 1>(tv, ti, lv[gg][c], li[gg][c]);
            }
            write_result<OP>(val, idx, s, tv, ti, n);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------

// gx[o, k, i] (+)= g[o, i] (sum's closure; mean reuses it, :1709-1721).
template <bool ACC>
__global__ void __launch_bounds__(kBlock) reduce_bwd_sum_kernel(const float* __restrict__ g, float* __restrict__ gx,
                                                                 int64_t outer, int64_t n, int64_t inner) {
    const int64_t total = outer * n * inner;
    const int64_t ni = n * inner;
    for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < total; e += (int64_t)gridDim.x * kBlock) {
        const int64_t o = e / ni;
        const int64_t i = (e - o * ni) % inner;
        const float c = g[o * inner + i];
        gx[e] = ACC ? gx[e] + c : c;
    }
}

// Vector variant: inner % 4 == 0 (4 adjacent i share o, k) or inner == 1 and
// n % 4 == 0 (4 adjacent k share o and g).
template <bool ACC, bool INNER1>
__global__ void __launch_bounds__(kBlock) reduce_bwd_sum_vec_kernel(const float* __restrict__ g,
                                                                     float4* __restrict__ gx, int64_t outer, int64_t n,
                                                                     int64_t inner) {
    const int64_t total4 = outer * n * inner / 4;
    const int64_t ni = n * inner;
    for (int64_t q = (int64_t)blockIdx.x * kBlock + threadIdx.x; q < total4; q += (int64_t)gridDim.x * kBlock) {
        const int64_t e = q * 4;
        float4 c;
        if constexpr (INNER1) {
            const float s = g[e / n];
            c = make_float4(s, s, s, s);
        } else {
            const int64_t o = e / ni;
            const int64_t i = (e - o * ni) % inner;
            c = *reinterpret_cast<const float4*>(g + o * inner + i);
        }
        if (ACC) {
            float4 old = gx[q];
            c.x += old.x; c.y += old.y; c.z += old.z; c.w += old.w;
        }
        gx[q] = c;
    }
}

// gx[o, idx[o,i], i] += g[o, i] (max/min closures route the gradient to the
// first winning position).
__global__ void __launch_bounds__(kBlock) reduce_bwd_scatter_kernel(const float* __restrict__ g,
                                                                     const int64_t* __restrict__ idx,
                                                                     float* __restrict__ gx, int64_t outer, int64_t n,
                                                                     int64_t inner) {
    const int64_t total = outer * inner;
    for (int64_t s = (int64_t)blockIdx.x * kBlock + threadIdx.x; s < total; s += (int64_t)gridDim.x * kBlock) {
        const int64_t o = s / inner, i = s - o * inner;
        const int64_t k = idx[s];
        if (k >= 0 && k < n) gx[(o * n + k) * inner + i] += g[s];
    }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------

template <int OP>
int launch_reduce(const float* x, int64_t outer, int64_t n, int64_t inner, float* val, int64_t* idx) {
    constexpr int KIND = kind_of(OP);
    hipStream_t st = stream();
    const int64_t target_waves = (int64_t)num_cus() * 32;
    if (inner == 1) {
        int64_t K = 1;
        if (outer < target_waves) K = std::min<int64_t>((target_waves + outer - 1) / outer, (n + 4095) / 4096);
        K = std::max<int64_t>(K, 1);
        int64_t chunk = (n + K - 1) / K;
        chunk = (chunk + 255) / 256 * 256;
        K = std::max<int64_t>(1, (n + chunk - 1) / chunk);
        Workspace wv(K > 1 ? (size_t)(outer * K) * sizeof(float) : 0);
        Workspace wi(K > 1 && KIND != 0 ? (size_t)(outer * K) * sizeof(int64_t) : 0);
        if (K > 1 && (!wv.p || (KIND != 0 && !wi.p))) return set_error(WM_ERR_NOMEM, "wm_reduce: workspace");
        const bool vec = (n % 4 == 0) && aligned16(x);
        dim3 grid(grid_for(outer * K, kBlock / 64, 32));
        if (vec)
            launch_kernel((reduce_rows_kernel<OP, true>), grid, dim3(kBlock), 0, st, x, outer, n, chunk, K, val,
                               idx, wv.as<float>(), wi.as<int64_t>());
        else
            launch_kernel((reduce_rows_kernel<OP, false>), grid, dim3(kBlock), 0, st, x, outer, n, chunk, K, val,
                               idx, wv.as<float>(), wi.as<int64_t>());
        WM_TRY(check_launch("wm_reduce(rows)"));
        if (K > 1) {
            launch_kernel(reduce_rows_finalize_kernel<OP>, dim3(grid_for(outer, 1, 8)), dim3(kBlock), 0, st,
                               wv.as<float>(), wi.as<int64_t>(), outer, K, n, val, idx);
            WM_TRY(check_launch("wm_reduce(rows finalize)"));
        }
        return WM_OK;
    }
    const bool vec = (inner % 4 == 0) && aligned16(x);
    const int64_t tile = (int64_t)64 * (vec ? 4 : 1);
    const int64_t tiles = (inner + tile - 1) / tile;
    // ~4 workgroups per CU, each wave walking at least 32 positions of n.
    const int64_t target_blocks = (int64_t)num_cus() * 4;
    int64_t K = 1;
    if (outer * tiles < target_blocks)
        K = std::min<int64_t>((target_blocks + outer * tiles - 1) / (outer * tiles), (n + 127) / 128);
    K = std::max<int64_t>(std::min<int64_t>(K, 4096), 1);
    const int64_t chunk = (n + K - 1) / K;
    K = std::max<int64_t>(1, (n + chunk - 1) / chunk);
    Workspace wv(K > 1 ? (size_t)(outer * K * inner) * sizeof(float) : 0);
    Workspace wi(K > 1 && KIND != 0 ? (size_t)(outer * K * inner) * sizeof(int64_t) : 0);
    if (K > 1 && (!wv.p || (KIND != 0 && !wi.p))) return set_error(WM_ERR_NOMEM, "wm_reduce: workspace");
    dim3 grid(grid_for(outer * K * tiles, 1, 32));
#define WM_RC(V, I)                                                                                          \
    launch_kernel((reduce_cols_kernel<OP, V, I>), grid, dim3(kBlock), 0, st, x, outer, n, inner, chunk, K, val, \
                       idx, wv.as<float>(), wi.as<int64_t>())
    const bool narrow = n <= (int64_t)INT32_MAX;
    if (vec) { if (narrow) WM_RC(true, int32_t); else WM_RC(true, int64_t); }
    else { if (narrow) WM_RC(false, int32_t); else WM_RC(false, int64_t); }
#undef WM_RC
    WM_TRY(check_launch("wm_reduce(cols)"));
    if (K > 1) {
        launch_kernel(reduce_cols_finalize_kernel<OP>, dim3(grid_for(outer * inner, 16, 8)), dim3(kBlock), 0,
                           st, wv.as<float>(), wi.as<int64_t>(), outer, K, inner, n, val, idx);
        WM_TRY(check_launch("wm_reduce(cols finalize)"));
    }
    return WM_OK;
}

}  // namespace wm

using namespace wm;

extern "C" {

int wm_reduce(int op, const float* x, int64_t outer, int64_t n, int64_t inner, float* val, int64_t* idx) {
    if (outer < 0 || n < 0 || inner < 0) return set_error(WM_ERR_INVALID, "wm_reduce: negative extent");
    if (op < WM_R_SUM || op > WM_R_ARGMIN) return set_error(WM_ERR_INVALID, "wm_reduce: unknown op");
    if (outer == 0 || inner == 0) return WM_OK;
    if (n == 0) {
        // An empty sum is 0 and an empty mean 0/0 (the reference's loops do
        // nothing, then divide); max/min/arg* would read data[0] there.
        if (op == WM_R_SUM || op == WM_R_MEAN) {
            if (!val) return set_error(WM_ERR_INVALID, "wm_reduce: null output");
            WM_CHECK_INIT();
            return wm_fill(val, op == WM_R_SUM ? 0.f : __builtin_nanf(""), outer * inner);
        }
        return set_error(WM_ERR_INVALID, "wm_reduce: empty reduction axis");
    }
    if (!x) return set_error(WM_ERR_INVALID, "wm_reduce: null input");
    if ((op == WM_R_SUM || op == WM_R_MEAN) && !val) return set_error(WM_ERR_INVALID, "wm_reduce: null output");
    if (op >= WM_R_MAX && !val && !idx) return set_error(WM_ERR_INVALID, "wm_reduce: no output requested");
    WM_CHECK_INIT();
    switch (op) {
        case WM_R_SUM: return launch_reduce<WM_R_SUM>(x, outer, n, inner, val, idx);
        case WM_R_MEAN: return launch_reduce<WM_R_MEAN>(x, outer, n, inner, val, idx);
        case WM_R_MAX: return launch_reduce<WM_R_MAX>(x, outer, n, inner, val, idx);
        case WM_R_MIN: return launch_reduce<WM_R_MIN>(x, outer, n, inner, val, idx);
        case WM_R_ARGMAX: return launch_reduce<WM_R_ARGMAX>(x, outer, n, inner, val, idx);
        default: return launch_reduce<WM_R_ARGMIN>(x, outer, n, inner, val, idx);
    }
}

int wm_reduce_bwd(int op, const float* g, const int64_t* idx, int64_t outer, int64_t n, int64_t inner, float* gx,
                  int accumulate) {
    if (outer < 0 || n < 0 || inner < 0) return set_error(WM_ERR_INVALID, "wm_reduce_bwd: negative extent");
    const int64_t total = outer * n * inner;
    if (total == 0) return WM_OK;
    if (!g || !gx) return set_error(WM_ERR_INVALID, "wm_reduce_bwd: null pointer");
    WM_CHECK_INIT();
    hipStream_t st = stream();
    if (op == WM_R_SUM || op == WM_R_MEAN) {
        const bool vec4 = aligned16(gx) && ((inner % 4 == 0 && aligned16(g)) || (inner == 1 && n % 4 == 0));
        if (vec4) {
            dim3 grid(grid_for(total / 4, kBlock, 16));
            if (inner == 1) {
                if (accumulate) launch_kernel((reduce_bwd_sum_vec_kernel<true, true>), grid, dim3(kBlock), 0, st, g, reinterpret_cast<float4*>(gx), outer, n, inner);
                else launch_kernel((reduce_bwd_sum_vec_kernel<false, true>), grid, dim3(kBlock), 0, st, g, reinterpret_cast<float4*>(gx), outer, n, inner);
            } else {
                if (accumulate) launch_kernel((reduce_bwd_sum_vec_kernel<true, false>), grid, dim3(kBlock), 0, st, g, reinterpret_cast<float4*>(gx), outer, n, inner);
                else launch_kernel((reduce_bwd_sum_vec_kernel<false, false>), grid, dim3(kBlock), 0, st, g, reinterpret_cast<float4*>(gx), outer, n, inner);
            }
        } else {
            dim3 grid(grid_for(total, kBlock, 16));
            if (accumulate) launch_kernel((reduce_bwd_sum_kernel<true>), grid, dim3(kBlock), 0, st, g, gx, outer, n, inner);
            else launch_kernel((reduce_bwd_sum_kernel<false>), grid, dim3(kBlock), 0, st, g, gx, outer, n, inner);
        }
        return check_launch("wm_reduce_bwd(sum)");
    }
    if (op == WM_R_MAX || op == WM_R_MIN) {
        if (!idx) return set_error(WM_ERR_INVALID, "wm_reduce_bwd: max/min backward needs the saved indices");
        if (!accumulate) WM_TRY(wm_fill(gx, 0.f, total));
        launch_kernel(reduce_bwd_scatter_kernel, dim3(grid_for(outer * inner, kBlock, 8)), dim3(kBlock), 0, st, g,
                           idx, gx, outer, n, inner);
        return check_launch("wm_reduce_bwd(scatter)");
    }
    return set_error(WM_ERR_INVALID, "wm_reduce_bwd: argmax/argmin have no backward (the reference output is not tracked)");
}

}  // extern "C"
