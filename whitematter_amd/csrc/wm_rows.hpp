// Row machinery shared by the softmax kernels and the fused loss heads: a
// row held in registers (RowTile), workgroup max / sum reductions, and the
// choice of register tile for a row length.
#pragma once

#include "wm_common.hpp"

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

    // CACHED = false: non-temporal loads (data read once); true: ordinary
    // cached loads for rows that other workgroups read again (a broadcast
    // mask row, per-column parameters).
    template <bool CACHED = false>
    __device__ __forceinline__ void load(const float* row, int64_t cols, float fill) {
#pragma unroll
        for (int t = 0; t < ITEMS; ++t) {
            if constexpr (VEC) {
                int64_t c = col(t, 0);
                if (c < cols) {
                    float4 q = CACHED ? *reinterpret_cast<const float4*>(row + c) : ld_stream(row + c);
                    v[t][0] = q.x; v[t][1] = q.y; v[t][2] = q.z; v[t][3] = q.w;
                } else {
                    v[t][0] = v[t][1] = v[t][2] = v[t][3] = fill;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    int64_t c = col(t, e);
                    v[t][e] = c < cols ? (CACHED ? row[c] : ld_stream1(row + c)) : fill;
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

// Row max and sum of exponentials of a row held in a RowTile.
// Each thread first takes the max m_t of its own slots and the sum
// s_t = sum exp(x - m_t) (replacing each slot by exp(x - m_t) when KEEP_EXP),
// so the exponentials are computed while the rest of the workgroup's loads
// are still arriving; the row max M and the sum S = sum_t s_t exp(m_t - M)
// then take one barrier each (block_max_1 / block_sum_1 on separate LDS
// arrays).  Padding slots hold -inf and contribute exp(-inf) = 0.  A thread
// whose slots are all -inf uses 0 in place of m_t and contributes nothing.
// ct = exp(m_t - M) is the thread's rescale factor.
struct RowMaxSum {
    float m, s, ct;
};

template <int NT, int ITEMS, bool VEC, bool KEEP_EXP>
__device__ __forceinline__ RowMaxSum row_max_sum(RowTile<NT, ITEMS, VEC>& tile, float* lds_m, float* lds_s) {
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
            if (KEEP_EXP) tile.v[t][e] = ex;
        }
    RowMaxSum r;
    r.m = block_max_1<NT>(mt, lds_m);
    r.ct = mt == -INFINITY ? 0.f : exp_rr(mt - r.m);
    r.s = block_sum_1<NT>(st * r.ct, lds_s);
    return r;
}

// Pick the register tile: NT = 64 for rows up to 2048 columns, else 1024;
// ITEMS the smallest power of two (<= 8) covering the row.
struct TileChoice {
    int nt = 0, items = 0;  // nt == 0: long-row path
};

inline TileChoice choose_tile(int64_t cols) {
    TileChoice t;
    const int nts[2] = {64, 1024};
    for (int nt : nts) {
        for (int items = 1; items <= 8; items *= 2) {
            if (cols <= (int64_t)nt * 4 * items) { t.nt = nt; t.items = items; return t; }
        }
    }
    return t;
}

}  // namespace wm
