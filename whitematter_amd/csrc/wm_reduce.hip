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
#include <memory>
#include <mutex>
#include <unordered_map>

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


// Reduction kinds: 0 = sum/mean, 1 = max family, 2 = min family.
__host__ __device__ constexpr int kind_of(int op) {
    return (op == WM_R_SUM || op == WM_R_MEAN) ? 0 : ((op == WM_R_MAX || op == WM_R_ARGMAX) ? 1 : 2);
}

// Write the final result of one output slot.
template <int OP, class I>
__device__ __forceinline__ void write_result(float* val, int64_t* idx, int64_t slot, float v, I i, int64_t n) {
    if constexpr (OP == WM_R_SUM) { val[slot] = v; }
    else if constexpr (OP == WM_R_MEAN) { val[slot] = v / (float)n; }
    else if constexpr (OP == WM_R_MAX || OP == WM_R_MIN) {
        if (val) val[slot] = v;
        if (idx) idx[slot] = (int64_t)i;
    } else {
        if (val) val[slot] = (float)i;
        if (idx) idx[slot] = (int64_t)i;
    }
}

// ---------------------------------------------------------------------------
// A thread's scan over its piece of a slice
// ---------------------------------------------------------------------------
//
// scan_fast folds with the reference's strict compare alone, starting from
// v = -inf (max) / +inf (min) and an empty position.  That takes every
// element the empty-state rule of scan_push takes except a first non-NaN
// element equal to -inf (+inf): a piece whose state is still empty after
// the loop (all its elements NaN or that infinity) is re-scanned with
// scan_push (scan_fix below).  A NaN at position 0 of the slice wins the
// whole scan; the thread whose piece starts there loads that element before
// its loop and, after the loop, replaces its state with it if it is a NaN
// (scan_start).
template <bool MAXOP>
__device__ __forceinline__ float scan_init() { return MAXOP ? -__builtin_inff() : __builtin_inff(); }

template <bool MAXOP, class I>
__device__ __forceinline__ void scan_fast(float& v, I& i, float x, I k) {
    const bool take = strictly_better<MAXOP>(x, v);
    v = take ? x : v;
    i = take ? k : i;
}

template <bool MAXOP, class I>
__device__ __forceinline__ void scan_start(float& v, I& i, float x0) {
    if (__builtin_isnan(x0)) { v = x0; i = 0; }
}

// Positions [p0, p1) of one slice, element p at base[p * stride]; returns
// the state (value, position).  Out of line: it is the rare path.
template <class I>
struct ScanState {
    float v;
    I i;
};

template <bool MAXOP, class I>
__device__ __noinline__ ScanState<I> scan_fix(const float* base, int64_t stride, int64_t p0, int64_t p1) {
    float v = 0.f;
    I i = (I)kEmpty;
    for (int64_t p = p0; p < p1; ++p) scan_push<MAXOP>(v, i, base[p * stride], (I)p);
    return {v, i};
}

template <bool MAXOP, class I>
__device__ __forceinline__ void wave_combine_t(float& v, I& i) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        float v2 = __shfl_xor(v, off, 64);
        I i2 = __shfl_xor(i, off, 64);
        combine<MAXOP>(v, i, v2, i2);
    }
}

// The state (v, pos) of a chunk as an unsigned 64-bit key whose order is
// the scan's preference between chunks.  The high word is the value in an
// order-preserving encoding (inverted for min; -0 and +0 encode alike, as
// they compare equal).  The low word ranks lower positions higher on equal
// values: with 32-bit positions it holds 2^31 - 1 - pos above one bit for
// the sign of a zero, so the key decodes back to (value, pos) with no load;
// with 64-bit positions it holds ~k for chunk k (chunks are in position
// order), and the second pass reads the winning chunk's saved position.  A
// NaN at position 0 (which wins the whole scan) is the largest key, an empty
// state 0.
template <bool MAXOP>
__device__ __forceinline__ uint32_t order_word(float v) {
    const uint32_t b = __float_as_uint(v == 0.f ? 0.f : v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return MAXOP ? o : ~o;
}

template <bool MAXOP, class I>
__device__ __forceinline__ uint64_t chunk_key(float v, I pos, uint32_t k) {
    if (pos == (I)kEmpty) return 0ull;
    if (pos == 0 && __builtin_isnan(v)) return ~0ull;
    uint32_t lo;
    if constexpr (sizeof(I) == 4) {
        const uint32_t zsign = v == 0.f ? (__float_as_uint(v) >> 31) : 0u;
        lo = ((0x7FFFFFFFu - (uint32_t)pos) << 1) | zsign;
    } else {
        lo = ~k;
    }
    return ((uint64_t)order_word<MAXOP>(v) << 32) | lo;
}

// Decode a winning key: its position (32-bit positions) or chunk (64-bit)
// and, for 32-bit positions, its value.  The NaN-at-0 key's value is read
// from the input by the caller (its payload is not in the key).
template <bool MAXOP>
__device__ __forceinline__ float key_value(uint64_t key) {
    uint32_t o = (uint32_t)(key >> 32);
    if (!MAXOP) o = ~o;
    uint32_t b = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
    if (b == 0u && (key & 1u)) b = 0x80000000u;  // -0
    return __uint_as_float(b);
}

__device__ __forceinline__ int64_t key_pos32(uint64_t key) { return 0x7FFFFFFF - (int64_t)(((uint32_t)key >> 1) & 0x7FFFFFFFu); }
__device__ __forceinline__ int64_t key_chunk(uint64_t key) { return (int64_t)(uint32_t)~(uint32_t)key; }

// The result slot's (value, position) from its winning key; x_at(pos) reads
// the input element at pos of the slot.
template <bool MAXOP, class I, class XAt>
__device__ __forceinline__ void decode_winner(uint64_t key, const I* pi_slot, int64_t pi_stride, XAt x_at, float& v,
                                              I& pos) {
    if constexpr (sizeof(I) == 4) {
        if (key == ~0ull) {
            pos = 0;
            v = x_at(0);
        } else {
            pos = (I)key_pos32(key);
            v = key_value<MAXOP>(key);
        }
    } else {
        pos = pi_slot[key_chunk(key) * pi_stride];
        v = x_at(pos);
    }
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = __shfl_xor(k, off, 64);
        k = o > k ? o : k;
    }
    return k;
}

// ---------------------------------------------------------------------------
// inner == 1: rows
// ---------------------------------------------------------------------------

// A wave's scan of row positions [c0, c1) (c0 a multiple of 4 when VEC).
// Each lane keeps four 128-bit loads in flight and folds them in increasing
// position order; the lanes are combined with DPP / shuffles.  Every lane
// returns the wave's state.
template <int KIND, bool VEC, class I>
__device__ __forceinline__ void lane_scan_row(const float* __restrict__ xr, int64_t c0, int64_t c1, int lane,
                                              float& v_out, I& pos_out) {
    constexpr bool MX = KIND == 1;
    float v = KIND == 0 ? 0.f : scan_init<MX>();
    I pos = (I)kEmpty;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    // Position 0's element, loaded now and looked at after the loop, so no
    // lane waits for it before its first stream load.
    const bool has0 = KIND != 0 && c0 == 0 && lane == 0 && c1 > 0;
    const float x0 = has0 ? xr[0] : 0.f;
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
                    const I p = (I)(c + u * 256);
                    scan_fast<MX>(v, pos, a[u].x, p);
                    scan_fast<MX>(v, pos, a[u].y, (I)(p + 1));
                    scan_fast<MX>(v, pos, a[u].z, (I)(p + 2));
                    scan_fast<MX>(v, pos, a[u].w, (I)(p + 3));
                }
            }
        }
        for (; c < c1; c += 256) {
            float4 a0 = ld_stream(xr + c);
            if constexpr (KIND == 0) {
                s.x += a0.x; s.y += a0.y; s.z += a0.z; s.w += a0.w;
            } else {
                scan_fast<MX>(v, pos, a0.x, (I)c);
                scan_fast<MX>(v, pos, a0.y, (I)(c + 1));
                scan_fast<MX>(v, pos, a0.z, (I)(c + 2));
                scan_fast<MX>(v, pos, a0.w, (I)(c + 3));
            }
        }
        if constexpr (KIND != 0) {
            // this lane's positions: c0 + 4 lane + 256 j + {0..3}
            if (__builtin_expect(pos == (I)kEmpty, 0)) {
                float fv = 0.f;
                I fi = (I)kEmpty;
                for (int64_t q = c0 + lane * 4; q < c1; q += 256)
                    for (int64_t e = q; e < q + 4 && e < c1; ++e) scan_push<MX>(fv, fi, xr[e], (I)e);
                v = fv;
                pos = fi;
            }
        }
    } else {
        for (int64_t c = c0 + lane; c < c1; c += 64) {
            float a0 = ld_stream1(xr + c);
            if constexpr (KIND == 0) s.x += a0;
            else scan_fast<MX>(v, pos, a0, (I)c);
        }
        if constexpr (KIND != 0) {
            if (__builtin_expect(pos == (I)kEmpty, 0)) {
                float fv = 0.f;
                I fi = (I)kEmpty;
                for (int64_t c = c0 + lane; c < c1; c += 64) scan_push<MX>(fv, fi, xr[c], (I)c);
                v = fv;
                pos = fi;
            }
        }
    }
    if constexpr (KIND != 0) {
        if (has0) scan_start<MX>(v, pos, x0);
    }
    if constexpr (KIND == 0) v = (s.x + s.y) + (s.z + s.w);
    v_out = v;
    pos_out = pos;
}

// The wave's state: its sum (every lane), or for the max family with 64-bit
// positions its (value, position) through pairwise combines (every lane).
template <int KIND, bool VEC, class I>
__device__ __forceinline__ void wave_scan_row(const float* __restrict__ xr, int64_t c0, int64_t c1, int lane,
                                              float& v, I& pos) {
    lane_scan_row<KIND, VEC, I>(xr, c0, c1, lane, v, pos);
    if constexpr (KIND == 0) v = wave_sum(v);
    else wave_combine_t<KIND == 1>(v, pos);
}

// The max family with 32-bit positions: the wave's state as its chunk key
// (every lane).  The key's order is combine's preference, so the fold is an
// unsigned maximum: no branches on NaN or emptiness between lanes.
template <int KIND, bool VEC, class I>
__device__ __forceinline__ uint64_t wave_scan_row_key(const float* __restrict__ xr, int64_t c0, int64_t c1,
                                                      int lane) {
    static_assert(KIND != 0 && sizeof(I) == 4, "keys hold 32-bit positions");
    float v;
    I pos;
    lane_scan_row<KIND, VEC, I>(xr, c0, c1, lane, v, pos);
    return wave_max_u64(chunk_key<KIND == 1>(v, pos, 0u));
}

// Two shapes of launch, chosen by K (uniform):
//   K == 1  one wave per row: the wave's state is the row's result;
//   K  > 1  one workgroup per (row, chunk of `chunk` positions): the four
//           waves take consecutive quarters of the chunk and their states
//           are combined through LDS (in wave order, or as chunk keys by an
//           unsigned maximum); the workgroup's state is the chunk's partial,
//           which reduce_rows_finalize_kernel combines.
template <int OP, bool VEC, class I>
__global__ void __launch_bounds__(kBlock) reduce_rows_kernel(const float* __restrict__ x, int64_t rows, int64_t n,
                                                              int64_t chunk, int64_t K, float* __restrict__ val,
                                                              int64_t* __restrict__ idx, float* __restrict__ pv,
                                                              uint64_t* __restrict__ pk, I* __restrict__ pi) {
    constexpr int KIND = kind_of(OP);
    constexpr bool MX = KIND == 1;
    constexpr bool KEYED = KIND != 0 && sizeof(I) == 4;  // states fold as chunk keys
    constexpr int NW = kBlock / 64;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (K == 1) {
        const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) >> 6;
        const int64_t nwaves = ((int64_t)gridDim.x * kBlock) >> 6;
        for (int64_t r = wave; r < rows; r += nwaves) {
            const float* xr = x + r * n;
            float v;
            I pos;
            if constexpr (KEYED) {
                // n >= 1, so the row's key is never the empty state's 0.
                const uint64_t key = wave_scan_row_key<KIND, VEC, I>(xr, 0, n, lane);
                if (lane == 0) {
                    decode_winner<MX>(key, (const I*)nullptr, 0, [&](int64_t p) { return xr[p]; }, v, pos);
                    write_result<OP>(val, idx, r, v, pos, n);
                }
            } else {
                wave_scan_row<KIND, VEC, I>(xr, 0, n, lane, v, pos);
                if (lane == 0) write_result<OP>(val, idx, r, v, pos, n);
            }
        }
        return;
    }
    __shared__ float lv[NW];
    __shared__ I li[NW];
    __shared__ uint64_t lk[NW];
    for (int64_t item = blockIdx.x; item < rows * K; item += gridDim.x) {
        const int64_t r = item / K, k = item - r * K;
        const int64_t c0 = k * chunk, c1 = min(n, c0 + chunk);
        const int64_t q = chunk / NW;  // a multiple of 256
        const int64_t a0 = min(c1, c0 + w * q), a1 = min(c1, a0 + q);
        if constexpr (KEYED) {
            const uint64_t key = wave_scan_row_key<KIND, VEC, I>(x + r * n, a0, a1, lane);
            if (lane == 0) lk[w] = key;
            __syncthreads();
            if (threadIdx.x == 0) {
                uint64_t best = lk[0];
#pragma unroll
                for (int ww = 1; ww < NW; ++ww) best = lk[ww] > best ? lk[ww] : best;
                pk[r * K + k] = best;
            }
            __syncthreads();  // LDS is reused by the next item
            continue;
        }
        float v;
        I pos;
        wave_scan_row<KIND, VEC, I>(x + r * n, a0, a1, lane, v, pos);
        if (lane == 0) { lv[w] = v; li[w] = pos; }
        __syncthreads();
        if (threadIdx.x == 0) {
            float tv = lv[0];
            I ti = li[0];
            if constexpr (KIND == 0) {
                tv = (lv[0] + lv[1]) + (lv[2] + lv[3]);
            } else {
#pragma unroll
                for (int ww = 1; ww < NW; ++ww) combine<MX>(tv, ti, lv[ww], li[ww]);
            }
            if constexpr (KIND == 0) {
                pv[r * K + k] = tv;
            } else {
                pk[r * K + k] = chunk_key<MX>(tv, ti, (uint32_t)k);
                if constexpr (sizeof(I) == 8) pi[r * K + k] = ti;
            }
        }
        __syncthreads();  // LDS is reused by the next item
    }
}

// Second pass for split rows: one workgroup per row; thread t folds chunks
// t, t + 256, ... in increasing order (sums) or takes the largest key (the
// max family), then a fixed block tree.
template <int OP, class I>
__global__ void __launch_bounds__(kBlock) reduce_rows_finalize_kernel(const float* __restrict__ x,
                                                                       const float* __restrict__ pv,
                                                                       const uint64_t* __restrict__ pk,
                                                                       const I* __restrict__ pi, int64_t rows,
                                                                       int64_t K, int64_t n, float* __restrict__ val,
                                                                       int64_t* __restrict__ idx) {
    constexpr int KIND = kind_of(OP);
    constexpr int NW = kBlock / 64;
    __shared__ float lv[NW];
    __shared__ uint64_t lk[NW];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        if constexpr (KIND == 0) {
            float a[4] = {0.f, 0.f, 0.f, 0.f};
            int64_t kk = threadIdx.x;
            for (; kk + 3 * kBlock < K; kk += 4 * kBlock) {
#pragma unroll
                for (int j = 0; j < 4; ++j) a[j] += pv[r * K + kk + j * kBlock];
            }
            for (int j = 0; kk < K; kk += kBlock, ++j) a[j & 3] += pv[r * K + kk];
            const float t = block_sum<kBlock>((a[0] + a[1]) + (a[2] + a[3]), lv);
            if (threadIdx.x == 0) write_result<OP>(val, idx, r, t, (I)0, n);
        } else {
            uint64_t best = 0;
            for (int64_t kk = threadIdx.x; kk < K; kk += kBlock) {
                const uint64_t c = pk[r * K + kk];
                best = c > best ? c : best;
            }
            best = wave_max_u64(best);
            if (lane == 0) lk[w] = best;
            __syncthreads();
            if (threadIdx.x == 0) {
#pragma unroll
                for (int ww = 1; ww < NW; ++ww) best = lk[ww] > best ? lk[ww] : best;
                float v;
                I pos;
                decode_winner<KIND == 1>(best, pi + r * K, 1, [&](int64_t p) { return x[r * n + p]; }, v, pos);
                write_result<OP>(val, idx, r, v, pos, n);
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
// [k0, k1) of n, each walking its quarter in increasing order with U loads
// in flight; the four wave states are combined through LDS (sums in wave
// order; the max family with 32-bit positions as chunk keys by an unsigned
// maximum, with 64-bit positions by pairwise combines in wave order).
// Items are (o, chunk, inner tile) triples, tile fastest; every thread of a
// workgroup walks the same items, so the barriers are uniform.
//
// With K > 1 chunks the workgroup's state is a partial per column (a sum, or
// the chunk key plus, for 64-bit positions, the position) that
// reduce_cols_finalize_kernel combines.
template <int OP, bool VEC, class I>
__global__ void __launch_bounds__(kBlock) reduce_cols_kernel(const float* __restrict__ x, int64_t outer, int64_t n,
                                                              int64_t inner, int64_t chunk, int64_t K,
                                                              float* __restrict__ val, int64_t* __restrict__ idx,
                                                              float* __restrict__ pv, uint64_t* __restrict__ pk,
                                                              I* __restrict__ pi) {
    constexpr int KIND = kind_of(OP);
    constexpr bool MX = KIND == 1;
    constexpr int W = VEC ? 4 : 1;
    constexpr int NW = kBlock / 64;
    constexpr int U = VEC ? 8 : 4;
    constexpr bool KEYED = KIND != 0 && sizeof(I) == 4;  // states fold as chunk keys
    __shared__ float lv[KEYED ? 1 : NW][KEYED ? 1 : 64 * W];
    __shared__ I li[KIND != 0 && !KEYED ? NW : 1][KIND != 0 && !KEYED ? 64 * W : 1];
    __shared__ uint64_t lk[KEYED ? NW : 1][KEYED ? W : 1][64];
    // w is the same for every lane of a wave: readfirstlane lets the compiler
    // keep each wave's row range, its loop and the scanned positions in
    // scalar registers.
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tile_elems = (int64_t)64 * W;
    const int64_t tiles = (inner + tile_elems - 1) / tile_elems;
    const int64_t items = outer * K * tiles;

    // The four wave states (v, pos) -> wave 0 lanes hold the workgroup's
    // state of their W columns (sums, and the max family with 64-bit
    // positions).
    auto lds_combine = [&](float (&v)[W], I (&pos)[W]) {
        if constexpr (!KEYED) {  // else lds_keys below
            __syncthreads();  // earlier LDS reads are done
#pragma unroll
            for (int j = 0; j < W; ++j) {
                lv[w][lane * W + j] = v[j];
                if constexpr (KIND != 0) li[w][lane * W + j] = pos[j];
            }
            __syncthreads();
            if (w == 0) {
#pragma unroll
                for (int j = 0; j < W; ++j) {
                    if constexpr (KIND == 0) {
                        v[j] = (lv[0][lane * W + j] + lv[1][lane * W + j]) + (lv[2][lane * W + j] + lv[3][lane * W + j]);
                    } else {
                        v[j] = lv[0][lane * W + j];
                        pos[j] = li[0][lane * W + j];
#pragma unroll
                        for (int ww = 1; ww < NW; ++ww) combine<MX>(v[j], pos[j], lv[ww][lane * W + j], li[ww][lane * W + j]);
                    }
                }
            }
        }
    };

    // The max family with 32-bit positions: the four wave states as chunk
    // keys, folded by an unsigned maximum (the keys' order is combine's
    // preference) -> wave 0 lanes hold the workgroup's keys of their W
    // columns.  Branch-free, where combine's NaN and emptiness tests cost
    // every workgroup's last wave a few hundred instructions at the end of
    // its item.
    auto lds_keys = [&](const float (&v)[W], const I (&pos)[W], uint64_t (&key)[W]) {
        __syncthreads();  // earlier LDS reads are done
#pragma unroll
        for (int j = 0; j < W; ++j) lk[w][j][lane] = chunk_key<MX>(v[j], pos[j], 0u);
        __syncthreads();
        if (w == 0) {
#pragma unroll
            for (int j = 0; j < W; ++j) {
                uint64_t b = lk[0][j][lane];
#pragma unroll
                for (int ww = 1; ww < NW; ++ww) b = lk[ww][j][lane] > b ? lk[ww][j][lane] : b;
                key[j] = b;
            }
        }
    };

    for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
        const int64_t t = item % tiles;
        const int64_t ok = item / tiles;
        const int64_t k = ok % K;
        const int64_t o = ok / K;
        const int64_t i0 = t * tile_elems + (int64_t)lane * W;
        const bool live = i0 < inner;
        const int64_t k0 = k * chunk, k1 = min(n, k0 + chunk);
        const int64_t q = (k1 - k0 + NW - 1) / NW;
        const int64_t r0 = min(k1, k0 + w * q), r1 = min(k1, r0 + q);
        const float* xp = x + o * n * inner + i0;
        float v[W];
        I pos[W];
#pragma unroll
        for (int j = 0; j < W; ++j) { v[j] = KIND == 0 ? 0.f : scan_init<MX>(); pos[j] = (I)kEmpty; }
        if (live) {
            // Row 0's elements, loaded now and looked at after the loop.
            const bool has0 = KIND != 0 && r0 == 0 && r1 > 0;
            float x0[W];
#pragma unroll
            for (int j = 0; j < W; ++j) x0[j] = has0 ? xp[j] : 0.f;
            int64_t p = r0;
            if constexpr (VEC && KIND != 0) {
                // The max family: the next U rows' loads are issued before
                // this batch is folded, so U loads stay in flight while the
                // wave compares (three vector instructions per element,
                // against the sum's one, otherwise leave the wave with no
                // load outstanding between batches).  On MI355X at
                // [16384, 4096] this took the first pass from 43.8 to
                // 41.2-42.5 us (the sum's is 40-41 us); a strict per-row
                // rolling order, 12 rows in flight, or 3, 5 or 6 workgroups
                // per CU were each 0.5-4 us slower.
                if (r1 - r0 >= U) {
                    float4 a[U];
#pragma unroll
                    for (int u = 0; u < U; ++u) a[u] = ld_stream(xp + (r0 + u) * inner);
                    for (; p + 2 * U <= r1; p += U) {
#pragma unroll
                        for (int u = 0; u < U; ++u) {
                            const float4 c = a[u];
                            a[u] = ld_stream(xp + (p + U + u) * inner);
                            scan_fast<MX>(v[0], pos[0], c.x, (I)(p + u));
                            scan_fast<MX>(v[1], pos[1], c.y, (I)(p + u));
                            scan_fast<MX>(v[2], pos[2], c.z, (I)(p + u));
                            scan_fast<MX>(v[3], pos[3], c.w, (I)(p + u));
                        }
                    }
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        scan_fast<MX>(v[0], pos[0], a[u].x, (I)(p + u));
                        scan_fast<MX>(v[1], pos[1], a[u].y, (I)(p + u));
                        scan_fast<MX>(v[2], pos[2], a[u].z, (I)(p + u));
                        scan_fast<MX>(v[3], pos[3], a[u].w, (I)(p + u));
                    }
                    p += U;
                }
            }
            for (; p + (U - 1) < r1; p += U) {
                float a[U][W];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    if constexpr (VEC) {
                        float4 qv = ld_stream(xp + (p + u) * inner);
                        a[u][0] = qv.x; a[u][1] = qv.y; a[u][2] = qv.z; a[u][3] = qv.w;
                    } else {
                        a[u][0] = ld_stream1(xp + (p + u) * inner);
                    }
                }
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int j = 0; j < W; ++j) {
                        if constexpr (KIND == 0) v[j] += a[u][j];
                        else scan_fast<MX>(v[j], pos[j], a[u][j], (I)(p + u));
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
                    else scan_fast<MX>(v[j], pos[j], a[j], (I)p);
                }
            }
            if constexpr (KIND != 0) {
#pragma unroll
                for (int j = 0; j < W; ++j) {
                    if (__builtin_expect(pos[j] == (I)kEmpty && r0 < r1, 0)) {
                        const ScanState<I> f = scan_fix<MX, I>(xp + j, inner, r0, r1);
                        v[j] = f.v;
                        pos[j] = f.i;
                    }
                    if (has0) scan_start<MX>(v[j], pos[j], x0[j]);
                }
            }
        }
        if constexpr (KEYED) {
            uint64_t key[W];
            lds_keys(v, pos, key);
            if (w == 0) {
#pragma unroll
                for (int j = 0; j < W; ++j) {
                    if (i0 + j >= inner) continue;
                    if (K == 1) {
                        // n >= 1, so the column's key is never the empty state's 0.
                        float rv;
                        I rp;
                        decode_winner<MX>(key[j], (const I*)nullptr, 0,
                                          [&](int64_t pp) { return xp[pp * inner + j]; }, rv, rp);
                        write_result<OP>(val, idx, o * inner + i0 + j, rv, rp, n);
                    } else {
                        pk[(o * K + k) * inner + i0 + j] = key[j];
                    }
                }
            }
            continue;
        }
        lds_combine(v, pos);
        if (K == 1) {
            if (w == 0) {
#pragma unroll
                for (int j = 0; j < W; ++j)
                    if (i0 + j < inner) write_result<OP>(val, idx, o * inner + i0 + j, v[j], pos[j], n);
            }
            continue;
        }
        if (w == 0) {
#pragma unroll
            for (int j = 0; j < W; ++j) {
                if (i0 + j < inner) {
                    const int64_t at = (o * K + k) * inner + i0 + j;
                    if constexpr (KIND == 0) {
                        pv[at] = v[j];
                    } else {
                        pk[at] = chunk_key<MX>(v[j], pos[j], (uint32_t)k);
                        if constexpr (sizeof(I) == 8) pi[at] = pos[j];
                    }
                }
            }
        }
    }
}

// Second pass for split columns.  A workgroup owns 16 adjacent output slots
// and its 256 threads form 16 groups of 16 lanes: group g folds chunks
// k = g, g + 16, g + 32, ... of its lane's slot (all its loads issued
// first) -- sums in increasing k, the max family by the largest key -- and
// the 16 group results are combined in group order through LDS.  Small
// slot tiles spread the pass over many workgroups, so each thread waits for
// one round of loads.
template <int OP, class I>
__global__ void __launch_bounds__(kBlock) reduce_cols_finalize_kernel(const float* __restrict__ x,
                                                                       const float* __restrict__ pv,
                                                                       const uint64_t* __restrict__ pk,
                                                                       const I* __restrict__ pi, int64_t outer,
                                                                       int64_t K, int64_t inner, int64_t n,
                                                                       float* __restrict__ val,
                                                                       int64_t* __restrict__ idx) {
    constexpr int KIND = kind_of(OP);
    constexpr int S = 16;          // slots per workgroup
    constexpr int G = kBlock / S;  // groups
    __shared__ float lv[KIND == 0 ? G : 1][S];
    __shared__ uint64_t lk[KIND != 0 ? G : 1][S];
    const int c = threadIdx.x & (S - 1), g = threadIdx.x / S;
    const int64_t total = outer * inner;
    for (int64_t s0 = (int64_t)blockIdx.x * S; s0 < total; s0 += (int64_t)gridDim.x * S) {
        const int64_t s = s0 + c;
        const int64_t o = s / inner, i = s - o * inner;
        if constexpr (KIND == 0) {
            float rv = 0.f;
            if (s < total) {
                const float* pvs = pv + o * K * inner + i;
                int64_t k = g;
                for (; k + 3 * G < K; k += 4 * G) {
                    float bv[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) bv[u] = pvs[(k + u * G) * inner];
                    rv = ((rv + bv[0]) + bv[1]) + (bv[2] + bv[3]);
                }
                for (; k < K; k += G) rv += pvs[k * inner];
            }
            lv[g][c] = rv;
            __syncthreads();
            if (g == 0 && s < total) {
                float tv = lv[0][c];
#pragma unroll
                for (int gg = 1; gg < G; ++gg) tv += lv[gg][c];
                write_result<OP>(val, idx, s, tv, (I)0, n);
            }
        } else {
            uint64_t best = 0;
            if (s < total) {
                const uint64_t* pks = pk + o * K * inner + i;
                int64_t k = g;
                for (; k + 3 * G < K; k += 4 * G) {
                    uint64_t b[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) b[u] = pks[(k + u * G) * inner];
#pragma unroll
                    for (int u = 0; u < 4; ++u) best = b[u] > best ? b[u] : best;
                }
                for (; k < K; k += G) {
                    const uint64_t b = pks[k * inner];
                    best = b > best ? b : best;
                }
            }
            lk[g][c] = best;
            __syncthreads();
            if (g == 0 && s < total) {
#pragma unroll
                for (int gg = 1; gg < G; ++gg) best = lk[gg][c] > best ? lk[gg][c] : best;
                float v;
                I pos;
                decode_winner<KIND == 1>(best, pi + o * K * inner + i, inner,
                                         [&](int64_t p) { return x[(o * n + p) * inner + i]; }, v, pos);
                write_result<OP>(val, idx, s, v, pos, n);
            }
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
// n % 4 == 0 (4 adjacent k share o and g).  kSlotsBwd float4s per thread,
// their values gathered before any store, on a grid that covers the tensor,
// with streaming stores: 74.7 % of the HBM peak for a [32768, 4096] mean
// backward against 63 % with one float4 per thread (each thread then waits
// on its g load before its only store).  IDX32: every index fits 32 bits,
// so the position arithmetic divides in 32 bits (a 64-bit division is a
// long instruction sequence).
constexpr int kSlotsBwd = 4;
template <bool ACC, bool INNER1, bool IDX32>
__global__ void __launch_bounds__(kBlock) reduce_bwd_sum_vec_kernel(const float* __restrict__ g,
                                                                     float* __restrict__ gx, int64_t outer, int64_t n,
                                                                     int64_t inner) {
    const int64_t total4 = outer * n * inner / 4;
    const int64_t ni = n * inner;
    const int64_t step = (int64_t)gridDim.x * kBlock * kSlotsBwd;
    for (int64_t q0 = (int64_t)blockIdx.x * kBlock * kSlotsBwd + threadIdx.x; q0 < total4; q0 += step) {
        float4 cc[kSlotsBwd];
#pragma unroll
        for (int u = 0; u < kSlotsBwd; ++u) {
            const int64_t q = q0 + (int64_t)u * kBlock;
            const int64_t e = q * 4;
            if (q >= total4) continue;
            float4 c;
            if constexpr (INNER1) {
                const float s = g[IDX32 ? (int64_t)((uint32_t)e / (uint32_t)n) : e / n];
                c = make_float4(s, s, s, s);
            } else {
                int64_t o, i;
                if constexpr (IDX32) {
                    const uint32_t o32 = (uint32_t)e / (uint32_t)ni;
                    o = o32;
                    i = ((uint32_t)e - o32 * (uint32_t)ni) % (uint32_t)inner;
                } else {
                    o = e / ni;
                    i = (e - o * ni) % inner;
                }
                c = *reinterpret_cast<const float4*>(g + o * inner + i);
            }
            if (ACC) {
                const float4 old = ld_stream(gx + e);
                c.x += old.x; c.y += old.y; c.z += old.z; c.w += old.w;
            }
            cc[u] = c;
        }
#pragma unroll
        for (int u = 0; u < kSlotsBwd; ++u) {
            const int64_t q = q0 + (int64_t)u * kBlock;
            if (q >= total4) continue;
            st_stream(gx + q * 4, cc[u]);
        }
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

// Where a launch's chunk partials live: blocks from the library's pool
// (base == null), or a fixed region of `cap` bytes (the allocation-free
// entry point's scratch array).
struct PartialArena {
    char* base = nullptr;
    size_t cap = 0;
};

// The partial arrays of one launch: floats for sums, order keys (+ 64-bit
// positions when positions are wide) for the max family.
struct Partials {
    Workspace wv, wk, wi;
    float* pv = nullptr;
    uint64_t* pk = nullptr;
    void* pi = nullptr;
    Partials(size_t fbytes, size_t kbytes, size_t ibytes, bool pool)
        : wv(pool ? fbytes : 0), wk(pool ? kbytes : 0), wi(pool ? ibytes : 0) {}
};

template <int KIND, class I>
int take_partials(size_t parts, const PartialArena& arena, std::unique_ptr<Partials>& P) {
    const size_t fb = KIND == 0 ? parts * sizeof(float) : 0;
    const size_t kb = KIND != 0 ? parts * sizeof(uint64_t) : 0;
    const size_t ib = KIND != 0 && sizeof(I) == 8 ? parts * sizeof(I) : 0;
    P.reset(new Partials(fb, kb, ib, arena.base == nullptr));
    if (parts == 0) return WM_OK;
    if (!arena.base) {
        if ((fb && !P->wv.p) || (kb && !P->wk.p) || (ib && !P->wi.p))
            return set_error(WM_ERR_NOMEM, "wm_reduce: workspace");
        P->pv = P->wv.as<float>();
        P->pk = P->wk.as<uint64_t>();
        P->pi = P->wi.p;
        return WM_OK;
    }
    const size_t first = (fb + kb + 255) / 256 * 256;
    if (first + ib > arena.cap)
        return set_error(WM_ERR_UNSUPPORTED, "wm_reduce_noalloc: this reduction needs " + std::to_string(first + ib) +
                                                 " bytes of partials; the scratch array holds " +
                                                 std::to_string(arena.cap) + " (use wm_reduce)");
    P->pv = reinterpret_cast<float*>(arena.base);
    P->pk = reinterpret_cast<uint64_t*>(arena.base);
    P->pi = ib ? arena.base + first : nullptr;
    return WM_OK;
}

template <int OP, class I>
int launch_rows(const float* x, int64_t rows, int64_t n, float* val, int64_t* idx, const PartialArena& arena) {
    constexpr int KIND = kind_of(OP);
    hipStream_t st = stream();
    const bool vec = (n % 4 == 0) && aligned16(x);
    // Enough rows: one wave per row.  Few long rows (a full reduction is one
    // row): each row in chunks of whole workgroups, ~8 workgroups per CU,
    // then a second pass over the chunk partials.
    const int64_t target_waves = (int64_t)num_cus() * 32;
    int64_t K = 1, chunk = n;
    if (rows < target_waves) {
        const int64_t target_wgs = (int64_t)num_cus() * 8;
        K = std::min<int64_t>((target_wgs + rows - 1) / rows, (n + 4095) / 4096);
        K = std::max<int64_t>(K, 1);
        if (K > 1) {
            chunk = (n + K - 1) / K;
            chunk = (chunk + 1023) / 1024 * 1024;  // four wave quarters of whole 256-float strides
            K = std::max<int64_t>(1, (n + chunk - 1) / chunk);
        }
    }
    if (K == 1) {
        dim3 grid(grid_for(rows, kBlock / 64, 32));
        if (vec) launch_kernel((reduce_rows_kernel<OP, true, I>), grid, dim3(kBlock), 0, st, x, rows, n, n, (int64_t)1,
                               val, idx, (float*)nullptr, (uint64_t*)nullptr, (I*)nullptr);
        else launch_kernel((reduce_rows_kernel<OP, false, I>), grid, dim3(kBlock), 0, st, x, rows, n, n, (int64_t)1,
                           val, idx, (float*)nullptr, (uint64_t*)nullptr, (I*)nullptr);
        return check_launch("wm_reduce(rows)");
    }
    std::unique_ptr<Partials> P;
    WM_TRY((take_partials<KIND, I>((size_t)(rows * K), arena, P)));
    I* pi = static_cast<I*>(P->pi);
    dim3 grid(grid_for(rows * K, 1, 8));
    if (vec) launch_kernel((reduce_rows_kernel<OP, true, I>), grid, dim3(kBlock), 0, st, x, rows, n, chunk, K, val,
                           idx, P->pv, P->pk, pi);
    else launch_kernel((reduce_rows_kernel<OP, false, I>), grid, dim3(kBlock), 0, st, x, rows, n, chunk, K, val, idx,
                       P->pv, P->pk, pi);
    WM_TRY(check_launch("wm_reduce(rows)"));
    launch_kernel((reduce_rows_finalize_kernel<OP, I>), dim3(grid_for(rows, 1, 8)), dim3(kBlock), 0, st, x, P->pv,
                  P->pk, pi, rows, K, n, val, idx);
    return check_launch("wm_reduce(rows finalize)");
}

template <int OP, class I>
int launch_cols(const float* x, int64_t outer, int64_t n, int64_t inner, float* val, int64_t* idx,
                const PartialArena& arena) {
    constexpr int KIND = kind_of(OP);
    hipStream_t st = stream();
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
    std::unique_ptr<Partials> P;
    WM_TRY((take_partials<KIND, I>(K > 1 ? (size_t)(outer * K * inner) : 0, arena, P)));
    I* pi = static_cast<I*>(P->pi);
    dim3 grid(grid_for(outer * K * tiles, 1, 32));
    if (vec) launch_kernel((reduce_cols_kernel<OP, true, I>), grid, dim3(kBlock), 0, st, x, outer, n, inner, chunk, K,
                           val, idx, P->pv, P->pk, pi);
    else launch_kernel((reduce_cols_kernel<OP, false, I>), grid, dim3(kBlock), 0, st, x, outer, n, inner, chunk, K,
                       val, idx, P->pv, P->pk, pi);
    WM_TRY(check_launch("wm_reduce(cols)"));
    if (K > 1) {
        launch_kernel((reduce_cols_finalize_kernel<OP, I>), dim3(grid_for(outer * inner, 16, 8)), dim3(kBlock), 0, st,
                      x, P->pv, P->pk, pi, outer, K, inner, n, val, idx);
        WM_TRY(check_launch("wm_reduce(cols finalize)"));
    }
    return WM_OK;
}

// Positions are tracked as 32-bit integers whenever the reduced extent fits
// (half the compare-and-select work and partial bytes of 64-bit ones).
template <int OP>
int launch_reduce(const float* x, int64_t outer, int64_t n, int64_t inner, float* val, int64_t* idx,
                  const PartialArena& arena) {
    const bool narrow = n <= (int64_t)INT32_MAX;
    if (inner == 1)
        return narrow ? launch_rows<OP, int32_t>(x, outer, n, val, idx, arena)
                      : launch_rows<OP, int64_t>(x, outer, n, val, idx, arena);
    return narrow ? launch_cols<OP, int32_t>(x, outer, n, inner, val, idx, arena)
                  : launch_cols<OP, int64_t>(x, outer, n, inner, val, idx, arena);
}

// The allocation-free entry point's partials: a file-scope device array (no
// counterpart in the reference), one copy per GPU the library runs on, held
// until the process ends.  Host code uses the address hipGetSymbolAddress
// gives for the current device, never the array's name.
constexpr size_t kScratchBytes = size_t(8) << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::unordered_map<int, void*> g_scratch_at;  // device -> its copy of scratch

// The address of `scratch` on the library's device, looked up once per device
// with that device current.
int scratch_address(void** out) {
    const int dev = device();
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch_at.find(dev);
    if (it != g_scratch_at.end()) {
        *out = it->second;
        return WM_OK;
    }
    int prev = -1;
    hipError_t e = hipGetDevice(&prev);
    if (e == hipSuccess && prev != dev) e = hipSetDevice(dev);
    void* p = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (prev >= 0 && prev != dev) (void)hipSetDevice(prev);
    if (e != hipSuccess || !p)
        return set_error(WM_ERR_HIP, std::string("wm_reduce_noalloc: scratch address: ") + hipGetErrorString(e));
    g_scratch_at[dev] = p;
    *out = p;
    return WM_OK;
}

}  // namespace wm

using namespace wm;

extern "C" {

static int reduce_entry(const char* name, int op, const float* x, int64_t outer, int64_t n, int64_t inner,
                        float* val, int64_t* idx, bool noalloc) {
    const std::string nm(name);
    if (outer < 0 || n < 0 || inner < 0) return set_error(WM_ERR_INVALID, nm + ": negative extent");
    if (op < WM_R_SUM || op > WM_R_ARGMIN) return set_error(WM_ERR_INVALID, nm + ": unknown op");
    if (outer == 0 || inner == 0) return WM_OK;
    if (n == 0) {
        // An empty sum is 0 and an empty mean 0/0 (the reference's loops do
        // nothing, then divide); max/min/arg* would read data[0] there.
        if (op == WM_R_SUM || op == WM_R_MEAN) {
            if (!val) return set_error(WM_ERR_INVALID, nm + ": null output");
            WM_CHECK_INIT();
            return wm_fill(val, op == WM_R_SUM ? 0.f : __builtin_nanf(""), outer * inner);
        }
        return set_error(WM_ERR_INVALID, nm + ": empty reduction axis");
    }
    if (!x) return set_error(WM_ERR_INVALID, nm + ": null input");
    if ((op == WM_R_SUM || op == WM_R_MEAN) && !val) return set_error(WM_ERR_INVALID, nm + ": null output");
    if (op >= WM_R_MAX && !val && !idx) return set_error(WM_ERR_INVALID, nm + ": no output requested");
    WM_CHECK_INIT();
    PartialArena arena;
    if (noalloc) {
        void* p = nullptr;
        WM_TRY(scratch_address(&p));
        arena.base = static_cast<char*>(p);
        arena.cap = kScratchBytes;
    }
    switch (op) {
        case WM_R_SUM: return launch_reduce<WM_R_SUM>(x, outer, n, inner, val, idx, arena);
        case WM_R_MEAN: return launch_reduce<WM_R_MEAN>(x, outer, n, inner, val, idx, arena);
        case WM_R_MAX: return launch_reduce<WM_R_MAX>(x, outer, n, inner, val, idx, arena);
        case WM_R_MIN: return launch_reduce<WM_R_MIN>(x, outer, n, inner, val, idx, arena);
        case WM_R_ARGMAX: return launch_reduce<WM_R_ARGMAX>(x, outer, n, inner, val, idx, arena);
        default: return launch_reduce<WM_R_ARGMIN>(x, outer, n, inner, val, idx, arena);
    }
}

int wm_reduce(int op, const float* x, int64_t outer, int64_t n, int64_t inner, float* val, int64_t* idx) {
    return reduce_entry("wm_reduce", op, x, outer, n, inner, val, idx, false);
}

int wm_reduce_noalloc(int op, const float* x, int64_t outer, int64_t n, int64_t inner, float* val, int64_t* idx) {
    return reduce_entry("wm_reduce_noalloc", op, x, outer, n, inner, val, idx, true);
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
            const dim3 grid(grid_for(total / 4, kBlock * kSlotsBwd, 1 << 12));
            const bool i32 = total < ((int64_t)1 << 32);
#define WM_RBS(A, I1, I32) \
    launch_kernel((reduce_bwd_sum_vec_kernel<A, I1, I32>), grid, dim3(kBlock), 0, st, g, gx, outer, n, inner)
            if (inner == 1) {
                if (accumulate) { if (i32) WM_RBS(true, true, true); else WM_RBS(true, true, false); }
                else { if (i32) WM_RBS(false, true, true); else WM_RBS(false, true, false); }
            } else {
                if (accumulate) { if (i32) WM_RBS(true, false, true); else WM_RBS(true, false, false); }
                else { if (i32) WM_RBS(false, false, true); else WM_RBS(false, false, false); }
            }
#undef WM_RBS
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
