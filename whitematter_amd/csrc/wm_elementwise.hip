// Elementwise kernels: fill, copy, fp16 conversion, broadcast binary forward
// and unary forward/backward.
//
// Layout: every tensor is contiguous row-major fp32, as in the reference
// (core/tensor.h:35).  Broadcasting follows NumPy's right-aligned rule
// (core/tensor.cpp:338-372); instead of the reference's per-element
// multi-index odometer (:375-387, :936-947) the host folds the output shape
// into as few dims as possible, the kernels give each broadcast operand a
// stride of 0 on the dims it repeats along, and the innermost dim is walked
// with 128-bit loads/stores in grid-stride loops.
#include "wm_ops.hpp"

#include <algorithm>

namespace wm {

constexpr int kBlock = 256;   // 4 waves
// Streaming kernels give each thread one float4 per operand and launch a
// grid that covers the whole tensor (kWholeGrid: the loops are still
// grid-stride, for tensors beyond a million workgroups).  On MI355X that
// measured 4-8 points of the HBM peak faster than a grid of 32 workgroups
// per CU looping over 4 float4s per thread (c2 A+r forward 72 -> 78 %, a
// same-shape backward 71 -> 79 %): short-lived workgroups keep the chip's
// accesses inside a narrow, advancing window of the tensor.
constexpr int kUnroll = 1;
constexpr int kWholeGrid = 1 << 12;  // grid_for cap, in workgroups per CU

// pow's forward evaluates ~40 vector instructions per element with 16
// doubles live per float4; it is issue-bound rather than latency-bound, and
// keeps 2 float4s per thread on a grid of 32 workgroups per CU, which
// measured faster for it than the whole-tensor grid.  Asking for 6
// workgroups of kBlock threads per CU (6 waves per SIMD) caps it at 80
// VGPRs, which pow(x, scalar) and pow with one exponent per row meet without
// spills (two tensor operands would spill).
template <int OP>
constexpr int fwd_unroll() {
    return OP == WM_POW || OP == WM_POWS ? 2 : kUnroll;
}
template <int OP>
constexpr int fwd_min_blocks() {
    return OP == WM_POW || OP == WM_POWS ? 6 : 1;
}
template <int OP>
constexpr int fwd_grid_cap() {
    return OP == WM_POW || OP == WM_POWS ? 32 : kWholeGrid;
}

// ---------------------------------------------------------------------------
// Broadcast layout (host)
// ---------------------------------------------------------------------------

struct BcastLayout {
    int nd = 0;                 // collapsed rank (>= 1)
    int64_t size[WM_MAX_DIMS];  // collapsed output sizes
    int64_t sa[WM_MAX_DIMS];    // element strides of a (0 = broadcast)
    int64_t sb[WM_MAX_DIMS];
    int64_t numel = 0;
};

// Reference semantics: right-align, each pair equal or one of them 1
// (core/tensor.cpp:338-358).
int broadcast_shape_impl(const int64_t* as, int an, const int64_t* bs, int bn,
                         int64_t* os, int* on) {
    if (an < 0 || bn < 0 || an > WM_MAX_DIMS || bn > WM_MAX_DIMS)
        return set_error(WM_ERR_INVALID, "broadcast: rank out of range (max 8)");
    int nd = std::max(an, bn);
    for (int i = 0; i < nd; ++i) {
        int64_t da = (i < nd - an) ? 1 : as[i - (nd - an)];
        int64_t db = (i < nd - bn) ? 1 : bs[i - (nd - bn)];
        if (da < 0 || db < 0) return set_error(WM_ERR_INVALID, "broadcast: negative dim");
        if (da == db) os[i] = da;
        else if (da == 1) os[i] = db;
        else if (db == 1) os[i] = da;
        else return set_error(WM_ERR_INVALID, "Shapes are not broadcastable");
    }
    *on = nd;
    return WM_OK;
}

// Per-output-dim strides of an operand (0 where it is broadcast), then merge
// dims that both operands walk contiguously (or both repeat).
int make_bcast_layout(const int64_t* as, int an, const int64_t* bs, int bn, BcastLayout& L) {
    int64_t os[WM_MAX_DIMS];
    int nd = 0;
    WM_TRY(broadcast_shape_impl(as, an, bs, bn, os, &nd));
    int64_t sa[WM_MAX_DIMS], sb[WM_MAX_DIMS];
    int64_t ra = 1, rb = 1;
    L.numel = 1;
    for (int i = nd - 1; i >= 0; --i) {
        int ia = i - (nd - an), ib = i - (nd - bn);
        int64_t da = ia >= 0 ? as[ia] : 1, db = ib >= 0 ? bs[ib] : 1;
        sa[i] = (da == 1) ? 0 : ra;
        sb[i] = (db == 1) ? 0 : rb;
        ra *= da;
        rb *= db;
        L.numel *= os[i];
    }
    // Drop size-1 dims, then merge neighbours.
    int k = 0;
    int64_t cs[WM_MAX_DIMS], ca[WM_MAX_DIMS], cb[WM_MAX_DIMS];
    for (int i = 0; i < nd; ++i) {
        if (os[i] == 1) continue;
        if (k > 0 && ca[k - 1] == sa[i] * os[i] && cb[k - 1] == sb[i] * os[i]) {
            cs[k - 1] *= os[i];
            ca[k - 1] = sa[i];
            cb[k - 1] = sb[i];
        } else {
            cs[k] = os[i]; ca[k] = sa[i]; cb[k] = sb[i];
            ++k;
        }
    }
    if (k == 0) { cs[0] = 1; ca[0] = 0; cb[0] = 0; k = 1; }
    L.nd = k;
    for (int i = 0; i < k; ++i) { L.size[i] = cs[i]; L.sa[i] = ca[i]; L.sb[i] = cb[i]; }
    return WM_OK;
}

int make_bcast_layout_public(const int64_t* as, int an, const int64_t* bs, int bn, int& nd, int64_t* size,
                             int64_t* sa, int64_t* sb, int64_t& numel) {
    BcastLayout L;
    WM_TRY(make_bcast_layout(as, an, bs, bn, L));
    nd = L.nd;
    numel = L.numel;
    for (int i = 0; i < L.nd; ++i) { size[i] = L.size[i]; sa[i] = L.sa[i]; sb[i] = L.sb[i]; }
    return WM_OK;
}

// Outer (row) dims of a collapsed layout, passed by value to kernels.
struct RowDims {
    int nd;                          // number of outer dims (0..7)
    int64_t size[WM_MAX_DIMS - 1];
    int64_t sa[WM_MAX_DIMS - 1];
    int64_t sb[WM_MAX_DIMS - 1];
};

__device__ __forceinline__ void row_offsets(const RowDims& d, int64_t row, int64_t& oa, int64_t& ob) {
    if (d.nd == 1) {  // one outer dim (the common folded case): row < size[0]
        oa = row * d.sa[0]; ob = row * d.sb[0];
        return;
    }
    oa = 0; ob = 0;
    for (int i = d.nd - 1; i >= 0; --i) {
        int64_t s = d.size[i];
        int64_t q = row / s;
        int64_t r = row - q * s;
        oa += r * d.sa[i];
        ob += r * d.sb[i];
        row = q;
    }
}

// ---------------------------------------------------------------------------
// Kernels
// ---------------------------------------------------------------------------

__global__ void __launch_bounds__(kBlock) fill_vec_kernel(float* __restrict__ out, float v, int64_t n4) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const float4 f = make_float4(v, v, v, v);
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) st_stream(out + 4 * i, f);
}

__global__ void __launch_bounds__(kBlock) fill_scalar_kernel(float* __restrict__ out, float v, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) out[i] = v;
}

// NT: non-temporal loads and stores (the streaming form every hot kernel
// uses); otherwise ordinary cached ones.  Both move the same bytes, so their
// counter readings calibrate each kind of access.
template <bool NT>
__global__ void __launch_bounds__(kBlock) copy_vec_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                           int64_t n4) {
    const int64_t stride = (int64_t)gridDim.x * kBlock * kUnroll;
    for (int64_t base = (int64_t)blockIdx.x * kBlock * kUnroll + threadIdx.x; base < n4; base += stride) {
        float4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            int64_t i = base + (int64_t)u * kBlock;
            if (i < n4) v[u] = NT ? ld_stream(src + 4 * i) : *reinterpret_cast<const float4*>(src + 4 * i);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            int64_t i = base + (int64_t)u * kBlock;
            if (i < n4) {
                if (NT)
                    st_stream(dst + 4 * i, v[u]);
                else
                    *reinterpret_cast<float4*>(dst + 4 * i) = v[u];
            }
        }
    }
}

__device__ __forceinline__ uint16_t f32_to_f16_rtz(float f) { return (uint16_t)float_to_half_bits_rtz(f); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) { return half_bits_to_float(h); }

__global__ void __launch_bounds__(kBlock) f32_to_f16_kernel(uint16_t* __restrict__ out, const float* __restrict__ x, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t n4 = n / 4;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
        float4 v = reinterpret_cast<const float4*>(x)[i];
        uint2 o;
        o.x = float2_to_half2_bits_rtz(v.x, v.y);
        o.y = float2_to_half2_bits_rtz(v.z, v.w);
        reinterpret_cast<uint2*>(out)[i] = o;
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        out[i] = f32_to_f16_rtz(x[i]);
}

__global__ void __launch_bounds__(kBlock) f16_to_f32_kernel(float* __restrict__ out, const uint16_t* __restrict__ x, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t n4 = n / 4;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n4; i += stride) {
        uint2 v = reinterpret_cast<const uint2*>(x)[i];
        float4 o = make_float4(f16_to_f32((uint16_t)(v.x & 0xFFFFu)), f16_to_f32((uint16_t)(v.x >> 16)),
                               f16_to_f32((uint16_t)(v.y & 0xFFFFu)), f16_to_f32((uint16_t)(v.y >> 16)));
        reinterpret_cast<float4*>(out)[i] = o;
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
        out[i] = f16_to_f32(x[i]);
}

// Same-shape binary op over float4s (the reference fast path, shape == other->shape).
template <int OP>
__global__ void __launch_bounds__(kBlock) binary_flat_kernel(float* __restrict__ out, const float* __restrict__ a,
                                                              const float* __restrict__ b, int64_t n4) {
    binary_prologue<OP>();
    constexpr int U = fwd_unroll<OP>();
    const int64_t stride = (int64_t)gridDim.x * kBlock * U;
    for (int64_t base = (int64_t)blockIdx.x * kBlock * U + threadIdx.x; base < n4; base += stride) {
        float4 va[U], vb[U], vr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int64_t i = base + (int64_t)u * kBlock;
            va[u] = vb[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < n4) { va[u] = ld_stream(a + 4 * i); vb[u] = ld_stream(b + 4 * i); }
        }
        binary_fwd_v<OP, U>(vr, va, vb);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int64_t i = base + (int64_t)u * kBlock;
            if (i < n4) st_stream(out + 4 * i, vr[u]);
        }
    }
}

// Broadcast binary op over [rows, inner]: each tile is one row segment of
// kBlock*4*fwd_unroll elements; the row's operand offsets come from the outer
// dims once per tile.  AI/BI: stride of a/b along inner (1 = contiguous,
// 0 = one value per row).  VEC: inner % 4 == 0 and 16-byte aligned bases.
// SA/SB: the operand is streamed (read once: it has a row stride), else it
// is a row vector reused by every row and stays on cached loads.
//
// With one outer dim, an even row count and rows of at least kPairMinInner
// floats, a matrix with a row vector or a column vector takes items of
// kRowPair rows instead: the item bookkeeping (row and tile indices, operand
// offsets) is shared by both rows and a row vector's float4 is loaded once
// for them.  Measured on 256 MiB operands: config 2 ([8192, 8192]) A + r
// forward 77.3 -> 81 %, A / r 74.8 -> 81 %, A * c 77 -> 81 % of the HBM
// peak, and 80.2 -> 81.9 % for a row vector at [4096, 16384]; with rows of
// 1024-4096 floats the pairs ran 1-3 points slower than single rows, which
// they keep.  pow pairs only with one exponent per row (A^c): one float4 per
// row instead of its single rows' two, at 7 waves per SIMD (72 VGPRs, no
// spills) on the same 32 workgroups per CU, 69.5 -> 72.0-72.4 % at config 2
// (pairs at 6 waves: 71 %; caps of 16-40 workgroups per CU within the
// spread, 64 and the whole-tensor grid 67 and 62 %).
//   AI = BI = 1: one operand has row stride 0 (the row vector);
//   one of AI, BI = 0: that operand is one value per row (a column vector).
template <int OP, int AI, int BI, bool VEC>
constexpr bool row_pairs() {
    return VEC && (OP != WM_POW ? (AI == 1 || BI == 1) : (AI == 1 && BI == 0));
}
constexpr int kRowPair = 2;
constexpr int64_t kPairMinInner = 8192;

template <int OP, int AI, int BI, bool VEC, bool PAIRS>
constexpr int rows_min_waves() {
    return BI != 0 ? 1 : (PAIRS && OP == WM_POW) ? 7 : fwd_min_blocks<OP>();
}
// Float4s per row and thread of a tile.
template <int OP, bool PAIRS>
constexpr int rows_unroll() {
    return PAIRS && OP == WM_POW ? 1 : fwd_unroll<OP>();
}

// PAIRS: the row-pair form (the host decides it, as row_pairs allows; a
// separate instantiation, because the pair code compiled into the single-row
// kernel slowed its own rows: a row vector at [16384, 4096] 77.7 -> 74.5 %).
template <int OP, int AI, int BI, bool VEC, bool PAIRS>
__global__ void __launch_bounds__(kBlock, (rows_min_waves<OP, AI, BI, VEC, PAIRS>()))
    binary_rows_kernel(float* __restrict__ out, const float* __restrict__ a, const float* __restrict__ b, int64_t rows,
                       int64_t inner, RowDims d, int stream_a, int stream_b) {
    static_assert(!PAIRS || row_pairs<OP, AI, BI, VEC>(), "row pairs: not for this operand layout");
    binary_prologue<OP>();
    constexpr int U = rows_unroll<OP, PAIRS>();
    constexpr int64_t kTile = (VEC ? 4 : 1) * kBlock * U;
    const int64_t items_rows = PAIRS ? rows / kRowPair : rows;
    const int64_t tiles_per_row = (inner + kTile - 1) / kTile;
    // Grid-stride over (row, tile) pairs, advanced incrementally so the loop
    // itself divides nothing (a 64-bit division costs ~40 instructions).
    const int64_t step_rows = (int64_t)gridDim.x / tiles_per_row;
    const int64_t step_tiles = (int64_t)gridDim.x - step_rows * tiles_per_row;
    int64_t row = (int64_t)blockIdx.x / tiles_per_row;
    int64_t tile = (int64_t)blockIdx.x - row * tiles_per_row;
    for (; row < items_rows; row += step_rows, tile += step_tiles) {
        if (tile >= tiles_per_row) { tile -= tiles_per_row; ++row; if (row >= items_rows) break; }
        const int64_t c0 = tile * kTile;
        if constexpr (PAIRS) {
            {
                // Rows kRowPair*row .. +kRowPair-1.
                float4 vr[kRowPair][U], va[kRowPair][U], vb[kRowPair][U];
                if constexpr (AI == 1 && BI == 1) {
                    // v: the row vector's float4; sv: the streamed operand's, per row
                    const bool a_vec = d.sa[0] == 0;
                    const float* sbase = a_vec ? b : a;
                    const int64_t sstride = a_vec ? d.sb[0] : d.sa[0];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int64_t c = c0 + ((int64_t)u * kBlock + threadIdx.x) * 4;
                        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                        if (c < inner) v = *reinterpret_cast<const float4*>((a_vec ? a : b) + c);
#pragma unroll
                        for (int q = 0; q < kRowPair; ++q) {
                            float4 sv = make_float4(0.f, 0.f, 0.f, 0.f);
                            if (c < inner) sv = ld_stream(sbase + (row * kRowPair + q) * sstride + c);
                            va[q][u] = a_vec ? v : sv;
                            vb[q][u] = a_vec ? sv : v;
                        }
                    }
                } else {
                    // One operand streamed (S*), the other one value per row (C*).
                    const float* sbase = AI ? a : b;
                    const float* cbase = AI ? b : a;
                    const int64_t sstride = AI ? d.sa[0] : d.sb[0];
                    const int64_t cstride = AI ? d.sb[0] : d.sa[0];
                    float cv[kRowPair];
#pragma unroll
                    for (int q = 0; q < kRowPair; ++q) cv[q] = cbase[(row * kRowPair + q) * cstride];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int64_t c = c0 + ((int64_t)u * kBlock + threadIdx.x) * 4;
#pragma unroll
                        for (int q = 0; q < kRowPair; ++q) {
                            float4 sv = make_float4(0.f, 0.f, 0.f, 0.f);
                            if (c < inner) sv = ld_stream(sbase + (row * kRowPair + q) * sstride + c);
                            const float4 v = make_float4(cv[q], cv[q], cv[q], cv[q]);
                            va[q][u] = AI ? sv : v;
                            vb[q][u] = AI ? v : sv;
                        }
                    }
                }
                if constexpr (OP == WM_POW) {
                    static_assert(kRowPair == 2 && U == 1, "pow pairs: one float4 of each of two rows");
                    pow_fwd_pair(vr[0][0], vr[1][0], va[0][0], va[1][0], vb[0][0].x, vb[1][0].x);
                } else {
#pragma unroll
                    for (int q = 0; q < kRowPair; ++q) binary_fwd_v<OP, U>(vr[q], va[q], vb[q]);
                }
#pragma unroll
                for (int q = 0; q < kRowPair; ++q)
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int64_t c = c0 + ((int64_t)u * kBlock + threadIdx.x) * 4;
                        if (c < inner) st_stream(out + (row * kRowPair + q) * inner + c, vr[q][u]);
                    }
            }
        } else {
        int64_t oa, ob;
        row_offsets(d, row, oa, ob);
        const float* ar = a + oa;
        const float* br = b + ob;
        float* orow = out + row * inner;
        if constexpr (VEC) {
            float4 va[U], vb[U], vr[U];
            float sa0 = AI ? 0.f : ar[0];
            float sb0 = BI ? 0.f : br[0];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int64_t c = c0 + ((int64_t)u * kBlock + threadIdx.x) * 4;
                va[u] = vb[u] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (c < inner) {
                    va[u] = AI ? (stream_a ? ld_stream(ar + c) : *reinterpret_cast<const float4*>(ar + c))
                               : make_float4(sa0, sa0, sa0, sa0);
                    vb[u] = BI ? (stream_b ? ld_stream(br + c) : *reinterpret_cast<const float4*>(br + c))
                               : make_float4(sb0, sb0, sb0, sb0);
                }
            }
            if constexpr (OP == WM_POW && BI == 0) pow_fwd_v_exp<U>(vr, va, sb0);  // one exponent per row
            else binary_fwd_v<OP, U>(vr, va, vb);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int64_t c = c0 + ((int64_t)u * kBlock + threadIdx.x) * 4;
                if (c < inner) st_stream(orow + c, vr[u]);
            }
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int64_t c = c0 + (int64_t)u * kBlock + threadIdx.x;
                if (c < inner) orow[c] = binary_fwd<OP>(ar[AI ? c : 0], br[BI ? c : 0]);
            }
        }
        }  // single rows
    }
}

// Fallback for any collapsed layout: per-element index math over all dims.
struct FullDims {
    int nd;
    int64_t size[WM_MAX_DIMS];
    int64_t sa[WM_MAX_DIMS];
    int64_t sb[WM_MAX_DIMS];
};

__device__ __forceinline__ void full_offsets(const FullDims& d, int64_t i, int64_t& oa, int64_t& ob) {
    oa = 0; ob = 0;
    for (int k = d.nd - 1; k >= 0; --k) {
        int64_t s = d.size[k];
        int64_t q = i / s;
        int64_t r = i - q * s;
        oa += r * d.sa[k];
        ob += r * d.sb[k];
        i = q;
    }
}

template <int OP>
__global__ void __launch_bounds__(kBlock) binary_generic_kernel(float* __restrict__ out, const float* __restrict__ a,
                                                                 const float* __restrict__ b, int64_t n, FullDims d) {
    binary_prologue<OP>();
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) {
        int64_t oa, ob;
        full_offsets(d, i, oa, ob);
        out[i] = binary_fwd<OP>(a[oa], b[ob]);
    }
}

template <int OP>
__global__ void __launch_bounds__(kBlock, fwd_min_blocks<OP>())
    unary_fwd_kernel(float* __restrict__ out, const float* __restrict__ x, int64_t n, float p0, float p1) {
    unary_prologue<OP>();
    constexpr int U = fwd_unroll<OP>();
    const int64_t n4 = n / 4;
    const int64_t stride = (int64_t)gridDim.x * kBlock * U;
    for (int64_t base = (int64_t)blockIdx.x * kBlock * U + threadIdx.x; base < n4; base += stride) {
        float4 v[U], r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int64_t i = base + (int64_t)u * kBlock;
            v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < n4) v[u] = ld_stream(x + 4 * i);
        }
        unary_fwd_v<OP, U>(r, v, p0, p1);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int64_t i = base + (int64_t)u * kBlock;
            if (i < n4) st_stream(out + 4 * i, r[u]);
        }
    }
    // Scalar tail (n % 4 elements).
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock)
        out[i] = unary_fwd<OP>(x[i], p0, p1);
}

template <int OP>
__global__ void __launch_bounds__(kBlock) unary_fwd_scalar_kernel(float* __restrict__ out, const float* __restrict__ x,
                                                                   int64_t n, float p0, float p1) {
    unary_prologue<OP>();
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock)
        out[i] = unary_fwd<OP>(x[i], p0, p1);
}

template <int OP, bool ACC>
__device__ __forceinline__ float ubwd1(float g, float x, float o, float gx, float p0, float p1) {
    float c = unary_bwd<OP>(g, x, o, p0, p1);
    return ACC ? gx + c : c;
}

template <int OP, bool ACC>
__global__ void __launch_bounds__(kBlock) unary_bwd_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                            const float* __restrict__ o, float* __restrict__ gx,
                                                            int64_t n, float p0, float p1) {
    unary_prologue<OP>();
    constexpr bool RX = unary_bwd_reads_x<OP>();
    constexpr bool RO = unary_bwd_reads_out<OP>();
    const int64_t n4 = n / 4;
    const int64_t stride = (int64_t)gridDim.x * kBlock * kUnroll;
    for (int64_t base = (int64_t)blockIdx.x * kBlock * kUnroll + threadIdx.x; base < n4; base += stride) {
        float4 vg[kUnroll], vx[kUnroll], vo[kUnroll], vgx[kUnroll], r[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            int64_t i = base + (int64_t)u * kBlock;
            vg[u] = vx[u] = vo[u] = vgx[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < n4) {
                vg[u] = ld_stream(g + 4 * i);
                vx[u] = RX ? ld_stream(x + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
                vo[u] = RO ? ld_stream(o + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
                vgx[u] = ACC ? ld_stream(gx + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        unary_bwd_v<OP, ACC, kUnroll>(r, vg, vx, vo, vgx, p0, p1);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            int64_t i = base + (int64_t)u * kBlock;
            if (i < n4) st_stream(gx + 4 * i, r[u]);
        }
    }
    for (int64_t i = n4 * 4 + (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock)
        gx[i] = ubwd1<OP, ACC>(g[i], RX ? x[i] : 0.f, RO ? o[i] : 0.f, ACC ? gx[i] : 0.f, p0, p1);
}

template <int OP, bool ACC>
__global__ void __launch_bounds__(kBlock) unary_bwd_scalar_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                                   const float* __restrict__ o, float* __restrict__ gx,
                                                                   int64_t n, float p0, float p1) {
    unary_prologue<OP>();
    constexpr bool RX = unary_bwd_reads_x<OP>();
    constexpr bool RO = unary_bwd_reads_out<OP>();
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock)
        gx[i] = ubwd1<OP, ACC>(g[i], RX ? x[i] : 0.f, RO ? o[i] : 0.f, ACC ? gx[i] : 0.f, p0, p1);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------

template <int OP>
int launch_binary(float* out, const float* a, const float* b, const BcastLayout& L) {
    hipStream_t s = stream();
    const int nd = L.nd;
    const int64_t inner = L.size[nd - 1];
    const int64_t ia = L.sa[nd - 1], ib = L.sb[nd - 1];
    // Same shape (or both fully contiguous after folding): flat float4 walk.
    if (nd == 1 && ia == 1 && ib == 1 && (inner % 4) == 0 && aligned16(out) && aligned16(a) && aligned16(b)) {
        int64_t n4 = inner / 4;
        launch_kernel(binary_flat_kernel<OP>, dim3(grid_for(n4, kBlock * fwd_unroll<OP>(), fwd_grid_cap<OP>())), dim3(kBlock), 0, s,
                           out, a, b, n4);
        return check_launch("wm_binary(flat)");
    }
    if (inner >= 64 && (ia == 0 || ia == 1) && (ib == 0 || ib == 1)) {
        RowDims d;
        d.nd = nd - 1;
        int64_t rows = 1;
        for (int i = 0; i < nd - 1; ++i) {
            d.size[i] = L.size[i]; d.sa[i] = L.sa[i]; d.sb[i] = L.sb[i];
            rows *= L.size[i];
        }
        // float4 path: every row start is a multiple of 4 floats when inner is.
        bool vec = (inner % 4) == 0 && aligned16(out) && aligned16(a) && aligned16(b);
        // Row pairs (binary_rows_kernel; pow only with one exponent per row):
        // half the items.
        const bool pairs = vec && (OP != WM_POW ? (ia || ib) : (ia && !ib)) && nd == 2 && rows % kRowPair == 0 &&
                           inner >= kPairMinInner && (!ia || !ib || L.sa[0] == 0 || L.sb[0] == 0);
        const int64_t tile = (vec ? 4 : 1) * kBlock * (pairs ? rows_unroll<OP, true>() : fwd_unroll<OP>());
        int64_t tiles = rows * ((inner + tile - 1) / tile);
        if (pairs) tiles /= kRowPair;
        dim3 grid(grid_for(tiles, 1, fwd_grid_cap<OP>()));
        // An operand with a row stride is read once; a row vector is re-read by every row.
        int stream_a = 0, stream_b = 0;
        for (int i = 0; i < nd - 1; ++i) {
            if (L.sa[i] != 0) stream_a = 1;
            if (L.sb[i] != 0) stream_b = 1;
        }
        if (nd == 1) stream_a = stream_b = 1;
#define WM_ROWS(AI, BI, V, P) \
    launch_kernel((binary_rows_kernel<OP, AI, BI, V, P>), grid, dim3(kBlock), 0, s, out, a, b, rows, inner, d, \
                       stream_a, stream_b)
        if (vec) {
            if constexpr (OP == WM_POW) {
                if (pairs) {
                    WM_ROWS(1, 0, true, true);
                    return check_launch("wm_binary(rows)");
                }
            } else {
                if (pairs) {
                    if (ia && ib) WM_ROWS(1, 1, true, true);
                    else if (ia) WM_ROWS(1, 0, true, true);
                    else WM_ROWS(0, 1, true, true);
                    return check_launch("wm_binary(rows)");
                }
            }
            if (ia && ib) WM_ROWS(1, 1, true, false);
            else if (ia) WM_ROWS(1, 0, true, false);
            else if (ib) WM_ROWS(0, 1, true, false);
            else WM_ROWS(0, 0, true, false);
        } else {
            if (ia && ib) WM_ROWS(1, 1, false, false);
            else if (ia) WM_ROWS(1, 0, false, false);
            else if (ib) WM_ROWS(0, 1, false, false);
            else WM_ROWS(0, 0, false, false);
        }
#undef WM_ROWS
        return check_launch("wm_binary(rows)");
    }
    FullDims d;
    d.nd = nd;
    for (int i = 0; i < nd; ++i) { d.size[i] = L.size[i]; d.sa[i] = L.sa[i]; d.sb[i] = L.sb[i]; }
    launch_kernel(binary_generic_kernel<OP>, dim3(grid_for(L.numel, kBlock)), dim3(kBlock), 0, s, out, a, b,
                       L.numel, d);
    return check_launch("wm_binary(generic)");
}

template <int OP>
int launch_unary(float* out, const float* x, int64_t n, float p0, float p1) {
    hipStream_t s = stream();
    if (aligned16(out) && aligned16(x)) {
        launch_kernel(unary_fwd_kernel<OP>, dim3(grid_for(n / 4 + 1, kBlock * fwd_unroll<OP>(), fwd_grid_cap<OP>())), dim3(kBlock), 0, s,
                           out, x, n, p0, p1);
    } else {
        launch_kernel(unary_fwd_scalar_kernel<OP>, dim3(grid_for(n, kBlock)), dim3(kBlock), 0, s, out, x, n,
                           p0, p1);
    }
    return check_launch("wm_unary");
}

template <int OP>
int launch_unary_bwd(const float* g, const float* x, const float* o, float* gx, int acc, int64_t n, float p0,
                     float p1) {
    hipStream_t s = stream();
    constexpr bool RX = unary_bwd_reads_x<OP>();
    constexpr bool RO = unary_bwd_reads_out<OP>();
    if (RX && !x) return set_error(WM_ERR_INVALID, "wm_unary_bwd: this op needs the forward input x");
    if (RO && !o) return set_error(WM_ERR_INVALID, "wm_unary_bwd: this op needs the forward output");
    bool vec = aligned16(g) && aligned16(gx) && (!RX || aligned16(x)) && (!RO || aligned16(o));
    dim3 grid_v(grid_for(n / 4 + 1, kBlock * kUnroll, kWholeGrid)), grid_s(grid_for(n, kBlock));
    if (vec) {
        if (acc) launch_kernel((unary_bwd_kernel<OP, true>), grid_v, dim3(kBlock), 0, s, g, x, o, gx, n, p0, p1);
        else launch_kernel((unary_bwd_kernel<OP, false>), grid_v, dim3(kBlock), 0, s, g, x, o, gx, n, p0, p1);
    } else {
        if (acc) launch_kernel((unary_bwd_scalar_kernel<OP, true>), grid_s, dim3(kBlock), 0, s, g, x, o, gx, n, p0, p1);
        else launch_kernel((unary_bwd_scalar_kernel<OP, false>), grid_s, dim3(kBlock), 0, s, g, x, o, gx, n, p0, p1);
    }
    return check_launch("wm_unary_bwd");
}

int check_shape(const int64_t* shape, int nd, const char* what) {
    if (nd < 0 || nd > WM_MAX_DIMS) return set_error(WM_ERR_INVALID, std::string(what) + ": rank out of range (max 8)");
    if (nd > 0 && !shape) return set_error(WM_ERR_INVALID, std::string(what) + ": null shape");
    for (int i = 0; i < nd; ++i)
        if (shape[i] < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative dim");
    return WM_OK;
}

int64_t shape_numel(const int64_t* shape, int nd) {
    int64_t n = 1;
    for (int i = 0; i < nd; ++i) n *= shape[i];
    return n;
}

}  // namespace wm

using namespace wm;

namespace {
template <bool NT>
int copy_entry(float* dst, const float* src, int64_t n, const char* what) {
    if (n < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative size");
    if (n == 0) return WM_OK;
    if (!dst || !src) return set_error(WM_ERR_INVALID, std::string(what) + ": null pointer");
    if (n % 4 || !aligned16(dst) || !aligned16(src))
        return set_error(WM_ERR_INVALID, std::string(what) + ": needs 16-byte aligned buffers and n % 4 == 0");
    WM_CHECK_INIT();
    launch_kernel(copy_vec_kernel<NT>, dim3(grid_for(n / 4, kBlock * kUnroll, kWholeGrid)), dim3(kBlock), 0, stream(), dst,
                  src, n / 4);
    return check_launch(what);
}
}  // namespace

extern "C" {

int wm_fill(float* out, float value, int64_t n) {
    if (n < 0) return set_error(WM_ERR_INVALID, "wm_fill: negative size");
    if (n == 0) return WM_OK;
    if (!out) return set_error(WM_ERR_INVALID, "wm_fill: null pointer");
    WM_CHECK_INIT();
    if (aligned16(out) && n % 4 == 0) {
        launch_kernel(fill_vec_kernel, dim3(grid_for(n / 4, kBlock, 64)), dim3(kBlock), 0, stream(), out,
                           value, n / 4);
    } else {
        launch_kernel(fill_scalar_kernel, dim3(grid_for(n, kBlock)), dim3(kBlock), 0, stream(), out, value, n);
    }
    return check_launch("wm_fill");
}

int wm_copy_kernel(float* dst, const float* src, int64_t n) { return copy_entry<true>(dst, src, n, "wm_copy_kernel"); }

int wm_copy_kernel_cached(float* dst, const float* src, int64_t n) {
    return copy_entry<false>(dst, src, n, "wm_copy_kernel_cached");
}

int wm_f32_to_f16_rtz(uint16_t* out, const float* x, int64_t n) {
    if (n < 0) return set_error(WM_ERR_INVALID, "wm_f32_to_f16_rtz: negative size");
    if (n == 0) return WM_OK;
    if (!out || !x) return set_error(WM_ERR_INVALID, "wm_f32_to_f16_rtz: null pointer");
    if (!aligned16(x) || ((uintptr_t)out & 7u))
        return set_error(WM_ERR_INVALID, "wm_f32_to_f16_rtz: x must be 16-byte and out 8-byte aligned");
    WM_CHECK_INIT();
    launch_kernel(f32_to_f16_kernel, dim3(grid_for(n / 4 + 1, kBlock, kWholeGrid)), dim3(kBlock), 0, stream(), out, x, n);
    return check_launch("wm_f32_to_f16_rtz");
}

int wm_f16_to_f32(float* out, const uint16_t* x, int64_t n) {
    if (n < 0) return set_error(WM_ERR_INVALID, "wm_f16_to_f32: negative size");
    if (n == 0) return WM_OK;
    if (!out || !x) return set_error(WM_ERR_INVALID, "wm_f16_to_f32: null pointer");
    if (!aligned16(out) || ((uintptr_t)x & 7u))
        return set_error(WM_ERR_INVALID, "wm_f16_to_f32: out must be 16-byte and x 8-byte aligned");
    WM_CHECK_INIT();
    launch_kernel(f16_to_f32_kernel, dim3(grid_for(n / 4 + 1, kBlock, kWholeGrid)), dim3(kBlock), 0, stream(), out, x, n);
    return check_launch("wm_f16_to_f32");
}

int wm_broadcast_shape(const int64_t* a_shape, int a_ndim, const int64_t* b_shape, int b_ndim, int64_t* out_shape,
                       int* out_ndim) {
    WM_TRY(check_shape(a_shape, a_ndim, "wm_broadcast_shape(a)"));
    WM_TRY(check_shape(b_shape, b_ndim, "wm_broadcast_shape(b)"));
    if (!out_shape || !out_ndim) return set_error(WM_ERR_INVALID, "wm_broadcast_shape: null output");
    return broadcast_shape_impl(a_shape, a_ndim, b_shape, b_ndim, out_shape, out_ndim);
}

int wm_binary(int op, float* out, const float* a, const int64_t* a_shape, int a_ndim, const float* b,
              const int64_t* b_shape, int b_ndim) {
    WM_TRY(check_shape(a_shape, a_ndim, "wm_binary(a)"));
    WM_TRY(check_shape(b_shape, b_ndim, "wm_binary(b)"));
    BcastLayout L;
    WM_TRY(make_bcast_layout(a_shape, a_ndim, b_shape, b_ndim, L));
    if (L.numel == 0) return WM_OK;
    if (!out || !a || !b) return set_error(WM_ERR_INVALID, "wm_binary: null pointer");
    WM_CHECK_INIT();
    switch (op) {
        case WM_ADD: return launch_binary<WM_ADD>(out, a, b, L);
        case WM_SUB: return launch_binary<WM_SUB>(out, a, b, L);
        case WM_MUL: return launch_binary<WM_MUL>(out, a, b, L);
        case WM_DIV: return launch_binary<WM_DIV>(out, a, b, L);
        case WM_POW: return launch_binary<WM_POW>(out, a, b, L);
        case WM_MAX: return launch_binary<WM_MAX>(out, a, b, L);
        case WM_MIN: return launch_binary<WM_MIN>(out, a, b, L);
        default: return set_error(WM_ERR_INVALID, "wm_binary: unknown op");
    }
}

int wm_unary(int op, float* out, const float* x, int64_t n, float p0, float p1) {
    if (n < 0) return set_error(WM_ERR_INVALID, "wm_unary: negative size");
    if (n == 0) return WM_OK;
    if (!out || !x) return set_error(WM_ERR_INVALID, "wm_unary: null pointer");
    WM_CHECK_INIT();
    switch (op) {
        case WM_RELU: return launch_unary<WM_RELU>(out, x, n, p0, p1);
        case WM_SIGMOID: return launch_unary<WM_SIGMOID>(out, x, n, p0, p1);
        case WM_TANH: return launch_unary<WM_TANH>(out, x, n, p0, p1);
        case WM_LOG: return launch_unary<WM_LOG>(out, x, n, p0, p1);
        case WM_EXP: return launch_unary<WM_EXP>(out, x, n, p0, p1);
        case WM_POWS: return launch_unary<WM_POWS>(out, x, n, p0, p1);
        case WM_SQRT: return launch_unary<WM_SQRT>(out, x, n, p0, p1);
        case WM_ABS: return launch_unary<WM_ABS>(out, x, n, p0, p1);
        case WM_CLAMP: return launch_unary<WM_CLAMP>(out, x, n, p0, p1);
        case WM_SCALE: return launch_unary<WM_SCALE>(out, x, n, p0, p1);
        default: return set_error(WM_ERR_INVALID, "wm_unary: unknown op");
    }
}

int wm_unary_bwd(int op, const float* g, const float* x, const float* out, float* gx, int accumulate, int64_t n,
                 float p0, float p1) {
    if (n < 0) return set_error(WM_ERR_INVALID, "wm_unary_bwd: negative size");
    if (n == 0) return WM_OK;
    if (!g || !gx) return set_error(WM_ERR_INVALID, "wm_unary_bwd: null pointer");
    WM_CHECK_INIT();
    switch (op) {
        case WM_RELU: return launch_unary_bwd<WM_RELU>(g, x, out, gx, accumulate, n, p0, p1);
        case WM_SIGMOID: return launch_unary_bwd<WM_SIGMOID>(g, x, out, gx, accumulate, n, p0, p1);
        case WM_TANH: return launch_unary_bwd<WM_TANH>(g, x, out, gx, accumulate, n, p0, p1);
        case WM_LOG: return launch_unary_bwd<WM_LOG>(g, x, out, gx, accumulate, n, p0, p1);
        case WM_EXP: return launch_unary_bwd<WM_EXP>(g, x, out, gx, accumulate, n, p0, p1);
        case WM_POWS: return launch_unary_bwd<WM_POWS>(g, x, out, gx, accumulate, n, p0, p1);
        case WM_SQRT: return launch_unary_bwd<WM_SQRT>(g, x, out, gx, accumulate, n, p0, p1);
        case WM_ABS: return launch_unary_bwd<WM_ABS>(g, x, out, gx, accumulate, n, p0, p1);
        case WM_CLAMP: return launch_unary_bwd<WM_CLAMP>(g, x, out, gx, accumulate, n, p0, p1);
        case WM_SCALE: return launch_unary_bwd<WM_SCALE>(g, x, out, gx, accumulate, n, p0, p1);
        default: return set_error(WM_ERR_INVALID, "wm_unary_bwd: unknown op");
    }
}

}  // extern "C"
