// wm_attention.hip -- MultiHeadAttention's forward and closure
// (include/wm_layers.h: wm_mha_fwd / wm_mha_bwd; reference core/layer.cpp:
// 1103-1437) on the one library stream: projections on the matrix cores
// (wm_gemm), bias gradients by the broadcast backward's column sums, and the
// per-head products, with the heads addressed as column blocks of the
// [B, S, E] activations, so nothing is copied or permuted.
//
// The score product and the softmax are one kernel (head_rows_kernel below):
// a workgroup holds 32 whole rows of a head's scores in its accumulators and
// writes only the attention weights, so the [B, H, Sq, Sk] scores never go to
// HBM and back.  Its backward twin computes dattn = dctx_h V_h^T the same way
// and writes d_scores = attn * (dattn - dot) directly.  Both take head
// widths up to 128 (multiples of 4); the forward up to 1024 keys (its rows
// live in registers), the backward any number.  Other shapes, and every
// shape when wm_mha_fused(0) is set, take the two-pass route: wm_gemm's
// per-head product into a scores buffer, then the attention-softmax kernels.
#include "wm_common.hpp"

#include "../../include/wm_gemm.h"
#include "../../include/wm_layers.h"

#include <atomic>
#include <cfloat>
#include <climits>
#include <cmath>
#include <initializer_list>
#include <type_traits>

namespace wm {
namespace {

struct MhaDims {
    int64_t B, Sq, Sk, E, H, hd;
};

std::atomic<int> g_fused{1};  // wm_mha_fused (read once per wm_mha_fwd / wm_mha_bwd call)

typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// Per-head products fused with the softmax and with its backward
// ---------------------------------------------------------------------------
//
// A workgroup of 4 waves takes 32 query rows i0 .. i0 + 31 of one (batch,
// head) and every key column: S = A_h B_h^T with A = Q (forward) or dctx
// (backward) and B = K or V.  Each row of S stays whole in the accumulators:
// wave w holds the columns 128 j + 32 w .. + 31 for j < NB as one 32 x 32
// v_mfma_f32_32x32x2_f32 block per j.  B's rows pass through LDS in chunks
// of 128 (two buffers, one barrier per chunk; the next chunk's loads -- the
// backward's, two chunks ahead -- are in flight while the matrix cores work
// on the current one); A's 32 rows are loaded once and kept in LDS, from
// which each chunk reads its fragments.  The k order is wm_gemm's (stages of 32, the
// half-wave h taking k = 16 h .. 16 h + 15 of each, four k per fragment), so
// S is bit for bit the product wm_gemm writes for the same operands.
//   forward:  attn_i = softmax(S_i * scale + mask_i), with the arithmetic of
//             attn_softmax_fwd_kernel (max from -FLT_MAX skipping NaN,
//             exp_rr, product with the row sum's reciprocal); only the sums'
//             order differs.
//   backward: d_scores_ij = attn_ij * (S_ij - dot_i), attn_softmax_bwd's
//             formula, with dot_i = dctx_i . ctx_i over the head's columns:
//             sum_j attn_ij S_ij = sum_j attn_ij sum_k dctx_ik V_jk =
//             sum_k dctx_ik ctx_ik since ctx_h = attn_h V_h, so the dot
//             needs hd products instead of the whole row of S.
// Accumulator element q of a block sits at row 8 (q / 4) + 4 half + q % 4
// of the workgroup's rows, column r (= lane % 32) of the block.
constexpr int kHRows = 32;    // query rows per workgroup
constexpr int kHChunk = 128;  // key rows per LDS chunk (4 waves x 32)
constexpr int kHMaxKeys = 8 * kHChunk;
constexpr int kHMaxWidth = 128;

struct HeadRows {
    const float* a;     // [B, Sq, E]: Q (forward) or dctx (backward)
    const float* b;     // [B, Sk, E]: K (forward) or V (backward)
    const float* mask;  // forward: NULL or [mask batches, Sq, Sk]
    const float* attn;  // backward: the forward's weights [B, H, Sq, Sk]
    const float* ctx;   // backward: the forward's context [B, Sq, E]
    float* out;         // attn (forward) or d_scores (backward)
    int64_t Sq, Sk, E, H, hd, mstride;
    float scale;
    int row_tiles, tiles, nch;
};

// Row reductions after quad_transpose: a row's values sit in the 8 lanes of
// a half-wave with the same lane % 4 (4 floats each).  Two DPP rotations
// inside each 16-lane row, then the half-wave's other row through ds_swizzle
// (lane ^ 16 inside each 32).  Fixed order, so the sums repeat bit for bit.
__device__ __forceinline__ float swz16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ float rows_max(float v) {
    v = fmaxf(v, dpp_mov<0x124>(v));  // row_ror:4
    v = fmaxf(v, dpp_mov<0x128>(v));  // row_ror:8
    return fmaxf(v, swz16(v));
}
__device__ __forceinline__ float rows_sum(float v) {
    v += dpp_mov<0x124>(v);
    v += dpp_mov<0x128>(v);
    return v + swz16(v);
}

// 4 x 4 transpose inside each quad of lanes (b = lane % 4): before, x holds
// rows 0..3 of the quad's block at column b; after, row b at columns 0..3.
// Two butterfly stages, each trading half the values with the lane whose
// index differs in one bit (DPP quad_perm), the kept half chosen by selects.
__device__ __forceinline__ float4 quad_transpose(float4 x) {
    const int b = (int)threadIdx.x & 3;
    const bool odd = (b & 1) != 0, hi = (b & 2) != 0;
    float s0 = dpp_mov<0xB1>(odd ? x.x : x.y);  // quad_perm [1, 0, 3, 2]
    float s1 = dpp_mov<0xB1>(odd ? x.z : x.w);
    x = make_float4(odd ? s0 : x.x, odd ? x.y : s0, odd ? s1 : x.z, odd ? x.w : s1);
    s0 = dpp_mov<0x4E>(hi ? x.x : x.z);  // quad_perm [2, 3, 0, 1]
    s1 = dpp_mov<0x4E>(hi ? x.y : x.w);
    return make_float4(hi ? s0 : x.x, hi ? s1 : x.y, hi ? x.z : s0, hi ? x.w : s1);
}

__device__ __forceinline__ float4 f4_of(const f32x16& a, int g) {
    return make_float4(a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]);
}
__device__ __forceinline__ void set_f4(f32x16& a, int g, float4 v) {
    a[4 * g] = v.x;
    a[4 * g + 1] = v.y;
    a[4 * g + 2] = v.z;
    a[4 * g + 3] = v.w;
}

// Buffer accesses: a descriptor (base, size in bytes) in scalar registers
// and a 32-bit byte offset per lane, constant parts folded into the
// instruction's offset field.  The hardware checks the lane offset against
// the size: a load past it returns 0 and a store past it is dropped, which
// is how the kernel below handles rows past the end of its operands.
typedef unsigned int wm_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf(const float* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes, 0x00020000);
}
template <int AUX = 0>  // 2: non-temporal
__device__ __forceinline__ float4 bld4(__amdgpu_buffer_rsrc_t r, int off) {
    const wm_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
__device__ __forceinline__ float bld1(__amdgpu_buffer_rsrc_t r, int off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ void bst4(__amdgpu_buffer_rsrc_t r, int off, float4 v) {
    const wm_u32x4 u = {__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z), __float_as_uint(v.w)};
    __builtin_amdgcn_raw_buffer_store_b128(u, r, off, 0, 2);
}
__device__ __forceinline__ void bst1(__amdgpu_buffer_rsrc_t r, int off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 2);
}

// One chunk of B's key rows (128 c .. + 127, the head's hd columns) on its
// way to LDS [row][k]: float4 loads along the rows, NSL per thread (rows
// row0 + (256 / F4) i, all at the same k), held in registers while the
// matrix cores work.  Rows past Sk read 0 (the descriptor ends at the last
// key row); k past hd, which would read the next head's columns, is zeroed
// on the way to LDS.
template <int KS>
struct KeyChunk {
    static constexpr int PK = 32 * KS + 4;          // LDS pitch of a key row (floats)
    static constexpr int F4 = 8 * KS;               // float4s of a key row
    static constexpr int NSL = kHChunk * F4 / 256;  // float4s per thread
    static constexpr int RSTEP = 256 / F4;          // rows between a thread's slots
    float4 v[NSL];

    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int off0, int64_t E, int c) {
#pragma unroll
        for (int i = 0; i < NSL; ++i) v[i] = bld4(r, off0 + (int)(((int64_t)c * kHChunk + RSTEP * i) * E * 4));
    }
    __device__ __forceinline__ void store(float* dst, bool kin) const {
        const int t = (int)threadIdx.x;
#pragma unroll
        for (int i = 0; i < NSL; ++i)
            *reinterpret_cast<float4*>(dst + (t / F4 + RSTEP * i) * PK + 4 * (t % F4)) =
                make_float4(kin ? v[i].x : 0.f, kin ? v[i].y : 0.f, kin ? v[i].z : 0.f, kin ? v[i].w : 0.f);
    }
};

// NB: 128-column chunks of the rows (NB * 128 >= Sk); KS: 32-wide k stages
// (32 * KS >= hd, the rest zero-filled); VEC: Sk % 4 == 0 with 16-byte
// aligned mask / attn / out, so row segments move as float4.
//
// After quad_transpose, block j's group g (accumulator elements 4 g .. 4 g
// + 3) holds row 8 g + 4 half + lane % 4 of the workgroup's rows, columns
// 128 j + 32 w + 4 (r / 4) .. + 3: a store instruction writes 8 rows x 128
// contiguous bytes.  Block j's vector work (transpose, scale and mask in the
// forward, the whole of d_scores in the backward) runs while the matrix
// cores compute block j + 1.  Columns past Sk are never stored; where a load
// of them stays inside the row tile it reads the next row's values, which
// the forward replaces by -inf and the backward never stores.
template <int NB, int KS, bool BWD, bool VEC>
__global__ void __launch_bounds__(256) head_rows_kernel(HeadRows P) {
    constexpr int PK = KeyChunk<KS>::PK;
    __shared__ __attribute__((aligned(16))) float lds[2][kHChunk * PK];  // B chunks
    __shared__ __attribute__((aligned(16))) float alds[kHRows * PK];      // the A tile
    __shared__ __attribute__((aligned(16))) float red[2][4][kHRows];

    // Workgroups are dealt to the 8 XCDs in turn; renumber them so each XCD
    // takes whole heads, whose B rows its L2 then holds for every row tile.
    int t = (int)blockIdx.x;
    if ((P.tiles & 7) == 0) t = (t & 7) * (P.tiles >> 3) + (t >> 3);
    const int64_t bh = t / P.row_tiles;
    const int64_t i0 = (int64_t)(t - bh * P.row_tiles) * kHRows;
    const int64_t bb = bh / P.H, hh = bh - bb * P.H;
    const int64_t nrows = min((int64_t)kHRows, P.Sq - i0);  // valid rows of this tile
    const int lane = (int)threadIdx.x & 63, w = (int)threadIdx.x >> 6;
    const int half = lane >> 5, r = lane & 31, qb = lane & 3, qa = r >> 2;

    // A fragments: row i0 + r, k = 32 st + 16 half + 4 kq .. + 3 (rows past
    // Sq read 0; k past hd is zeroed).
    const int64_t a0 = (bb * P.Sq + i0) * P.E + hh * P.hd;
    const int64_t abytes = ((nrows - 1) * P.E + P.hd) * 4;
    const __amdgpu_buffer_rsrc_t rA = buf(P.a + a0, abytes);
    const int aoff = (int)((r * P.E + 16 * half) * 4);
    float4 af[KS][4];
#pragma unroll
    for (int st = 0; st < KS; ++st)
#pragma unroll
        for (int kq = 0; kq < 4; ++kq) af[st][kq] = bld4(rA, aoff + (32 * st + 4 * kq) * 4);
    if constexpr (BWD) {
        // dot of row i0 + r: this half's terms, then the other half's.
        const __amdgpu_buffer_rsrc_t rC = buf(P.ctx + a0, abytes);
        float d = 0.f;
#pragma unroll
        for (int st = 0; st < KS; ++st)
#pragma unroll
            for (int kq = 0; kq < 4; ++kq) {
                const float4 c4 = bld4(rC, aoff + (32 * st + 4 * kq) * 4);
                if (32 * st + 16 * half + 4 * kq < P.hd) {
                    d += af[st][kq].x * c4.x;
                    d += af[st][kq].y * c4.y;
                    d += af[st][kq].z * c4.z;
                    d += af[st][kq].w * c4.w;
                }
            }
        d += __shfl_xor(d, 32);
        if (w == 0 && half == 0) red[0][0][r] = d;  // read after the first barrier
    }
#pragma unroll
    for (int st = 0; st < KS; ++st)
#pragma unroll
        for (int kq = 0; kq < 4; ++kq)
            if (32 * st + 16 * half + 4 * kq >= P.hd) af[st][kq] = make_float4(0.f, 0.f, 0.f, 0.f);

    const __amdgpu_buffer_rsrc_t rB =
        buf(P.b + bb * P.Sk * P.E + hh * P.hd, ((P.Sk - 1) * P.E + P.hd) * 4);
    const int bk = 4 * ((int)threadIdx.x % KeyChunk<KS>::F4);
    const int boff = (int)(((int)threadIdx.x / KeyChunk<KS>::F4) * P.E * 4) + bk * 4;
    const bool bkin = bk < P.hd;
    // Staging for B chunks: the forward (whose accumulators hold whole rows)
    // loads one chunk ahead; the backward two, from alternate register sets.
    KeyChunk<KS> kc[BWD ? 2 : 1];
    kc[0].load(rB, boff, P.E, 0);
    if constexpr (BWD) {
        if (P.nch > 1) kc[1].load(rB, boff, P.E, 1);
    }
    kc[0].store(lds[0], bkin);
    // The A fragments go to LDS (re-read per chunk), which frees their
    // registers for the loads in flight.
    if (w == 0)
#pragma unroll
        for (int st = 0; st < KS; ++st)
#pragma unroll
            for (int kq = 0; kq < 4; ++kq)
                *reinterpret_cast<float4*>(alds + r * PK + 32 * st + 16 * half + 4 * kq) = af[st][kq];
    __syncthreads();

    // This lane's transposed values: group g of block j is row
    // 8 g + 4 half + qb of the tile, columns 128 j + 32 w + 4 qa .. + 3,
    // at byte offset so(g) + 512 j of the tile's [rows, Sk] slab.
    const int64_t orow = bh * P.Sq + i0;  // first output row of this tile
    const int64_t tbytes = nrows * P.Sk * 4;
    const __amdgpu_buffer_rsrc_t rO = buf(P.out + orow * P.Sk, tbytes);
    const float* side = BWD ? P.attn + orow * P.Sk : (P.mask ? P.mask + bb * P.mstride + i0 * P.Sk : nullptr);
    const __amdgpu_buffer_rsrc_t rS = buf(side ? side : P.out, tbytes);
    const int so0 = (int)(((4 * half + qb) * P.Sk + 32 * w + 4 * qa) * 4);
    const int sog = (int)(8 * P.Sk * 4);
    const int64_t cl = 32 * w + 4 * qa;  // column of block 0

    auto load_side = [&](int j, float4 (&dst)[4]) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int off = so0 + g * sog + 512 * j;
            if constexpr (VEC) {
                dst[g] = BWD ? bld4<2>(rS, off) : bld4<0>(rS, off);
            } else {
                dst[g] = make_float4(bld1(rS, off), bld1(rS, off + 4), bld1(rS, off + 8), bld1(rS, off + 12));
            }
        }
    };
    auto store_out = [&](int j, int g, float4 o) {
        const int off = so0 + g * sog + 512 * j;
        const int64_t c0 = cl + (int64_t)j * kHChunk;
        if constexpr (VEC) {
            if (c0 < P.Sk) bst4(rO, off, o);
        } else {
            if (c0 < P.Sk) bst1(rO, off, o.x);
            if (c0 + 1 < P.Sk) bst1(rO, off + 4, o.y);
            if (c0 + 2 < P.Sk) bst1(rO, off + 8, o.z);
            if (c0 + 3 < P.Sk) bst1(rO, off + 12, o.w);
        }
    };

    f32x16 acc[BWD ? 2 : NB];
    float4 sd[2][4];  // side values of block j (slot j & 1)
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    float dt[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (BWD) {
#pragma unroll
        for (int g = 0; g < 4; ++g) dt[g] = red[0][0][8 * g + 4 * half + qb];
    }

    // Block j's vector work once its products (in a) are done; sv4 holds its
    // mask or attn values.
    auto finish_block = [&](int j, f32x16& a, const float4 (&sv4)[4]) {
        const int64_t c0 = cl + (int64_t)j * kHChunk;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float4 x = quad_transpose(f4_of(a, g));
            const float4 sv = sv4[g];
            if constexpr (BWD) {
                // d_scores = attn * (dattn - dot)
                store_out(j, g, make_float4(sv.x * (x.x - dt[g]), sv.y * (x.y - dt[g]), sv.z * (x.z - dt[g]),
                                            sv.w * (x.w - dt[g])));
            } else {
                x = make_float4(x.x * P.scale, x.y * P.scale, x.z * P.scale, x.w * P.scale);
                if (side) x = make_float4(x.x + sv.x, x.y + sv.y, x.z + sv.z, x.w + sv.w);
                x.x = c0 < P.Sk ? x.x : -INFINITY;
                x.y = c0 + 1 < P.Sk ? x.y : -INFINITY;
                x.z = c0 + 2 < P.Sk ? x.z : -INFINITY;
                x.w = c0 + 3 < P.Sk ? x.w : -INFINITY;
                set_f4(a, g, x);
                mx[g] = fmaxf(fmaxf(fmaxf(mx[g], x.x), fmaxf(x.y, x.z)), x.w);
            }
        }
    };

    // One chunk's products into a, from LDS buffer buf.
    auto mma = [&](f32x16& a, const float* buf) {
#pragma unroll
        for (int q = 0; q < 16; ++q) a[q] = 0.0f;
        const float* As = alds + r * PK + 16 * half;
        const float* Bs = buf + (32 * w + r) * PK + 16 * half;
#pragma unroll
        for (int st = 0; st < KS; ++st)
#pragma unroll
            for (int kq = 0; kq < 4; ++kq) {
                const float4 av = *reinterpret_cast<const float4*>(As + 32 * st + 4 * kq);
                const float4 bv = *reinterpret_cast<const float4*>(Bs + 32 * st + 4 * kq);
                a = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, bv.x, a, 0, 0, 0);
                a = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, bv.y, a, 0, 0, 0);
                a = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, bv.z, a, 0, 0, 0);
                a = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, bv.w, a, 0, 0, 0);
            }
    };

    if constexpr (BWD) {
        // Any number of chunks: two blocks live, the step for chunk c
        // specialised on c's parity (the accumulator, side slot, register
        // set and LDS buffer it uses).
        auto step = [&](auto parity, int c) {
            constexpr int S = decltype(parity)::value;
            const bool more = c + 1 < P.nch;
            if (c + 2 < P.nch) kc[S].load(rB, boff, P.E, c + 2);
            // block c's attn values, used once its products are done (in
            // the next chunk)
            load_side(c, sd[S]);
            __builtin_amdgcn_sched_barrier(0);  // the loads go out before the products
            mma(acc[S], lds[S]);
            if (c > 0) finish_block(c - 1, acc[S ^ 1], sd[S ^ 1]);
            if (!more) finish_block(c, acc[S], sd[S]);
            if (more) kc[S ^ 1].store(lds[S ^ 1], bkin);
            __syncthreads();
        };
        for (int c = 0; c < P.nch; c += 2) {
            step(std::integral_constant<int, 0>{}, c);
            if (c + 1 < P.nch) step(std::integral_constant<int, 1>{}, c + 1);
        }
        return;
    } else {
#pragma unroll
        for (int c = 0; c < NB; ++c) {
            if (c < P.nch) {
                const bool more = c + 1 < P.nch;
                if (more) kc[0].load(rB, boff, P.E, c + 1);
                // block c's mask values, added once its products are done
                // (in the next chunk)
                if (side) load_side(c, sd[c & 1]);
                __builtin_amdgcn_sched_barrier(0);  // the loads go out before the products
                mma(acc[c], lds[c & 1]);
                if (c > 0) finish_block(c - 1, acc[c - 1], sd[(c - 1) & 1]);
                if (!more) finish_block(c, acc[c], sd[c & 1]);
                if (more) kc[0].store(lds[(c + 1) & 1], bkin);
                __syncthreads();
            }
        }
    }

    // Forward: the row maxima, the exponentials and their sums, the weights.
#pragma unroll
    for (int g = 0; g < 4; ++g) mx[g] = rows_max(mx[g]);
    if (qa == 0)
#pragma unroll
        for (int g = 0; g < 4; ++g) red[0][w][8 * g + 4 * half + qb] = mx[g];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int rr = 8 * g + 4 * half + qb;
        // max_val starts at -FLT_MAX (core/layer.cpp:1215); fmaxf skips NaN as std::max does there
        mx[g] = fmaxf(fmaxf(fmaxf(red[0][0][rr], red[0][1][rr]), fmaxf(red[0][2][rr], red[0][3][rr])), -FLT_MAX);
    }
    float sm[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        if (j >= P.nch) break;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float4 x = f4_of(acc[j], g);  // columns past Sk: exp(-inf) = 0
            x = make_float4(exp_rr(x.x - mx[g]), exp_rr(x.y - mx[g]), exp_rr(x.z - mx[g]), exp_rr(x.w - mx[g]));
            sm[g] += x.x;
            sm[g] += x.y;
            sm[g] += x.z;
            sm[g] += x.w;
            set_f4(acc[j], g, x);
        }
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) sm[g] = rows_sum(sm[g]);
    if (qa == 0)
#pragma unroll
        for (int g = 0; g < 4; ++g) red[1][w][8 * g + 4 * half + qb] = sm[g];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int rr = 8 * g + 4 * half + qb;
        sm[g] = 1.0f / ((red[1][0][rr] + red[1][1][rr]) + (red[1][2][rr] + red[1][3][rr]));
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        if (j >= P.nch) break;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const float4 e = f4_of(acc[j], g);
            store_out(j, g, make_float4(e.x * sm[g], e.y * sm[g], e.z * sm[g], e.w * sm[g]));
        }
    }
}

// Whether the fused kernels take this shape: keys and head width within
// the register tile, float4 operand rows, every operand 16-byte aligned.
bool head_rows_fit(const MhaDims& d, int64_t max_keys, std::initializer_list<const void*> ptrs) {
    if (!g_fused.load(std::memory_order_relaxed)) return false;
    if (d.Sk < 1 || d.Sk > max_keys || d.hd < 1 || d.hd > kHMaxWidth || d.hd % 4 != 0 || d.E % 4 != 0)
        return false;
    const int64_t tiles = (d.Sq + kHRows - 1) / kHRows * d.B * d.H;
    if (tiles > INT_MAX) return false;
    // 32-bit byte offsets into a head's key rows (every chunk, padding
    // included) and into a row tile's [32, Sk] slab
    if ((d.Sk + kHChunk) * d.E * 4 > INT_MAX || (int64_t)kHRows * d.Sk * 4 > INT_MAX) return false;
    for (const void* p : ptrs)
        if (!aligned16(p)) return false;
    return true;
}

// One workgroup per 32 query rows of each (batch, head); BH = batch * heads.
template <bool BWD>
int launch_head_rows(HeadRows P, int64_t BH, const char* who) {
    P.row_tiles = (int)((P.Sq + kHRows - 1) / kHRows);
    P.tiles = (int)(P.row_tiles * BH);
    P.nch = (int)((P.Sk + kHChunk - 1) / kHChunk);
    // the forward's accumulators hold whole rows (NB chunks); the backward
    // loops over any number of chunks
    const int nb = BWD || P.nch <= 1 ? 1 : P.nch <= 2 ? 2 : P.nch <= 4 ? 4 : 8;
    const int ks = P.hd <= 32 ? 1 : P.hd <= 64 ? 2 : 4;
    const dim3 grid((unsigned)P.tiles), block(256);
    hipStream_t st = stream();
    const bool vec = P.Sk % 4 == 0 && aligned16(P.out) && aligned16(BWD ? P.attn : P.mask);
#define WM_HR(NBv, KSv)                                                                          \
    if constexpr (!BWD || NBv == 1) {                                                            \
        if (nb == NBv && ks == KSv) {                                                            \
            if (vec)                                                                             \
                launch_kernel((head_rows_kernel<NBv, KSv, BWD, true>), grid, block, 0, st, P);   \
            else                                                                                 \
                launch_kernel((head_rows_kernel<NBv, KSv, BWD, false>), grid, block, 0, st, P);  \
            return check_launch(who);                                                            \
        }                                                                                        \
    }
    WM_HR(1, 1) WM_HR(1, 2) WM_HR(1, 4) WM_HR(2, 1) WM_HR(2, 2) WM_HR(2, 4)
    WM_HR(4, 1) WM_HR(4, 2) WM_HR(4, 4) WM_HR(8, 1) WM_HR(8, 2) WM_HR(8, 4)
#undef WM_HR
    return set_error(WM_ERR_INVALID, std::string(who) + ": no tile");
}

int check_dims(const MhaDims& d, const char* who) {
    if (d.B < 0 || d.Sq < 0 || d.Sk < 0 || d.E < 0 || d.H < 1)
        return set_error(WM_ERR_INVALID, std::string(who) + ": negative extent or no heads");
    if (d.E % d.H != 0) return set_error(WM_ERR_INVALID, std::string(who) + ": embed_dim % num_heads != 0");
    return WM_OK;
}

// y [rows, E] = x [rows, E] W^T + bias (W [E, E], row = output feature).
int project(const float* x, const float* W, const float* bias, int64_t rows, int64_t E, float* y) {
    return wm_gemm(0, 1, rows, E, E, 1.0f, x, E, W, E, y, E, 0, bias, 1, 1, nullptr);
}

// gb [E] += column sums of dy [rows, E] (the broadcast add's backward).
int bias_grad(const float* dy, int64_t rows, int64_t E, float* gb) {
    const int64_t ys[2] = {rows, E}, bs[1] = {E};
    return wm_binary_bwd(WM_ADD, dy, dy, ys, 2, gb, bs, 1, nullptr, nullptr, 0, gb, 1);
}

}  // namespace
}  // namespace wm

using namespace wm;

int wm_mha_fwd(const float* q, const float* k, const float* v, const float* mask, int64_t mask_batches,
               const float* Wq, const float* Wk, const float* Wv, const float* Wo, const float* bq, const float* bk,
               const float* bv, const float* bo, int64_t batch, int64_t seq_q, int64_t seq_k, int64_t embed,
               int64_t heads, float* out, float* attn, float* Q, float* K, float* V, float* ctx) {
    const MhaDims d{batch, seq_q, seq_k, embed, heads, heads > 0 ? embed / heads : 0};
    WM_TRY(check_dims(d, "wm_mha_fwd"));
    if (d.B == 0 || d.Sq == 0 || d.E == 0) return WM_OK;
    if (mask && mask_batches != 1 && mask_batches != d.B)
        return set_error(WM_ERR_INVALID, "wm_mha_fwd: mask batch must be 1 or the batch size");
    if (!q || !k || !v || !Wq || !Wk || !Wv || !Wo || !bq || !bk || !bv || !bo || !out || !attn || !Q || !K || !V ||
        !ctx)
        return set_error(WM_ERR_INVALID, "wm_mha_fwd: null pointer");
    WM_CHECK_INIT();
    const float scale = 1.0f / std::sqrt((float)d.hd);  // layer.cpp:1178
    WM_TRY(project(q, Wq, bq, d.B * d.Sq, d.E, Q));
    WM_TRY(project(k, Wk, bk, d.B * d.Sk, d.E, K));
    WM_TRY(project(v, Wv, bv, d.B * d.Sk, d.E, V));
    if (d.Sk > 0 && head_rows_fit(d, kHMaxKeys, {Q, K, V})) {
        // attn[b, h] = softmax(Q_h K_h^T * scale + mask) in one pass
        HeadRows P{};
        P.a = Q;
        P.b = K;
        P.mask = mask;
        P.out = attn;
        P.Sq = d.Sq, P.Sk = d.Sk, P.E = d.E, P.H = d.H, P.hd = d.hd;
        P.mstride = mask && mask_batches != 1 ? d.Sq * d.Sk : 0;
        P.scale = scale;
        WM_TRY(launch_head_rows<false>(P, d.B * d.H, "wm_mha_fwd(scores)"));
    } else if (d.Sk > 0) {
        // scores[b, h] = Q_h K_h^T * scale, one problem per (b, h)
        Workspace scores((size_t)(d.B * d.H * d.Sq * d.Sk) * sizeof(float));
        const int64_t st[6] = {d.Sq * d.E, d.hd, d.Sk * d.E, d.hd, d.H * d.Sq * d.Sk, d.Sq * d.Sk};
        WM_TRY(wm_gemm(0, 1, d.Sq, d.Sk, d.hd, scale, Q, d.E, K, d.E, scores.as<float>(), d.Sk, 0, nullptr,
                       d.B * d.H, d.H, st));
        WM_TRY(wm_attention_softmax_fwd(scores.as<float>(), mask, mask ? mask_batches : 0, d.B, d.H, d.Sq, d.Sk,
                                        attn));
    }
    // ctx[b, :, h] = attn[b, h] V_h
    const int64_t sc[6] = {d.H * d.Sq * d.Sk, d.Sq * d.Sk, d.Sk * d.E, d.hd, d.Sq * d.E, d.hd};
    WM_TRY(wm_gemm(0, 0, d.Sq, d.hd, d.Sk, 1.0f, attn, std::max<int64_t>(d.Sk, 1), V, d.E, ctx, d.E, 0, nullptr,
                   d.B * d.H, d.H, sc));
    return project(ctx, Wo, bo, d.B * d.Sq, d.E, out);
}

int wm_mha_bwd(const float* dout, const float* q, const float* k, const float* v, const float* Wq, const float* Wk,
               const float* Wv, const float* Wo, const float* Q, const float* K, const float* V, const float* attn,
               const float* ctx, int64_t batch, int64_t seq_q, int64_t seq_k, int64_t embed, int64_t heads,
               float* gWq, float* gWk, float* gWv, float* gWo, float* gbq, float* gbk, float* gbv, float* gbo,
               float* gq, float* gk, float* gv) {
    const MhaDims d{batch, seq_q, seq_k, embed, heads, heads > 0 ? embed / heads : 0};
    WM_TRY(check_dims(d, "wm_mha_bwd"));
    if (d.B == 0 || d.Sq == 0 || d.E == 0) return WM_OK;
    if (!dout || !q || !k || !v || !Wq || !Wk || !Wv || !Wo || !Q || !K || !V || !attn || !ctx || !gWq || !gWk ||
        !gWv || !gWo || !gbq || !gbk || !gbv || !gbo)
        return set_error(WM_ERR_INVALID, "wm_mha_bwd: null pointer");
    WM_CHECK_INIT();
    const float scale = 1.0f / std::sqrt((float)d.hd);
    const int64_t Rq = d.B * d.Sq, Rk = d.B * d.Sk, E = d.E;
    // output projection (:1305-1318): gbo += sum dout; gWo += dout^T ctx; dctx = dout Wo
    WM_TRY(bias_grad(dout, Rq, E, gbo));
    WM_TRY(wm_gemm(1, 0, E, E, Rq, 1.0f, dout, E, ctx, E, gWo, E, 1, nullptr, 1, 1, nullptr));
    Workspace dctx((size_t)(Rq * E) * sizeof(float));
    WM_TRY(wm_gemm(0, 0, Rq, E, E, 1.0f, dout, E, Wo, E, dctx.as<float>(), E, 0, nullptr, 1, 1, nullptr));
    Workspace dV((size_t)(Rk * E) * sizeof(float));
    Workspace dK((size_t)(Rk * E) * sizeof(float));
    Workspace dQ((size_t)(Rq * E) * sizeof(float));
    if (d.Sk > 0) {
        const size_t n_att = (size_t)(d.B * d.H * d.Sq * d.Sk);
        Workspace ds(n_att * sizeof(float));
        // attn @ V (:1320-1339): dV_h = attn_h^T dctx_h; dattn_h = dctx_h V_h^T
        const int64_t s2[6] = {d.H * d.Sq * d.Sk, d.Sq * d.Sk, d.Sq * E, d.hd, d.Sk * E, d.hd};
        WM_TRY(wm_gemm(1, 0, d.Sk, d.hd, d.Sq, 1.0f, attn, d.Sk, dctx.as<float>(), E, dV.as<float>(), E, 0, nullptr,
                       d.B * d.H, d.H, s2));
        if (head_rows_fit(d, INT64_MAX, {dctx.p, V, ctx})) {
            // dattn and the softmax's backward (:1341-1360) in one pass
            HeadRows P{};
            P.a = dctx.as<float>();
            P.b = V;
            P.attn = attn;
            P.ctx = ctx;
            P.out = ds.as<float>();
            P.Sq = d.Sq, P.Sk = d.Sk, P.E = d.E, P.H = d.H, P.hd = d.hd;
            P.scale = 1.0f;
            WM_TRY(launch_head_rows<true>(P, d.B * d.H, "wm_mha_bwd(scores)"));
        } else {
            Workspace dattn(n_att * sizeof(float));
            const int64_t s1[6] = {d.Sq * E, d.hd, d.Sk * E, d.hd, d.H * d.Sq * d.Sk, d.Sq * d.Sk};
            WM_TRY(wm_gemm(0, 1, d.Sq, d.Sk, d.hd, 1.0f, dctx.as<float>(), E, V, E, dattn.as<float>(), d.Sk, 0,
                           nullptr, d.B * d.H, d.H, s1));
            // softmax (:1341-1360)
            WM_TRY(wm_attention_softmax_bwd(attn, dattn.as<float>(), d.B * d.H * d.Sq, d.Sk, ds.as<float>()));
        }
        // Q K^T (:1362-1383): dQ_h = scale ds_h K_h; dK_h = scale ds_h^T Q_h
        const int64_t s3[6] = {d.H * d.Sq * d.Sk, d.Sq * d.Sk, d.Sk * E, d.hd, d.Sq * E, d.hd};
        WM_TRY(wm_gemm(0, 0, d.Sq, d.hd, d.Sk, scale, ds.as<float>(), d.Sk, K, E, dQ.as<float>(), E, 0, nullptr,
                       d.B * d.H, d.H, s3));
        const int64_t s4[6] = {d.H * d.Sq * d.Sk, d.Sq * d.Sk, d.Sq * E, d.hd, d.Sk * E, d.hd};
        WM_TRY(wm_gemm(1, 0, d.Sk, d.hd, d.Sq, scale, ds.as<float>(), d.Sk, Q, E, dK.as<float>(), E, 0, nullptr,
                       d.B * d.H, d.H, s4));
    } else {
        // no keys: the context is zero and so are dV, dK and dQ
        WM_TRY(wm_fill(dQ.as<float>(), 0.0f, Rq * E));
    }
    // V, K, Q projections (:1385-1433): gb += sum dY; gW += dY^T x; gx += dY W
    struct Proj {
        const float* dY;
        const float* x;
        const float* W;
        float *gW, *gb, *gx;
        int64_t rows;
    };
    const Proj proj[3] = {{dV.as<float>(), v, Wv, gWv, gbv, gv, Rk},
                          {dK.as<float>(), k, Wk, gWk, gbk, gk, Rk},
                          {dQ.as<float>(), q, Wq, gWq, gbq, gq, Rq}};
    for (const Proj& p : proj) {
        if (p.rows == 0) continue;
        WM_TRY(bias_grad(p.dY, p.rows, E, p.gb));
        WM_TRY(wm_gemm(1, 0, E, E, p.rows, 1.0f, p.dY, E, p.x, E, p.gW, E, 1, nullptr, 1, 1, nullptr));
        if (p.gx) WM_TRY(wm_gemm(0, 0, p.rows, E, E, 1.0f, p.dY, E, p.W, E, p.gx, E, 1, nullptr, 1, 1, nullptr));
    }
    return WM_OK;
}

int wm_mha_fused(int mode) {
    if (mode == 0 || mode == 1) g_fused.store(mode, std::memory_order_relaxed);
    return g_fused.load(std::memory_order_relaxed);
}
