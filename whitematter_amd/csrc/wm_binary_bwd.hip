// Backward of the broadcast binary ops, including the reduction of each
// broadcast operand's gradient over the dims it was repeated along.
//
// The reference closures (core/tensor.cpp:956-976 and the same loop in
// sub/mul/div/pow/max/min) walk the output in row-major order and scatter
// "grad[src_idx] += contribution" one element at a time.  Here the output is
// folded to the fewest dims (as in the forward) and three layouts get their
// own kernels:
//   flat    both operands have the output's shape: one fused elementwise pass;
//   colsum  one operand is full [R,C], the other a row vector [1,C]: column
//           tiles x row chunks, per-column partial sums in registers, then a
//           fixed-order second pass (c1 bias grad, c2 r.grad, c5 g.grad);
//   rowsum  one operand is full, the other a column vector [R,1] (or a
//           scalar): one wave per (row, column chunk), DPP wave reduction,
//           then a fixed-order second pass when a row is split (c2 c.grad).
// Everything else goes through a generic kernel: one thread per operand
// element, summing its contributions in the reference's row-major order.
// Every path is deterministic: no atomics, fixed partition, fixed order.
#include "wm_ops.hpp"

#include <algorithm>

namespace wm {

int make_bcast_layout_public(const int64_t* as, int an, const int64_t* bs, int bn, int& nd, int64_t* size,
                             int64_t* sa, int64_t* sb, int64_t& numel);

constexpr int kBlock = 256;
constexpr int kSlotsFlat = 1;  // float4s per thread in bwd_flat_kernel

// ---------------------------------------------------------------------------
// flat: same shape
// ---------------------------------------------------------------------------

template <int OP>
__global__ void __launch_bounds__(kBlock) bwd_flat_kernel(const float* __restrict__ g, const float* __restrict__ a,
                                                           const float* __restrict__ b, const float* __restrict__ o,
                                                           float* __restrict__ ga, int acc_a, float* __restrict__ gb,
                                                           int acc_b, int64_t n4) {
    binary_prologue<OP>();
    const bool need_a = (ga && da_reads_a<OP>()) || (gb && db_reads_a<OP>());
    const bool need_b = (ga && da_reads_b<OP>()) || (gb && db_reads_b<OP>()) || (gb && db_reads_out<OP>() && !o);
    const bool need_o = gb && db_reads_out<OP>() && o;
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    // One float4 per thread on a grid that covers the tensor: measured 71 ->
    // 79 % of the HBM peak against 4 float4s per thread on 32 workgroups
    // per CU (the loop stays grid-stride for very large tensors).
    constexpr int kSlots = kSlotsFlat;
    const int64_t stride = (int64_t)gridDim.x * kBlock * kSlots;
    for (int64_t i0 = (int64_t)blockIdx.x * kBlock * kSlots + threadIdx.x; i0 < n4; i0 += stride) {
        float4 vg[kSlots], va[kSlots], vb[kSlots], vo[kSlots], oa[kSlots], ob[kSlots];
#pragma unroll
        for (int u = 0; u < kSlots; ++u) {
            const int64_t i = i0 + (int64_t)u * kBlock;
            const bool in = i < n4;
            const int64_t e = 4 * i;
            vg[u] = in ? ld_stream(g + e) : z;
            va[u] = in && need_a ? ld_stream(a + e) : z;
            vb[u] = in && need_b ? ld_stream(b + e) : z;
            vo[u] = in && need_o ? ld_stream(o + e) : z;
            oa[u] = in && ga && acc_a ? ld_stream(ga + e) : z;
            ob[u] = in && gb && acc_b ? ld_stream(gb + e) : z;
        }
#pragma unroll
        for (int u = 0; u < kSlots; ++u) {
            const int64_t i = i0 + (int64_t)u * kBlock;
            if (i >= n4) continue;
            const int64_t e = 4 * i;
            const float eg[4] = {vg[u].x, vg[u].y, vg[u].z, vg[u].w}, ea[4] = {va[u].x, va[u].y, va[u].z, va[u].w},
                        eb[4] = {vb[u].x, vb[u].y, vb[u].z, vb[u].w}, eo[4] = {vo[u].x, vo[u].y, vo[u].z, vo[u].w};
            float da[4], db[4];
            binary_grads_n<OP, 4>(eg, ea, eb, eo, need_o, ga != nullptr, gb != nullptr, da, db);
            if (ga) {
                float4 r = make_float4(da[0], da[1], da[2], da[3]);
                if (acc_a) { r.x += oa[u].x; r.y += oa[u].y; r.z += oa[u].z; r.w += oa[u].w; }
                st_stream(ga + e, r);
            }
            if (gb) {
                float4 r = make_float4(db[0], db[1], db[2], db[3]);
                if (acc_b) { r.x += ob[u].x; r.y += ob[u].y; r.z += ob[u].z; r.w += ob[u].w; }
                st_stream(gb + e, r);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// colsum: F full [R,C], V row vector [1,C]; C % 4 == 0, 16-byte aligned
// ---------------------------------------------------------------------------

// One thread owns 4 adjacent columns of one column tile.  Row group k
// (blockIdx.y, of K = gridDim.y) takes rows k, k + K, k + 2K, ...: at any
// moment the resident workgroups read a narrow band of adjacent rows that
// advances down the matrix, which measured 4-5 points of the HBM peak faster
// than giving each group a contiguous block of R/K rows (every group then
// reads its own distant row).  The partial of group k is a sum in a fixed
// order, so results stay deterministic.  VB: the vector operand is b (else a).
template <int OP, bool VB>
__global__ void __launch_bounds__(kBlock) bwd_colsum_kernel(const float* __restrict__ g, const float* __restrict__ F,
                                                             const float* __restrict__ V, const float* __restrict__ o,
                                                             float* __restrict__ gF, int accF, float* __restrict__ part,
                                                             int64_t R, int64_t C) {
    binary_prologue<OP>();
    const int64_t c = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * 4;
    if (c >= C) return;
    const bool want_v = part != nullptr;
    // Which tensors the contributions read.
    const bool gF_reads_F = VB ? da_reads_a<OP>() : db_reads_b<OP>();
    const bool gF_reads_V = VB ? da_reads_b<OP>() : db_reads_a<OP>();
    const bool gV_reads_F = VB ? db_reads_a<OP>() : da_reads_b<OP>();
    const bool gV_reads_V = VB ? db_reads_b<OP>() : da_reads_a<OP>();
    const bool want_o = VB ? (want_v && db_reads_out<OP>()) : (gF && db_reads_out<OP>());
    const bool need_o = want_o && o;
    const bool need_F = (gF && gF_reads_F) || (want_v && gV_reads_F) || (want_o && !o);
    const bool need_V = (gF && gF_reads_V) || (want_v && gV_reads_V) || (want_o && !o);
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 vv = need_V ? *reinterpret_cast<const float4*>(V + c) : z;
    float4 s = z;
    // a / b with b the row vector: each column's divisor is fixed, so the
    // gradients multiply by its reciprocal (g / b -> g * q, g a / b^2 ->
    // g a q q; a few ulp, within the gradients' 1e-5) instead of dividing twice per
    // element, when |b| is in [2^-62, 2^62], where neither q nor q * q can
    // overflow or underflow.  Other divisors (zero, infinite, NaN, tiny,
    // huge) keep the divisions.
    float q[4] = {0.f, 0.f, 0.f, 0.f};
    bool rcp = false;
    if constexpr (OP == WM_DIV && VB) {
        const float bv4[4] = {vv.x, vv.y, vv.z, vv.w};
        rcp = true;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float m = fabsf(bv4[j]);
            rcp = rcp && m >= 0x1p-62f && m <= 0x1p62f;
            q[j] = 1.0f / bv4[j];
        }
    }
    // One row per iteration (several rows' loads in flight per thread
    // measured slower than one; more workgroups carry the memory-level
    // parallelism instead).
#pragma unroll 1
    for (int64_t r = blockIdx.y; r < R; r += gridDim.y) {
        const int64_t off = r * C + c;
        float4 vg = ld_stream(g + off);
        float4 vf = need_F ? ld_stream(F + off) : z;
        float4 vo = need_o ? ld_stream(o + off) : z;
        float4 old = (gF && accF) ? ld_stream(gF + off) : z;
        const float4 av = VB ? vf : vv, bv = VB ? vv : vf;
        const float eg[4] = {vg.x, vg.y, vg.z, vg.w}, ea[4] = {av.x, av.y, av.z, av.w},
                    eb[4] = {bv.x, bv.y, bv.z, bv.w}, eo[4] = {vo.x, vo.y, vo.z, vo.w};
        float da[4], db[4];
        if (OP == WM_DIV && VB && rcp) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                da[j] = eg[j] * q[j];
                db[j] = -((eg[j] * ea[j]) * q[j] * q[j]);
            }
        } else {
            binary_grads_n<OP, 4>(eg, ea, eb, eo, need_o, VB ? gF != nullptr : want_v, VB ? want_v : gF != nullptr,
                                  da, db);
        }
        const float* dF = VB ? da : db;
        const float* dV = VB ? db : da;
        if (gF) {
            float4 d = make_float4(dF[0], dF[1], dF[2], dF[3]);
            if (accF) { d.x += old.x; d.y += old.y; d.z += old.z; d.w += old.w; }
            st_stream(gF + off, d);
        }
        if (want_v) { s.x += dV[0]; s.y += dV[1]; s.z += dV[2]; s.w += dV[3]; }
    }
    if (want_v) *reinterpret_cast<float4*>(part + (int64_t)blockIdx.y * C + c) = s;
}

// out[c] (+)= sum_k part[k, c], k in 0..K-1.  A workgroup owns S adjacent
// columns and its threads form G = 256 / S groups: group g folds partial
// rows k = g, g + G, g + 2G, ... (8 interleaved accumulators, combined in a
// fixed order), and the G group sums are added in group order through LDS.
// S is chosen so the grid has ~256 workgroups or more: with few columns
// and many partial rows (a Linear bias gradient, 1024 columns over 1024
// row groups) 64-column workgroups left 16 workgroups each walking 256
// rows per wave (13.6 us).
template <int S>
__global__ void __launch_bounds__(kBlock) colsum_finalize_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                                  int acc, int64_t K, int64_t C) {
    constexpr int G = kBlock / S;
    __shared__ float lds[G][S];
    const int cl = threadIdx.x % S, g = threadIdx.x / S;
    for (int64_t c0 = (int64_t)blockIdx.x * S; c0 < C; c0 += (int64_t)gridDim.x * S) {
        const int64_t c = c0 + cl;
        float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (c < C) {
            int64_t k = g;
            for (; k + 7 * G < K; k += 8 * G) {
#pragma unroll
                for (int j = 0; j < 8; ++j) s[j] += part[(k + j * G) * C + c];
            }
            for (int j = 0; k < K; k += G, ++j) s[j & 7] += part[k * C + c];
        }
        lds[g][cl] = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
        __syncthreads();
        if (g == 0 && c < C) {
            float t = lds[0][cl];
#pragma unroll
            for (int gg = 1; gg < G; ++gg) t += lds[gg][cl];
            out[c] = acc ? out[c] + t : t;
        }
        __syncthreads();
    }
}

// colsum_finalize_kernel with its column slot width chosen for C.
int launch_colsum_finalize(const float* part, float* out, int acc, int64_t K, int64_t C, hipStream_t st) {
    const int64_t want = (int64_t)num_cus();
    if (C >= 64 * want)
        launch_kernel(colsum_finalize_kernel<64>, dim3(grid_for(C, 64, 8)), dim3(kBlock), 0, st, part, out, acc, K, C);
    else if (C >= 16 * want)
        launch_kernel(colsum_finalize_kernel<16>, dim3(grid_for(C, 16, 8)), dim3(kBlock), 0, st, part, out, acc, K, C);
    else
        launch_kernel(colsum_finalize_kernel<4>, dim3(grid_for(C, 4, 8)), dim3(kBlock), 0, st, part, out, acc, K, C);
    return check_launch("wm_binary_bwd(colsum finalize)");
}

// ---------------------------------------------------------------------------
// rowsum: F full [R,C], V column vector [R,1] (R = 1 covers a scalar operand)
// ---------------------------------------------------------------------------

// One wave per (row, chunk) item; lanes walk the chunk 4 columns at a time.
// VEC: C % 4 == 0 and 16-byte aligned bases.  FULL (pow with VB only): both
// gradients are wanted and the forward output is recomputed (not given), so
// the gradient code carries no runtime flags.
template <int OP, bool VB, bool VEC, bool FULL = false>
__global__ void __launch_bounds__(kBlock) bwd_rowsum_kernel(const float* __restrict__ g, const float* __restrict__ F,
                                                             const float* __restrict__ V, const float* __restrict__ o,
                                                             float* __restrict__ gF, int accF, float* __restrict__ gV,
                                                             int accV, float* __restrict__ part, int64_t R, int64_t C,
                                                             int64_t chunk, int64_t K) {
    binary_prologue<OP>();
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * kBlock + threadIdx.x) >> 6;
    const int64_t nwaves = ((int64_t)gridDim.x * kBlock) >> 6;
    static_assert(!FULL || (OP == WM_POW && VB), "FULL is pow's specialisation");
    const bool want_v = FULL || gV != nullptr;
    const bool gF_reads_F = VB ? da_reads_a<OP>() : db_reads_b<OP>();
    const bool gF_reads_V = VB ? da_reads_b<OP>() : db_reads_a<OP>();
    const bool gV_reads_F = VB ? db_reads_a<OP>() : da_reads_b<OP>();
    const bool gV_reads_V = VB ? db_reads_b<OP>() : da_reads_a<OP>();
    const bool want_o = VB ? (want_v && db_reads_out<OP>()) : (gF && db_reads_out<OP>());
    const bool need_o = !FULL && want_o && o;
    const bool need_F = FULL || (gF && gF_reads_F) || (want_v && gV_reads_F) || (want_o && !o);
    const bool need_V = FULL || (gF && gF_reads_V) || (want_v && gV_reads_V) || (want_o && !o);
    for (int64_t item = wave; item < R * K; item += nwaves) {
        const int64_t r = item / K;
        const int64_t k = item - r * K;
        const int64_t c0 = k * chunk;
        const int64_t c1 = min(C, c0 + chunk);
        const float v = need_V ? V[r] : 0.f;
        const float* gr = g + r * C;
        const float* fr = F + r * C;
        const float* orow = o + r * C;
        float* gfr = (FULL || gF) ? gF + r * C : nullptr;
        float s = 0.f;
        if constexpr (VEC) {
            // kSlots float4 per lane per step (256 columns apart), every load
            // of the step issued before any store.  pow's gradient math is
            // long and register-heavy: one slot, its next step's loads issued
            // before the current step's math so they overlap it, and the
            // elements taken two at a time (4 waves per SIMD; measured 69 %
            // of the HBM peak against 66 % for two slots without the
            // prefetch).
            constexpr int kSlots = OP == WM_POW ? 1 : 4;
            constexpr bool kPipe = OP == WM_POW;
            constexpr int kGroup = OP == WM_POW ? 2 : 4;
            const PowGradExponent pq = pow_grad_exponent(OP == WM_POW && VB ? v : 0.0f);
            const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
            float4 s4 = z4;
            float4 vg[kSlots], vf[kSlots], vo[kSlots], old[kSlots];
            auto load = [&](int64_t cb, float4(&lg)[kSlots], float4(&lf)[kSlots], float4(&lo)[kSlots],
                            float4(&lold)[kSlots]) {
#pragma unroll
                for (int u = 0; u < kSlots; ++u) {
                    const int64_t c = cb + u * 256;
                    const bool in = c < c1;
                    lg[u] = in ? ld_stream(gr + c) : z4;
                    lf[u] = in && need_F ? ld_stream(fr + c) : z4;
                    lo[u] = in && need_o ? ld_stream(orow + c) : z4;
                    lold[u] = in && gfr && accF ? ld_stream(gfr + c) : z4;
                }
            };
            if constexpr (kPipe) load(c0 + lane * 4, vg, vf, vo, old);
            for (int64_t cb = c0 + lane * 4; cb < c1; cb += 256 * kSlots) {
                float4 ng[kSlots], nf[kSlots], no[kSlots], nold[kSlots];
                if constexpr (kPipe) load(cb + 256 * kSlots, ng, nf, no, nold);
                else load(cb, vg, vf, vo, old);
#pragma unroll
                for (int u = 0; u < kSlots; ++u) {
                    const int64_t c = cb + u * 256;
                    if (c >= c1) continue;
                    const float e[4] = {vf[u].x, vf[u].y, vf[u].z, vf[u].w},
                                gg[4] = {vg[u].x, vg[u].y, vg[u].z, vg[u].w},
                                oo[4] = {vo[u].x, vo[u].y, vo[u].z, vo[u].w};
                    float da[4], db[4];
#pragma unroll
                    for (int h = 0; h < 4; h += kGroup) {
                        float gh[kGroup], ah[kGroup], bh[kGroup], oh[kGroup], dah[kGroup], dbh[kGroup];
#pragma unroll
                        for (int j = 0; j < kGroup; ++j) {
                            gh[j] = gg[h + j];
                            ah[j] = VB ? e[h + j] : v;
                            bh[j] = VB ? v : e[h + j];
                            oh[j] = oo[h + j];
                        }
                        if constexpr (OP == WM_POW && VB)  // one exponent per row
                            pow_grads_n_exp<kGroup>(gh, ah, v, pq, oh, !FULL && need_o, FULL || gfr != nullptr,
                                                    FULL || want_v, dah, dbh);
                        else
                            binary_grads_n<OP, kGroup>(gh, ah, bh, oh, need_o, VB ? gfr != nullptr : want_v,
                                                       VB ? want_v : gfr != nullptr, dah, dbh);
#pragma unroll
                        for (int j = 0; j < kGroup; ++j) {
                            da[h + j] = dah[j];
                            db[h + j] = dbh[j];
                        }
                    }
                    const float* d = VB ? da : db;
                    const float* sv = VB ? db : da;
                    if (gfr) {
                        float4 nd = make_float4(d[0], d[1], d[2], d[3]);
                        if (accF) { nd.x += old[u].x; nd.y += old[u].y; nd.z += old[u].z; nd.w += old[u].w; }
                        st_stream(gfr + c, nd);
                    }
                    s4.x += sv[0]; s4.y += sv[1]; s4.z += sv[2]; s4.w += sv[3];
                }
                if constexpr (kPipe) {
#pragma unroll
                    for (int u = 0; u < kSlots; ++u) {
                        vg[u] = ng[u];
                        vf[u] = nf[u];
                        vo[u] = no[u];
                        old[u] = nold[u];
                    }
                }
            }
            s = (s4.x + s4.y) + (s4.z + s4.w);
        } else {
            for (int64_t c = c0 + lane; c < c1; c += 64) {
                float vg = gr[c];
                float vf = need_F ? fr[c] : 0.f;
                const float av = VB ? vf : v, bv = VB ? v : vf;
                const float vo = need_o ? orow[c] : 0.f;
                float da, db;
                binary_grads<OP>(vg, av, bv, vo, need_o, VB ? gfr != nullptr : want_v,
                                 VB ? want_v : gfr != nullptr, da, db);
                const float d = VB ? da : db, sv = VB ? db : da;
                if (gfr) gfr[c] = accF ? gfr[c] + d : d;
                s += sv;
            }
        }
        if (want_v) {
            s = wave_sum(s);
            if (lane == 0) {
                if (K == 1) gV[r] = accV ? gV[r] + s : s;
                else part[r * K + k] = s;
            }
        }
    }
}

// One workgroup per row for rows of up to NT * 4 * IT floats: the row's
// loads are all issued before any math, then one fixed-order block sum.  A
// short-lived workgroup reading one contiguous row measured 2-3 points of
// the HBM peak faster than a wave walking each row (c2 A*c backward 73 ->
// 75.6 %); pow's gradient keeps the wave kernel, whose register budget and
// prefetch suit its long math.
template <int OP, bool VB, int NT, int IT>
__global__ void __launch_bounds__(NT) rowsum_wg_kernel(const float* __restrict__ g, const float* __restrict__ F,
                                                       const float* __restrict__ V, const float* __restrict__ o,
                                                       float* __restrict__ gF, int accF, float* __restrict__ gV,
                                                       int accV, int64_t R, int64_t C) {
    binary_prologue<OP>();
    __shared__ float lds[NT / 64];
    const bool want_v = gV != nullptr;
    const bool gF_reads_F = VB ? da_reads_a<OP>() : db_reads_b<OP>();
    const bool gF_reads_V = VB ? da_reads_b<OP>() : db_reads_a<OP>();
    const bool gV_reads_F = VB ? db_reads_a<OP>() : da_reads_b<OP>();
    const bool gV_reads_V = VB ? db_reads_b<OP>() : da_reads_a<OP>();
    const bool want_o = VB ? (want_v && db_reads_out<OP>()) : (gF && db_reads_out<OP>());
    const bool need_o = want_o && o;
    const bool need_F = (gF && gF_reads_F) || (want_v && gV_reads_F) || (want_o && !o);
    const bool need_V = (gF && gF_reads_V) || (want_v && gV_reads_V) || (want_o && !o);
    constexpr int kGroup = OP == WM_POW ? 2 : 4;
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int64_t r = blockIdx.x; r < R; r += gridDim.x) {
        const float v = need_V ? V[r] : 0.f;
        const int64_t base = r * C;
        float4 vg[IT], vf[IT], vo[IT], old[IT];
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int64_t c = ((int64_t)it * NT + threadIdx.x) * 4;
            const bool in = c < C;
            vg[it] = in ? ld_stream(g + base + c) : z4;
            vf[it] = in && need_F ? ld_stream(F + base + c) : z4;
            vo[it] = in && need_o ? ld_stream(o + base + c) : z4;
            old[it] = in && gF && accF ? ld_stream(gF + base + c) : z4;
        }
        float4 s4 = z4;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int64_t c = ((int64_t)it * NT + threadIdx.x) * 4;
            if (c >= C) continue;
            const float e[4] = {vf[it].x, vf[it].y, vf[it].z, vf[it].w},
                        gg[4] = {vg[it].x, vg[it].y, vg[it].z, vg[it].w},
                        oo[4] = {vo[it].x, vo[it].y, vo[it].z, vo[it].w};
            float da[4], db[4];
#pragma unroll
            for (int h = 0; h < 4; h += kGroup) {
                float gh[kGroup], ah[kGroup], bh[kGroup], oh[kGroup], dah[kGroup], dbh[kGroup];
#pragma unroll
                for (int j = 0; j < kGroup; ++j) {
                    gh[j] = gg[h + j];
                    ah[j] = VB ? e[h + j] : v;
                    bh[j] = VB ? v : e[h + j];
                    oh[j] = oo[h + j];
                }
                binary_grads_n<OP, kGroup>(gh, ah, bh, oh, need_o, VB ? gF != nullptr : want_v,
                                           VB ? want_v : gF != nullptr, dah, dbh);
#pragma unroll
                for (int j = 0; j < kGroup; ++j) {
                    da[h + j] = dah[j];
                    db[h + j] = dbh[j];
                }
            }
            const float* d = VB ? da : db;
            const float* sv = VB ? db : da;
            if (gF) {
                float4 nd = make_float4(d[0], d[1], d[2], d[3]);
                if (accF) { nd.x += old[it].x; nd.y += old[it].y; nd.z += old[it].z; nd.w += old[it].w; }
                st_stream(gF + base + c, nd);
            }
            s4.x += sv[0]; s4.y += sv[1]; s4.z += sv[2]; s4.w += sv[3];
        }
        if (want_v) {
            const float s = block_sum<NT>((s4.x + s4.y) + (s4.z + s4.w), lds);
            if (threadIdx.x == 0) gV[r] = accV ? gV[r] + s : s;
        }
    }
}

// gV[r] (+)= sum_k part[r, k]: one block per row, fixed-order tree.
__global__ void __launch_bounds__(kBlock) rowsum_finalize_kernel(const float* __restrict__ part, float* __restrict__ gV,
                                                                  int acc, int64_t R, int64_t K) {
    __shared__ float lds[kBlock / 64];
    for (int64_t r = blockIdx.x; r < R; r += gridDim.x) {
        float s = 0.f;
        for (int64_t k = threadIdx.x; k < K; k += kBlock) s += part[r * K + k];
        s = block_sum<kBlock>(s, lds);
        if (threadIdx.x == 0) gV[r] = acc ? gV[r] + s : s;
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// generic: one thread per operand element
// ---------------------------------------------------------------------------

struct GenDims {
    int nd;
    int64_t size[WM_MAX_DIMS];
    int64_t sa[WM_MAX_DIMS];
    int64_t sb[WM_MAX_DIMS];
    int64_t so[WM_MAX_DIMS];  // output strides
};

// WB: the gradient being produced is b's (else a's).  The thread for operand
// element e visits every output element that reads e in row-major order and
// sums the contributions (the reference's order, core/tensor.cpp:958-975).
template <int OP, bool WB>
__global__ void __launch_bounds__(kBlock) bwd_generic_kernel(const float* __restrict__ g, const float* __restrict__ a,
                                                              const float* __restrict__ b, const float* __restrict__ o,
                                                              float* __restrict__ gx, int acc, int64_t nx, GenDims d) {
    binary_prologue<OP>();
    for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < nx; e += (int64_t)gridDim.x * kBlock) {
        // Output base index from the kept dims of this operand.
        int64_t base = 0;
        int64_t idx[WM_MAX_DIMS];
        int64_t red_total = 1;
        for (int k = 0; k < d.nd; ++k) {
            int64_t s = WB ? d.sb[k] : d.sa[k];
            if (s != 0) {
                int64_t ik = (e / s) % d.size[k];
                base += ik * d.so[k];
                idx[k] = ik;
            } else {
                idx[k] = 0;
                red_total *= d.size[k];
            }
        }
        float acc_v = 0.f;
        for (int64_t j = 0; j < red_total; ++j) {
            int64_t i = base, oa = 0, ob = 0;
            for (int k = 0; k < d.nd; ++k) {
                i += ((WB ? d.sb[k] : d.sa[k]) == 0 ? idx[k] * d.so[k] : 0);
                oa += idx[k] * d.sa[k];
                ob += idx[k] * d.sb[k];
            }
            float vg = g[i], va = a[oa], vb = b[ob];
            if constexpr (WB) acc_v += binary_db<OP>(vg, va, vb, db_reads_out<OP>() ? fwd_out_or<OP>(o, i, va, vb) : 0.f);
            else acc_v += binary_da<OP>(vg, va, vb);
            // Odometer over the reduced dims, last dim fastest.
            for (int k = d.nd - 1; k >= 0; --k) {
                if ((WB ? d.sb[k] : d.sa[k]) != 0) continue;
                if (++idx[k] < d.size[k]) break;
                idx[k] = 0;
            }
        }
        gx[e] = acc ? gx[e] + acc_v : acc_v;
    }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------

template <int OP>
int launch_binary_bwd(const float* g, const float* a, const float* b, const float* o, float* ga, int acc_a, float* gb,
                      int acc_b, int nd, const int64_t* size, const int64_t* sa, const int64_t* sb, int64_t numel,
                      int64_t na, int64_t nb) {
    hipStream_t st = stream();
    auto contiguous_full = [&](const int64_t* s) {
        int64_t expect = 1;
        for (int k = nd - 1; k >= 0; --k) {
            if (s[k] != expect) return false;
            expect *= size[k];
        }
        return true;
    };
    const bool a_full = contiguous_full(sa), b_full = contiguous_full(sb);
    bool aligned = aligned16(g) && aligned16(a) && aligned16(b) && (!o || aligned16(o)) && (!ga || aligned16(ga)) &&
                   (!gb || aligned16(gb));

    // flat
    if (a_full && b_full) {
        if (numel % 4 == 0 && aligned) {
            int64_t n4 = numel / 4;
            launch_kernel(bwd_flat_kernel<OP>, dim3(grid_for(n4, kBlock * kSlotsFlat, 1 << 12)), dim3(kBlock), 0, st, g, a, b, o,
                               ga, acc_a, gb, acc_b, n4);
            return check_launch("wm_binary_bwd(flat)");
        }
    }

    // 2-D layouts: [R, C] with one full operand.
    if ((a_full || b_full) && !(a_full && b_full) && (nd == 2 || nd == 1)) {
        const bool vb = a_full;  // the vector operand is b
        const int64_t* sv = vb ? sb : sa;
        const int64_t R = nd == 2 ? size[0] : 1;
        const int64_t C = size[nd - 1];
        const float* F = vb ? a : b;
        const float* V = vb ? b : a;
        float* gF = vb ? ga : gb;
        float* gV = vb ? gb : ga;
        const int accF = vb ? acc_a : acc_b, accV = vb ? acc_b : acc_a;
        const bool rowvec = nd == 2 && sv[0] == 0 && sv[1] == 1;
        const bool colvec = (nd == 2 && sv[0] == 1 && sv[1] == 0) || (nd == 1 && sv[0] == 0);
        if (rowvec && C % 4 == 0 && aligned) {
            const int64_t col_tiles = (C + kBlock * 4 - 1) / (kBlock * 4);
            // ~1024 workgroups (4 per CU), each group of at least 4 rows (a
            // thread walks its group's rows one at a time, so a small R needs
            // many groups: at R = C = 1024 the column pass took 12 µs with
            // groups of 16 rows, 6 µs with 4; a large R reaches the 1024
            // first)
            int64_t K = std::min<int64_t>((1024 + col_tiles - 1) / col_tiles, (R + 3) / 4);
            K = std::max<int64_t>(1, std::min<int64_t>(K, 65535));
            Workspace ws(gV ? (size_t)(K * C) * sizeof(float) : 0);
            if (gV && !ws.p) return set_error(WM_ERR_NOMEM, "wm_binary_bwd: workspace");
            dim3 grid((unsigned)col_tiles, (unsigned)K);
            if (vb)
                launch_kernel((bwd_colsum_kernel<OP, true>), grid, dim3(kBlock), 0, st, g, F, V, o, gF, accF,
                                   ws.as<float>(), R, C);
            else
                launch_kernel((bwd_colsum_kernel<OP, false>), grid, dim3(kBlock), 0, st, g, F, V, o, gF, accF,
                                   ws.as<float>(), R, C);
            WM_TRY(check_launch("wm_binary_bwd(colsum)"));
            if (gV) {
                WM_TRY(launch_colsum_finalize(ws.as<float>(), gV, accV, K, C, st));
            }
            return WM_OK;
        }
        if (colvec) {
            // Split rows into chunks only when there are too few rows to fill the chip.
            const int64_t target_waves = (int64_t)num_cus() * 32;
            int64_t K = 1;
            if (R < target_waves) K = std::min<int64_t>((target_waves + R - 1) / R, (C + 1023) / 1024);
            K = std::max<int64_t>(K, 1);
            int64_t chunk = (C + K - 1) / K;
            chunk = (chunk + 255) / 256 * 256;
            K = (C + chunk - 1) / chunk;
            if (K < 1) K = 1;
            Workspace ws(gV && K > 1 ? (size_t)(R * K) * sizeof(float) : 0);
            if (gV && K > 1 && !ws.p) return set_error(WM_ERR_NOMEM, "wm_binary_bwd: workspace");
            const bool vec = C % 4 == 0 && aligned;
            if constexpr (OP != WM_POW) {
                if (K == 1 && vec && C >= 1024 && C <= 8192) {
                    // rowsum_wg_kernel with 2 float4s per thread: 256, 512 or 1024 threads
                    const dim3 g1(grid_for(R, 1, 1 << 12));
#define WM_RW(NTv)                                                                                                \
    do {                                                                                                          \
        if (vb) launch_kernel((rowsum_wg_kernel<OP, true, NTv, 2>), g1, dim3(NTv), 0, st, g, F, V, o, gF, accF, gV, \
                              accV, R, C);                                                                        \
        else launch_kernel((rowsum_wg_kernel<OP, false, NTv, 2>), g1, dim3(NTv), 0, st, g, F, V, o, gF, accF, gV, \
                           accV, R, C);                                                                           \
    } while (0)
                    if (C <= 2048) WM_RW(256);
                    else if (C <= 4096) WM_RW(512);
                    else WM_RW(1024);
#undef WM_RW
                    return check_launch("wm_binary_bwd(rowsum, workgroup per row)");
                }
            }
            dim3 grid(grid_for(R * K, kBlock / 64, 32));
#define WM_RS(VBv, VECv)                                                                                          \
    launch_kernel((bwd_rowsum_kernel<OP, VBv, VECv>), grid, dim3(kBlock), 0, st, g, F, V, o, gF, accF, gV, accV, \
                       ws.as<float>(), R, C, chunk, K)
            if constexpr (OP == WM_POW) {
                if (vb && vec && gF && gV && !o) {
                    launch_kernel((bwd_rowsum_kernel<OP, true, true, true>), grid, dim3(kBlock), 0, st, g, F, V, o,
                                  gF, accF, gV, accV, ws.as<float>(), R, C, chunk, K);
                    WM_TRY(check_launch("wm_binary_bwd(rowsum)"));
                    if (K > 1) {
                        launch_kernel(rowsum_finalize_kernel, dim3(grid_for(R, 1, 8)), dim3(kBlock), 0, st,
                                      ws.as<float>(), gV, accV, R, K);
                        WM_TRY(check_launch("wm_binary_bwd(rowsum finalize)"));
                    }
                    return WM_OK;
                }
            }
            if (vb) { if (vec) WM_RS(true, true); else WM_RS(true, false); }
            else { if (vec) WM_RS(false, true); else WM_RS(false, false); }
#undef WM_RS
            WM_TRY(check_launch("wm_binary_bwd(rowsum)"));
            if (gV && K > 1) {
                launch_kernel(rowsum_finalize_kernel, dim3(grid_for(R, 1, 8)), dim3(kBlock), 0, st,
                                   ws.as<float>(), gV, accV, R, K);
                WM_TRY(check_launch("wm_binary_bwd(rowsum finalize)"));
            }
            return WM_OK;
        }
    }

    // generic
    GenDims d;
    d.nd = nd;
    int64_t so = 1;
    for (int k = nd - 1; k >= 0; --k) {
        d.size[k] = size[k]; d.sa[k] = sa[k]; d.sb[k] = sb[k]; d.so[k] = so;
        so *= size[k];
    }
    if (ga) {
        launch_kernel((bwd_generic_kernel<OP, false>), dim3(grid_for(na, kBlock)), dim3(kBlock), 0, st, g, a, b,
                           o, ga, acc_a, na, d);
        WM_TRY(check_launch("wm_binary_bwd(generic a)"));
    }
    if (gb) {
        launch_kernel((bwd_generic_kernel<OP, true>), dim3(grid_for(nb, kBlock)), dim3(kBlock), 0, st, g, a, b,
                           o, gb, acc_b, nb, d);
        WM_TRY(check_launch("wm_binary_bwd(generic b)"));
    }
    return WM_OK;
}

int check_shape(const int64_t* shape, int nd, const char* what);
int64_t shape_numel(const int64_t* shape, int nd);

}  // namespace wm

using namespace wm;

extern "C" int wm_binary_bwd(int op, const float* g, const float* a, const int64_t* a_shape, int a_ndim,
                             const float* b, const int64_t* b_shape, int b_ndim, const float* out, float* ga,
                             int ga_accumulate, float* gb, int gb_accumulate) {
    WM_TRY(check_shape(a_shape, a_ndim, "wm_binary_bwd(a)"));
    WM_TRY(check_shape(b_shape, b_ndim, "wm_binary_bwd(b)"));
    int nd = 0;
    int64_t size[WM_MAX_DIMS], sa[WM_MAX_DIMS], sb[WM_MAX_DIMS], numel = 0;
    WM_TRY(make_bcast_layout_public(a_shape, a_ndim, b_shape, b_ndim, nd, size, sa, sb, numel));
    if (!ga && !gb) return WM_OK;
    const int64_t na = shape_numel(a_shape, a_ndim), nb = shape_numel(b_shape, b_ndim);
    if (numel == 0) {
        // Nothing flows back; an overwrite request still has to leave zeros.
        WM_CHECK_INIT();
        if (ga && !ga_accumulate) WM_TRY(wm_fill(ga, 0.f, na));
        if (gb && !gb_accumulate) WM_TRY(wm_fill(gb, 0.f, nb));
        return WM_OK;
    }
    if (!g || !a || !b) return set_error(WM_ERR_INVALID, "wm_binary_bwd: null pointer");
    WM_CHECK_INIT();
    switch (op) {
#define WM_CASE(OPC) \
    case OPC: return launch_binary_bwd<OPC>(g, a, b, out, ga, ga_accumulate, gb, gb_accumulate, nd, size, sa, sb, numel, na, nb)
        WM_CASE(WM_ADD);
        WM_CASE(WM_SUB);
        WM_CASE(WM_MUL);
        WM_CASE(WM_DIV);
        WM_CASE(WM_POW);
        WM_CASE(WM_MAX);
        WM_CASE(WM_MIN);
#undef WM_CASE
        default: return set_error(WM_ERR_INVALID, "wm_binary_bwd: unknown op");
    }
}
