// Normalisation and attention-softmax kernels (reference core/layer.cpp).
//
// LayerNorm (core/layer.cpp:395-504).  One row (instance) per workgroup,
// held in registers (RowTile): the forward is the reference's two passes
// (mean, then the sum of squared deviations) over registers, so the row is
// read once and written once.  The backward computes both row sums of the
// closure with one barrier, writes dx, and keeps the dgamma / dbeta column
// partials of the rows it visits in registers (a thread owns the same
// columns in every row), so the parameter gradients cost one
// [workgroups, n] partial write and a fixed-order column pass instead of a
// second read of g and x.  Rows longer than 8192 elements stream through
// global memory instead and take the parameter gradients in a separate
// column pass.
//
// BatchNorm2d (core/layer.cpp:202-374).  x is [batch, channels, spatial];
// a channel's elements are `batch` planes of `spatial` contiguous floats.
// Every kernel works on (channel, chunk) workgroups: a chunk is a run of
// 4096-float plane segments of one channel, so the channel's constants are
// loaded once per workgroup and each segment is one contiguous span.  The
// statistics accumulate sum(x) and sum(x^2) (forward) and sum(g),
// sum(g (x - mean)), sum(x - mean) (backward) in double per thread and per
// chunk, combined in a fixed order: one pass over the data, no cancellation
// problem at fp32 data magnitudes, deterministic.  Normalisation and dx are
// a second, element-wise pass.
//
// MultiHeadAttention's softmax (core/layer.cpp:1198-1237, backward
// :1343-1360): one row of scores per workgroup with the mask row added in
// registers, the reference's max-from--FLT_MAX, and its plain backward
// attn * (d_attn - sum(attn * d_attn)).  The reference divides each
// exponential by the row sum; here they are multiplied by one reciprocal per
// row (within an ulp of the quotient, inside the softmax tolerance, and an
// IEEE division per element would cost more than the row's memory traffic).
#include "wm_rows.hpp"

#include <algorithm>
#include <cfloat>

#include "../../include/wm_layers.h"

namespace wm {
namespace {

// Two sums across the workgroup with one barrier.  `lds` must not be
// written again until every thread has read it: callers alternate between
// two arrays per row (see ln_bwd_kernel).
template <int NT>
__device__ __forceinline__ float2 block_sum2_1(float a, float b, float2* lds) {
    constexpr int NW = NT / 64;
    a = wave_sum(a);
    b = wave_sum(b);
    if (NW == 1) return make_float2(a, b);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = make_float2(a, b);
    __syncthreads();
    float2 t = make_float2(0.f, 0.f);
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        t.x += lds[i].x;
        t.y += lds[i].y;
    }
    return t;
}

// Sum of a double over a 256-thread workgroup into thread 0 (fixed order).
__device__ __forceinline__ double block_sum_d256(double v, double* lds) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
    if (threadIdx.x == 0) t = (lds[0] + lds[1]) + (lds[2] + lds[3]);
    __syncthreads();
    return t;
}

// ---------------------------------------------------------------------------
// LayerNorm
// ---------------------------------------------------------------------------

template <int NT, int ITEMS, bool VEC>
__global__ void __launch_bounds__(NT) ln_fwd_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                     const float* __restrict__ beta, int64_t rows, int64_t n,
                                                     float eps, float* __restrict__ y, float* __restrict__ mean_out,
                                                     float* __restrict__ inv_out) {
    using Tile = RowTile<NT, ITEMS, VEC>;
    __shared__ float lds_a[NT / 64], lds_b[NT / 64];
    Tile gt, bt;  // this thread's columns of gamma / beta, the same in every row
    gt.template load<true>(gamma, n, 0.f);
    bt.template load<true>(beta, n, 0.f);
    const float nf = (float)n;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        Tile t;
        t.load(x + r * n, n, 0.f);
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) s += t.v[i][e];
        const float mean = block_sum_1<NT>(s, lds_a) / nf;
        float q = 0.f;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (Tile::col(i, e) < n) {
                    const float d = t.v[i][e] - mean;
                    q += d * d;
                }
        const float var = block_sum_1<NT>(q, lds_b) / nf;
        const float inv = 1.0f / sqrtf(var + eps);
#pragma unroll
        for (int i = 0; i < ITEMS; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) t.v[i][e] = gt.v[i][e] * ((t.v[i][e] - mean) * inv) + bt.v[i][e];
        t.store(y + r * n, n);
        if (threadIdx.x == 0) {
            mean_out[r] = mean;
            inv_out[r] = inv;
        }
    }
}

// pgamma / pbeta: [gridDim.x, n] partials of this workgroup's rows (NULL
// when that gradient is not wanted).
//
// The second __launch_bounds__ argument is HIP's minimum waves per SIMD: a
// 1024-thread workgroup puts 4 waves on each SIMD, so 8 keeps the kernel
// within 64 VGPRs and two workgroups resident per CU (one float4 per
// thread and row; the compiler's own choice, 66, left one: 67 -> 71 % of
// the HBM peak at [32768, 4096]).  Two float4s per thread need more than
// 64 without spilling.
template <int NT, int ITEMS>
constexpr int ln_bwd_min_waves() { return NT == 1024 && ITEMS == 1 ? 8 : 1; }

template <int NT, int ITEMS, bool VEC>
__global__ void __launch_bounds__(NT, (ln_bwd_min_waves<NT, ITEMS>())) ln_bwd_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                     const float* __restrict__ gamma, const float* __restrict__ mean,
                                                     const float* __restrict__ inv_std, int64_t rows, int64_t n,
                                                     float* __restrict__ gx, int acc, float* __restrict__ pgamma,
                                                     float* __restrict__ pbeta) {
    using Tile = RowTile<NT, ITEMS, VEC>;
    __shared__ float2 lds2[2][NT / 64];
    Tile gt;
    gt.template load<true>(gamma, n, 0.f);
    float pg[ITEMS][4], pb[ITEMS][4];
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) pg[i][e] = pb[i][e] = 0.f;
    const float nf = (float)n;
    int k = 0;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x, ++k) {
        Tile dy, xv;
        dy.load(g + r * n, n, 0.f);
        xv.load(x + r * n, n, 0.f);
        const float m = mean[r], iv = inv_std[r];
        float s1 = 0.f, s2 = 0.f;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float xn = (xv.v[i][e] - m) * iv;
                xv.v[i][e] = xn;
                const float dg = dy.v[i][e] * gt.v[i][e];
                s1 += dg;
                s2 += dg * xn;
                pg[i][e] += dy.v[i][e] * xn;  // padding: dy = 0
                pb[i][e] += dy.v[i][e];
            }
        const float2 S = block_sum2_1<NT>(s1, s2, lds2[k & 1]);
        if (gx) {
            const float mdg = S.x / nf, mdgx = S.y / nf;
#pragma unroll
            for (int i = 0; i < ITEMS; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    dy.v[i][e] = iv * (dy.v[i][e] * gt.v[i][e] - mdg - xv.v[i][e] * mdgx);
            if (acc) {
                Tile old;
                old.load(gx + r * n, n, 0.f);
#pragma unroll
                for (int i = 0; i < ITEMS; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) dy.v[i][e] = old.v[i][e] + dy.v[i][e];
            }
            dy.store(gx + r * n, n);
        }
    }
    float* pgr = pgamma ? pgamma + (int64_t)blockIdx.x * n : nullptr;
    float* pbr = pbeta ? pbeta + (int64_t)blockIdx.x * n : nullptr;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t c = Tile::col(i, e);
            if (c < n) {
                if (pgr) pgr[c] = pg[i][e];
                if (pbr) pbr[c] = pb[i][e];
            }
        }
}

// Column sums of [parts, n] partials: out[c] (+)= sum_w part[w][c], w in
// order.  64 columns per workgroup; the 4 waves take every 4th partial row
// and combine in LDS.  blockIdx.z picks one of two independent sums (the
// weight and bias gradients share the launch).
__global__ void __launch_bounds__(256) colsum_parts_kernel(const float* __restrict__ part0,
                                                            const float* __restrict__ part1, int64_t parts, int64_t n,
                                                            float* __restrict__ out0, float* __restrict__ out1,
                                                            int acc0, int acc1) {
    __shared__ float lds[4][64];
    const float* part = blockIdx.z ? part1 : part0;
    float* out = blockIdx.z ? out1 : out0;
    const int acc = blockIdx.z ? acc1 : acc0;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t c = (int64_t)blockIdx.x * 64 + lane;
    float s = 0.f;
    if (c < n)
        for (int64_t p = w; p < parts; p += 4) s += part[p * n + c];
    lds[w][lane] = s;
    __syncthreads();
    if (w == 0 && c < n) {
        const float t = (lds[0][lane] + lds[1][lane]) + (lds[2][lane] + lds[3][lane]);
        out[c] = acc ? out[c] + t : t;
    }
}

// First stage for many partial rows: workgroup (x, y, z) sums partial rows
// [y * chunk, (y + 1) * chunk) of 64 columns of sum z into out2_z[y][c]; each
// wave takes every 4th row with four independent accumulators (loads in
// flight), the waves combine in LDS in a fixed order.  colsum_parts_kernel
// then sums the out2 rows.
__global__ void __launch_bounds__(256) colsum_stage_kernel(const float* __restrict__ part0,
                                                            const float* __restrict__ part1, int64_t parts, int64_t n,
                                                            int64_t chunk, float* __restrict__ out2_0,
                                                            float* __restrict__ out2_1) {
    __shared__ float lds[4][64];
    const float* part = blockIdx.z ? part1 : part0;
    float* out2 = blockIdx.z ? out2_1 : out2_0;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t c = (int64_t)blockIdx.x * 64 + lane;
    const int64_t p0 = (int64_t)blockIdx.y * chunk;
    const int64_t p1 = p0 + chunk < parts ? p0 + chunk : parts;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (c < n) {
        int64_t p = p0 + w;
        for (; p + 12 < p1; p += 16) {
            a0 += part[p * n + c];
            a1 += part[(p + 4) * n + c];
            a2 += part[(p + 8) * n + c];
            a3 += part[(p + 12) * n + c];
        }
        for (; p < p1; p += 4) a0 += part[p * n + c];
    }
    lds[w][lane] = (a0 + a1) + (a2 + a3);
    __syncthreads();
    if (w == 0 && c < n) out2[(int64_t)blockIdx.y * n + c] = (lds[0][lane] + lds[1][lane]) + (lds[2][lane] + lds[3][lane]);
}

// Column sums of [parts, n] partial rows into out_g and out_b (+= when
// acc_*; a null partial array skips its sum): one pass for up to 64 rows,
// else colsum_stage_kernel first.  Both sums share each launch, so the
// weight and bias gradients cost two dispatches, not four (LayerNorm
// backward at [32768, 4096]: 283.5-284.1 -> 278.0-280.8 us).
int colsum_parts(const float* part_g, float* out_g, int acc_g, const float* part_b, float* out_b, int acc_b,
                 int64_t parts, int64_t n, const char* what) {
    hipStream_t st = stream();
    if (!part_g) {  // the bias sum alone: slot 0
        part_g = part_b; out_g = out_b; acc_g = acc_b;
        part_b = nullptr;
    }
    if (!part_g) return WM_OK;
    const unsigned jobs = part_b ? 2u : 1u;
    const dim3 cg((unsigned)((n + 63) / 64), 1u, jobs);
    if (parts <= 64) {
        launch_kernel(colsum_parts_kernel, cg, dim3(256), 0, st, part_g, part_b, parts, n, out_g, out_b, acc_g,
                      acc_b);
        return check_launch(what);
    }
    const int64_t chunk = 64, parts2 = (parts + chunk - 1) / chunk;
    Workspace w2((size_t)(jobs * parts2 * n) * sizeof(float));
    if (!w2.p) return set_error(WM_ERR_NOMEM, std::string(what) + ": workspace");
    float* s0 = w2.as<float>();
    float* s1 = jobs == 2 ? s0 + parts2 * n : nullptr;
    launch_kernel(colsum_stage_kernel, dim3(cg.x, (unsigned)parts2, jobs), dim3(256), 0, st, part_g, part_b, parts,
                  n, chunk, s0, s1);
    WM_TRY(check_launch(what));
    launch_kernel(colsum_parts_kernel, cg, dim3(256), 0, st, (const float*)s0, (const float*)s1, parts2, n, out_g,
                  out_b, acc_g, acc_b);
    return check_launch(what);
}

// Rows longer than the register tile: three streaming passes per row.
__global__ void __launch_bounds__(1024) ln_fwd_long_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                            const float* __restrict__ beta, int64_t rows, int64_t n,
                                                            float eps, float* __restrict__ y,
                                                            float* __restrict__ mean_out, float* __restrict__ inv_out) {
    __shared__ float lds_a[16], lds_b[16];
    const float nf = (float)n;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * n;
        float s = 0.f;
        for (int64_t c = threadIdx.x; c < n; c += 1024) s += xr[c];
        const float mean = block_sum_1<1024>(s, lds_a) / nf;
        float q = 0.f;
        for (int64_t c = threadIdx.x; c < n; c += 1024) {
            const float d = xr[c] - mean;
            q += d * d;
        }
        const float inv = 1.0f / sqrtf(block_sum_1<1024>(q, lds_b) / nf + eps);
        for (int64_t c = threadIdx.x; c < n; c += 1024) y[r * n + c] = gamma[c] * ((xr[c] - mean) * inv) + beta[c];
        if (threadIdx.x == 0) {
            mean_out[r] = mean;
            inv_out[r] = inv;
        }
    }
}

__global__ void __launch_bounds__(1024) ln_bwd_long_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ mean,
                                                            const float* __restrict__ inv_std, int64_t rows, int64_t n,
                                                            float* __restrict__ gx, int acc) {
    __shared__ float2 lds2[2][16];
    const float nf = (float)n;
    int k = 0;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x, ++k) {
        const float* gr = g + r * n;
        const float* xr = x + r * n;
        const float m = mean[r], iv = inv_std[r];
        float s1 = 0.f, s2 = 0.f;
        for (int64_t c = threadIdx.x; c < n; c += 1024) {
            const float dg = gr[c] * gamma[c];
            s1 += dg;
            s2 += dg * ((xr[c] - m) * iv);
        }
        const float2 S = block_sum2_1<1024>(s1, s2, lds2[k & 1]);
        const float mdg = S.x / nf, mdgx = S.y / nf;
        for (int64_t c = threadIdx.x; c < n; c += 1024) {
            const float d = iv * (gr[c] * gamma[c] - mdg - ((xr[c] - m) * iv) * mdgx);
            gx[r * n + c] = acc ? gx[r * n + c] + d : d;
        }
    }
}

// dgamma / dbeta partials for the long-row path: [chunks, n], each thread a
// column, each workgroup a chunk of rows.
__global__ void __launch_bounds__(256) ln_param_parts_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                              const float* __restrict__ mean,
                                                              const float* __restrict__ inv_std, int64_t rows,
                                                              int64_t n, int64_t rows_per_chunk,
                                                              float* __restrict__ pgamma, float* __restrict__ pbeta) {
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t r0 = (int64_t)blockIdx.y * rows_per_chunk;
    const int64_t r1 = r0 + rows_per_chunk < rows ? r0 + rows_per_chunk : rows;
    if (c >= n) return;
    float sg = 0.f, sb = 0.f;
    for (int64_t r = r0; r < r1; ++r) {
        const float dy = g[r * n + c];
        sg += dy * ((x[r * n + c] - mean[r]) * inv_std[r]);
        sb += dy;
    }
    if (pgamma) pgamma[(int64_t)blockIdx.y * n + c] = sg;
    if (pbeta) pbeta[(int64_t)blockIdx.y * n + c] = sb;
}

// ---------------------------------------------------------------------------
// BatchNorm2d
// ---------------------------------------------------------------------------

// A (channel, chunk) workgroup walks segments [seg0, seg1) of its channel;
// segment s is plane s / spp, units [(s % spp) * kSeg, ...) of that plane.
// A unit is a float4 (VEC: spatial % 4 == 0 and x aligned) or a float.
constexpr int64_t kSeg = 1024;

struct BnGeom {
    int64_t C, S, units;   // units per plane
    int64_t spp, nseg;     // segments per plane, per channel
    int64_t chunks;        // chunks per channel (gridDim.x)
};

// Visit every unit of this workgroup's chunk (blockIdx.x) of its channel
// (blockIdx.y): f(plane_offset_in_floats, unit_index_in_plane), four units
// per thread per step, loads first.
template <bool VEC, class F>
__device__ __forceinline__ void bn_for_chunk(const BnGeom& gm, F&& f) {
    const int64_t k = blockIdx.x, c = blockIdx.y;
    const int64_t s0 = gm.nseg * k / gm.chunks, s1 = gm.nseg * (k + 1) / gm.chunks;
    for (int64_t sg = s0; sg < s1; ++sg) {
        const int64_t b = sg / gm.spp, u0 = (sg - b * gm.spp) * kSeg;
        const int64_t base = (b * gm.C + c) * gm.S;
        f(base, u0);
    }
}

// Cached loads: the apply pass reads x again right after, and for a tensor
// of a few tens of MiB part of that re-read then comes from the caches
// (measured: a re-read of 64 MiB 2-15 % faster, of 192 MiB no faster).
template <bool VEC>
__global__ void __launch_bounds__(256) bn_stats_kernel(const float* __restrict__ x, BnGeom gm,
                                                        double* __restrict__ part) {
    __shared__ double lds[4];
    double s = 0.0, q = 0.0;
    bn_for_chunk<VEC>(gm, [&](int64_t base, int64_t u0) {
        const float* p = x + base;
        if (VEC) {
            float4 v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                v[k] = u < gm.units && u < u0 + kSeg ? *reinterpret_cast<const float4*>(p + u * 4)
                                                     : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const double a = v[k].x, b = v[k].y, cc = v[k].z, d = v[k].w;
                s += (a + b) + (cc + d);
                q += (a * a + b * b) + (cc * cc + d * d);
            }
        } else {
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                v[k] = u < gm.units && u < u0 + kSeg ? p[u] : 0.f;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const double a = v[k];
                s += a;
                q += a * a;
            }
        }
    });
    s = block_sum_d256(s, lds);
    q = block_sum_d256(q, lds);
    if (threadIdx.x == 0) {
        double* o = part + ((int64_t)blockIdx.y * gm.chunks + blockIdx.x) * 2;
        o[0] = s;
        o[1] = q;
    }
}

// Channel c's statistics: the chunk partials combined in order, then the
// reference's float arithmetic for the running statistics and 1/std.  With
// `update`, the running statistics and the saved mean / 1/std are written.
struct BnStats {
    const double* part;
    int64_t chunks;
    int64_t n;
    float eps, momentum;
    int training;
    float* running_mean;
    float* running_var;
    float* mean_out;
    float* inv_out;
};

__device__ __forceinline__ float2 bn_channel_stats(const BnStats& a, int64_t c, bool update) {
#pragma clang fp contract(off)
    float mean, var;
    if (a.training) {
        double s = 0.0, q = 0.0;
        for (int64_t k = 0; k < a.chunks; ++k) {
            s += a.part[(c * a.chunks + k) * 2];
            q += a.part[(c * a.chunks + k) * 2 + 1];
        }
        const double md = s / (double)a.n;
        const double m2 = q - s * md;
        mean = (float)md;
        var = (float)((m2 > 0.0 ? m2 : 0.0) / (double)a.n);
        if (update) {
            a.running_mean[c] = (1.0f - a.momentum) * a.running_mean[c] + a.momentum * mean;
            a.running_var[c] = (1.0f - a.momentum) * a.running_var[c] + a.momentum * var;
        }
    } else {
        mean = a.running_mean[c];
        var = a.running_var[c];
    }
    const float inv = 1.0f / sqrtf(var + a.eps);
    if (update) {
        a.mean_out[c] = mean;
        a.inv_out[c] = inv;
    }
    return make_float2(mean, inv);
}

// One lane per channel (the statistics alone, when no output is wanted).
__global__ void __launch_bounds__(256) bn_stats_finalize_kernel(BnStats a, int64_t C) {
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < C; c += (int64_t)gridDim.x * 256)
        (void)bn_channel_stats(a, c, true);
}

// Each workgroup combines its channel's partials itself (chunk 0's also
// writes the running and saved statistics): no finalize launch between the
// two passes.
template <bool VEC>
__global__ void __launch_bounds__(256) bn_apply_kernel(const float* __restrict__ x, const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, BnStats sa, BnGeom gm,
                                                        float* __restrict__ y) {
    const int64_t c = blockIdx.y;
    __shared__ float2 s_mi;
    if (threadIdx.x == 0) s_mi = bn_channel_stats(sa, c, blockIdx.x == 0);
    __syncthreads();
    const float gc = gamma[c], bc = beta[c], mc = s_mi.x, ic = s_mi.y;
    auto nrm = [&](float v) { return gc * ((v - mc) * ic) + bc; };
    bn_for_chunk<VEC>(gm, [&](int64_t base, int64_t u0) {
        if (VEC) {
            float4 v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                if (u < gm.units && u < u0 + kSeg) v[k] = ld_stream(x + base + u * 4);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                if (u < gm.units && u < u0 + kSeg)
                    st_stream(y + base + u * 4, make_float4(nrm(v[k].x), nrm(v[k].y), nrm(v[k].z), nrm(v[k].w)));
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                if (u < gm.units && u < u0 + kSeg) st_stream1(y + base + u, nrm(ld_stream1(x + base + u)));
            }
        }
    });
}

// Backward sums per chunk: sum(g), sum(g (x - mean)), sum(x - mean), with
// x - mean in float as the closure computes it (cached loads, as in
// bn_stats_kernel: the dx pass re-reads g and x).
template <bool VEC>
__global__ void __launch_bounds__(256) bn_bwd_sums_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                           const float* __restrict__ mean, BnGeom gm,
                                                           double* __restrict__ part) {
    __shared__ double lds[4];
    const float mc = mean[blockIdx.y];
    double s1 = 0.0, s2 = 0.0, s3 = 0.0;
    bn_for_chunk<VEC>(gm, [&](int64_t base, int64_t u0) {
        if (VEC) {
            float4 gv[4], xv[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                const bool in = u < gm.units && u < u0 + kSeg;
                gv[k] = in ? *reinterpret_cast<const float4*>(g + base + u * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
                xv[k] = in ? *reinterpret_cast<const float4*>(x + base + u * 4) : make_float4(mc, mc, mc, mc);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float d0 = xv[k].x - mc, d1 = xv[k].y - mc, d2 = xv[k].z - mc, d3 = xv[k].w - mc;
                s1 += ((double)gv[k].x + (double)gv[k].y) + ((double)gv[k].z + (double)gv[k].w);
                s2 += ((double)gv[k].x * d0 + (double)gv[k].y * d1) + ((double)gv[k].z * d2 + (double)gv[k].w * d3);
                s3 += ((double)d0 + (double)d1) + ((double)d2 + (double)d3);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                if (u < gm.units && u < u0 + kSeg) {
                    const float gv = g[base + u], d = x[base + u] - mc;
                    s1 += gv;
                    s2 += (double)gv * d;
                    s3 += d;
                }
            }
        }
    });
    s1 = block_sum_d256(s1, lds);
    s2 = block_sum_d256(s2, lds);
    s3 = block_sum_d256(s3, lds);
    if (threadIdx.x == 0) {
        double* o = part + ((int64_t)blockIdx.y * gm.chunks + blockIdx.x) * 3;
        o[0] = s1;
        o[1] = s2;
        o[2] = s3;
    }
}

// Channel c's backward coefficients from the chunk sums: the closure's
// dvar, dmean; with `update`, dgamma and dbeta (accumulated as requested).
struct BnBwdCoef {
    const double* part;
    int64_t chunks;
    int64_t n;
    const float* gamma;
    const float* inv_std;
    float* dgamma;
    int acc_gamma;
    float* dbeta;
    int acc_beta;
};

__device__ __forceinline__ float2 bn_channel_coef(const BnBwdCoef& a, int64_t c, bool update) {
    double s1 = 0.0, s2 = 0.0, s3 = 0.0;
    for (int64_t k = 0; k < a.chunks; ++k) {
        const double* p = a.part + (c * a.chunks + k) * 3;
        s1 += p[0];
        s2 += p[1];
        s3 += p[2];
    }
    const double iv = a.inv_std[c], gm = a.gamma[c];
    if (update && a.dgamma) {
        const float dg = (float)(s2 * iv);
        a.dgamma[c] = a.acc_gamma ? a.dgamma[c] + dg : dg;
    }
    if (update && a.dbeta) {
        const float db = (float)s1;
        a.dbeta[c] = a.acc_beta ? a.dbeta[c] + db : db;
    }
    const float dvar = (float)(gm * s2 * -0.5 * iv * iv * iv);
    const float dmean = (float)(-gm * iv * s1 + (double)dvar * (-2.0 * s3) / (double)a.n);
    return make_float2(dvar, dmean);
}

// One lane per channel: dgamma, dbeta when no input gradient is wanted.
__global__ void __launch_bounds__(256) bn_bwd_finalize_kernel(BnBwdCoef a, int64_t C) {
    for (int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x; c < C; c += (int64_t)gridDim.x * 256)
        (void)bn_channel_coef(a, c, true);
}

// Each workgroup combines its channel's sums itself (chunk 0's also writes
// dgamma / dbeta): no finalize launch between the two passes.
template <bool VEC>
__global__ void __launch_bounds__(256) bn_bwd_apply_kernel(const float* __restrict__ g, const float* __restrict__ x,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ mean,
                                                            const float* __restrict__ inv_std, BnBwdCoef ca,
                                                            BnGeom gm, float nf, float* __restrict__ gx, int acc) {
    const int64_t c = blockIdx.y;
    __shared__ float2 s_cf;
    if (threadIdx.x == 0) s_cf = bn_channel_coef(ca, c, blockIdx.x == 0);
    __syncthreads();
    const float gc = gamma[c], mc = mean[c], ic = inv_std[c];
    const float2 cf = s_cf;
    const float dm = cf.y / nf;
    auto dx = [&](float gv, float xv) { return gv * gc * ic + cf.x * 2.0f * (xv - mc) / nf + dm; };
    bn_for_chunk<VEC>(gm, [&](int64_t base, int64_t u0) {
        if (VEC) {
            float4 gv[4], xv[4], ov[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                if (u < gm.units && u < u0 + kSeg) {
                    gv[k] = ld_stream(g + base + u * 4);
                    xv[k] = ld_stream(x + base + u * 4);
                    if (acc) ov[k] = ld_stream(gx + base + u * 4);
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                if (u < gm.units && u < u0 + kSeg) {
                    float4 d = make_float4(dx(gv[k].x, xv[k].x), dx(gv[k].y, xv[k].y), dx(gv[k].z, xv[k].z),
                                           dx(gv[k].w, xv[k].w));
                    if (acc) d = make_float4(ov[k].x + d.x, ov[k].y + d.y, ov[k].z + d.z, ov[k].w + d.w);
                    st_stream(gx + base + u * 4, d);
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int64_t u = u0 + threadIdx.x + k * 256;
                if (u < gm.units && u < u0 + kSeg) {
                    float d = dx(ld_stream1(g + base + u), ld_stream1(x + base + u));
                    if (acc) d = ld_stream1(gx + base + u) + d;
                    st_stream1(gx + base + u, d);
                }
            }
        }
    });
}

// ---------------------------------------------------------------------------
// Attention softmax
// ---------------------------------------------------------------------------

template <int NT, int ITEMS, bool VEC>
__global__ void __launch_bounds__(NT) attn_softmax_fwd_kernel(const float* __restrict__ scores,
                                                               const float* __restrict__ mask, int64_t mask_bstride,
                                                               int64_t heads_tq, int64_t tq, int64_t rows, int64_t tk,
                                                               float* __restrict__ attn) {
    using Tile = RowTile<NT, ITEMS, VEC>;
    __shared__ float lds_m[NT / 64], lds_s[NT / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        Tile t;
        t.load(scores + r * tk, tk, -INFINITY);
        if (mask) {
            const int64_t b = r / heads_tq, i = r % tq;
            Tile mt;
            mt.template load<true>(mask + b * mask_bstride + i * tk, tk, 0.f);
#pragma unroll
            for (int k = 0; k < ITEMS; ++k)
#pragma unroll
                for (int e = 0; e < 4; ++e) t.v[k][e] = t.v[k][e] + mt.v[k][e];
        }
        float mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) mx = fmaxf(mx, t.v[k][e]);
        // max_val starts at -FLT_MAX (core/layer.cpp:1215); std::max skips NaN like fmaxf
        const float m = fmaxf(block_max_1<NT>(mx, lds_m), -FLT_MAX);
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                t.v[k][e] = exp_rr(t.v[k][e] - m);  // padding: exp(-inf) = 0
                s += t.v[k][e];
            }
        const float rs = 1.0f / block_sum_1<NT>(s, lds_s);
#pragma unroll
        for (int k = 0; k < ITEMS; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) t.v[k][e] = t.v[k][e] * rs;
        t.store(attn + r * tk, tk);
    }
}

template <int NT, int ITEMS, bool VEC>
__global__ void __launch_bounds__(NT) attn_softmax_bwd_kernel(const float* __restrict__ attn,
                                                               const float* __restrict__ da, int64_t rows, int64_t tk,
                                                               float* __restrict__ ds) {
    using Tile = RowTile<NT, ITEMS, VEC>;
    __shared__ float lds[2][NT / 64];
    int k2 = 0;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x, ++k2) {
        Tile a, d;
        a.load(attn + r * tk, tk, 0.f);
        d.load(da + r * tk, tk, 0.f);
        float dot = 0.f;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) dot += a.v[k][e] * d.v[k][e];
        dot = block_sum_1<NT>(dot, lds[k2 & 1]);
#pragma unroll
        for (int k = 0; k < ITEMS; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) d.v[k][e] = a.v[k][e] * (d.v[k][e] - dot);
        d.store(ds + r * tk, tk);
    }
}

// Rows longer than the register tile.
__global__ void __launch_bounds__(1024) attn_softmax_fwd_long_kernel(const float* __restrict__ scores,
                                                                      const float* __restrict__ mask,
                                                                      int64_t mask_bstride, int64_t heads_tq,
                                                                      int64_t tq, int64_t rows, int64_t tk,
                                                                      float* __restrict__ attn) {
    __shared__ float lds_m[16], lds_s[16];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* sr = scores + r * tk;
        const float* mr = mask ? mask + (r / heads_tq) * mask_bstride + (r % tq) * tk : nullptr;
        float* ar = attn + r * tk;
        float mx = -INFINITY;
        for (int64_t c = threadIdx.x; c < tk; c += 1024) mx = fmaxf(mx, mr ? sr[c] + mr[c] : sr[c]);
        const float m = fmaxf(block_max_1<1024>(mx, lds_m), -FLT_MAX);
        float s = 0.f;
        for (int64_t c = threadIdx.x; c < tk; c += 1024) {
            const float e = exp_rr((mr ? sr[c] + mr[c] : sr[c]) - m);
            ar[c] = e;
            s += e;
        }
        const float rs = 1.0f / block_sum_1<1024>(s, lds_s);
        for (int64_t c = threadIdx.x; c < tk; c += 1024) ar[c] = ar[c] * rs;
        __syncthreads();
    }
}

__global__ void __launch_bounds__(1024) attn_softmax_bwd_long_kernel(const float* __restrict__ attn,
                                                                      const float* __restrict__ da, int64_t rows,
                                                                      int64_t tk, float* __restrict__ ds) {
    __shared__ float lds[2][16];
    int k2 = 0;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x, ++k2) {
        const float* ar = attn + r * tk;
        const float* dr = da + r * tk;
        float dot = 0.f;
        for (int64_t c = threadIdx.x; c < tk; c += 1024) dot += ar[c] * dr[c];
        dot = block_sum_1<1024>(dot, lds[k2 & 1]);
        for (int64_t c = threadIdx.x; c < tk; c += 1024) ds[r * tk + c] = ar[c] * (dr[c] - dot);
    }
}

// ---------------------------------------------------------------------------
// Dropout mask
// ---------------------------------------------------------------------------

// splitmix64 (Vigna): one 64-bit state step, a bijective mix of the counter.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void __launch_bounds__(256) dropout_mask_kernel(float* __restrict__ mask, int64_t n, float p, float scale,
                                                            uint64_t seed) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float u = (float)(uint32_t)(splitmix64(seed + (uint64_t)i) >> 40) * 0x1p-24f;
        mask[i] = u > p ? scale : 0.0f;
    }
}

// ---------------------------------------------------------------------------
// host
// ---------------------------------------------------------------------------

// LayerNorm register tiles: NT in {64, 256, 1024}, ITEMS in {1, 2}; rows
// over 8192 elements take the streaming path (nt == 0).
TileChoice ln_tile(int64_t n) {
    TileChoice t;
    const int nts[3] = {64, 256, 1024};
    for (int nt : nts)
        for (int items = 1; items <= 2; ++items)
            if (n <= (int64_t)nt * 4 * items) {
                t.nt = nt;
                t.items = items;
                return t;
            }
    return t;
}

int ln_waves(int nt) { return nt == 64 ? 16 : nt == 256 ? 4 : 2; }  // workgroups per CU in the grid

int launch_ln_fwd(const float* x, const float* gamma, const float* beta, int64_t rows, int64_t n, float eps,
                  float* y, float* mean, float* inv) {
    hipStream_t st = stream();
    const TileChoice tc = ln_tile(n);
    const bool vec = n % 4 == 0 && aligned16(x) && aligned16(y) && aligned16(gamma) && aligned16(beta);
    if (tc.nt == 0) {
        dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * 2));
        launch_kernel(ln_fwd_long_kernel, grid, dim3(1024), 0, st, x, gamma, beta, rows, n, eps, y, mean, inv);
        return check_launch("wm_layernorm_fwd(long)");
    }
    dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * ln_waves(tc.nt) * 2));
#define WM_LNF(NTv, IT)                                                                                         \
    if (tc.nt == NTv && tc.items == IT) {                                                                       \
        if (vec)                                                                                                \
            launch_kernel((ln_fwd_kernel<NTv, IT, true>), grid, dim3(NTv), 0, st, x, gamma, beta, rows, n, \
                               eps, y, mean, inv);                                                              \
        else                                                                                                    \
            launch_kernel((ln_fwd_kernel<NTv, IT, false>), grid, dim3(NTv), 0, st, x, gamma, beta, rows,   \
                               n, eps, y, mean, inv);                                                           \
        return check_launch("wm_layernorm_fwd");                                                                \
    }
    WM_LNF(64, 1) WM_LNF(64, 2) WM_LNF(256, 1) WM_LNF(256, 2) WM_LNF(1024, 1) WM_LNF(1024, 2)
#undef WM_LNF
    return set_error(WM_ERR_INVALID, "wm_layernorm_fwd: no tile");
}

int launch_ln_bwd(const float* g, const float* x, const float* gamma, const float* mean, const float* inv,
                  int64_t rows, int64_t n, float* gx, int acc_x, float* dgamma, int acc_g, float* dbeta, int acc_b) {
    hipStream_t st = stream();
    const TileChoice tc = ln_tile(n);
    const bool want_p = dgamma || dbeta;
    if (tc.nt == 0) {
        if (gx) {
            dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * 2));
            launch_kernel(ln_bwd_long_kernel, grid, dim3(1024), 0, st, g, x, gamma, mean, inv, rows, n, gx,
                               acc_x);
            WM_TRY(check_launch("wm_layernorm_bwd(long)"));
        }
        if (!want_p) return WM_OK;
        const int64_t chunks = std::max<int64_t>(1, std::min<int64_t>(rows / 64, 256));
        const int64_t rpc = (rows + chunks - 1) / chunks;
        Workspace wg(dgamma ? (size_t)(chunks * n) * sizeof(float) : 0);
        Workspace wb(dbeta ? (size_t)(chunks * n) * sizeof(float) : 0);
        if ((dgamma && !wg.p) || (dbeta && !wb.p)) return set_error(WM_ERR_NOMEM, "wm_layernorm_bwd: workspace");
        launch_kernel(ln_param_parts_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)chunks), dim3(256), 0,
                           st, g, x, mean, inv, rows, n, rpc, wg.as<float>(), wb.as<float>());
        WM_TRY(check_launch("wm_layernorm_bwd(params)"));
        return colsum_parts(dgamma ? wg.as<float>() : nullptr, dgamma, acc_g, dbeta ? wb.as<float>() : nullptr,
                            dbeta, acc_b, chunks, n, "wm_layernorm_bwd(colsum)");
    }
    // Fused path: G workgroups, each leaving one [n] partial per parameter
    // gradient.  G also bounds the partial traffic: at least 32 rows each.
    int64_t G = std::min<int64_t>(rows, (int64_t)num_cus() * ln_waves(tc.nt) * 2);
    if (want_p) G = std::max<int64_t>(1, std::min<int64_t>(G, (rows + 31) / 32));
    Workspace wg(dgamma ? (size_t)(G * n) * sizeof(float) : 0);
    Workspace wb(dbeta ? (size_t)(G * n) * sizeof(float) : 0);
    if ((dgamma && !wg.p) || (dbeta && !wb.p)) return set_error(WM_ERR_NOMEM, "wm_layernorm_bwd: workspace");
    const bool vec = n % 4 == 0 && aligned16(g) && aligned16(x) && aligned16(gamma) && (!gx || aligned16(gx));
    dim3 grid((unsigned)G);
    bool launched = false;
#define WM_LNB(NTv, IT)                                                                                         \
    if (!launched && tc.nt == NTv && tc.items == IT) {                                                          \
        if (vec)                                                                                                \
            launch_kernel((ln_bwd_kernel<NTv, IT, true>), grid, dim3(NTv), 0, st, g, x, gamma, mean, inv,  \
                               rows, n, gx, acc_x, wg.as<float>(), wb.as<float>());                             \
        else                                                                                                    \
            launch_kernel((ln_bwd_kernel<NTv, IT, false>), grid, dim3(NTv), 0, st, g, x, gamma, mean, inv, \
                               rows, n, gx, acc_x, wg.as<float>(), wb.as<float>());                             \
        launched = true;                                                                                        \
    }
    WM_LNB(64, 1) WM_LNB(64, 2) WM_LNB(256, 1) WM_LNB(256, 2) WM_LNB(1024, 1) WM_LNB(1024, 2)
#undef WM_LNB
    if (!launched) return set_error(WM_ERR_INVALID, "wm_layernorm_bwd: no tile");
    WM_TRY(check_launch("wm_layernorm_bwd"));
    return colsum_parts(dgamma ? wg.as<float>() : nullptr, dgamma, acc_g, dbeta ? wb.as<float>() : nullptr, dbeta,
                        acc_b, G, n, "wm_layernorm_bwd(colsum)");
}

// Workgroups per CU for a pass of two kernels: as many as both keep
// resident, at most 8, so the grid runs in one round (the backward's
// kernels hold 7 per CU: a grid of 8 per CU ran as 7 plus a one-per-CU
// tail, 178.7 against 164.2 us at [64, 256, 56, 56]).
template <class K1, class K2>
int bn_per_cu(K1 k1, K2 k2) {
    int a = 0, b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&a, k1, 256, 0) != hipSuccess || a < 1) a = 1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, k2, 256, 0) != hipSuccess || b < 1) b = 1;
    return std::min(8, std::min(a, b));
}

// per_cu: workgroups per CU the grid aims at.
BnGeom bn_geom(int64_t B, int64_t C, int64_t S, bool vec, int per_cu) {
    BnGeom gm;
    gm.C = C;
    gm.S = S;
    gm.units = vec ? S / 4 : S;
    gm.spp = (gm.units + kSeg - 1) / kSeg;
    gm.nseg = B * gm.spp;
    const int64_t target = (int64_t)num_cus() * per_cu;
    gm.chunks = std::max<int64_t>(1, std::min<int64_t>(gm.nseg, (target + C - 1) / C));
    return gm;
}

int check_bn(int64_t B, int64_t C, int64_t S, const char* what) {
    if (B < 0 || C < 0 || S < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative extent");
    if (C > 65535) return set_error(WM_ERR_UNSUPPORTED, std::string(what) + ": more than 65535 channels");
    return WM_OK;
}

}  // namespace
}  // namespace wm

using namespace wm;

extern "C" {

int wm_layernorm_fwd(const float* x, const float* gamma, const float* beta, int64_t rows, int64_t n, float eps,
                     float* y, float* mean, float* inv_std) {
    if (rows < 0 || n < 0) return set_error(WM_ERR_INVALID, "wm_layernorm_fwd: negative extent");
    if (rows == 0 || n == 0) return WM_OK;
    if (!x || !gamma || !beta || !y || !mean || !inv_std)
        return set_error(WM_ERR_INVALID, "wm_layernorm_fwd: null pointer");
    WM_CHECK_INIT();
    return launch_ln_fwd(x, gamma, beta, rows, n, eps, y, mean, inv_std);
}

int wm_layernorm_bwd(const float* g, const float* x, const float* gamma, const float* mean, const float* inv_std,
                     int64_t rows, int64_t n, float* gx, int acc_x, float* dgamma, int acc_gamma, float* dbeta,
                     int acc_beta) {
    if (rows < 0 || n < 0) return set_error(WM_ERR_INVALID, "wm_layernorm_bwd: negative extent");
    if (n == 0 || (!gx && !dgamma && !dbeta)) return WM_OK;
    if (rows == 0) {
        // no instances: the parameter gradients receive zero contributions
        WM_CHECK_INIT();
        if (dgamma && !acc_gamma) WM_TRY(wm_fill(dgamma, 0.0f, n));
        if (dbeta && !acc_beta) WM_TRY(wm_fill(dbeta, 0.0f, n));
        return WM_OK;
    }
    if (!g || !x || !gamma || !mean || !inv_std) return set_error(WM_ERR_INVALID, "wm_layernorm_bwd: null pointer");
    WM_CHECK_INIT();
    return launch_ln_bwd(g, x, gamma, mean, inv_std, rows, n, gx, acc_x, dgamma, acc_gamma, dbeta, acc_beta);
}

int wm_batchnorm2d_fwd(const float* x, const float* gamma, const float* beta, float* running_mean,
                       float* running_var, int64_t batch, int64_t channels, int64_t spatial, float eps,
                       float momentum, int training, float* y, float* mean, float* inv_std) {
    WM_TRY(check_bn(batch, channels, spatial, "wm_batchnorm2d_fwd"));
    if (channels == 0) return WM_OK;
    if (!gamma || !beta || !running_mean || !running_var || !mean || !inv_std)
        return set_error(WM_ERR_INVALID, "wm_batchnorm2d_fwd: null pointer");
    const int64_t n = batch * spatial;
    if (n > 0 && (!x || !y)) return set_error(WM_ERR_INVALID, "wm_batchnorm2d_fwd: null pointer");
    WM_CHECK_INIT();
    hipStream_t st = stream();
    const bool vec = spatial % 4 == 0 && aligned16(x) && aligned16(y);
    const BnGeom gm = bn_geom(batch, channels, spatial, vec,
                              vec ? bn_per_cu(bn_stats_kernel<true>, bn_apply_kernel<true>)
                                  : bn_per_cu(bn_stats_kernel<false>, bn_apply_kernel<false>));
    Workspace part(training ? (size_t)(channels * gm.chunks) * 2 * sizeof(double) : 0);
    if (training && !part.p) return set_error(WM_ERR_NOMEM, "wm_batchnorm2d_fwd: workspace");
    const BnStats sa{part.as<double>(), gm.chunks, n, eps, momentum, training, running_mean, running_var, mean,
                     inv_std};
    if (n == 0) {  // no elements: the statistics of empty sums (the reference's 0 / 0)
        if (training) {
            launch_kernel(bn_stats_kernel<false>, dim3((unsigned)gm.chunks, (unsigned)channels), dim3(256), 0, st, x,
                          gm, part.as<double>());
            WM_TRY(check_launch("wm_batchnorm2d_fwd(stats)"));
        }
        launch_kernel(bn_stats_finalize_kernel, dim3((unsigned)((channels + 255) / 256)), dim3(256), 0, st, sa,
                      channels);
        return check_launch("wm_batchnorm2d_fwd(finalize)");
    }
    const dim3 grid((unsigned)gm.chunks, (unsigned)channels);
    if (training) {
        if (vec) launch_kernel(bn_stats_kernel<true>, grid, dim3(256), 0, st, x, gm, part.as<double>());
        else launch_kernel(bn_stats_kernel<false>, grid, dim3(256), 0, st, x, gm, part.as<double>());
        WM_TRY(check_launch("wm_batchnorm2d_fwd(stats)"));
    }
    if (vec) launch_kernel(bn_apply_kernel<true>, grid, dim3(256), 0, st, x, gamma, beta, sa, gm, y);
    else launch_kernel(bn_apply_kernel<false>, grid, dim3(256), 0, st, x, gamma, beta, sa, gm, y);
    return check_launch("wm_batchnorm2d_fwd(apply)");
}

int wm_batchnorm2d_bwd(const float* g, const float* x, const float* gamma, const float* mean, const float* inv_std,
                       int64_t batch, int64_t channels, int64_t spatial, float* gx, int acc_x, float* dgamma,
                       int acc_gamma, float* dbeta, int acc_beta) {
    WM_TRY(check_bn(batch, channels, spatial, "wm_batchnorm2d_bwd"));
    if (channels == 0 || (!gx && !dgamma && !dbeta)) return WM_OK;
    if (!gamma || !mean || !inv_std) return set_error(WM_ERR_INVALID, "wm_batchnorm2d_bwd: null pointer");
    const int64_t n = batch * spatial;
    if (n > 0 && (!g || !x)) return set_error(WM_ERR_INVALID, "wm_batchnorm2d_bwd: null pointer");
    WM_CHECK_INIT();
    hipStream_t st = stream();
    const bool vec = spatial % 4 == 0 && aligned16(g) && aligned16(x) && (!gx || aligned16(gx));
    const BnGeom gm = bn_geom(batch, channels, spatial, vec,
                              vec ? bn_per_cu(bn_bwd_sums_kernel<true>, bn_bwd_apply_kernel<true>)
                                  : bn_per_cu(bn_bwd_sums_kernel<false>, bn_bwd_apply_kernel<false>));
    Workspace part((size_t)(channels * gm.chunks) * 3 * sizeof(double));
    if (!part.p) return set_error(WM_ERR_NOMEM, "wm_batchnorm2d_bwd: workspace");
    const BnBwdCoef ca{part.as<double>(), gm.chunks, n, gamma, inv_std, dgamma, acc_gamma, dbeta, acc_beta};
    const float nf = (float)n;
    const dim3 grid((unsigned)gm.chunks, (unsigned)channels);
    if (vec) launch_kernel(bn_bwd_sums_kernel<true>, grid, dim3(256), 0, st, g, x, mean, gm, part.as<double>());
    else launch_kernel(bn_bwd_sums_kernel<false>, grid, dim3(256), 0, st, g, x, mean, gm, part.as<double>());
    WM_TRY(check_launch("wm_batchnorm2d_bwd(sums)"));
    if (!gx || n == 0) {  // the parameter gradients alone
        launch_kernel(bn_bwd_finalize_kernel, dim3((unsigned)((channels + 255) / 256)), dim3(256), 0, st, ca,
                      channels);
        return check_launch("wm_batchnorm2d_bwd(finalize)");
    }
    if (vec)
        launch_kernel(bn_bwd_apply_kernel<true>, grid, dim3(256), 0, st, g, x, gamma, mean, inv_std, ca, gm, nf, gx,
                      acc_x);
    else
        launch_kernel(bn_bwd_apply_kernel<false>, grid, dim3(256), 0, st, g, x, gamma, mean, inv_std, ca, gm, nf, gx,
                      acc_x);
    return check_launch("wm_batchnorm2d_bwd(apply)");
}

int wm_attention_softmax_fwd(const float* scores, const float* mask, int64_t mask_batches, int64_t batch,
                             int64_t heads, int64_t tq, int64_t tk, float* attn) {
    if (batch < 0 || heads < 0 || tq < 0 || tk < 0)
        return set_error(WM_ERR_INVALID, "wm_attention_softmax_fwd: negative extent");
    if (mask && mask_batches != 1 && mask_batches != batch)
        return set_error(WM_ERR_INVALID, "wm_attention_softmax_fwd: mask batch must be 1 or the batch size");
    const int64_t rows = batch * heads * tq;
    if (rows == 0 || tk == 0) return WM_OK;
    if (!scores || !attn) return set_error(WM_ERR_INVALID, "wm_attention_softmax_fwd: null pointer");
    WM_CHECK_INIT();
    hipStream_t st = stream();
    const int64_t mstride = mask_batches == 1 ? 0 : tq * tk;
    const TileChoice tc = choose_tile(tk);
    const bool vec = tk % 4 == 0 && aligned16(scores) && aligned16(attn) && (!mask || aligned16(mask));
    // One row per workgroup on a grid that covers every row: 68.4 -> 75.7 %
    // of the HBM peak at [8, 16, 1024, 1024] (backward 66.5 -> 79.6 %)
    // against 32 one-wave workgroups per CU looping over rows.
    dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * (1 << 12)));
    if (tc.nt == 0) {
        launch_kernel(attn_softmax_fwd_long_kernel, grid, dim3(1024), 0, st, scores, mask, mstride, heads * tq,
                           tq, rows, tk, attn);
        return check_launch("wm_attention_softmax_fwd(long)");
    }
#define WM_ASF(NTv, IT)                                                                                          \
    if (tc.nt == NTv && tc.items == IT) {                                                                        \
        if (vec)                                                                                                 \
            launch_kernel((attn_softmax_fwd_kernel<NTv, IT, true>), grid, dim3(NTv), 0, st, scores, mask,   \
                               mstride, heads * tq, tq, rows, tk, attn);                                         \
        else                                                                                                     \
            launch_kernel((attn_softmax_fwd_kernel<NTv, IT, false>), grid, dim3(NTv), 0, st, scores, mask,  \
                               mstride, heads * tq, tq, rows, tk, attn);                                         \
        return check_launch("wm_attention_softmax_fwd");                                                         \
    }
    WM_ASF(64, 1) WM_ASF(64, 2) WM_ASF(64, 4) WM_ASF(64, 8)
    WM_ASF(1024, 1) WM_ASF(1024, 2) WM_ASF(1024, 4) WM_ASF(1024, 8)
#undef WM_ASF
    return set_error(WM_ERR_INVALID, "wm_attention_softmax_fwd: no tile");
}

int wm_attention_softmax_bwd(const float* attn, const float* d_attn, int64_t rows, int64_t tk, float* d_scores) {
    if (rows < 0 || tk < 0) return set_error(WM_ERR_INVALID, "wm_attention_softmax_bwd: negative extent");
    if (rows == 0 || tk == 0) return WM_OK;
    if (!attn || !d_attn || !d_scores) return set_error(WM_ERR_INVALID, "wm_attention_softmax_bwd: null pointer");
    WM_CHECK_INIT();
    hipStream_t st = stream();
    const TileChoice tc = choose_tile(tk);
    const bool vec = tk % 4 == 0 && aligned16(attn) && aligned16(d_attn) && aligned16(d_scores);
    dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * (1 << 12)));  // as in the forward
    if (tc.nt == 0) {
        launch_kernel(attn_softmax_bwd_long_kernel, grid, dim3(1024), 0, st, attn, d_attn, rows, tk, d_scores);
        return check_launch("wm_attention_softmax_bwd(long)");
    }
#define WM_ASB(NTv, IT)                                                                                         \
    if (tc.nt == NTv && tc.items == IT) {                                                                       \
        if (vec)                                                                                                \
            launch_kernel((attn_softmax_bwd_kernel<NTv, IT, true>), grid, dim3(NTv), 0, st, attn, d_attn,  \
                               rows, tk, d_scores);                                                             \
        else                                                                                                    \
            launch_kernel((attn_softmax_bwd_kernel<NTv, IT, false>), grid, dim3(NTv), 0, st, attn, d_attn, \
                               rows, tk, d_scores);                                                             \
        return check_launch("wm_attention_softmax_bwd");                                                        \
    }
    WM_ASB(64, 1) WM_ASB(64, 2) WM_ASB(64, 4) WM_ASB(64, 8)
    WM_ASB(1024, 1) WM_ASB(1024, 2) WM_ASB(1024, 4) WM_ASB(1024, 8)
#undef WM_ASB
    return set_error(WM_ERR_INVALID, "wm_attention_softmax_bwd: no tile");
}

int wm_dropout_mask(float* mask, int64_t n, float p, uint64_t seed) {
    if (n < 0) return set_error(WM_ERR_INVALID, "wm_dropout_mask: negative size");
    if (n == 0) return WM_OK;
    if (!mask) return set_error(WM_ERR_INVALID, "wm_dropout_mask: null pointer");
    WM_CHECK_INIT();
    const float scale = 1.0f / (1.0f - p);  // core/layer.cpp:55
    launch_kernel(dropout_mask_kernel, dim3(grid_for(n, 256)), dim3(256), 0, stream(), mask, n, p, scale, seed);
    return check_launch("wm_dropout_mask");
}

}  // extern "C"
