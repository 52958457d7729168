// Loss heads on the device (reference core/loss.cpp).
//
// Classification heads (CrossEntropyLoss, FocalLoss).  The reference runs
// log_softmax / softmax over the whole [batch, classes] prediction, writes it
// to a new tensor, and then gathers the label entries in a host loop
// (core/loss.cpp:74-82, :271-285); the backward scatters into that tensor's
// gradient and lets the (log_)softmax closure expand it to the logits
// (:86-93, then core/tensor.cpp:1621-1632), or loops over every class on the
// host (:296-328).  Here:
//   forward   one row per workgroup, the row held in registers (RowTile, as
//             in the softmax kernels, through the same row_max_sum), the
//             label entry gathered by one lane; per-row statistics and the
//             row's loss term go to a small stats array.  Nothing of size
//             batch x classes is written.
//   backward  one streaming pass over the logits: each element's probability
//             is recomputed from the saved row statistics, so the gradient
//             costs one read of the logits and one write (or read-modify-
//             write) of the gradient.
// Rows longer than the register tile use an online single pass (running max
// and rescaled sum per thread), which still reads the row once.
//
// The batch mean is a fixed-order sum of the per-row terms (a single
// workgroup, or chunk partials then a single workgroup), so the loss is
// deterministic on a given device.
//
// NLLLoss is a gather (forward) and a scatter or one-hot row write
// (backward).  The element-wise losses whose reference bodies are host loops
// (SmoothL1, BCE, BCEWithLogits, KLDiv, BinaryFocal) are one grid-stride
// pass each way.
#include "wm_rows.hpp"

#include <algorithm>

#include "../../include/wm_loss.h"

namespace wm {
namespace {

// The eps of core/loss.cpp:137 (BCE), :276 (Focal), :342 (BinaryFocal).
constexpr float kProbEps = 1e-7f;

// static_cast<size_t>(t) when that is a class index in [0, classes):
// truncation toward zero; -1 for anything else (negative, too large, NaN).
__device__ __forceinline__ int64_t label_of(float t, int64_t classes) {
    if (!(t > -1.0f) || !(t < 9.0e18f)) return -1;
    const int64_t c = (int64_t)t;
    return c < classes ? c : -1;
}

// std::max / std::min on two floats: (a < b) ? b : a and (b < a) ? b : a, so
// a NaN first argument is returned (fmaxf / fminf would drop it).
__device__ __forceinline__ float std_max(float a, float b) { return a < b ? b : a; }
__device__ __forceinline__ float std_min(float a, float b) { return b < a ? b : a; }

// ---------------------------------------------------------------------------
// Per-row epilogue of the fused forward, run by one lane per row.
// ---------------------------------------------------------------------------

// Cross entropy: stats = {log_sum, x_label - log_sum}, the log_softmax entry
// at the label computed exactly as softmax_fwd_kernel computes it.
// Focal: stats = {max, 1/sum, p_label, 0}; focal_rows_kernel then turns
// p_label into the closure's per-row factors.  (Keeping the pow / log work
// out of the row kernel keeps it at the cross-entropy kernel's register
// count, and so at two 1024-thread workgroups per CU.)
template <bool FOCAL>
__device__ __forceinline__ void head_row_epilogue(const float* __restrict__ xr, float label, int64_t cols, float m,
                                                  float s, float* __restrict__ st) {
    const int64_t lab = label_of(label, cols);
    if (!FOCAL) {
        const float log_sum = m + logf(s);
        const float term = lab >= 0 ? xr[lab] - log_sum : NAN;
        *reinterpret_cast<float2*>(st) = make_float2(log_sum, term);
    } else {
        const float inv = 1.0f / s;
        const float pl = lab >= 0 ? exp_rr(xr[lab] - m) * inv : NAN;
        *reinterpret_cast<float4*>(st) = make_float4(m, inv, pl, 0.f);
    }
}

// Focal per-row factors, one lane per row: with p_t the clamped label
// probability and q = 1 - p_t (core/loss.cpp:279-285, :300-316),
//   stats = {max, 1/sum, F, K, B, l, 0, 0}
//   B = q^gamma,  K = gamma log(p_t) q^gamma + (-q^gamma),
//   F = q^(gamma-1) (gamma p_t log(p_t) + q),  l = -B log(p_t) (* alpha)
__global__ void __launch_bounds__(256) focal_rows_kernel(float* __restrict__ stats, int64_t rows, float gamma,
                                                          float alpha) {
    for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < rows; r += (int64_t)gridDim.x * 256) {
        float4* s4 = reinterpret_cast<float4*>(stats + r * WM_FOCAL_STATS);
        const float4 a = s4[0];
        const float pt = std_max(a.z, kProbEps);
        const float q = 1.0f - pt;
        const float b = powf(q, gamma);
        const float lg = logf(pt);
        float l = -b * lg;
        if (alpha >= 0.0f) l *= alpha;
        const float k = gamma * lg * b + -b;
        const float f = powf(q, gamma - 1.0f) * (gamma * pt * lg + q);
        s4[0] = make_float4(a.x, a.y, f, k);
        s4[1] = make_float4(b, l, 0.f, 0.f);
    }
}

template <bool FOCAL>
constexpr int head_stats() { return FOCAL ? WM_FOCAL_STATS : WM_CE_STATS; }

template <int NT, int ITEMS, bool VEC, bool FOCAL>
__global__ void __launch_bounds__(NT) head_fwd_kernel(const float* __restrict__ x, const float* __restrict__ labels,
                                                       int64_t rows, int64_t cols, float* __restrict__ stats) {
    __shared__ float lds_m[NT / 64], lds_s[NT / 64];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        RowTile<NT, ITEMS, VEC> tile;
        tile.load(x + r * cols, cols, -INFINITY);
        const RowMaxSum ms = row_max_sum<NT, ITEMS, VEC, false>(tile, lds_m, lds_s);
        if (threadIdx.x == 0)
            head_row_epilogue<FOCAL>(x + r * cols, labels[r], cols, ms.m, ms.s, stats + r * head_stats<FOCAL>());
    }
}

// Online single pass for long rows: each thread keeps a running max m_t and
// the sum s_t of exp(x - m_t) over its elements, rescaling s_t when m_t
// grows; the workgroup then combines them as row_max_sum does.  -inf
// elements contribute nothing (exp(-inf) = 0); an element equal to a +inf
// max contributes exp(inf - inf) = NaN, as in the reference.
template <bool FOCAL>
__global__ void __launch_bounds__(1024) head_fwd_long_kernel(const float* __restrict__ x,
                                                              const float* __restrict__ labels, int64_t rows,
                                                              int64_t cols, float* __restrict__ stats) {
    __shared__ float lds_m[16], lds_s[16];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * cols;
        float mt = -INFINITY, st = 0.f;
        for (int64_t c = threadIdx.x; c < cols; c += 1024) {
            const float v = ld_stream1(xr + c);
            if (v > mt) {
                st = st * exp_rr(mt - v) + (1.0f + (v - v));
                mt = v;
            } else if (v != -INFINITY) {
                st += exp_rr(v - mt);
            }
        }
        const float m = block_max_1<1024>(mt, lds_m);
        const float ct = mt == -INFINITY ? 0.f : exp_rr(mt - m);
        const float s = block_sum_1<1024>(st * ct, lds_s);
        if (threadIdx.x == 0) head_row_epilogue<FOCAL>(xr, labels[r], cols, m, s, stats + r * head_stats<FOCAL>());
    }
}

// ---------------------------------------------------------------------------
// Backward: one streaming pass per row.
// ---------------------------------------------------------------------------

enum HeadMode { kCrossEntropy = 0, kFocal = 1, kOneHot = 2 };

// Per-row constants of the backward.
struct HeadRow {
    int64_t lab;
    float a, b, c, d, e;
};

template <int MODE>
__device__ __forceinline__ HeadRow head_row(const float* __restrict__ stats, float label, int64_t r, int64_t cols,
                                            float scale) {
    HeadRow h{};
    h.lab = label_of(label, cols);
    if (MODE == kCrossEntropy) {
        // a = log_sum, b = the label's upstream gradient 0 - scale, c = the
        // row's gradient sum (the same value; NaN poisons a bad row).
        h.a = stats[r * WM_CE_STATS];
        h.b = 0.0f - scale;
        h.c = h.lab >= 0 ? h.b : NAN;
    } else if (MODE == kFocal) {
        const float4 s0 = *reinterpret_cast<const float4*>(stats + r * WM_FOCAL_STATS);
        h.a = s0.x;                        // max
        h.b = h.lab >= 0 ? s0.y : NAN;     // 1/sum
        h.c = s0.z;                        // F
        h.d = s0.w;                        // K
        h.e = stats[r * WM_FOCAL_STATS + 4];  // B
    } else {
        h.b = 0.0f - scale;
    }
    return h;
}

template <int MODE>
__device__ __forceinline__ float head_elem(float xv, bool is_label, const HeadRow& h, float scale, float alpha) {
    if (MODE == kCrossEntropy) {
        // log_softmax closure on the scattered gradient: g - exp(y) * sum(g).
        const float g = is_label ? h.b : 0.0f;
        const float y = xv - h.a;
        return g - exp_rr(y) * h.c;
    } else if (MODE == kFocal) {
        const float p = exp_rr(xv - h.a) * h.b;
        float g = is_label ? p * h.d + h.e : -p * h.c;
        if (alpha >= 0.0f) g *= alpha;
        return scale * g;
    } else {
        return is_label ? h.b : 0.0f;
    }
}

// Element-wise loss backward (pw_bwd_kernel): kUnroll float4 slots per
// thread (slot u of thread t at float4 q0 + u * 256), on a grid that covers
// the tensor: one slot measured 69.9 -> 82.1 % of the HBM peak for
// BCE-with-logits against 4 slots on 4 workgroups per CU.
constexpr int kUnroll = 1;

// Vector path of the head backward: one workgroup per 1024-column tile of a
// row (one float4 per thread), items (row, tile) with the tile fastest, on
// a grid that covers the matrix.  Short-lived workgroups reading adjacent
// tiles measured 64.6 -> 78.9 % of the HBM peak for cross entropy on
// [8192, 32000] (focal 64.8 -> 77 %, NLL's one-hot write 65 -> 76.9 %)
// against a workgroup walking each whole row.
template <int MODE>
__global__ void __launch_bounds__(256) head_bwd_tile_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ labels,
                                                             const float* __restrict__ stats,
                                                             const float* __restrict__ loss_grad,
                                                             float* __restrict__ gx, int acc, int64_t rows,
                                                             int64_t cols, float alpha) {
    const float scale = loss_grad[0] / (float)rows;
    const int64_t n4 = cols >> 2;
    const int64_t tiles = (n4 + 255) / 256;
    // rows * tiles < 2^32 (the host falls back to the row kernel otherwise).
    // The one-hot write (NLL, no loads) divides in 32 bits: 76.9 -> 83.7 %
    // of the HBM peak against the 64-bit division (~130 instructions per
    // workgroup); the modes that read the logits measured 2 points slower
    // with it (cross entropy 78.9 -> 77 %) and keep the 64-bit one.
    for (int64_t item = blockIdx.x; item < rows * tiles; item += gridDim.x) {
        const int64_t r = MODE == kOneHot ? (int64_t)((uint32_t)item / (uint32_t)tiles) : item / tiles;
        const int64_t q = (item - r * tiles) * 256 + threadIdx.x;
        const HeadRow h = head_row<MODE>(stats, labels[r], r, cols, scale);
        if (q >= n4) continue;
        const float* xr = x + r * cols;
        float* gr = gx + r * cols;
        const float4 xv = MODE != kOneHot ? ld_stream(xr + q * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 ov = acc ? ld_stream(gr + q * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
        const int64_t c0 = q * 4;
        float d0 = head_elem<MODE>(xv.x, c0 == h.lab, h, scale, alpha);
        float d1 = head_elem<MODE>(xv.y, c0 + 1 == h.lab, h, scale, alpha);
        float d2 = head_elem<MODE>(xv.z, c0 + 2 == h.lab, h, scale, alpha);
        float d3 = head_elem<MODE>(xv.w, c0 + 3 == h.lab, h, scale, alpha);
        if (acc) {
            d0 = ov.x + d0; d1 = ov.y + d1; d2 = ov.z + d2; d3 = ov.w + d3;
        }
        st_stream(gr + c0, make_float4(d0, d1, d2, d3));
    }
}

// Scalar path (cols % 4 != 0 or unaligned): one workgroup per row.
template <int MODE>
__global__ void __launch_bounds__(256) head_bwd_kernel(const float* __restrict__ x, const float* __restrict__ labels,
                                                        const float* __restrict__ stats,
                                                        const float* __restrict__ loss_grad, float* __restrict__ gx,
                                                        int acc, int64_t rows, int64_t cols, float alpha) {
    const float scale = loss_grad[0] / (float)rows;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const HeadRow h = head_row<MODE>(stats, labels[r], r, cols, scale);
        const float* xr = x + r * cols;
        float* gr = gx + r * cols;
        for (int64_t c = threadIdx.x; c < cols; c += 256) {
            const float xv = MODE != kOneHot ? ld_stream1(xr + c) : 0.f;
            float d = head_elem<MODE>(xv, c == h.lab, h, scale, alpha);
            if (acc) d = ld_stream1(gr + c) + d;
            st_stream1(gr + c, d);
        }
    }
}

// NLL: one lane per row.
__global__ void __launch_bounds__(256) nll_gather_kernel(const float* __restrict__ pred,
                                                          const float* __restrict__ labels, int64_t rows,
                                                          int64_t cols, float* __restrict__ terms) {
    for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < rows; r += (int64_t)gridDim.x * 256) {
        const int64_t lab = label_of(labels[r], cols);
        terms[r] = lab >= 0 ? pred[r * cols + lab] : NAN;
    }
}

__global__ void __launch_bounds__(256) nll_scatter_kernel(const float* __restrict__ labels,
                                                           const float* __restrict__ loss_grad, float* __restrict__ gx,
                                                           int64_t rows, int64_t cols) {
    const float scale = loss_grad[0] / (float)rows;
    for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < rows; r += (int64_t)gridDim.x * 256) {
        const int64_t lab = label_of(labels[r], cols);
        if (lab >= 0) gx[r * cols + lab] = gx[r * cols + lab] - scale;
    }
}

// ---------------------------------------------------------------------------
// Element-wise losses.
// ---------------------------------------------------------------------------

// One loss term per element, written as the reference's loop body adds it to
// the result (a subtracted quantity is returned negated).
template <int KIND>
__device__ __forceinline__ float pw_term(float x, float y, float p0, float p1) {
    if (KIND == WM_L_SMOOTH_L1) {  // :29-38
        const float d = x - y, ad = fabsf(d);
        return ad < p0 ? 0.5f * d * d / p0 : ad - 0.5f * p0;
    } else if (KIND == WM_L_BCE) {  // :140-144
        const float p = std_max(std_min(x, 1.0f - kProbEps), kProbEps);
        return -(y * logf(p) + (1.0f - y) * logf(1.0f - p));
    } else if (KIND == WM_L_BCE_LOGITS) {  // :175-181
        return std_max(x, 0.0f) - x * y + logf(1.0f + expf(-fabsf(x)));
    } else if (KIND == WM_L_KLDIV) {  // :228-233
        return y > 0.0f ? y * (logf(y) - x) : 0.0f;
    } else if (KIND == WM_L_KLDIV_LOG) {  // :218-226
        const float t = expf(y);
        return t > 0.0f ? t * (y - x) : 0.0f;
    } else {  // WM_L_BINARY_FOCAL, :344-364
        float p = 1.0f / (1.0f + expf(-x));
        p = std_max(std_min(p, 1.0f - kProbEps), kProbEps);
        const float pt = y * p + (1.0f - y) * (1.0f - p);
        const float fw = powf(1.0f - pt, p0);
        const float at = p1 >= 0.0f ? y * p1 + (1.0f - y) * (1.0f - p1) : 1.0f;
        return -(at * fw * logf(pt));
    }
}

// scale * d term / d x, the reference closure's increment.
template <int KIND>
__device__ __forceinline__ float pw_grad(float x, float y, float p0, float p1, float scale) {
    if (KIND == WM_L_SMOOTH_L1) {  // :49-61
        const float d = x - y;
        return fabsf(d) < p0 ? scale * d / p0 : scale * (d > 0.0f ? 1.0f : -1.0f);
    } else if (KIND == WM_L_BCE) {  // :153-159
        const float p = std_max(std_min(x, 1.0f - kProbEps), kProbEps);
        return scale * (-y / p + (1.0f - y) / (1.0f - p));
    } else if (KIND == WM_L_BCE_LOGITS) {  // :190-197
        const float s = 1.0f / (1.0f + expf(-x));
        return scale * (s - y);
    } else if (KIND == WM_L_KLDIV) {  // :244-253
        return scale * (-y);
    } else if (KIND == WM_L_KLDIV_LOG) {
        return scale * (-expf(y));
    } else {  // WM_L_BINARY_FOCAL, :375-414
        float p = 1.0f / (1.0f + expf(-x));
        p = std_max(std_min(p, 1.0f - kProbEps), kProbEps);
        const float pt = y * p + (1.0f - y) * (1.0f - p);
        const float q = 1.0f - pt;
        const float at = p1 >= 0.0f ? y * p1 + (1.0f - y) * (1.0f - p1) : 1.0f;
        const float dpt = (2.0f * y - 1.0f) * (p * (1.0f - p));
        float fg;
        if (p0 == 0.0f) {
            fg = -at / pt * dpt;
        } else {
            const float br = q / pt - p0 * logf(pt);
            fg = -at * dpt * powf(q, p0 - 1.0f) * br;
        }
        return scale * fg;
    }
}

// Per-workgroup partial sums of the terms; grid-stride, fixed order.
template <int KIND, bool VEC>
__global__ void __launch_bounds__(256) pw_fwd_kernel(const float* __restrict__ x, const float* __restrict__ y,
                                                      int64_t n, float p0, float p1, float* __restrict__ partials) {
    __shared__ float lds[4];
    float acc = 0.f;
    const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x, nthreads = (int64_t)gridDim.x * 256;
    int64_t tail0 = 0;
    if (VEC) {
        const int64_t n4 = n >> 2;
        for (int64_t q = tid; q < n4; q += nthreads) {
            const float4 a = ld_stream(x + q * 4), b = ld_stream(y + q * 4);
            acc += pw_term<KIND>(a.x, b.x, p0, p1);
            acc += pw_term<KIND>(a.y, b.y, p0, p1);
            acc += pw_term<KIND>(a.z, b.z, p0, p1);
            acc += pw_term<KIND>(a.w, b.w, p0, p1);
        }
        tail0 = n4 * 4;
    }
    for (int64_t i = tail0 + tid; i < n; i += nthreads) acc += pw_term<KIND>(ld_stream1(x + i), ld_stream1(y + i), p0, p1);
    acc = block_sum<256>(acc, lds);
    if (threadIdx.x == 0) partials[blockIdx.x] = acc;
}

template <int KIND, bool VEC>
__global__ void __launch_bounds__(256) pw_bwd_kernel(const float* __restrict__ x, const float* __restrict__ y,
                                                      int64_t n, float p0, float p1, float denom,
                                                      const float* __restrict__ loss_grad, float* __restrict__ gx,
                                                      int acc) {
    const float scale = loss_grad[0] / denom;
    const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x, nthreads = (int64_t)gridDim.x * 256;
    int64_t tail0 = 0;
    if (VEC) {
        // kUnroll float4 slots per thread per iteration, all loads first.
        const int64_t n4 = n >> 2;
        for (int64_t q0 = (int64_t)blockIdx.x * 256 * kUnroll + threadIdx.x; q0 < n4; q0 += nthreads * kUnroll) {
            float4 a[kUnroll], b[kUnroll], o[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t q = q0 + u * 256;
                if (q < n4) {
                    a[u] = ld_stream(x + q * 4);
                    b[u] = ld_stream(y + q * 4);
                    if (acc) o[u] = ld_stream(gx + q * 4);
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int64_t q = q0 + u * 256;
                if (q >= n4) continue;
                float4 d = make_float4(pw_grad<KIND>(a[u].x, b[u].x, p0, p1, scale),
                                       pw_grad<KIND>(a[u].y, b[u].y, p0, p1, scale),
                                       pw_grad<KIND>(a[u].z, b[u].z, p0, p1, scale),
                                       pw_grad<KIND>(a[u].w, b[u].w, p0, p1, scale));
                if (acc) d = make_float4(o[u].x + d.x, o[u].y + d.y, o[u].z + d.z, o[u].w + d.w);
                st_stream(gx + q * 4, d);
            }
        }
        tail0 = n4 * 4;
    }
    for (int64_t i = tail0 + tid; i < n; i += nthreads) {
        float d = pw_grad<KIND>(ld_stream1(x + i), ld_stream1(y + i), p0, p1, scale);
        if (acc) d = ld_stream1(gx + i) + d;
        st_stream1(gx + i, d);
    }
}

// ---------------------------------------------------------------------------
// The batch mean: out = (sign * sum_i v[i * stride]) / denom.
// ---------------------------------------------------------------------------

// Chunk partials: workgroup b sums v[i * stride] for i in [b*chunk, (b+1)*chunk).
__global__ void __launch_bounds__(256) sum_chunks_kernel(const float* __restrict__ v, int64_t n, int64_t stride,
                                                          int64_t chunk, float* __restrict__ partials) {
    __shared__ float lds[4];
    const int64_t lo = (int64_t)blockIdx.x * chunk, hi = n < lo + chunk ? n : lo + chunk;
    float acc = 0.f;
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) acc += v[i * stride];
    acc = block_sum<256>(acc, lds);
    if (threadIdx.x == 0) partials[blockIdx.x] = acc;
}

__global__ void __launch_bounds__(1024) sum_finalize_kernel(const float* __restrict__ v, int64_t n, int64_t stride,
                                                             float sign, float denom, float* __restrict__ out) {
    __shared__ float lds[16];
    float acc = 0.f;
    for (int64_t i = threadIdx.x; i < n; i += 1024) acc += v[i * stride];
    acc = block_sum<1024>(acc, lds);
    if (threadIdx.x == 0) out[0] = (sign * acc) / denom;
}

// Up to kDirect values go straight to the single-workgroup finalize; more go
// through chunk partials first.
constexpr int64_t kDirect = 65536;
constexpr int64_t kChunk = 16384;

int sum_to_loss(const float* v, int64_t n, int64_t stride, float sign, float denom, float* out, const char* what) {
    hipStream_t st = stream();
    if (n <= kDirect) {
        launch_kernel(sum_finalize_kernel, dim3(1), dim3(1024), 0, st, v, n, stride, sign, denom, out);
        return check_launch(what);
    }
    const int64_t parts = (n + kChunk - 1) / kChunk;
    Workspace ws((size_t)parts * sizeof(float));
    if (!ws.p) return set_error(WM_ERR_NOMEM, std::string(what) + ": workspace");
    launch_kernel(sum_chunks_kernel, dim3((unsigned)parts), dim3(256), 0, st, v, n, stride, kChunk,
                       ws.as<float>());
    WM_TRY(check_launch(what));
    launch_kernel(sum_finalize_kernel, dim3(1), dim3(1024), 0, st, ws.as<float>(), parts, (int64_t)1, sign,
                       denom, out);
    return check_launch(what);
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------

template <bool FOCAL>
int launch_head_fwd(const float* x, const float* labels, int64_t rows, int64_t cols, float gamma, float alpha,
                    float* stats, float* loss, const char* what) {
    hipStream_t st = stream();
    if (rows > 0) {
        const TileChoice tc = choose_tile(cols);
        const bool vec = cols % 4 == 0 && aligned16(x);
        dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * (tc.nt == 64 ? 32 : 4)));
        bool launched = false;
        if (tc.nt == 0) {
            launch_kernel(head_fwd_long_kernel<FOCAL>, grid, dim3(1024), 0, st, x, labels, rows, cols, stats);
            launched = true;
        }
#define WM_HF(NTv, IT)                                                                                          \
    if (!launched && tc.nt == NTv && tc.items == IT) {                                                          \
        if (vec)                                                                                                \
            launch_kernel((head_fwd_kernel<NTv, IT, true, FOCAL>), grid, dim3(NTv), 0, st, x, labels, rows, \
                               cols, stats);                                                                    \
        else                                                                                                    \
            launch_kernel((head_fwd_kernel<NTv, IT, false, FOCAL>), grid, dim3(NTv), 0, st, x, labels,    \
                               rows, cols, stats);                                                              \
        launched = true;                                                                                        \
    }
        WM_HF(64, 1) WM_HF(64, 2) WM_HF(64, 4) WM_HF(64, 8)
        WM_HF(1024, 1) WM_HF(1024, 2) WM_HF(1024, 4) WM_HF(1024, 8)
#undef WM_HF
        if (!launched) return set_error(WM_ERR_INVALID, std::string(what) + ": no tile");
        WM_TRY(check_launch(what));
        if (FOCAL) {
            launch_kernel(focal_rows_kernel, dim3(grid_for(rows, 256)), dim3(256), 0, st, stats, rows, gamma,
                               alpha);
            WM_TRY(check_launch(what));
        }
    }
    // CE: loss = -(sum of log-probabilities) / rows; focal: (sum of l_r) / rows.
    // No rows: 0 / 0 = NaN, as the reference's division gives.
    const int64_t ns = FOCAL ? WM_FOCAL_STATS : WM_CE_STATS;
    const float* terms = rows > 0 ? stats + (FOCAL ? 5 : 1) : nullptr;
    return sum_to_loss(terms, rows, ns, FOCAL ? 1.0f : -1.0f, (float)rows, loss, what);
}

template <int MODE>
int launch_head_bwd(const float* x, const float* labels, const float* stats, const float* loss_grad, float* gx,
                    int acc, int64_t rows, int64_t cols, float alpha, const char* what) {
    const bool vec = cols % 4 == 0 && aligned16(gx) && (MODE == kOneHot || aligned16(x));
    dim3 grid((unsigned)std::min<int64_t>(rows, (int64_t)num_cus() * 8));
    const int64_t tiles = (cols / 4 + 255) / 256;
    if (vec && rows * tiles < ((int64_t)1 << 32)) {
        launch_kernel((head_bwd_tile_kernel<MODE>), dim3(grid_for(rows * tiles, 1, 1 << 12)), dim3(256), 0,
                      stream(), x, labels, stats, loss_grad, gx, acc, rows, cols, alpha);
    } else
        launch_kernel((head_bwd_kernel<MODE>), grid, dim3(256), 0, stream(), x, labels, stats, loss_grad, gx,
                      acc, rows, cols, alpha);
    return check_launch(what);
}

template <int KIND>
int launch_pw_fwd(const float* x, const float* y, int64_t n, float p0, float p1, float denom, float* loss) {
    const bool vec = aligned16(x) && aligned16(y);
    const unsigned grid = grid_for((n + 3) / 4, 256, 4);
    Workspace ws((size_t)grid * sizeof(float));
    if (!ws.p) return set_error(WM_ERR_NOMEM, "wm_pointwise_loss_fwd: workspace");
    if (vec)
        launch_kernel((pw_fwd_kernel<KIND, true>), dim3(grid), dim3(256), 0, stream(), x, y, n, p0, p1,
                           ws.as<float>());
    else
        launch_kernel((pw_fwd_kernel<KIND, false>), dim3(grid), dim3(256), 0, stream(), x, y, n, p0, p1,
                           ws.as<float>());
    WM_TRY(check_launch("wm_pointwise_loss_fwd"));
    return sum_to_loss(ws.as<float>(), grid, 1, 1.0f, denom, loss, "wm_pointwise_loss_fwd");
}

template <int KIND>
int launch_pw_bwd(const float* x, const float* y, int64_t n, float p0, float p1, float denom, const float* loss_grad,
                  float* gx, int acc) {
    const bool vec = aligned16(x) && aligned16(y) && aligned16(gx);
    const unsigned grid = grid_for((n + 3) / 4, 256 * kUnroll, 1 << 12);
    if (vec)
        launch_kernel((pw_bwd_kernel<KIND, true>), dim3(grid), dim3(256), 0, stream(), x, y, n, p0, p1, denom,
                           loss_grad, gx, acc);
    else
        launch_kernel((pw_bwd_kernel<KIND, false>), dim3(grid), dim3(256), 0, stream(), x, y, n, p0, p1, denom,
                           loss_grad, gx, acc);
    return check_launch("wm_pointwise_loss_bwd");
}

int check_head(int64_t rows, int64_t cols, const void* x, const void* labels, const char* what) {
    if (rows < 0 || cols < 0) return set_error(WM_ERR_INVALID, std::string(what) + ": negative extent");
    if (rows > 0 && (!labels || (cols > 0 && !x))) return set_error(WM_ERR_INVALID, std::string(what) + ": null pointer");
    return WM_OK;
}

}  // namespace
}  // namespace wm

using namespace wm;

extern "C" {

int wm_cross_entropy_fwd(const float* logits, const float* labels, int64_t rows, int64_t classes, float* stats,
                         float* loss) {
    WM_TRY(check_head(rows, classes, logits, labels, "wm_cross_entropy_fwd"));
    if (!loss || (rows > 0 && !stats)) return set_error(WM_ERR_INVALID, "wm_cross_entropy_fwd: null output");
    if (rows > 0 && classes == 0)
        return set_error(WM_ERR_INVALID, "wm_cross_entropy_fwd: zero classes (no label can be valid)");
    if (rows > 0 && ((uintptr_t)stats & 7u))
        return set_error(WM_ERR_INVALID, "wm_cross_entropy_fwd: stats must be 8-byte aligned");
    WM_CHECK_INIT();
    return launch_head_fwd<false>(logits, labels, rows, classes, 0.f, 0.f, stats, loss, "wm_cross_entropy_fwd");
}

int wm_cross_entropy_bwd(const float* logits, const float* labels, const float* stats, const float* loss_grad,
                         float* grad, int accumulate, int64_t rows, int64_t classes) {
    WM_TRY(check_head(rows, classes, logits, labels, "wm_cross_entropy_bwd"));
    if (rows == 0 || classes == 0) return WM_OK;
    if (!stats || !loss_grad || !grad) return set_error(WM_ERR_INVALID, "wm_cross_entropy_bwd: null pointer");
    WM_CHECK_INIT();
    return launch_head_bwd<kCrossEntropy>(logits, labels, stats, loss_grad, grad, accumulate, rows, classes, 0.f,
                                          "wm_cross_entropy_bwd");
}

int wm_nll_fwd(const float* pred, const float* labels, int64_t rows, int64_t classes, float* loss) {
    WM_TRY(check_head(rows, classes, pred, labels, "wm_nll_fwd"));
    if (!loss) return set_error(WM_ERR_INVALID, "wm_nll_fwd: null output");
    WM_CHECK_INIT();
    Workspace terms((size_t)std::max<int64_t>(rows, 1) * sizeof(float));
    if (!terms.p) return set_error(WM_ERR_NOMEM, "wm_nll_fwd: workspace");
    if (rows > 0) {
        launch_kernel(nll_gather_kernel, dim3(grid_for(rows, 256)), dim3(256), 0, stream(), pred, labels, rows,
                           classes, terms.as<float>());
        WM_TRY(check_launch("wm_nll_fwd"));
    }
    return sum_to_loss(terms.as<float>(), rows, 1, -1.0f, (float)rows, loss, "wm_nll_fwd");
}

int wm_nll_bwd(const float* labels, const float* loss_grad, float* grad, int accumulate, int64_t rows,
               int64_t classes) {
    WM_TRY(check_head(rows, classes, grad, labels, "wm_nll_bwd"));
    if (rows == 0 || classes == 0) return WM_OK;
    if (!loss_grad) return set_error(WM_ERR_INVALID, "wm_nll_bwd: null loss_grad");
    WM_CHECK_INIT();
    if (accumulate) {
        launch_kernel(nll_scatter_kernel, dim3(grid_for(rows, 256)), dim3(256), 0, stream(), labels, loss_grad,
                           grad, rows, classes);
        return check_launch("wm_nll_bwd");
    }
    return launch_head_bwd<kOneHot>(nullptr, labels, nullptr, loss_grad, grad, 0, rows, classes, 0.f, "wm_nll_bwd");
}

int wm_focal_fwd(const float* logits, const float* labels, int64_t rows, int64_t classes, float gamma, float alpha,
                 float* stats, float* loss) {
    WM_TRY(check_head(rows, classes, logits, labels, "wm_focal_fwd"));
    if (!loss || (rows > 0 && !stats)) return set_error(WM_ERR_INVALID, "wm_focal_fwd: null output");
    if (rows > 0 && classes == 0) return set_error(WM_ERR_INVALID, "wm_focal_fwd: zero classes (no label can be valid)");
    if (rows > 0 && ((uintptr_t)stats & 15u))
        return set_error(WM_ERR_INVALID, "wm_focal_fwd: stats must be 16-byte aligned");
    WM_CHECK_INIT();
    return launch_head_fwd<true>(logits, labels, rows, classes, gamma, alpha, stats, loss, "wm_focal_fwd");
}

int wm_focal_bwd(const float* logits, const float* labels, const float* stats, const float* loss_grad, float* grad,
                 int accumulate, int64_t rows, int64_t classes, float gamma, float alpha) {
    (void)gamma;  // folded into the saved per-row factors
    WM_TRY(check_head(rows, classes, logits, labels, "wm_focal_bwd"));
    if (rows == 0 || classes == 0) return WM_OK;
    if (!stats || !loss_grad || !grad) return set_error(WM_ERR_INVALID, "wm_focal_bwd: null pointer");
    if ((uintptr_t)stats & 15u) return set_error(WM_ERR_INVALID, "wm_focal_bwd: stats must be 16-byte aligned");
    WM_CHECK_INIT();
    return launch_head_bwd<kFocal>(logits, labels, stats, loss_grad, grad, accumulate, rows, classes, alpha,
                                   "wm_focal_bwd");
}

int wm_pointwise_loss_fwd(int kind, const float* pred, const float* target, int64_t n, float p0, float p1,
                          float denom, float* loss) {
    if (n < 0) return set_error(WM_ERR_INVALID, "wm_pointwise_loss_fwd: negative size");
    if (!loss || (n > 0 && (!pred || !target))) return set_error(WM_ERR_INVALID, "wm_pointwise_loss_fwd: null pointer");
    WM_CHECK_INIT();
    switch (kind) {
        case WM_L_SMOOTH_L1: return launch_pw_fwd<WM_L_SMOOTH_L1>(pred, target, n, p0, p1, denom, loss);
        case WM_L_BCE: return launch_pw_fwd<WM_L_BCE>(pred, target, n, p0, p1, denom, loss);
        case WM_L_BCE_LOGITS: return launch_pw_fwd<WM_L_BCE_LOGITS>(pred, target, n, p0, p1, denom, loss);
        case WM_L_KLDIV: return launch_pw_fwd<WM_L_KLDIV>(pred, target, n, p0, p1, denom, loss);
        case WM_L_KLDIV_LOG: return launch_pw_fwd<WM_L_KLDIV_LOG>(pred, target, n, p0, p1, denom, loss);
        case WM_L_BINARY_FOCAL: return launch_pw_fwd<WM_L_BINARY_FOCAL>(pred, target, n, p0, p1, denom, loss);
        default: return set_error(WM_ERR_INVALID, "wm_pointwise_loss_fwd: unknown kind");
    }
}

int wm_pointwise_loss_bwd(int kind, const float* pred, const float* target, int64_t n, float p0, float p1,
                          float denom, const float* loss_grad, float* grad, int accumulate) {
    if (n < 0) return set_error(WM_ERR_INVALID, "wm_pointwise_loss_bwd: negative size");
    if (kind < WM_L_SMOOTH_L1 || kind > WM_L_BINARY_FOCAL)
        return set_error(WM_ERR_INVALID, "wm_pointwise_loss_bwd: unknown kind");
    if (n == 0) return WM_OK;
    if (!pred || !target || !loss_grad || !grad) return set_error(WM_ERR_INVALID, "wm_pointwise_loss_bwd: null pointer");
    WM_CHECK_INIT();
    switch (kind) {
        case WM_L_SMOOTH_L1: return launch_pw_bwd<WM_L_SMOOTH_L1>(pred, target, n, p0, p1, denom, loss_grad, grad, accumulate);
        case WM_L_BCE: return launch_pw_bwd<WM_L_BCE>(pred, target, n, p0, p1, denom, loss_grad, grad, accumulate);
        case WM_L_BCE_LOGITS: return launch_pw_bwd<WM_L_BCE_LOGITS>(pred, target, n, p0, p1, denom, loss_grad, grad, accumulate);
        case WM_L_KLDIV: return launch_pw_bwd<WM_L_KLDIV>(pred, target, n, p0, p1, denom, loss_grad, grad, accumulate);
        case WM_L_KLDIV_LOG: return launch_pw_bwd<WM_L_KLDIV_LOG>(pred, target, n, p0, p1, denom, loss_grad, grad, accumulate);
        default: return launch_pw_bwd<WM_L_BINARY_FOCAL>(pred, target, n, p0, p1, denom, loss_grad, grad, accumulate);
    }
}

}  // extern "C"
