// Scalar semantics of every elementwise op, shared by the forward and
// backward kernels.  Each function is the per-element body of a reference
// loop (file:line relative to the reference root); the kernels around them
// only decide which elements to visit.
#pragma once

#include "wm_common.hpp"

namespace wm {

// ---- binary forward -------------------------------------------------------
// std::max(a,b) is (a < b) ? b : a and std::min(a,b) is (b < a) ? b : a; the
// reference's element-wise max/min use them directly (core/tensor.cpp:1909,
// :1996), so NaN and signed-zero behaviour follow those two expressions.
template <int OP>
__device__ __forceinline__ float binary_fwd(float a, float b) {
    if constexpr (OP == WM_ADD) return a + b;          // :906 / :939
    else if constexpr (OP == WM_SUB) return a - b;     // :990 / :1022
    else if constexpr (OP == WM_MUL) return a * b;     // :1072 / :1104
    else if constexpr (OP == WM_DIV) return a / b;     // :1155 / :1191 (IEEE)
    else if constexpr (OP == WM_POW) return powf(a, b);  // :1394 / :1430
    else if constexpr (OP == WM_MAX) return (a < b) ? b : a;  // :1910
    else return (b < a) ? b : a;                        // :1997
}

// ---- binary backward ------------------------------------------------------
// Contribution to dL/da and dL/db from one output element.  `o` is the
// forward output (only pow's d/db reads it).
template <int OP>
__device__ __forceinline__ float binary_da(float g, float a, float b) {
    if constexpr (OP == WM_ADD || OP == WM_SUB) return g;             // :913, :997
    else if constexpr (OP == WM_MUL) return g * b;                     // :1080
    else if constexpr (OP == WM_DIV) return g / b;                     // :1167
    else if constexpr (OP == WM_POW) return g * b * powf(a, b - 1.0f); // :1405-1406
    else if constexpr (OP == WM_MAX) return (a >= b) ? g : 0.0f;       // :1920
    else return (a <= b) ? g : 0.0f;                                   // :2007
}

template <int OP>
__device__ __forceinline__ float binary_db(float g, float a, float b, float o) {
    if constexpr (OP == WM_ADD) return g;                              // :917
    else if constexpr (OP == WM_SUB) return -g;                        // :1001 (grad -= g)
    else if constexpr (OP == WM_MUL) return g * a;                     // :1085
    else if constexpr (OP == WM_DIV) return -(g * a / (b * b));        // :1171-1172 (grad -= ...)
    else if constexpr (OP == WM_POW) return g * o * logf(a);           // :1410-1411, no eps
    else if constexpr (OP == WM_MAX) return (a >= b) ? 0.0f : g;       // :1923
    else return (a <= b) ? 0.0f : g;                                   // :2010
}

// Whether the op's d/da or d/db needs the other operand / the output.
template <int OP> constexpr bool da_reads_b() { return OP != WM_ADD && OP != WM_SUB; }
template <int OP> constexpr bool da_reads_a() { return OP == WM_POW || OP == WM_MAX || OP == WM_MIN; }
template <int OP> constexpr bool db_reads_a() { return OP != WM_ADD && OP != WM_SUB; }
template <int OP> constexpr bool db_reads_b() { return OP == WM_DIV || OP == WM_MAX || OP == WM_MIN; }
template <int OP> constexpr bool db_reads_out() { return OP == WM_POW; }

// pow's d/db reads the forward output; when the caller passes no output
// buffer it is recomputed bit-identically (same powf on the same operands),
// which saves one full-size read.
template <int OP>
__device__ __forceinline__ float fwd_out_or(const float* o, int64_t i, float a, float b) {
    return o ? o[i] : binary_fwd<OP>(a, b);
}

// ---- unary forward --------------------------------------------------------
template <int OP>
__device__ __forceinline__ float unary_fwd(float x, float p0, float p1) {
    if constexpr (OP == WM_RELU) return x > 0.0f ? x : 0.0f;            // simd_relu :139-158
    else if constexpr (OP == WM_SIGMOID) return 1.0f / (1.0f + expf(-x)); // :1286
    else if constexpr (OP == WM_TANH) return tanhf(x);                  // :1307
    else if constexpr (OP == WM_LOG)                                    // :1328
        // The +1e-8f is the reference's fp32 add; the log itself is taken in
        // double and rounded once, which keeps it within 1 ulp (logf's
        // device implementation measured 2.25 ulp at worst).
        return (float)log((double)(x + 1e-8f));
    else if constexpr (OP == WM_EXP) return expf(x);                    // :1348
    else if constexpr (OP == WM_POWS) return powf(x, p0);               // :1368
    else if constexpr (OP == WM_SQRT) return sqrtf(x);                  // :1482
    else if constexpr (OP == WM_ABS) return fabsf(x);                   // :1503
    else if constexpr (OP == WM_CLAMP) {                                // :1529
        float m = (x < p1) ? x : p1;     // std::min(max_val, x)
        return (p0 < m) ? m : p0;        // std::max(min_val, m)
    } else return x * p0;                                               // simd_scale :117-136
}

// ---- unary backward -------------------------------------------------------
// Returns the value the reference closure adds to grad[i].  `x` is the
// forward input, `o` the forward output.
template <int OP>
__device__ __forceinline__ float unary_bwd(float g, float x, float o, float p0, float p1) {
    if constexpr (OP == WM_RELU) return g * (x > 0.0f ? 1.0f : 0.0f);   // :1274
    else if constexpr (OP == WM_SIGMOID) return g * o * (1.0f - o);     // :1295-1296
    else if constexpr (OP == WM_TANH) return g * (1.0f - o * o);        // :1316-1317
    else if constexpr (OP == WM_LOG) return g / (x + 1e-8f);            // :1336
    else if constexpr (OP == WM_EXP) return g * o;                      // :1356
    else if constexpr (OP == WM_POWS) return g * p0 * powf(x, p0 - 1.0f);  // :1377-1378
    else if constexpr (OP == WM_SQRT) return g / (2.0f * o);            // :1492
    else if constexpr (OP == WM_ABS)                                    // :1512-1517
        return x > 0.0f ? g : (x < 0.0f ? -g : 0.0f);
    else if constexpr (OP == WM_CLAMP)                                  // :1538-1540
        return (x > p0 && x < p1) ? g : 0.0f;
    else return g * p0;                                                 // :1248
}

// Ops whose "no contribution" case leaves grad[i] untouched in the reference
// (abs at 0 / NaN, clamp outside the open interval).  Adding 0.0f instead is
// identical for every grad value except -0.0f, which becomes +0.0f; gradients
// are compared with a tolerance, so the kernels add the 0.
template <int OP> constexpr bool unary_bwd_reads_x() {
    return OP == WM_RELU || OP == WM_LOG || OP == WM_POWS || OP == WM_ABS || OP == WM_CLAMP;
}
template <int OP> constexpr bool unary_bwd_reads_out() {
    return OP == WM_SIGMOID || OP == WM_TANH || OP == WM_EXP || OP == WM_SQRT;
}

}  // namespace wm
