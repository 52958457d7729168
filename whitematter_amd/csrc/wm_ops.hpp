// Scalar semantics of every elementwise op, shared by the forward and
// backward kernels.  Each function is the per-element body of a reference
// loop (file:line relative to the reference root); the kernels around them
// only decide which elements to visit.
#pragma once

#include "wm_common.hpp"
#include "wm_pow.hpp"

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
    else if constexpr (OP == WM_POW) return pow_f32(a, b);  // :1394 / :1430
    else if constexpr (OP == WM_MAX) return (a < b) ? b : a;  // :1910
    else return (b < a) ? b : a;                        // :1997
}

// Kernel prologues: a kernel templated on a binary (unary) op code calls
// binary_prologue<OP>() (unary_prologue<OP>()) first, with all its threads;
// for pow it loads the pow tables into LDS.
template <int OP>
__device__ __forceinline__ void binary_prologue() {
    if constexpr (OP == WM_POW) pow_tables_to_lds();
}

template <int OP>
__device__ __forceinline__ void unary_prologue() {
    if constexpr (OP == WM_POWS) pow_tables_to_lds();
}

// ---- binary backward ------------------------------------------------------
// Contribution to dL/da and dL/db from one output element.  `o` is the
// forward output (only pow's d/db reads it).
template <int OP>
__device__ __forceinline__ float binary_da(float g, float a, float b) {
    if constexpr (OP == WM_ADD || OP == WM_SUB) return g;             // :913, :997
    else if constexpr (OP == WM_MUL) return g * b;                     // :1080
    else if constexpr (OP == WM_DIV) return g / b;                     // :1167
    else if constexpr (OP == WM_POW) return g * b * pow_f32(a, b - 1.0f); // :1405-1406
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
// buffer it is recomputed bit-identically (same pow on the same operands),
// which saves one full-size read.
template <int OP>
__device__ __forceinline__ float fwd_out_or(const float* o, int64_t i, float a, float b) {
    return o ? o[i] : binary_fwd<OP>(a, b);
}

// d/da and d/db of one output element together (only the requested ones are
// meaningful).  `o` is the forward output when `have_o`, else it is
// recomputed.  For pow the two share one log2|a|: it feeds the recomputed
// pow(a, b), pow(a, b - 1) and log(a), which costs about as much as one
// pow instead of three transcendental calls; those three carry a relative
// error of ~2e-7 (gradient precision), where binary_da / binary_db use the
// 1-ulp pow.
template <int OP>
__device__ __forceinline__ void binary_grads(float g, float a, float b, float o, bool have_o, bool want_da,
                                             bool want_db, float& da, float& db) {
    if constexpr (OP == WM_POW) {
        const PowGrad p = pow_grad_parts(a, b, want_db && !have_o, want_da, want_db);
        da = g * b * p.pbm1;
        db = g * (have_o ? o : p.out) * p.lga;
    } else {
        da = binary_da<OP>(g, a, b);
        db = binary_db<OP>(g, a, b, (db_reads_out<OP>() && !have_o) ? binary_fwd<OP>(a, b) : o);
    }
}

// binary_grads over N elements.  pow runs the branch-free table path for all
// N first and fixes up special operands in one branch afterwards, so the N
// table lookups overlap instead of each waiting behind its own branch.
template <int OP, int N>
__device__ __forceinline__ void binary_grads_n(const float (&g)[N], const float (&a)[N], const float (&b)[N],
                                               const float (&o)[N], bool have_o, bool want_da, bool want_db,
                                               float (&da)[N], float (&db)[N]) {
    if constexpr (OP == WM_POW) {
        const bool want_out = want_db && !have_o;
        PowGrad p[N];
        bool fix = false;
#pragma unroll
        for (int j = 0; j < N; ++j) {
            p[j] = pow_grad_table(a[j], b[j], want_out, want_da, want_db);
            fix |= pow_grad_needs_fix(a[j], b[j], p[j]);
        }
        if (fix) {
#pragma unroll
            for (int j = 0; j < N; ++j)
                if (pow_grad_needs_fix(a[j], b[j], p[j])) pow_grad_fix(a[j], b[j], want_out, want_da, want_db, p[j]);
        }
#pragma unroll
        for (int j = 0; j < N; ++j) {
            da[j] = g[j] * b[j] * p[j].pbm1;
            db[j] = g[j] * (have_o ? o[j] : p[j].out) * p[j].lga;
        }
    } else {
#pragma unroll
        for (int j = 0; j < N; ++j) binary_grads<OP>(g[j], a[j], b[j], o[j], have_o, want_da, want_db, da[j], db[j]);
    }
}

// pow's gradients over N elements that share the exponent b (q =
// pow_grad_exponent(b)): bit for bit binary_grads_n<WM_POW, N> with b
// everywhere, the exponent's share computed once.
template <int N>
__device__ __forceinline__ void pow_grads_n_exp(const float (&g)[N], const float (&a)[N], float b,
                                                const PowGradExponent& q, const float (&o)[N], bool have_o,
                                                bool want_da, bool want_db, float (&da)[N], float (&db)[N]) {
    const bool want_out = want_db && !have_o;
    PowGrad p[N];
    bool fix = false;
#pragma unroll
    for (int j = 0; j < N; ++j) {
        p[j] = pow_grad_table_exp(a[j], q, want_out, want_da, want_db);
        fix |= pow_grad_needs_fix_exp(a[j], q, p[j]);
    }
    if (fix) {
#pragma unroll
        for (int j = 0; j < N; ++j)
            if (pow_grad_needs_fix_exp(a[j], q, p[j])) pow_grad_fix(a[j], b, want_out, want_da, want_db, p[j]);
    }
#pragma unroll
    for (int j = 0; j < N; ++j) {
        da[j] = g[j] * b * p[j].pbm1;
        db[j] = g[j] * (have_o ? o[j] : p[j].out) * p[j].lga;
    }
}

// binary_fwd over U float4s, with pow's table path first and one fix-up
// branch after (as in binary_grads_n).
template <int OP, int U>
__device__ __forceinline__ void binary_fwd_v(float4 (&r)[U], const float4 (&a)[U], const float4 (&b)[U]) {
    if constexpr (OP == WM_POW) {
        bool fix = false;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            r[u] = make_float4(pow_table(a[u].x, b[u].x), pow_table(a[u].y, b[u].y), pow_table(a[u].z, b[u].z),
                               pow_table(a[u].w, b[u].w));
            fix |= pow_needs_fix(a[u].x, b[u].x) || pow_needs_fix(a[u].y, b[u].y) || pow_needs_fix(a[u].z, b[u].z) ||
                   pow_needs_fix(a[u].w, b[u].w);
        }
        if (fix) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (pow_needs_fix(a[u].x, b[u].x)) r[u].x = powf(a[u].x, b[u].x);
                if (pow_needs_fix(a[u].y, b[u].y)) r[u].y = powf(a[u].y, b[u].y);
                if (pow_needs_fix(a[u].z, b[u].z)) r[u].z = powf(a[u].z, b[u].z);
                if (pow_needs_fix(a[u].w, b[u].w)) r[u].w = powf(a[u].w, b[u].w);
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < U; ++u)
            r[u] = make_float4(binary_fwd<OP>(a[u].x, b[u].x), binary_fwd<OP>(a[u].y, b[u].y),
                               binary_fwd<OP>(a[u].z, b[u].z), binary_fwd<OP>(a[u].w, b[u].w));
    }
}

// ---- unary forward --------------------------------------------------------
template <int OP>
__device__ __forceinline__ float unary_fwd(float x, float p0, float p1) {
    if constexpr (OP == WM_RELU) return x > 0.0f ? x : 0.0f;            // simd_relu :139-158
    else if constexpr (OP == WM_SIGMOID) {                              // :1286
        // Below -80, 1 + exp(-x) rounds past FLT_MAX to inf (from -88.7) and
        // sigmoid(x) = exp(x) / (1 + exp(x)) is exp(x) to within 2e-35
        // relative: exp(x) keeps the results that fall in fp32's subnormal
        // range within the 2-ulp contract (the quotient gives 0 there).
        const bool far = x < -80.0f;
        const float e = expf(far ? x : -x);
        return far ? e : 1.0f / (1.0f + e);
    }
    else if constexpr (OP == WM_TANH) return tanh_fast(x);              // :1307
    else if constexpr (OP == WM_LOG)                                    // :1328
        // The +1e-8f is the reference's fp32 add; the log itself is taken in
        // double and rounded once, which keeps it within 1 ulp (logf's
        // device implementation measured 2.25 ulp at worst).
        return (float)log((double)(x + 1e-8f));
    else if constexpr (OP == WM_EXP) return expf(x);                    // :1348
    else if constexpr (OP == WM_POWS) return pow_f32(x, p0);            // :1368
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
    else if constexpr (OP == WM_POWS) return g * p0 * pow_f32(x, p0 - 1.0f);  // :1377-1378
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

// pow over U float4s that share one exponent y (a per-row or scalar
// exponent): the exponent's part of the table path and of the special-operand
// test is computed once (pow_exponent), the rest as in binary_fwd_v; equal
// to binary_fwd_v with b = y everywhere, bit for bit.
template <int U>
__device__ __forceinline__ void pow_fwd_v_exp(float4 (&r)[U], const float4 (&a)[U], float y) {
    const PowExponent e = pow_exponent(y);
    bool fix = false;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        r[u] = make_float4(pow_table_exp(a[u].x, e), pow_table_exp(a[u].y, e), pow_table_exp(a[u].z, e),
                           pow_table_exp(a[u].w, e));
        fix |= pow_needs_fix_exp(a[u].x, e) || pow_needs_fix_exp(a[u].y, e) || pow_needs_fix_exp(a[u].z, e) ||
               pow_needs_fix_exp(a[u].w, e);
    }
    if (fix) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (pow_needs_fix_exp(a[u].x, e)) r[u].x = powf(a[u].x, y);
            if (pow_needs_fix_exp(a[u].y, e)) r[u].y = powf(a[u].y, y);
            if (pow_needs_fix_exp(a[u].z, e)) r[u].z = powf(a[u].z, y);
            if (pow_needs_fix_exp(a[u].w, e)) r[u].w = powf(a[u].w, y);
        }
    }
}

// pow over the float4s of two rows, each row with its own exponent (y0 for
// a0, y1 for a1): pow_fwd_v_exp<1> of each, with one special-operand branch
// for both.  Bit for bit equal to binary_fwd_v with b = y0 / y1.
__device__ __forceinline__ void pow_fwd_pair(float4& r0, float4& r1, const float4& a0, const float4& a1, float y0,
                                             float y1) {
    const PowExponent e0 = pow_exponent(y0), e1 = pow_exponent(y1);
    r0 = make_float4(pow_table_exp(a0.x, e0), pow_table_exp(a0.y, e0), pow_table_exp(a0.z, e0),
                     pow_table_exp(a0.w, e0));
    r1 = make_float4(pow_table_exp(a1.x, e1), pow_table_exp(a1.y, e1), pow_table_exp(a1.z, e1),
                     pow_table_exp(a1.w, e1));
    const bool f0 = pow_needs_fix_exp(a0.x, e0) || pow_needs_fix_exp(a0.y, e0) || pow_needs_fix_exp(a0.z, e0) ||
                    pow_needs_fix_exp(a0.w, e0);
    const bool f1 = pow_needs_fix_exp(a1.x, e1) || pow_needs_fix_exp(a1.y, e1) || pow_needs_fix_exp(a1.z, e1) ||
                    pow_needs_fix_exp(a1.w, e1);
    if (f0 || f1) {
        if (pow_needs_fix_exp(a0.x, e0)) r0.x = powf(a0.x, y0);
        if (pow_needs_fix_exp(a0.y, e0)) r0.y = powf(a0.y, y0);
        if (pow_needs_fix_exp(a0.z, e0)) r0.z = powf(a0.z, y0);
        if (pow_needs_fix_exp(a0.w, e0)) r0.w = powf(a0.w, y0);
        if (pow_needs_fix_exp(a1.x, e1)) r1.x = powf(a1.x, y1);
        if (pow_needs_fix_exp(a1.y, e1)) r1.y = powf(a1.y, y1);
        if (pow_needs_fix_exp(a1.z, e1)) r1.z = powf(a1.z, y1);
        if (pow_needs_fix_exp(a1.w, e1)) r1.w = powf(a1.w, y1);
    }
}

// unary_fwd over U float4s; pow(x, p0) through pow_fwd_v_exp.
template <int OP, int U>
__device__ __forceinline__ void unary_fwd_v(float4 (&r)[U], const float4 (&x)[U], float p0, float p1) {
    if constexpr (OP == WM_POWS) {
        pow_fwd_v_exp<U>(r, x, p0);
    } else {
#pragma unroll
        for (int u = 0; u < U; ++u)
            r[u] = make_float4(unary_fwd<OP>(x[u].x, p0, p1), unary_fwd<OP>(x[u].y, p0, p1),
                               unary_fwd<OP>(x[u].z, p0, p1), unary_fwd<OP>(x[u].w, p0, p1));
    }
}

// unary_bwd over U float4s, plus the existing gradient when ACC; pow's
// pow(x, p0 - 1) through pow_fwd_v_exp.
template <int OP, bool ACC, int U>
__device__ __forceinline__ void unary_bwd_v(float4 (&r)[U], const float4 (&g)[U], const float4 (&x)[U],
                                            const float4 (&o)[U], const float4 (&gx)[U], float p0, float p1) {
    if constexpr (OP == WM_POWS) {
        float4 q[U];
        pow_fwd_v_exp<U>(q, x, p0 - 1.0f);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            r[u] = make_float4(g[u].x * p0 * q[u].x, g[u].y * p0 * q[u].y, g[u].z * p0 * q[u].z, g[u].w * p0 * q[u].w);
            if (ACC) { r[u].x += gx[u].x; r[u].y += gx[u].y; r[u].z += gx[u].z; r[u].w += gx[u].w; }
        }
    } else {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            r[u] = make_float4(unary_bwd<OP>(g[u].x, x[u].x, o[u].x, p0, p1), unary_bwd<OP>(g[u].y, x[u].y, o[u].y, p0, p1),
                               unary_bwd<OP>(g[u].z, x[u].z, o[u].z, p0, p1), unary_bwd<OP>(g[u].w, x[u].w, o[u].w, p0, p1));
            if (ACC) { r[u].x = gx[u].x + r[u].x; r[u].y = gx[u].y + r[u].y; r[u].z = gx[u].z + r[u].z; r[u].w = gx[u].w + r[u].w; }
        }
    }
}

}  // namespace wm
