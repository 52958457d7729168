/*
 * wm_oracle.c -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * A CPU restatement of whitematter's Tensor elementwise / broadcast /
 * reduction / softmax hot path (reference core/tensor.cpp, core/amp.h), used
 * only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 * Nothing under whitematter_amd/ links, loads or calls it.
 *
 * Each function follows the reference loop it cites: same visiting order,
 * same accumulation order, same strict comparisons.  The file is compiled
 * three times (oracle/Makefile):
 *   liboracle_f32.so  REAL=float, IEEE, no contraction: the bit-exact oracle
 *                     for add/sub/mul/div/neg/relu/abs/clamp/max/min/arg*;
 *   liboracle_f64.so  REAL=double: the fp64 oracle for the tolerance
 *                     contracts (transcendentals, sums, softmax, gradients);
 *   liboracle_abs.so  REAL=double with OR_ABS: every accumulation adds |term|
 *                     and the two subtractions of independently rounded
 *                     quantities (log_softmax's x - log_sum and g - e*sum(g))
 *                     add magnitudes, giving the "sum of |terms|" scale of
 *                     each result, so a tolerance can be stated relative to
 *                     the terms that cancel.
 * Inputs are always fp32 arrays (what the reference stores); outputs and
 * gradient accumulators are REAL.  Backward functions read the forward output
 * as fp32 -- the value the reference closure reads from result->data.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifndef REAL
#define REAL double
#endif

#ifdef OR_ABS
#define MAG(x) fabs((double)(x))
#define ACC(dst, term) ((dst) += MAG(term))
#define MINUS(x, y) (MAG(x) + MAG(y))
#else
#define MAG(x) (x)
#define ACC(dst, term) ((dst) += (term))
#define MINUS(x, y) ((x) - (y))
#endif

/* Floating-point mode.  A library built with -ffast-math elsewhere in the
 * process (the reference's, for one) may have switched flush-to-zero and
 * denormals-are-zero on for the calling thread; every entry point below sets
 * the mode it is defined with for its own duration and restores the caller's
 * on return: IEEE (both off) for the strict oracles, both on for the port
 * build, as in the reference's -ffast-math executables. */
#if defined(__x86_64__) || defined(__i386__)
#include <xmmintrin.h>
static void or_fp_restore(unsigned* saved) { _mm_setcsr(*saved); }
#ifdef OR_REF_FP_MODE
#define OR_FP_MODE(c) ((c) | 0x8040u)
#else
#define OR_FP_MODE(c) ((c) & ~0x8040u)
#endif
#define OR_FP_SCOPE                                                                  \
    unsigned or_fp_saved_ __attribute__((cleanup(or_fp_restore))) = _mm_getcsr(); \
    _mm_setcsr(OR_FP_MODE(or_fp_saved_))
#else
#define OR_FP_SCOPE (void)0
#endif

#define OR_MAX_DIMS 8

enum { OR_ADD, OR_SUB, OR_MUL, OR_DIV, OR_POW, OR_MAX, OR_MIN };
enum { OR_RELU, OR_SIGMOID, OR_TANH, OR_LOG, OR_EXP, OR_POWS, OR_SQRT, OR_ABSOP, OR_CLAMP, OR_SCALE };
enum { OR_R_SUM, OR_R_MEAN, OR_R_MAX, OR_R_MIN, OR_R_ARGMAX, OR_R_ARGMIN };

/* ---- broadcasting: core/tensor.cpp:338-398 ------------------------------ */

/* broadcast_shape, :338-358 (right-aligned; equal, or one side 1). */
int or_broadcast_shape(const int64_t* as, int an, const int64_t* bs, int bn, int64_t* os, int* on) {
    int nd = an > bn ? an : bn;
    for (int i = 0; i < nd; i++) {
        int64_t da = (i < nd - an) ? 1 : as[i - (nd - an)];
        int64_t db = (i < nd - bn) ? 1 : bs[i - (nd - bn)];
        if (da == db) os[i] = da;
        else if (da == 1) os[i] = db;
        else if (db == 1) os[i] = da;
        else return -1;
    }
    *on = nd;
    return 0;
}

/* compute_strides, :390-398. */
static void strides_of(const int64_t* shape, int nd, int64_t* st) {
    if (nd == 0) return;
    st[nd - 1] = 1;
    for (int i = nd - 2; i >= 0; i--) st[i] = st[i + 1] * shape[i + 1];
}

/* broadcast_index, :375-387: source offset of output multi-index idx. */
static int64_t bindex(const int64_t* idx, const int64_t* src_shape, const int64_t* src_st, int src_nd, int nd) {
    int64_t lin = 0;
    for (int i = 0; i < src_nd; i++) {
        int d = nd - src_nd + i;
        int64_t si = (src_shape[i] == 1) ? 0 : idx[d];
        lin += si * src_st[i];
    }
    return lin;
}

/* Odometer increment, :942-946. */
static void bump(int64_t* idx, const int64_t* os, int nd) {
    for (int d = nd - 1; d >= 0; d--) {
        idx[d]++;
        if (idx[d] < os[d]) break;
        idx[d] = 0;
    }
}

static int64_t numel_of(const int64_t* s, int nd) {
    int64_t n = 1;
    for (int i = 0; i < nd; i++) n *= s[i];
    return n;
}

/* ---- binary ops --------------------------------------------------------- */

/* One output element.  std::max/std::min expressions of :1910 / :1997. */
static REAL bin_fwd(int op, float a, float b) {
    switch (op) {
        case OR_ADD: return (REAL)a + (REAL)b;
        case OR_SUB: return (REAL)a - (REAL)b;
        case OR_MUL: return (REAL)a * (REAL)b;
        case OR_DIV: return (REAL)a / (REAL)b;
        case OR_POW: return (REAL)pow((REAL)a, (REAL)b);
        case OR_MAX: return (a < b) ? (REAL)b : (REAL)a;
        default: return (b < a) ? (REAL)b : (REAL)a;
    }
}

/* add :897-979, sub :981-1061, mul :1063-1145, div :1147-1235,
 * pow(Tensor) :1385-1475, max(Tensor) :1901-1984, min(Tensor) :1986-2073.
 * Same-shape fast path and broadcast path visit outputs in the same order. */
int or_binary(int op, REAL* out, const float* a, const int64_t* as, int an, const float* b, const int64_t* bs,
              int bn) {
    OR_FP_SCOPE;
    int64_t os[OR_MAX_DIMS], ast[OR_MAX_DIMS], bst[OR_MAX_DIMS], idx[OR_MAX_DIMS] = {0};
    int nd;
    if (or_broadcast_shape(as, an, bs, bn, os, &nd)) return -1;
    strides_of(as, an, ast);
    strides_of(bs, bn, bst);
    int64_t n = numel_of(os, nd);
    for (int64_t i = 0; i < n; i++) {
        out[i] = bin_fwd(op, a[bindex(idx, as, ast, an, nd)], b[bindex(idx, bs, bst, bn, nd)]);
        bump(idx, os, nd);
    }
    return 0;
}

/* Backward closures, output row-major order, accumulating into ga / gb
 * (either may be NULL = that input does not require grad).  out is the
 * forward output as stored (fp32), read only by pow's d/db.
 *   add  :956-976   ga += g;           gb += g
 *   sub  :1039-1058 ga += g;           gb -= g
 *   mul  :1122-1142 ga += g*b;         gb += g*a
 *   div  :1209-1232 ga += g/b;         gb -= g*a/(b*b)
 *   pow  :1448-1472 ga += g*b*pow(a,b-1); gb += g*out*log(a)
 *   max  :1962-1984 a >= b ? ga += g : gb += g
 *   min  :2049-2071 a <= b ? ga += g : gb += g                      */
int or_binary_bwd(int op, const float* g, const float* a, const int64_t* as, int an, const float* b,
                  const int64_t* bs, int bn, const float* out, REAL* ga, REAL* gb) {
    OR_FP_SCOPE;
    int64_t os[OR_MAX_DIMS], ast[OR_MAX_DIMS], bst[OR_MAX_DIMS], idx[OR_MAX_DIMS] = {0};
    int nd;
    if (or_broadcast_shape(as, an, bs, bn, os, &nd)) return -1;
    strides_of(as, an, ast);
    strides_of(bs, bn, bst);
    int64_t n = numel_of(os, nd);
    for (int64_t i = 0; i < n; i++) {
        int64_t ia = bindex(idx, as, ast, an, nd), ib = bindex(idx, bs, bst, bn, nd);
        REAL gg = g[i], va = a[ia], vb = b[ib];
        switch (op) {
            case OR_ADD:
                if (ga) ACC(ga[ia], gg);
                if (gb) ACC(gb[ib], gg);
                break;
            case OR_SUB:
                if (ga) ACC(ga[ia], gg);
                if (gb) ACC(gb[ib], -gg);
                break;
            case OR_MUL:
                if (ga) ACC(ga[ia], gg * vb);
                if (gb) ACC(gb[ib], gg * va);
                break;
            case OR_DIV:
                if (ga) ACC(ga[ia], gg / vb);
                if (gb) ACC(gb[ib], -(gg * va / (vb * vb)));
                break;
            case OR_POW:
                /* b - 1.0f is the reference's float subtraction: it rounds
                 * (-1.0000001f - 1.0f == -2.0f), which decides pow's domain */
                if (ga) ACC(ga[ia], gg * vb * (REAL)pow(va, (REAL)(b[ib] - 1.0f)));
                if (gb) ACC(gb[ib], gg * (REAL)out[i] * (REAL)log(va));
                break;
            case OR_MAX:
                if (a[ia] >= b[ib]) { if (ga) ACC(ga[ia], gg); }
                else if (gb) ACC(gb[ib], gg);
                break;
            default:
                if (a[ia] <= b[ib]) { if (ga) ACC(ga[ia], gg); }
                else if (gb) ACC(gb[ib], gg);
                break;
        }
        bump(idx, os, nd);
    }
    return 0;
}

/* ---- unary ops ---------------------------------------------------------- */

/* relu :1263-1279 (simd_relu :139-158: x > 0 ? x : 0), sigmoid :1281-1300,
 * tanh_ :1302-1321, log_ :1323-1341 (log(x + 1e-8f); the +1e-8f is the
 * reference's fp32 add and stays fp32 here), exp_ :1343-1361, pow(float)
 * :1363-1383, sqrt :1477-1496, abs :1498-1522, clamp :1524-1546
 * (std::max(lo, std::min(hi, x))), mul(float) :1237-1253. */
int or_unary(int op, REAL* out, const float* x, int64_t n, float p0, float p1) {
    OR_FP_SCOPE;
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        REAL r;
        switch (op) {
            case OR_RELU: r = v > 0 ? (REAL)v : (REAL)0; break;
            case OR_SIGMOID: r = (REAL)1 / ((REAL)1 + (REAL)exp(-(REAL)v)); break;
            case OR_TANH: r = (REAL)tanh((REAL)v); break;
            case OR_LOG: { float t = v + 1e-8f; r = (REAL)log((REAL)t); break; }
            case OR_EXP: r = (REAL)exp((REAL)v); break;
            case OR_POWS: r = (REAL)pow((REAL)v, (REAL)p0); break;
            case OR_SQRT: r = (REAL)sqrt((REAL)v); break;
            case OR_ABSOP: r = (REAL)fabsf(v); break;
            case OR_CLAMP: { float m = (v < p1) ? v : p1; r = (REAL)((p0 < m) ? m : p0); break; }
            default: r = (REAL)v * (REAL)p0; break;
        }
        out[i] = r;
    }
    return 0;
}

/* Closures: relu :1272-1276, sigmoid :1293-1298 (reads out), tanh :1314-1319
 * (reads out), log :1334-1339, exp :1354-1359 (reads out), pow(float)
 * :1374-1380, sqrt :1489-1494 (reads out), abs :1508-1519, clamp
 * :1533-1544, mul(float) :1246-1251.  gx accumulates. */
int or_unary_bwd(int op, const float* g, const float* x, const float* out, REAL* gx, int64_t n, float p0, float p1) {
    OR_FP_SCOPE;
    for (int64_t i = 0; i < n; i++) {
        REAL gg = g[i];
        switch (op) {
            case OR_RELU: ACC(gx[i], gg * (x[i] > 0 ? (REAL)1 : (REAL)0)); break;
            case OR_SIGMOID: { REAL s = out[i]; ACC(gx[i], gg * s * ((REAL)1 - s)); break; }
            case OR_TANH: { REAL t = out[i]; ACC(gx[i], gg * ((REAL)1 - t * t)); break; }
            case OR_LOG: { float t = x[i] + 1e-8f; ACC(gx[i], gg / (REAL)t); break; }
            case OR_EXP: ACC(gx[i], gg * (REAL)out[i]); break;
            case OR_POWS: ACC(gx[i], gg * (REAL)p0 * (REAL)pow((REAL)x[i], (REAL)(p0 - 1.0f))); break;
            case OR_SQRT: ACC(gx[i], gg / ((REAL)2 * (REAL)out[i])); break;
            case OR_ABSOP:
                if (x[i] > 0) ACC(gx[i], gg);
                else if (x[i] < 0) ACC(gx[i], -gg);
                break;
            case OR_CLAMP:
                if (x[i] > p0 && x[i] < p1) ACC(gx[i], gg);
                break;
            default: ACC(gx[i], gg * (REAL)p0); break;
        }
    }
    return 0;
}

/* ---- reductions --------------------------------------------------------- */

/* x viewed as [outer, n, inner], reduced over n, each output slot scanned in
 * increasing position order:
 *   sum full :1638-1645, dim 0 :1662-1671, dim 1 :1684-1693
 *   mean :1709-1721 (sum, then divide by n)
 *   max/min full :1727-1738 / :1816-1827, dim 0 :1755-1768 / :1844-1857,
 *   dim 1 :1783-1796 / :1872-1885 (start at the first element, replace only
 *   on strictly greater / smaller)
 *   argmax/argmin N-d :2096-2142 / :2170-2216 (same scan; index as fp32)
 * val: REAL values (or fp32-representable indices for arg*); idx: positions. */
int or_reduce(int op, const float* x, int64_t outer, int64_t n, int64_t inner, REAL* val, int64_t* idx) {
    OR_FP_SCOPE;
    if (n == 0 && op > OR_R_MEAN) return -1;
    for (int64_t o = 0; o < outer; o++) {
        for (int64_t i = 0; i < inner; i++) {
            const float* p = x + o * n * inner + i;
            int64_t slot = o * inner + i;
            if (op == OR_R_SUM || op == OR_R_MEAN) {
                REAL s = 0;
                for (int64_t k = 0; k < n; k++) ACC(s, (REAL)p[k * inner]);
                if (op == OR_R_MEAN) s = s / (REAL)(float)n;
                val[slot] = s;
            } else {
                int want_max = (op == OR_R_MAX || op == OR_R_ARGMAX);
                float best = p[0];
                int64_t bi = 0;
                for (int64_t k = 1; k < n; k++) {
                    float v = p[k * inner];
                    if (want_max ? (v > best) : (v < best)) { best = v; bi = k; }
                }
                if (val) val[slot] = (op == OR_R_MAX || op == OR_R_MIN) ? (REAL)best : (REAL)(float)bi;
                if (idx) idx[slot] = bi;
            }
        }
    }
    return 0;
}

/* Closures: sum/mean gx[o,k,i] += g[o,i] (:1649-1653, :1675-1681,
 * :1697-1703; mean reuses them, so no 1/n); max/min gx[o, idx, i] += g
 * (:1743-1745, :1774-1778, :1802-1806 and the min twins). */
int or_reduce_bwd(int op, const float* g, const int64_t* idx, int64_t outer, int64_t n, int64_t inner, REAL* gx) {
    OR_FP_SCOPE;
    for (int64_t o = 0; o < outer; o++) {
        for (int64_t i = 0; i < inner; i++) {
            int64_t slot = o * inner + i;
            if (op == OR_R_SUM || op == OR_R_MEAN) {
                for (int64_t k = 0; k < n; k++) ACC(gx[(o * n + k) * inner + i], (REAL)g[slot]);
            } else if (op == OR_R_MAX || op == OR_R_MIN) {
                ACC(gx[(o * n + idx[slot]) * inner + i], (REAL)g[slot]);
            } else {
                return -1;
            }
        }
    }
    return 0;
}

/* ---- softmax ------------------------------------------------------------ */

/* softmax :1556-1572: row max (std::max scan), out = exp(x - max), sum,
 * multiply by 1/sum. */
int or_softmax(REAL* out, const float* x, int64_t rows, int64_t cols) {
    OR_FP_SCOPE;
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * cols;
        REAL* orow = out + r * cols;
        float m = xr[0];
        for (int64_t j = 1; j < cols; j++) m = (m < xr[j]) ? xr[j] : m;
        REAL s = 0;
        for (int64_t j = 0; j < cols; j++) {
            orow[j] = (REAL)exp((REAL)xr[j] - (REAL)m);
            s += orow[j];
        }
        REAL inv = (REAL)1 / s;
        for (int64_t j = 0; j < cols; j++) orow[j] *= inv;
    }
    return 0;
}

/* log_softmax :1601-1616: out = x - (max + log(sum exp(x - max))). */
int or_log_softmax(REAL* out, const float* x, int64_t rows, int64_t cols) {
    OR_FP_SCOPE;
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * cols;
        float m = xr[0];
        for (int64_t j = 1; j < cols; j++) m = (m < xr[j]) ? xr[j] : m;
        REAL s = 0;
        for (int64_t j = 0; j < cols; j++) s += (REAL)exp((REAL)xr[j] - (REAL)m);
        REAL log_sum = (REAL)m + (REAL)log(s);
        for (int64_t j = 0; j < cols; j++) out[r * cols + j] = MINUS((REAL)xr[j], log_sum);
    }
    return 0;
}

/* softmax closure :1577-1588, the explicit Jacobian:
 *   gx[j] += sum_k g[k] * (j == k ? s_j (1 - s_j) : -s_j s_k)
 * with s = the stored fp32 output. */
int or_softmax_bwd(const float* g, const float* out, REAL* gx, int64_t rows, int64_t cols) {
    OR_FP_SCOPE;
    for (int64_t r = 0; r < rows; r++) {
        const float* yr = out + r * cols;
        const float* gr = g + r * cols;
        for (int64_t j = 0; j < cols; j++) {
            REAL sj = yr[j];
            for (int64_t k = 0; k < cols; k++) {
                REAL sk = yr[k];
                REAL d = (j == k) ? sj * ((REAL)1 - sj) : -sj * sk;
                ACC(gx[r * cols + j], (REAL)gr[k] * d);
            }
        }
    }
    return 0;
}

/* log_softmax closure :1621-1632: gx[j] += g[j] - exp(out[j]) * sum_k g[k]. */
int or_log_softmax_bwd(const float* g, const float* out, REAL* gx, int64_t rows, int64_t cols) {
    OR_FP_SCOPE;
    for (int64_t r = 0; r < rows; r++) {
        const float* gr = g + r * cols;
        const float* yr = out + r * cols;
        REAL gs = 0;
        for (int64_t j = 0; j < cols; j++) ACC(gs, (REAL)gr[j]);
        for (int64_t j = 0; j < cols; j++) {
            REAL sm = (REAL)exp((REAL)yr[j]);
            ACC(gx[r * cols + j], MINUS((REAL)gr[j], sm * gs));
        }
    }
    return 0;
}

/* ---- fp16 storage: core/amp.h:15-72 ------------------------------------- */

/* float_to_half :15-38 (truncating). */
static uint16_t f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    int32_t e = (int32_t)((x >> 23) & 0xFFu) - 127 + 15;
    uint32_t m = x & 0x7FFFFFu;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m = (m | 0x800000u) >> (1 - e);
        return (uint16_t)(sign | (m >> 13));
    } else if (e == 0xFF - 127 + 15) {
        if (m == 0) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7C00u | (m >> 13));
    } else if (e > 30) {
        return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | (m >> 13));
}

/* half_to_float :40-72 (normalising loop for subnormals). */
static float h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    float f;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
            memcpy(&f, &bits, 4);
            return f;
        }
        while ((m & 0x400u) == 0) { m <<= 1; e--; }
        e++;
        m &= ~0x400u;
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
        memcpy(&f, &bits, 4);
        return f;
    }
    bits = sign | ((e + 127 - 15) << 23) | (m << 13);
    memcpy(&f, &bits, 4);
    return f;
}

int or_f32_to_f16(uint16_t* out, const float* x, int64_t n) {
    OR_FP_SCOPE;
    for (int64_t i = 0; i < n; i++) out[i] = f2h(x[i]);
    return 0;
}

int or_f16_to_f32(float* out, const uint16_t* x, int64_t n) {
    OR_FP_SCOPE;
    for (int64_t i = 0; i < n; i++) out[i] = h2f(x[i]);
    return 0;
}

/* ---- parameter updates: core/optimizer.cpp, core/amp.h ---------------------
 * The steps are float arithmetic in every build (the reference's types); the
 * strict builds evaluate the reference's expressions in source order with
 * IEEE operations and no contraction, which is the bit-exact target of the
 * device kernels.  The sum of squares accumulates in REAL. */

/* Adam/AdamW's `1.0f - std::pow(beta, t)`: std::pow(float, int) is the
 * double pow, the subtraction is double and the assignment rounds to float
 * (core/optimizer.cpp:48-49, :78-79). */
float or_bias_correction(float beta, int t) {
    OR_FP_SCOPE;
    return (float)(1.0 - pow((double)beta, (double)t));
}

/* SGD::step, core/optimizer.cpp:22-36 */
int or_sgd_step(float* p, const float* g, float* vel, int64_t n, float lr, float momentum) {
    OR_FP_SCOPE;
    for (int64_t j = 0; j < n; j++) {
        if (momentum > 0.0f) {
            vel[j] = momentum * vel[j] + g[j];
            p[j] -= lr * vel[j];
        } else {
            p[j] -= lr * g[j];
        }
    }
    return 0;
}

/* Adam::step :46-66 (decoupled = 0) and AdamW::step :76-100 (decoupled = 1),
 * for one parameter tensor with the bias corrections of the current t. */
int or_adam_step(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                 float eps, float bc1, float bc2, float weight_decay, int decoupled) {
    OR_FP_SCOPE;
    for (int64_t j = 0; j < n; j++) {
        float gj = g[j];
        m[j] = beta1 * m[j] + (1.0f - beta1) * gj;
        v[j] = beta2 * v[j] + (1.0f - beta2) * gj * gj;
        float m_hat = m[j] / bc1;
        float v_hat = v[j] / bc2;
        if (decoupled) p[j] -= lr * (m_hat / (sqrtf(v_hat) + eps) + weight_decay * p[j]);
        else p[j] -= lr * m_hat / (sqrtf(v_hat) + eps);
    }
    return 0;
}

/* RMSprop::step, core/optimizer.cpp:112-138 */
int or_rmsprop_step(float* p, const float* g, float* v, float* buf, int64_t n, float lr, float alpha, float eps,
                    float momentum, float weight_decay) {
    OR_FP_SCOPE;
    for (int64_t j = 0; j < n; j++) {
        float gj = g[j];
        if (weight_decay != 0.0f) gj += weight_decay * p[j];
        v[j] = alpha * v[j] + (1.0f - alpha) * gj * gj;
        float avg = sqrtf(v[j]) + eps;
        if (momentum > 0.0f) {
            buf[j] = momentum * buf[j] + gj / avg;
            p[j] -= lr * buf[j];
        } else {
            p[j] -= lr * gj / avg;
        }
    }
    return 0;
}

/* get_grad_norm's accumulation for one tensor, core/optimizer.cpp:145-153,
 * in REAL (the fp64 build is the sum contract's reference). */
double or_grad_sumsq(const float* g, int64_t n) {
    OR_FP_SCOPE;
    REAL t = 0;
    for (int64_t i = 0; i < n; i++) t += (REAL)g[i] * (REAL)g[i];
    return (double)t;
}

/* clip_grad_value_, core/optimizer.cpp:166-177 */
int or_clip_grad_value(float* g, int64_t n, float c) {
    OR_FP_SCOPE;
    for (int64_t i = 0; i < n; i++) {
        if (g[i] > c) g[i] = c;
        else if (g[i] < -c) g[i] = -c;
    }
    return 0;
}

/* GradScaler::unscale's inner loop for one tensor, core/amp.h:134-142:
 * scales g in place up to the first element whose product is not finite
 * and returns that position (n when there is none). */
int64_t or_unscale_tensor(float* g, int64_t n, float inv_scale) {
    OR_FP_SCOPE;
    for (int64_t i = 0; i < n; i++) {
        float v = g[i] * inv_scale;
        if (!isfinite(v)) return i;
        g[i] = v;
    }
    return n;
}

/* ---- losses: core/loss.cpp ------------------------------------------------
 * Every function returns the loss through *loss (REAL) and accumulates the
 * prediction's gradient into gx (+=, caller-initialised), given the value of
 * the loss tensor's grad[0] (loss_grad) that the closure reads.
 *
 * Labels: the reference reads static_cast<size_t>(target->data[i])
 * (loss.cpp:80); a value that does not truncate to a class in [0, classes)
 * is an out-of-bounds access there.  Here such a row's loss term is NaN and
 * its gradient row NaN (cross entropy, focal) or untouched (NLL): the
 * behaviour the device heads define for it. */

static int64_t or_label(float t, int64_t classes) {
    if (!(t > -1.0f) || !(t < 9.0e18f)) return -1;
    int64_t c = (int64_t)t;
    return c < classes ? c : -1;
}

/* std::max / std::min on floats: (a < b) ? b : a and (b < a) ? b : a. */
static REAL or_std_max(REAL a, REAL b) { return a < b ? b : a; }
static REAL or_std_min(REAL a, REAL b) { return b < a ? b : a; }

#ifdef OR_ABS
#define PLUS(x, y) (MAG(x) + MAG(y))
#else
#define PLUS(x, y) ((x) + (y))
#endif

/* Row max and log(sum exp(x - max)) of log_softmax, core/tensor.cpp:1601-1612. */
static REAL or_row_log_sum(const float* xr, int64_t cols) {
    float m = xr[0];
    for (int64_t j = 1; j < cols; j++) m = (m < xr[j]) ? xr[j] : m;
    REAL s = 0;
    for (int64_t j = 0; j < cols; j++) s += (REAL)exp((REAL)xr[j] - (REAL)m);
    return (REAL)m + (REAL)log(s);
}

/* CrossEntropyLoss::forward, loss.cpp:67-84: log_probs = log_softmax(x)
 * (:74), result -= log_probs[i, label] over the batch, result /= batch. */
int or_cross_entropy(const float* x, const float* labels, int64_t rows, int64_t cols, REAL* loss) {
    OR_FP_SCOPE;
    REAL res = 0;
    for (int64_t r = 0; r < rows; r++) {
        int64_t lab = or_label(labels[r], cols);
        REAL lp = lab >= 0 ? MINUS((REAL)x[r * cols + lab], or_row_log_sum(x + r * cols, cols)) : (REAL)NAN;
        ACC(res, -lp);
    }
    *loss = res / (REAL)(float)rows;
    return 0;
}

/* Its backward: the closure at loss.cpp:87-93 (log_probs->grad[label] -=
 * scale, scale = grad / batch) followed by log_softmax's closure
 * (core/tensor.cpp:1621-1632) on that gradient. */
int or_cross_entropy_bwd(const float* x, const float* labels, int64_t rows, int64_t cols, float loss_grad, REAL* gx) {
    OR_FP_SCOPE;
    REAL scale = (REAL)loss_grad / (REAL)(float)rows;
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * cols;
        int64_t lab = or_label(labels[r], cols);
        REAL log_sum = or_row_log_sum(xr, cols);
        REAL gl = (REAL)0 - scale;            /* log_probs->grad[label], from 0 */
        REAL gs = lab >= 0 ? gl : (REAL)NAN;  /* the row's gradient sum */
        for (int64_t j = 0; j < cols; j++) {
            REAL lp = (REAL)xr[j] - log_sum;  /* log_probs[j] */
            REAL sm = (REAL)exp(lp);
            REAL g = (j == lab) ? gl : (REAL)0;
            ACC(gx[r * cols + j], MINUS(g, sm * gs));
        }
    }
    return 0;
}

/* NLLLoss::forward, loss.cpp:99-115. */
int or_nll(const float* pred, const float* labels, int64_t rows, int64_t cols, REAL* loss) {
    OR_FP_SCOPE;
    REAL res = 0;
    for (int64_t r = 0; r < rows; r++) {
        int64_t lab = or_label(labels[r], cols);
        ACC(res, -(lab >= 0 ? (REAL)pred[r * cols + lab] : (REAL)NAN));
    }
    *loss = res / (REAL)(float)rows;
    return 0;
}

/* NLLLoss's closure, loss.cpp:118-124: grad[i, label] -= grad / batch. */
int or_nll_bwd(const float* labels, int64_t rows, int64_t cols, float loss_grad, REAL* gx) {
    OR_FP_SCOPE;
    REAL scale = (REAL)loss_grad / (REAL)(float)rows;
    for (int64_t r = 0; r < rows; r++) {
        int64_t lab = or_label(labels[r], cols);
        if (lab >= 0) ACC(gx[r * cols + lab], -scale);
    }
    return 0;
}

/* softmax of one row as core/tensor.cpp:1556-1572 computes it. */
static void or_row_softmax(const float* xr, int64_t cols, REAL* p) {
    float m = xr[0];
    for (int64_t j = 1; j < cols; j++) m = (m < xr[j]) ? xr[j] : m;
    REAL s = 0;
    for (int64_t j = 0; j < cols; j++) {
        p[j] = (REAL)exp((REAL)xr[j] - (REAL)m);
        s += p[j];
    }
    REAL inv = (REAL)1 / s;
    for (int64_t j = 0; j < cols; j++) p[j] *= inv;
}

/* FocalLoss::forward, loss.cpp:260-294. */
int or_focal(const float* x, const float* labels, int64_t rows, int64_t cols, float gamma, float alpha, REAL* loss) {
    OR_FP_SCOPE;
    REAL* p = (REAL*)malloc(sizeof(REAL) * (size_t)(cols > 0 ? cols : 1));
    if (!p) return 1;
    const REAL eps = (REAL)1e-7f;
    REAL res = 0;
    for (int64_t r = 0; r < rows; r++) {
        int64_t lab = or_label(labels[r], cols);
        or_row_softmax(x + r * cols, cols, p);
        REAL pt = or_std_max(lab >= 0 ? p[lab] : (REAL)NAN, eps);
        REAL fw = (REAL)pow((REAL)1 - pt, (REAL)gamma);
        REAL li = -fw * (REAL)log(pt);
        if (alpha >= 0) li *= (REAL)alpha;
        ACC(res, li);
    }
    free(p);
    *loss = res / (REAL)(float)rows;
    return 0;
}

/* FocalLoss's closure, loss.cpp:296-328, over every class of every row. */
int or_focal_bwd(const float* x, const float* labels, int64_t rows, int64_t cols, float gamma, float alpha,
                 float loss_grad, REAL* gx) {
    OR_FP_SCOPE;
    REAL* p = (REAL*)malloc(sizeof(REAL) * (size_t)(cols > 0 ? cols : 1));
    if (!p) return 1;
    const REAL eps = (REAL)1e-7f, gm = (REAL)gamma;
    REAL scale = (REAL)loss_grad / (REAL)(float)rows;
    for (int64_t r = 0; r < rows; r++) {
        int64_t lab = or_label(labels[r], cols);
        or_row_softmax(x + r * cols, cols, p);
        REAL pt = or_std_max(lab >= 0 ? p[lab] : (REAL)NAN, eps);
        REAL q = (REAL)1 - pt;
        for (int64_t c = 0; c < cols; c++) {
            REAL pc = lab >= 0 ? p[c] : (REAL)NAN;
            REAL gv;
            if (c == lab) {
                REAL term1 = gm * (REAL)log(pt) * (REAL)pow(q, gm);
                REAL term2 = -(REAL)pow(q, gm);
                gv = PLUS(pc * PLUS(term1, term2), (REAL)pow(q, gm));
            } else {
                REAL ft = (REAL)pow(q, gm - (REAL)1);
                gv = -pc * (ft * PLUS(gm * pt * (REAL)log(pt), q));
            }
            if (alpha >= 0) gv *= (REAL)alpha;
            ACC(gx[r * cols + c], scale * gv);
        }
    }
    free(p);
    return 0;
}

/* The element-wise losses: one term per element (the quantity the loop adds
 * to the result; a subtracted one negated) and one gradient increment.
 * kind: 0 SmoothL1 (p0 = beta), 1 BCE, 2 BCEWithLogits, 3 KLDiv,
 * 4 KLDiv with log_target, 5 BinaryFocal (p0 = gamma, p1 = alpha). */
static REAL or_pw_term(int kind, float xf, float yf, float p0, float p1) {
    const REAL x = xf, y = yf, one = 1;
    const REAL eps = (REAL)1e-7f, hi = (REAL)(1.0f - 1e-7f);
    switch (kind) {
        case 0: { /* loss.cpp:29-38 */
            REAL ad = x - y, b = p0;
            if (ad < 0) ad = -ad;
            REAL d = MINUS(x, y); /* |x| + |y| in the magnitude build */
            return ad < b ? (REAL)0.5f * d * d / b : MINUS(ad, (REAL)0.5f * b);
        }
        case 1: { /* :140-144 */
            REAL p = or_std_max(or_std_min(x, hi), eps);
            return -PLUS(y * (REAL)log(p), (one - y) * (REAL)log(one - p));
        }
        case 2: /* :175-181 */
            return PLUS(MINUS(or_std_max(x, 0), x * y), (REAL)log(one + (REAL)exp(-fabs((double)x))));
        case 3: /* :228-233 */
            return y > 0 ? y * MINUS((REAL)log(y), x) : (REAL)0;
        case 4: { /* :218-226 */
            REAL t = (REAL)exp(y);
            return t > 0 ? t * MINUS(y, x) : (REAL)0;
        }
        default: { /* :344-364 */
            REAL p = one / (one + (REAL)exp(-x));
            p = or_std_max(or_std_min(p, hi), eps);
            REAL pt = y * p + (one - y) * (one - p);
            REAL fw = (REAL)pow(one - pt, (REAL)p0);
            REAL at = p1 >= 0 ? y * (REAL)p1 + (one - y) * (one - (REAL)p1) : one;
            return -(at * fw * (REAL)log(pt));
        }
    }
}

static REAL or_pw_grad(int kind, float xf, float yf, float p0, float p1, REAL scale) {
    const REAL x = xf, y = yf, one = 1;
    const REAL eps = (REAL)1e-7f, hi = (REAL)(1.0f - 1e-7f);
    switch (kind) {
        case 0: { /* :49-61 */
            REAL d = x - y, b = p0;
            REAL ad = d < 0 ? -d : d;
            return ad < b ? scale * d / b : scale * (d > 0 ? one : -one);
        }
        case 1: { /* :153-159 */
            REAL p = or_std_max(or_std_min(x, hi), eps);
            return scale * PLUS(-y / p, (one - y) / (one - p));
        }
        case 2: { /* :190-197 */
            REAL s = one / (one + (REAL)exp(-x));
            return scale * MINUS(s, y);
        }
        case 3: /* :244-253 */
            return scale * (-y);
        case 4:
            return scale * (-(REAL)exp(y));
        default: { /* :375-414 */
            REAL p = one / (one + (REAL)exp(-x));
            p = or_std_max(or_std_min(p, hi), eps);
            REAL pt = y * p + (one - y) * (one - p);
            REAL q = one - pt;
            REAL at = p1 >= 0 ? y * (REAL)p1 + (one - y) * (one - (REAL)p1) : one;
            REAL dpt = ((REAL)2 * y - one) * (p * (one - p));
            REAL fg;
            if (p0 == 0) {
                fg = -at / pt * dpt;
            } else {
                REAL br = PLUS(q / pt, -(REAL)p0 * (REAL)log(pt));
                fg = -at * dpt * (REAL)pow(q, (REAL)p0 - one) * br;
            }
            return scale * fg;
        }
    }
}

/* The loop over the elements and the final division (by n, or by the batch
 * size for the KL divergence): loss.cpp:29-39 and the matching lines of each
 * loss. */
int or_pointwise_loss(int kind, const float* x, const float* y, int64_t n, float p0, float p1, float denom, REAL* loss) {
    OR_FP_SCOPE;
    REAL res = 0;
    for (int64_t i = 0; i < n; i++) ACC(res, or_pw_term(kind, x[i], y[i], p0, p1));
    *loss = res / (REAL)denom;
    return 0;
}

int or_pointwise_loss_bwd(int kind, const float* x, const float* y, int64_t n, float p0, float p1, float denom,
                          float loss_grad, REAL* gx) {
    OR_FP_SCOPE;
    REAL scale = (REAL)loss_grad / (REAL)denom;
    for (int64_t i = 0; i < n; i++) ACC(gx[i], or_pw_grad(kind, x[i], y[i], p0, p1, scale));
    return 0;
}

/* ---- normalisation layers and the attention softmax: core/layer.cpp -------
 * Statistics the backward captures (mean, inv_std) are outputs of the
 * forward (REAL) and inputs of the backward (float: the values the closure
 * captured).  Gradients accumulate (+=) into caller-initialised arrays; a
 * NULL gradient array is skipped. */

/* LayerNorm::forward, layer.cpp:395-446.  The statistics are computed
 * with plain arithmetic in every build (the magnitude build's scales use the
 * true mean and 1/std); only the output takes magnitudes. */
int or_layernorm(const float* x, const float* gamma, const float* beta, int64_t rows, int64_t n, float eps, REAL* y,
                 REAL* mean, REAL* inv_std) {
    OR_FP_SCOPE;
    const REAL nf = (REAL)(float)n;
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * n;
        REAL s = 0;
        for (int64_t i = 0; i < n; i++) s += (REAL)xr[i];
        REAL m = s / nf;
        REAL q = 0;
        for (int64_t i = 0; i < n; i++) {
            REAL d = (REAL)xr[i] - m;
            q += d * d;
        }
        REAL var = q / nf;
        REAL iv = (REAL)1 / (REAL)sqrt(var + (REAL)eps);
        for (int64_t i = 0; i < n; i++) {
            REAL xn = MINUS((REAL)xr[i], m) * iv;
            y[r * n + i] = PLUS((REAL)gamma[i] * xn, (REAL)beta[i]);
        }
        mean[r] = m;
        inv_std[r] = iv;
    }
    return 0;
}

/* LayerNorm's closure, layer.cpp:453-504. */
int or_layernorm_bwd(const float* g, const float* x, const float* gamma, const float* mean, const float* inv_std,
                     int64_t rows, int64_t n, REAL* gx, REAL* dgamma, REAL* dbeta) {
    OR_FP_SCOPE;
    const REAL nf = (REAL)(float)n;
    for (int64_t r = 0; r < rows; r++) {
        const float* gr = g + r * n;
        const float* xr = x + r * n;
        const REAL m = mean[r], iv = inv_std[r];
        for (int64_t i = 0; i < n; i++) {
            REAL xn = MINUS((REAL)xr[i], m) * iv;
            if (dgamma) ACC(dgamma[i], (REAL)gr[i] * xn);
            if (dbeta) ACC(dbeta[i], (REAL)gr[i]);
        }
        REAL s1 = 0, s2 = 0;
        for (int64_t i = 0; i < n; i++) {
            REAL dy = gr[i];
            REAL xn = MINUS((REAL)xr[i], m) * iv;
            ACC(s1, dy * (REAL)gamma[i]);
            ACC(s2, dy * (REAL)gamma[i] * xn);
        }
        REAL mdg = s1 / nf, mdgx = s2 / nf;
        if (gx)
            for (int64_t i = 0; i < n; i++) {
                REAL dy = gr[i];
                REAL xn = MINUS((REAL)xr[i], m) * iv;
                ACC(gx[r * n + i], iv * MINUS(MINUS(dy * (REAL)gamma[i], mdg), xn * mdgx));
            }
    }
    return 0;
}

/* BatchNorm2d::forward, layer.cpp:202-280, x [B, C, S].  running_mean /
 * running_var are updated in place when training (rounded to float, what the
 * reference stores).  Statistics in plain arithmetic in every build, as for
 * LayerNorm. */
int or_batchnorm2d(const float* x, const float* gamma, const float* beta, float* running_mean, float* running_var,
                   int64_t B, int64_t C, int64_t S, float eps, float momentum, int training, REAL* y, REAL* mean,
                   REAL* inv_std) {
    OR_FP_SCOPE;
    const REAL nf = (REAL)(float)(B * S);
    for (int64_t c = 0; c < C; c++) {
        REAL m, var;
        if (training) {
            REAL s = 0;
            for (int64_t b = 0; b < B; b++)
                for (int64_t i = 0; i < S; i++) s += (REAL)x[(b * C + c) * S + i];
            m = s / nf;
            REAL q = 0;
            for (int64_t b = 0; b < B; b++)
                for (int64_t i = 0; i < S; i++) {
                    REAL d = (REAL)x[(b * C + c) * S + i] - m;
                    q += d * d;
                }
            var = q / nf;
            const REAL mo = (REAL)momentum;
            running_mean[c] = (float)(((REAL)1 - mo) * (REAL)running_mean[c] + mo * m);
            running_var[c] = (float)(((REAL)1 - mo) * (REAL)running_var[c] + mo * var);
        } else {
            m = running_mean[c];
            var = running_var[c];
        }
        mean[c] = m;
        inv_std[c] = (REAL)1 / (REAL)sqrt(var + (REAL)eps);
    }
    for (int64_t b = 0; b < B; b++)
        for (int64_t c = 0; c < C; c++)
            for (int64_t i = 0; i < S; i++) {
                int64_t idx = (b * C + c) * S + i;
                REAL xn = MINUS((REAL)x[idx], mean[c]) * inv_std[c];
                y[idx] = PLUS((REAL)gamma[c] * xn, (REAL)beta[c]);
            }
    return 0;
}

/* BatchNorm2d's closure, layer.cpp:287-374, with the captured mean / inv_std. */
int or_batchnorm2d_bwd(const float* g, const float* x, const float* gamma, const float* mean, const float* inv_std,
                       int64_t B, int64_t C, int64_t S, REAL* gx, REAL* dgamma, REAL* dbeta) {
    OR_FP_SCOPE;
    const REAL nf = (REAL)(float)(B * S);
    for (int64_t c = 0; c < C; c++) {
        const REAL m = mean[c], iv = inv_std[c], gm = gamma[c];
        REAL dg = 0, db = 0, dvar = 0, sdx = 0, sxd = 0;
        for (int64_t b = 0; b < B; b++)
            for (int64_t i = 0; i < S; i++) {
                int64_t idx = (b * C + c) * S + i;
                REAL xn = MINUS((REAL)x[idx], m) * iv;
                ACC(dg, (REAL)g[idx] * xn);
                ACC(db, (REAL)g[idx]);
            }
        for (int64_t b = 0; b < B; b++)
            for (int64_t i = 0; i < S; i++) {
                int64_t idx = (b * C + c) * S + i;
                REAL dxn = (REAL)g[idx] * gm;
                ACC(dvar, dxn * MINUS((REAL)x[idx], m) * (REAL)-0.5f * iv * iv * iv);
            }
        for (int64_t b = 0; b < B; b++)
            for (int64_t i = 0; i < S; i++) {
                int64_t idx = (b * C + c) * S + i;
                ACC(sdx, (REAL)g[idx] * gm * (-iv));
                ACC(sxd, (REAL)-2.0f * MINUS((REAL)x[idx], m));
            }
        REAL dmean = PLUS(sdx, dvar * sxd / nf);
        if (gx)
            for (int64_t b = 0; b < B; b++)
                for (int64_t i = 0; i < S; i++) {
                    int64_t idx = (b * C + c) * S + i;
                    REAL dxn = (REAL)g[idx] * gm;
                    REAL t = PLUS(PLUS(dxn * iv, dvar * (REAL)2.0f * MINUS((REAL)x[idx], m) / nf), dmean / nf);
                    ACC(gx[idx], t);
                }
        if (dgamma) ACC(dgamma[c], dg);
        if (dbeta) ACC(dbeta[c], db);
    }
    return 0;
}

/* MultiHeadAttention's mask add (layer.cpp:1198-1204) and softmax
 * (:1210-1237): max from -FLT_MAX, exp, sum, division.  mask NULL or
 * [mask_batches, 1, tq, tk]. */
int or_attention_softmax(const float* scores, const float* mask, int64_t mask_batches, int64_t B, int64_t H,
                         int64_t tq, int64_t tk, REAL* attn) {
    OR_FP_SCOPE;
    for (int64_t b = 0; b < B; b++)
        for (int64_t h = 0; h < H; h++)
            for (int64_t i = 0; i < tq; i++) {
                const int64_t r = (b * H + h) * tq + i;
                const float* mr = mask ? mask + ((mask_batches == 1 ? 0 : b) * tq + i) * tk : NULL;
                REAL* ar = attn + r * tk;
                REAL mx = (REAL)-3.40282347e+38f;
                for (int64_t j = 0; j < tk; j++) {
                    REAL s = mr ? (REAL)scores[r * tk + j] + (REAL)mr[j] : (REAL)scores[r * tk + j];
                    ar[j] = s;
                    mx = (mx < s) ? s : mx;
                }
                REAL sum = 0;
                for (int64_t j = 0; j < tk; j++) {
                    ar[j] = (REAL)exp(ar[j] - mx);
                    sum += ar[j];
                }
                for (int64_t j = 0; j < tk; j++) ar[j] /= sum;
            }
    return 0;
}

/* Its backward, layer.cpp:1343-1360: d = attn * (d_attn - sum(attn * d_attn)). */
int or_attention_softmax_bwd(const float* attn, const float* d_attn, int64_t rows, int64_t tk, REAL* ds) {
    OR_FP_SCOPE;
    for (int64_t r = 0; r < rows; r++) {
        const float* ar = attn + r * tk;
        const float* dr = d_attn + r * tk;
        REAL dot = 0;
        for (int64_t j = 0; j < tk; j++) ACC(dot, (REAL)ar[j] * (REAL)dr[j]);
        for (int64_t j = 0; j < tk; j++) ds[r * tk + j] = (REAL)ar[j] * MINUS((REAL)dr[j], dot);
    }
    return 0;
}

/* Dropout's mask as the device draws it (the generator is this build's own:
 * splitmix64 of seed + i, top 24 bits as u in [0, 1)); keep when u > p
 * (core/layer.cpp:59), scale 1 / (1 - p) in float (:55). */
int or_dropout_mask(float* mask, int64_t n, float p, uint64_t seed) {
    OR_FP_SCOPE;
    const float scale = 1.0f / (1.0f - p);
    for (int64_t i = 0; i < n; i++) {
        uint64_t z = seed + (uint64_t)i + 0x9E3779B97F4A7C15ull;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        float u = (float)(uint32_t)(z >> 40) * 0x1p-24f;
        mask[i] = u > p ? scale : 0.0f;
    }
    return 0;
}

/* ---- matrix products: core/tensor.cpp:281-331, :783-895 ----------------- */

/* Tensor::matmul / bmm forward (:783-795, :827-852) through matmul_blocked
 * (:281-331): C starts at zero and, for a fixed (i, j), the blocked loop adds
 * a_ik * b_kj for k ascending (k blocks in order, k in order inside a
 * block), one product and one addition each.  a [batch, m, k], b [batch, k,
 * n], c [batch, m, n]. */
int or_bmm(const float* a, const float* b, int64_t batch, int64_t m, int64_t k, int64_t n, REAL* c) {
    OR_FP_SCOPE;
    for (int64_t p = 0; p < batch; p++) {
        const float* A = a + p * m * k;
        const float* B = b + p * k * n;
        REAL* Cp = c + p * m * n;
        for (int64_t i = 0; i < m; i++)
            for (int64_t j = 0; j < n; j++) {
                REAL s = 0;
                for (int64_t l = 0; l < k; l++) ACC(s, (REAL)A[i * k + l] * (REAL)B[l * n + j]);
                Cp[i * n + j] = s;
            }
    }
    return 0;
}

/* Their closures (:797-815, :857-893), adding into ga / gb (NULL = no grad):
 *   ga[i][l] += sum_j g[i][j] * b[l][j]   (j ascending; simd_dot's scalar
 *                                           form in a build without AVX)
 *   gb[l][j] += sum_i a[i][l] * g[i][j]   (i ascending)
 * Each sum is formed first and then added to the gradient. */
int or_bmm_bwd(const float* g, const float* a, const float* b, int64_t batch, int64_t m, int64_t k, int64_t n,
               REAL* ga, REAL* gb) {
    OR_FP_SCOPE;
    for (int64_t p = 0; p < batch; p++) {
        const float* G = g + p * m * n;
        const float* A = a + p * m * k;
        const float* B = b + p * k * n;
        if (ga)
            for (int64_t i = 0; i < m; i++)
                for (int64_t l = 0; l < k; l++) {
                    REAL s = 0;
                    for (int64_t j = 0; j < n; j++) ACC(s, (REAL)G[i * n + j] * (REAL)B[l * n + j]);
                    REAL* d = ga + p * m * k + i * k + l;
                    *d = PLUS(*d, s);
                }
        if (gb)
            for (int64_t l = 0; l < k; l++)
                for (int64_t j = 0; j < n; j++) {
                    REAL s = 0;
                    for (int64_t i = 0; i < m; i++) ACC(s, (REAL)A[i * k + l] * (REAL)G[i * n + j]);
                    REAL* d = gb + p * k * n + l * n + j;
                    *d = PLUS(*d, s);
                }
    }
    return 0;
}

/* ---- MultiHeadAttention: core/layer.cpp:1103-1437 ------------------------- */

/* y[r][d] = bias[d] + sum_k x[r][k] * W[d][k], k ascending, the sum starting
 * from the bias (:1133-1175, :1262-1276). */
static void or_proj(const float* x, const float* W, const float* bias, int64_t rows, int64_t E, REAL* y) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t d = 0; d < E; d++) {
            REAL s = (REAL)bias[d];
            for (int64_t k = 0; k < E; k++) ACC(s, (REAL)x[r * E + k] * (REAL)W[d * E + k]);
            y[r * E + d] = s;
        }
}

/* MultiHeadAttention::forward(query, key, value, mask), :1103-1280.
 * q [B, Sq, E]; k, v [B, Sk, E]; mask NULL or [Bm, 1, Sq, Sk]; W [E, E]
 * (row d = output feature d), b [E].  Writes out [B, Sq, E], attn
 * [B, H, Sq, Sk] and the intermediates the closure captures: Q [B, Sq, E],
 * K, V [B, Sk, E], ctx [B, Sq, E].  The f32 build rounds every product and
 * sum as the reference's loops do. */
int or_mha_forward(const float* q, const float* k, const float* v, const float* mask, int64_t mask_batches,
                   const float* Wq, const float* Wk, const float* Wv, const float* Wo, const float* bq,
                   const float* bk, const float* bv, const float* bo, int64_t B, int64_t Sq, int64_t Sk, int64_t E,
                   int64_t H, REAL* out, REAL* attn, REAL* Q, REAL* K, REAL* V, REAL* ctx) {
    OR_FP_SCOPE;
    const int64_t hd = E / H;
    const float scale = 1.0f / sqrtf((float)hd);
    or_proj(q, Wq, bq, B * Sq, E, Q);
    or_proj(k, Wk, bk, B * Sk, E, K);
    or_proj(v, Wv, bv, B * Sk, E, V);
    /* scores: dot over the head's slice, times scale, plus the mask (:1180-1208);
     * softmax over Sk (:1210-1237), as or_attention_softmax. */
    for (int64_t b = 0; b < B; b++)
        for (int64_t h = 0; h < H; h++)
            for (int64_t i = 0; i < Sq; i++) {
                REAL* ar = attn + ((b * H + h) * Sq + i) * Sk;
                const float* mr = mask ? mask + ((mask_batches == 1 ? 0 : b) * Sq + i) * Sk : NULL;
                for (int64_t j = 0; j < Sk; j++) {
                    REAL dot = 0;
                    for (int64_t d = 0; d < hd; d++)
                        ACC(dot, Q[(b * Sq + i) * E + h * hd + d] * K[(b * Sk + j) * E + h * hd + d]);
                    REAL s = dot * (REAL)scale;
                    if (mr) s = PLUS(s, (REAL)mr[j]);
                    ar[j] = s;
                }
                REAL mx = (REAL)-3.40282347e+38f;
                for (int64_t j = 0; j < Sk; j++) mx = (mx < ar[j]) ? ar[j] : mx;
                REAL sum = 0;
                for (int64_t j = 0; j < Sk; j++) {
                    ar[j] = (REAL)exp(ar[j] - mx);
                    sum += ar[j];
                }
                for (int64_t j = 0; j < Sk; j++) ar[j] /= sum;
            }
    /* context[b, i, h*hd + d] = sum_j attn * V (:1242-1259) */
    for (int64_t b = 0; b < B; b++)
        for (int64_t h = 0; h < H; h++)
            for (int64_t i = 0; i < Sq; i++)
                for (int64_t d = 0; d < hd; d++) {
                    REAL s = 0;
                    for (int64_t j = 0; j < Sk; j++)
                        ACC(s, attn[((b * H + h) * Sq + i) * Sk + j] * V[(b * Sk + j) * E + h * hd + d]);
                    ctx[(b * Sq + i) * E + h * hd + d] = s;
                }
    /* output projection (:1262-1276), from the context as stored (fp32 in the
     * reference; REAL here) */
    for (int64_t r = 0; r < B * Sq; r++)
        for (int64_t d = 0; d < E; d++) {
            REAL s = (REAL)bo[d];
            for (int64_t kk = 0; kk < E; kk++) ACC(s, ctx[r * E + kk] * (REAL)Wo[d * E + kk]);
            out[r * E + d] = s;
        }
    return 0;
}

/* Its closure, :1299-1433, given dout [B, Sq, E] and the captured
 * intermediates (fp32, as the reference stores them).  Parameter gradients
 * are always added (the reference does not test their requires_grad); gq,
 * gk, gv may be NULL (input does not require grad) and may alias (self
 * attention adds all three into one gradient).  Accumulation order follows
 * the reference's loops: every += goes straight into its target. */
int or_mha_backward(const float* dout, const float* q, const float* k, const float* v, const float* Wq,
                    const float* Wk, const float* Wv, const float* Wo, const float* Q, const float* K,
                    const float* V, const float* attn, const float* ctx, int64_t B, int64_t Sq, int64_t Sk,
                    int64_t E, int64_t H, REAL* gWq, REAL* gWk, REAL* gWv, REAL* gWo, REAL* gbq, REAL* gbk,
                    REAL* gbv, REAL* gbo, REAL* gq, REAL* gk, REAL* gv) {
    OR_FP_SCOPE;
    const int64_t hd = E / H;
    const float scale = 1.0f / sqrtf((float)hd);
    REAL* dctx = (REAL*)calloc((size_t)(B * Sq * E), sizeof(REAL));
    REAL* dattn = (REAL*)calloc((size_t)(B * H * Sq * Sk), sizeof(REAL));
    REAL* dV = (REAL*)calloc((size_t)(B * Sk * E), sizeof(REAL));
    REAL* ds = (REAL*)calloc((size_t)(B * H * Sq * Sk), sizeof(REAL));
    REAL* dQ = (REAL*)calloc((size_t)(B * Sq * E), sizeof(REAL));
    REAL* dK = (REAL*)calloc((size_t)(B * Sk * E), sizeof(REAL));
    if (!dctx || !dattn || !dV || !ds || !dQ || !dK) {
        free(dctx), free(dattn), free(dV), free(ds), free(dQ), free(dK);
        return 1;
    }
    /* output projection (:1305-1318) */
    for (int64_t r = 0; r < B * Sq; r++)
        for (int64_t d = 0; d < E; d++) {
            const REAL g = (REAL)dout[r * E + d];
            gbo[d] = PLUS(gbo[d], g);
            for (int64_t kk = 0; kk < E; kk++) {
                ACC(gWo[d * E + kk], g * (REAL)ctx[r * E + kk]);
                ACC(dctx[r * E + kk], g * (REAL)Wo[d * E + kk]);
            }
        }
    /* attn @ V (:1320-1339) */
    for (int64_t b = 0; b < B; b++)
        for (int64_t h = 0; h < H; h++)
            for (int64_t i = 0; i < Sq; i++)
                for (int64_t d = 0; d < hd; d++) {
                    const REAL dc = dctx[(b * Sq + i) * E + h * hd + d];
                    for (int64_t j = 0; j < Sk; j++) {
                        const int64_t ai = ((b * H + h) * Sq + i) * Sk + j;
                        const int64_t vi = (b * Sk + j) * E + h * hd + d;
                        ACC(dattn[ai], dc * (REAL)V[vi]);
                        ACC(dV[vi], dc * (REAL)attn[ai]);
                    }
                }
    /* softmax (:1341-1360): ds = attn * (dattn - sum(attn * dattn)) */
    for (int64_t r = 0; r < B * H * Sq; r++) {
        REAL dot = 0;
        for (int64_t j = 0; j < Sk; j++) ACC(dot, (REAL)attn[r * Sk + j] * dattn[r * Sk + j]);
        for (int64_t j = 0; j < Sk; j++) ds[r * Sk + j] = (REAL)attn[r * Sk + j] * MINUS(dattn[r * Sk + j], dot);
    }
    /* Q @ K^T (:1362-1383): d_s = ds * scale, then into dQ and dK */
    for (int64_t b = 0; b < B; b++)
        for (int64_t h = 0; h < H; h++)
            for (int64_t i = 0; i < Sq; i++)
                for (int64_t j = 0; j < Sk; j++) {
                    const REAL d_s = ds[((b * H + h) * Sq + i) * Sk + j] * (REAL)scale;
                    for (int64_t d = 0; d < hd; d++) {
                        const int64_t qi = (b * Sq + i) * E + h * hd + d;
                        const int64_t ki = (b * Sk + j) * E + h * hd + d;
                        ACC(dQ[qi], d_s * (REAL)K[ki]);
                        ACC(dK[ki], d_s * (REAL)Q[qi]);
                    }
                }
    /* V, K, Q projections (:1385-1433) */
    const struct {
        const REAL* dY;
        const float* x;
        const float* W;
        REAL *gW, *gb, *gx;
        int64_t S;
    } proj[3] = {{dV, v, Wv, gWv, gbv, gv, Sk}, {dK, k, Wk, gWk, gbk, gk, Sk}, {dQ, q, Wq, gWq, gbq, gq, Sq}};
    for (int t = 0; t < 3; t++)
        for (int64_t r = 0; r < B * proj[t].S; r++)
            for (int64_t d = 0; d < E; d++) {
                const REAL dy = proj[t].dY[r * E + d];
                proj[t].gb[d] = PLUS(proj[t].gb[d], dy);
                for (int64_t kk = 0; kk < E; kk++) {
                    ACC(proj[t].gW[d * E + kk], dy * (REAL)proj[t].x[r * E + kk]);
                    if (proj[t].gx) ACC(proj[t].gx[r * E + kk], dy * (REAL)proj[t].W[d * E + kk]);
                }
            }
    free(dctx), free(dattn), free(dV), free(ds), free(dQ), free(dK);
    return 0;
}
