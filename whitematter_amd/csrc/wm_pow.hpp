// Table-driven float pow for the pow kernels.
//
// The device powf costs ~166 vector instructions per element on gfx950,
// which makes pow(Tensor) compute-bound (about a third of the HBM rate).
// This one evaluates y * log2|x| and the power of two in double precision,
// where small tables make both halves short:
//   log2|x|: |x| = 2^k * z with z in [0.699, 1.398); 16 sub-intervals of z
//            with invc ~ 1/c (20 significant bits, so z * invc is exact in
//            double) and logc = log2(c); r = z * invc - 1 with |r| < 0.0297;
//            log2(1 + r) by its series to r^6 (truncation < 4.2e-12).
//   2^t:     t = kd/128 + r with |r| <= 1/256; 2^(kd/128) from a
//            128-entry table and an exponent shift; 2^r by 1 + E1 r + E2 r^2
//            with E1, E2 minimising the largest relative error on
//            [-1/256, 1/256]: 8.3e-10.  (The
//            Taylor series to degree 3 on a 32-entry table, 5.7e-10, took
//            one more FMA per element; degree 2 on 64 entries, 6.6e-9,
//            rounded results near ties in the subnormal range the other way
//            from the C library noticeably more often.)
// The double result is within ~9e-10 (relative) of the exact power, so its
// one rounding to float is within 1 ulp.  A negative base takes C pow's sign
// rule (NaN for a non-integer exponent, the magnitude's sign flipped for an
// odd one) without a branch.  The operands the tables do not cover (zero,
// subnormal, infinite or NaN bases, |x| == 1, and infinite, NaN or zero
// exponents) go to the device powf in a branch that a wave skips when none
// of its lanes needs it.
//
// The backward needs pow(a, b), pow(a, b - 1) and log(a) only inside
// gradients, so it shares one log2|a| and takes the powers of two from the
// hardware exp2 on a reduced argument (relative error ~2e-7).
//
// The method is the published table-driven one: P. T. P. Tang,
// "Table-driven implementation of the exponential function in IEEE
// floating-point arithmetic", ACM TOMS 15(2), 1989, and "... of the
// logarithm function ...", ACM TOMS 16(4), 1990, in the double-precision
// arrangement for powf of the ARM Optimized Routines (Szabolcs Nagy, 2018;
// the same scheme is in musl and in glibc's powf since 2.28): log2 of the
// reduced argument from a 16-entry table of (1/c, log2 c) and a polynomial
// in r = z/c - 1, the product with y in double, then 2^t from a table of
// 2^(j/N) and a short polynomial.  The table sizes (N = 128 here), the
// polynomial degrees and the coefficients are this file's own, generated and
// fitted for this build.
//
// The file is plain C++ with explicit fma(), so the same code compiles for
// the host and is checked there against long double powl
// (tests/cpp/pow_table_check.cpp).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>

#ifdef __HIPCC__
#define WM_HD __host__ __device__
#else
#define WM_HD
#endif

namespace wm {
namespace powdetail {

struct LogEntry {
    double invc, logc;
};

struct alignas(16) PowTables {
    LogEntry log[16];  // {1/c, log2(c)} for the 16 sub-intervals of z
    double exp2[128];  // 2^(j/128), j = 0..127, correctly rounded
};

WM_HD inline const PowTables& pow_table_data() {
    static constexpr PowTables t = {
        {
            {1.3989067077636719, -0.48429975325710395}, {1.3403148651123047, -0.4225719566348825},
            {1.2864322662353516, -0.3633754976944188},  {1.236715316772461, -0.3065134402105001},
            {1.1906986236572266, -0.2518083005440589},  {1.1479816436767578, -0.19909957338273085},
            {1.108224868774414, -0.14825064686535408},  {1.0711288452148438, -0.09913203113589106},
            {1.03643798828125, -0.051633800310858485},  {0.9980506896972656, 0.002815004858138399},
            {0.9481477737426758, 0.07681616674347436},  {0.8951053619384766, 0.15987058435448812},
            {0.847681999206543, 0.23840494355449127},   {0.8050317764282227, 0.31288236409411413},
            {0.7664670944213867, 0.38370423872947484},  {0.7314281463623047, 0.4512119502479954},
        },
        {
            1.0, 1.0054299011128027, 1.0108892860517005, 1.016378314910953,
            1.0218971486541166, 1.0274459491187637, 1.0330248790212284, 1.0386341019613787,
            1.0442737824274138, 1.0499440858006872, 1.0556451783605572, 1.061377227289262,
            1.0671404006768237, 1.0729348675259756, 1.0787607977571199, 1.0846183622133092,
            1.0905077326652577, 1.0964290818163769, 1.102382583307841, 1.1083684117236787,
            1.1143867425958924, 1.1204377524096067, 1.1265216186082418, 1.1326385195987192,
            1.1387886347566916, 1.1449721444318042, 1.1511892299529827, 1.1574400736337511,
            1.1637248587775775, 1.1700437696832502, 1.1763969916502812, 1.182784710984341,
            1.189207115002721, 1.1956643920398273, 1.202156731452703, 1.2086843236265816,
            1.215247359980469, 1.2218460329727576, 1.22848053610687, 1.2351510639369334,
            1.241857812073484, 1.2486009771892048, 1.255380757024691, 1.2621973503942507,
            1.2690509571917332, 1.275941778396392, 1.2828700160787783, 1.2898358734066657,
            1.2968395546510096, 1.3038812651919358, 1.3109612115247644, 1.318079601266064,
            1.3252366431597413, 1.3324325470831615, 1.339667524053303, 1.3469417862329458,
            1.3542555469368927, 1.3616090206382248, 1.3690024229745905, 1.3764359707545302,
            1.383909881963832, 1.3914243757719262, 1.3989796725383112, 1.4065759938190154,
            1.4142135623730951, 1.4218926021691656, 1.42961333839197, 1.4373759974489824,
            1.4451808069770467, 1.4530279958490526, 1.460917794180647, 1.4688504333369818,
            1.4768261459394993, 1.4848451658727524, 1.4929077282912648, 1.5010140696264256,
            1.5091644275934228, 1.5173590411982147, 1.5255981507445384, 1.533881997840956,
            1.5422108254079407, 1.550584877685, 1.559004400237837, 1.567469639965553,
            1.5759808451078865, 1.5845382652524937, 1.593142151342267, 1.6017927556826934,
            1.6104903319492543, 1.6192351351948637, 1.6280274218573478, 1.6368674497669644,
            1.645755478153965, 1.6546917676561943, 1.6636765803267364, 1.6727101796415966,
            1.681792830507429, 1.6909247992693053, 1.7001063537185235, 1.709337763100463,
            1.718619298122478, 1.7279512309618377, 1.7373338352737062, 1.746767386199169,
            1.7562521603732995, 1.7657884359332727, 1.7753764925265212, 1.785016611318935,
            1.7947090750031072, 1.804454167806624, 1.8142521755003989, 1.8241033854070534,
            1.8340080864093424, 1.843966568958626, 1.8539791250833855, 1.864046048397789,
            1.8741676341103, 1.8843441790323345, 1.8945759815869656, 1.9048633418176741,
            1.9152065613971474, 1.925605943636125, 1.9360617934922943, 1.9465744175792332,
            1.9571441241754002, 1.9677712232331759, 1.978456026387951, 1.9891988469672663,
        },
    };
    return t;
}

#ifdef __HIP_DEVICE_COMPILE__
// On the device the lookups read a copy of the tables in LDS, which every
// kernel that evaluates pow fills first (pow_tables_to_lds).  Each log
// entry sits in its own LDS banks; exp2 entries j, j + 32, j + 64 and
// j + 96 share theirs, so a wave's exp2 lookups conflict at most four ways.  The lookups stay off
// the texture path, which per-lane gathers from global memory had
// saturated.
static __shared__ PowTables wm_pow_lds;
#endif

WM_HD inline const PowTables& pow_tables() {
#ifdef __HIP_DEVICE_COMPILE__
    return wm_pow_lds;
#else
    return pow_table_data();
#endif
}

WM_HD inline uint32_t bits_of(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

WM_HD inline float float_of(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

WM_HD inline uint32_t low_word(double d) {
    uint64_t u;
    std::memcpy(&u, &d, 8);
    return (uint32_t)u;
}

// log2(ax) for a normal ax > 0.  Branch-free; any other input gives a
// meaningless value, but the table index always stays in range.
WM_HD inline double log2_normal(float ax) {
    const uint32_t ix = bits_of(ax);
    const uint32_t OFF = 0x3f330000u;
    const uint32_t tmp = ix - OFF;
    const int i = (int)((tmp >> 19) & 15u);
    const int k = (int)((int32_t)tmp >> 23);
    const double z = (double)float_of(ix - (tmp & 0xff800000u));
    const LogEntry e = pow_tables().log[i];
    const double r = std::fma(z, e.invc, -1.0);
    // log2(1 + r) = r * (C1 + C2 r + ... + C6 r^5), Cn = (-1)^(n+1) / (n ln 2)
    const double C1 = 1.4426950408889634, C2 = -0.7213475204444817, C3 = 0.48089834696298783,
                 C4 = -0.36067376022224085, C5 = 0.28853900817779266, C6 = -0.24044917348149392;
    double q = std::fma(C6, r, C5);
    q = std::fma(q, r, C4);
    q = std::fma(q, r, C3);
    q = std::fma(q, r, C2);
    q = std::fma(q, r, C1);
    return std::fma(q, r, (double)k + e.logc);
}

// 2^t rounded once to float, within 1 ulp: overflow -> inf, underflow -> 0
// or a rounded subnormal.  t is clamped to [-200, 200] (NaN -> 200), so the
// integer conversion is exact and the table index in range.
WM_HD inline float exp2_to_float(double t) {
    t = std::fmax(std::fmin(t, 200.0), -200.0);
    // kd = rint(128 t) by adding 1.5 * 2^52: the low word is then rint(128 t)
    // in two's complement (|128 t| <= 25600).
    const double SHIFT = 6755399441055744.0;
    const double kds = std::fma(t, 128.0, SHIFT);
    const int ki = (int)low_word(kds);
    const double kd = kds - SHIFT;
    const double r = std::fma(kd, -1.0 / 128.0, t);  // exact, |r| <= 1/256
    // 2^r ~ 1 + E1 r + E2 r^2: the coefficients minimise the largest
    // relative error on the range (8.3e-10) with the constant held at 1, so
    // r = 0 gives exactly the table entry: an exact power of two stays
    // exact (2^-150, a tie between 0 and the smallest subnormal, must round
    // to even as the C library's powf does).
    const double E1 = 0.6931478155387308, E2 = 0.24022650685171912;
    const double p = std::fma(std::fma(E2, r, E1), r, 1.0);
    return (float)std::ldexp(pow_tables().exp2[ki & 127] * p, ki >> 7);
}

// 2^t for values used only inside gradients: relative error ~2e-7 (the
// hardware exp2 of a float argument in [-0.5, 0.5], then an exact shift;
// results in the subnormal range round once more).
WM_HD inline float exp2_grad(double t) {
    t = std::fmax(std::fmin(t, 200.0), -200.0);
    const double n = std::rint(t);
    const float f = (float)(t - n);
#ifdef __HIP_DEVICE_COMPILE__
    const float p = __builtin_amdgcn_exp2f(f);
#else
    const float p = std::exp2(f);
#endif
    return std::ldexp(p, (int)n);
}

// Operands the table path covers: |x| normal and != 1, y finite and
// non-zero.  |x| == 1 is excluded because pow(+-1, y) must be exactly +-1,
// and the table's log2(1) is only zero to ~1e-19, which a huge y would
// amplify.
WM_HD inline bool table_ok(float x, float y) {
    return std::isnormal(x) && std::fabs(x) != 1.0f && std::isfinite(y) && y != 0.0f;
}

// C pow's sign rule for a finite non-zero base, given the magnitude
// |x|^y: a negative base gives NaN for a non-integer exponent and flips
// the sign for an odd one.  Branch-free.
WM_HD inline float apply_sign(float x, float y, float mag) {
    const float yi = std::rint(y);
    const bool is_int = yi == y;
    // |y| >= 2^24 is always even; the clamp keeps the conversion in range.
    const bool odd = ((int)std::fmin(std::fabs(yi), 16777216.0f) & 1) != 0;
    const float s = odd ? -mag : mag;
    return x < 0.0f ? (is_int ? s : NAN) : mag;
}

}  // namespace powdetail

#ifdef __HIPCC__
// Copies the pow tables into LDS.  Every kernel that evaluates pow_table,
// pow_f32 or pow_grad_* calls this first, with all its threads (it contains
// a barrier).
__device__ inline void pow_tables_to_lds() {
#ifdef __HIP_DEVICE_COMPILE__
    constexpr int kWords = (int)(sizeof(powdetail::PowTables) / 16);
    static_assert(kWords * 16 == sizeof(powdetail::PowTables), "pow tables are whole 16-byte words");
    for (int i = threadIdx.x; i < kWords; i += blockDim.x)
        reinterpret_cast<uint4*>(&powdetail::wm_pow_lds)[i] =
            reinterpret_cast<const uint4*>(&powdetail::pow_table_data())[i];
    __syncthreads();
#endif
}
#endif

// The table path alone: equal to pow(x, y) within 1 ulp wherever
// pow_needs_fix(x, y) is false.  Branch-free, so kernels evaluate it for a
// whole vector of elements (the table lookups overlap) before fixing up the
// rare specials.
WM_HD inline float pow_table(float x, float y) {
    using namespace powdetail;
    return apply_sign(x, y, exp2_to_float((double)y * log2_normal(std::fabs(x))));
}

WM_HD inline bool pow_needs_fix(float x, float y) { return !powdetail::table_ok(x, y); }

// The exponent's share of pow_table and pow_needs_fix, for a run of
// elements that share one exponent (a per-row or scalar exponent): its
// double, C pow's sign rule for a negative base (NaN unless y is an integer;
// an odd y flips the sign bit of |x|^y) and its half of table_ok.
struct PowExponent {
    double yd;
    uint32_t odd_mask;  // 0x80000000 for an odd integer y
    bool is_int;
    bool ok;            // finite and non-zero
};

WM_HD inline PowExponent pow_exponent(float y) {
    const float yi = std::rint(y);
    const bool odd = ((int)std::fmin(std::fabs(yi), 16777216.0f) & 1) != 0;
    return {(double)y, odd ? 0x80000000u : 0u, yi == y, std::isfinite(y) && y != 0.0f};
}

// pow_table(x, y) for y described by e: the same value, bit for bit (the
// magnitude is never NaN, so flipping its sign bit is negation).
WM_HD inline float pow_table_exp(float x, const PowExponent& e) {
    using namespace powdetail;
    const float mag = exp2_to_float(e.yd * log2_normal(std::fabs(x)));
    const float neg = e.is_int ? float_of(bits_of(mag) ^ e.odd_mask) : NAN;
    return x < 0.0f ? neg : mag;
}

WM_HD inline bool pow_needs_fix_exp(float x, const PowExponent& e) {
    return !(e.ok && std::isnormal(x) && std::fabs(x) != 1.0f);
}

// pow(x, y) with C semantics, within 1 ulp.
WM_HD inline float pow_f32(float x, float y) {
    return pow_needs_fix(x, y) ? powf(x, y) : pow_table(x, y);
}

// The three values pow's backward needs, sharing one log2|a| and one power
// of two:
//   out  = pow(a, b)            (the forward output, recomputed; d/db)
//   pbm1 = pow(a, b - 1.0f)     (d/da = g * b * pbm1) = out * (1 / a)
//   lga  = log(a)               (d/db = g * out * lga)
// Only the requested ones are computed (the others are 0).  On the table
// path out carries a relative error of ~2e-7 and pbm1 ~3e-7 against the
// exact pow(a, b - 1) (the reciprocal adds at most 1 ulp); the reference's
// pow(a, b - 1.0f) rounds the exponent to float first, which moves it by up
// to |(b - 1) ln a| 2^-24 < 5.3e-6 relative (see below).  lga is log(a) rounded once
// from double (NaN for a < 0).  The quotient stands for pow(a, b - 1) while |b| < 2^24, pow(a, b)
// stays in the normal range (or is the NaN of a negative base) and 1 / a
// does too (|a| < 2^126); other lanes set `slow`, for pow_grad_fix.
struct PowGrad {
    float out, pbm1, lga;
    bool slow;
};

WM_HD inline float recip_normal(float a) {
#ifdef __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_rcpf(a);  // within 1 ulp for normal a with |a| < 2^126
#else
    return 1.0f / a;
#endif
}

WM_HD inline PowGrad pow_grad_table(float a, float b, bool want_out, bool want_pbm1, bool want_lga) {
    using namespace powdetail;
    PowGrad r = {0.0f, 0.0f, 0.0f, false};
    const double l2 = log2_normal(std::fabs(a));
    if (want_out || want_pbm1) {
        const float o = apply_sign(a, b, exp2_grad((double)b * l2));
        if (want_out) r.out = o;
        if (want_pbm1) {
            r.pbm1 = o * recip_normal(a);
            // pow(a, b - 1.0f) takes b - 1 rounded to float, at most
            // |b - 1| 2^-24 from the exact b - 1, which changes the power by
            // at most |(b - 1) ln a| 2^-24 relative: below 5.3e-6 wherever
            // the power is a normal float (|(b - 1) ln a| < 88.8).  From
            // |b| = 2^24 up the rounding can drop the "- 1" altogether, so
            // those lanes are slow.  A NaN power (a < 0, b not an integer) is
            // pow(a, b - 1) too unless b - 1 rounded to an integer (|b| below
            // 2^-25).
            const float bm1 = b - 1.0f;
            const bool ok = std::isnormal(o) || (std::isnan(o) && std::rint(bm1) != bm1);
            r.slow = !ok || !(std::fabs(b) < 0x1p24f) || !(std::fabs(a) < 0x1p126f);
        }
    }
    if (want_lga) r.lga = a > 0.0f ? (float)(l2 * 0.6931471805599453) : NAN;
    return r;
}

WM_HD inline bool pow_grad_needs_fix(float a, float b) {
    return !powdetail::table_ok(a, b) || !powdetail::table_ok(a, b - 1.0f);
}

WM_HD inline bool pow_grad_needs_fix(float a, float b, const PowGrad& r) {
    return r.slow || pow_grad_needs_fix(a, b);
}

// Operands outside the table path: all three from powf / logf.  A lane that
// is only `slow` keeps out and lga and takes pow(a, b - 1) from the table
// path's own power of two of (b - 1) log2|a|.
WM_HD inline void pow_grad_fix(float a, float b, bool want_out, bool want_pbm1, bool want_lga, PowGrad& r) {
    using namespace powdetail;
    if (!pow_grad_needs_fix(a, b)) {
        const float bm1 = b - 1.0f;
        r.pbm1 = apply_sign(a, bm1, exp2_grad((double)bm1 * log2_normal(std::fabs(a))));
        return;
    }
    if (want_out) r.out = powf(a, b);
    if (want_pbm1) r.pbm1 = powf(a, b - 1.0f);
    if (want_lga) r.lga = logf(a);
}

// The exponent's share of pow_grad_table and pow_grad_needs_fix, for
// elements that share one exponent b (a per-row exponent): computed once,
// the per-element work is then pow_grad_table_exp, bit for bit
// pow_grad_table.
struct PowGradExponent {
    PowExponent e;  // b: its double, sign rule, finite and non-zero
    bool ok_bm1;    // b - 1.0f finite and non-zero
    bool bm1_int;   // b - 1.0f an integer
    bool b_small;   // |b| < 2^24
};

WM_HD inline PowGradExponent pow_grad_exponent(float b) {
    const float bm1 = b - 1.0f;
    return {pow_exponent(b), std::isfinite(bm1) && bm1 != 0.0f, std::rint(bm1) == bm1, std::fabs(b) < 0x1p24f};
}

WM_HD inline PowGrad pow_grad_table_exp(float a, const PowGradExponent& q, bool want_out, bool want_pbm1,
                                        bool want_lga) {
    using namespace powdetail;
    PowGrad r = {0.0f, 0.0f, 0.0f, false};
    const double l2 = log2_normal(std::fabs(a));
    if (want_out || want_pbm1) {
        const float mag = exp2_grad(q.e.yd * l2);  // never NaN: flipping its sign bit is negation
        const float o = a < 0.0f ? (q.e.is_int ? float_of(bits_of(mag) ^ q.e.odd_mask) : NAN) : mag;
        if (want_out) r.out = o;
        if (want_pbm1) {
            r.pbm1 = o * recip_normal(a);
            const bool ok = std::isnormal(o) || (std::isnan(o) && !q.bm1_int);
            r.slow = !ok || !q.b_small || !(std::fabs(a) < 0x1p126f);
        }
    }
    if (want_lga) r.lga = a > 0.0f ? (float)(l2 * 0.6931471805599453) : NAN;
    return r;
}

WM_HD inline bool pow_grad_needs_fix_exp(float a, const PowGradExponent& q, const PowGrad& r) {
    return r.slow || !(q.e.ok && q.ok_bm1 && std::isnormal(a) && std::fabs(a) != 1.0f);
}

WM_HD inline PowGrad pow_grad_parts(float a, float b, bool want_out, bool want_pbm1, bool want_lga) {
    PowGrad r = pow_grad_table(a, b, want_out, want_pbm1, want_lga);
    if (pow_grad_needs_fix(a, b, r)) pow_grad_fix(a, b, want_out, want_pbm1, want_lga, r);
    return r;
}

}  // namespace wm
