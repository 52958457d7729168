// Host build of the device pow (whitematter_amd/csrc/wm_pow.hpp: the same
// source, plain C++ with explicit fma) against long double powl / logl on
// random and special operands.  Contract checked, per the header:
//   pow_f32            within 1 ulp of powl; NaN / infinity / zero exactly
//                      where the C library's powf has them; exact powers of
//                      two (ties to even among subnormals) bit for bit
//   pow_grad_parts     out within 1e-6 relative of powl(a, b);
//                      pbm1 within |(b - 1) ln a| 2^-24 + 1e-6 relative
//                      of powl(a, (float)(b - 1)) (the reference rounds
//                      b - 1 to float first, which moves its power by up to
//                      |(b - 1) ln a| 2^-24); lga within 1 ulp of logl(a)
//   pow_table_exp, pow_grad_table_exp (one exponent shared by many
//                      elements) equal pow_table, pow_grad_table bit for bit
// Prints "POW CHECK PASSED" and exits 0 when every case holds.
#include "../../whitematter_amd/csrc/wm_pow.hpp"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

namespace {

int64_t ulp_dist(float a, long double ref) {
    if (std::isnan(a) && std::isnan((double)ref)) return 0;
    if (std::isnan(a) || std::isnan((double)ref)) return INT64_C(1) << 40;
    const float rf = (float)ref;
    if (std::isinf(a) || std::isinf(rf)) return a == rf ? 0 : INT64_C(1) << 40;
    int32_t ia, ib;
    std::memcpy(&ia, &a, 4);
    std::memcpy(&ib, &rf, 4);
    if (ia < 0) ia = INT32_MIN - ia;
    if (ib < 0) ib = INT32_MIN - ib;
    const int64_t d = (int64_t)ia - ib;
    return d < 0 ? -d : d;
}

bool rel_close(float a, long double ref, long double tol) {
    if (std::isnan(a) && std::isnan((double)ref)) return true;
    if (std::isnan(a) || std::isnan((double)ref)) return false;
    const float rf = (float)ref;
    if (std::isinf(rf) || std::isinf(a)) return a == rf || fabsl(ref) > 3.3e38L;  // at the overflow edge
    if (fabsl(ref) < 1e-37L) return fabsl(a - ref) < 1e-44L + tol * fabsl(ref);  // subnormal results
    return fabsl(a - ref) <= tol * fabsl(ref);
}

}  // namespace

int main(int argc, char** argv) {
    const long long N = argc > 1 ? atoll(argv[1]) : 1000000;
    std::mt19937_64 gen(20240611);
    long long n = 0, bad = 0;
    int64_t worst = 0;
    auto fail = [&](const char* what, float x, float y, double got, long double ref) {
        if (bad < 10) printf("%s x=%a y=%a got=%a ref=%La\n", what, x, y, got, ref);
        ++bad;
    };
    auto check = [&](float x, float y) {
        ++n;
        const float r = wm::pow_f32(x, y);
        const long double ref = powl((long double)x, (long double)y);
        const float lib = powf(x, y);
        if (std::isnan(r) != std::isnan(lib) || std::isinf(r) != std::isinf(lib) || (r == 0.f) != (lib == 0.f))
            fail("special", x, y, r, lib);
        const int64_t d = ulp_dist(r, ref);
        if (d > worst) worst = d;
        if (d > 1) fail("pow", x, y, r, ref);
        const wm::PowGrad gp = wm::pow_grad_parts(x, y, true, true, true);
        if (!rel_close(gp.out, ref, 1e-6L)) fail("grad out", x, y, gp.out, ref);
        const long double ref2 = powl((long double)x, (long double)(float)(y - 1.0f));
        long double tol2 = fabsl(logl(fabsl((long double)x)) * ((long double)y - 1.0L)) * 0x1p-24L + 1e-6L;
        if (!std::isfinite((double)tol2)) tol2 = 1e-6L;  // zero or infinite bases: exact results
        if (!rel_close(gp.pbm1, ref2, tol2)) fail("grad pbm1", x, y, gp.pbm1, ref2);
        const long double l = logl((long double)x);
        if (ulp_dist(gp.lga, l) > 1 && !(x == 1.0f && gp.lga == 0.f)) fail("grad lga", x, y, gp.lga, l);
        // the shared-exponent forms equal the per-element ones bit for bit
        const wm::PowExponent pe = wm::pow_exponent(y);
        const float t1 = wm::pow_table(x, y), t2 = wm::pow_table_exp(x, pe);
        if (std::memcmp(&t1, &t2, 4) != 0 || wm::pow_needs_fix(x, y) != wm::pow_needs_fix_exp(x, pe))
            fail("shared exponent", x, y, t2, t1);
        const wm::PowGradExponent pq = wm::pow_grad_exponent(y);
        const wm::PowGrad g1 = wm::pow_grad_table(x, y, true, true, true);
        const wm::PowGrad g2 = wm::pow_grad_table_exp(x, pq, true, true, true);
        if (std::memcmp(&g1.out, &g2.out, 4) != 0 || std::memcmp(&g1.pbm1, &g2.pbm1, 4) != 0 ||
            std::memcmp(&g1.lga, &g2.lga, 4) != 0 || g1.slow != g2.slow ||
            wm::pow_grad_needs_fix(x, y, g1) != wm::pow_grad_needs_fix_exp(x, pq, g2))
            fail("shared exponent (grad)", x, y, g2.pbm1, g1.pbm1);
    };
    std::uniform_real_distribution<float> u(-3.f, 3.f), e(-20.f, 20.f);
    std::uniform_int_distribution<uint32_t> bits;
    for (long long i = 0; i < N; ++i) {
        float x, y;
        switch (i % 6) {
            case 0: x = std::fabs(u(gen)) + 1e-3f; y = u(gen); break;
            case 1: {  // any magnitude, exponent scaled so the power stays in range
                const uint32_t b = bits(gen);
                std::memcpy(&x, &b, 4);
                x = std::fabs(x);
                const float l2 = std::fabs(std::log2(x));
                y = e(gen) / (l2 == 0.f || !std::isfinite(l2) ? 1.f : l2);
                break;
            }
            case 2: x = u(gen); y = (float)(int)e(gen); break;  // negative bases, integer exponents
            case 3: {  // any bit patterns
                const uint32_t b = bits(gen), c = bits(gen);
                std::memcpy(&x, &b, 4);
                std::memcpy(&y, &c, 4);
                break;
            }
            case 4: x = u(gen); y = 0.5f + 1.5f * (u(gen) + 3.f) / 6.f; break;  // config 2's exponents
            default: x = 1.0f + u(gen) * 1e-6f; y = e(gen) * 1e6f; break;      // bases near 1, huge exponents
        }
        check(x, y);
    }
    const float sp[] = {0.f, -0.f, 1.f, -1.f, INFINITY, -INFINITY, NAN, 2.f, 0.5f, -2.f, -0.5f, 1e-45f, -1e-45f,
                        3e38f, 1.17549435e-38f, 1.1754942e-38f, 16777216.f, 16777217.f, -16777216.f, 3.f, -3.f,
                        0.3f, 1e30f, -1e30f, 2147483648.f, 4294967296.f, -4294967296.f, 1.0000001f, 0.99999994f};
    for (float x : sp)
        for (float y : sp) check(x, y);
    // Exact powers of two, ties to even in the subnormal range included
    // (2^-150 -> 0, 3 * 2^-151 -> 2^-149): bit for bit the C library's.
    for (int k = -160; k <= 130; ++k) {
        const float bases[3] = {2.0f, 0.5f, 4.0f};
        const float exps[3] = {(float)k, (float)-k, 0.5f * (float)k};
        for (int j = 0; j < 3; ++j) {
            const float r = wm::pow_f32(bases[j], exps[j]), lib = powf(bases[j], exps[j]);
            if (std::memcmp(&r, &lib, 4) != 0) fail("power of two", bases[j], exps[j], r, lib);
            ++n;
        }
    }
    printf("%lld operand pairs, worst %lld ulp, %lld failures\n", n, (long long)worst, bad);
    if (bad == 0) printf("POW CHECK PASSED\n");
    return bad == 0 ? 0 : 1;
}
