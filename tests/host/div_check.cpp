// Host check of shp_div.hpp: (float)((double)q * y) == q / a (IEEE f32
// division) for y = 1/a rounded to double and for y one ulp above or below it.
// Inputs: random f32 pairs over the whole finite range (both signs), Snake's
// range (q in [0, 1], a log-uniform in [1e-3, 1e3]), divisors with power-of-two
// significands (exact ties into the subnormal range), subnormal q and a, and
// quotients that overflow or underflow.
// Also checks that the device's two Newton steps reach 1/a to within 1 ulp
// from a start 2^-20 off, and exactly for power-of-two significands (where a
// quotient can be an exact f32 tie, which a reciprocal 1 ulp off would round
// the wrong way).
// Prints "<pairs> <mismatches> <reciprocals> <bad reciprocals>" and exits
// non-zero on any failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

#include "shp_div.hpp"

static long checked = 0, bad = 0;

static float from_bits(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// The device's two Newton steps (shp::rcp_d) from a crude start: within 1 ulp
// of 1/a in general, and exactly 1/a when a's significand is a power of two.
static long rcp_checked = 0, rcp_bad = 0;

static double newton2(double a, double y) {
    double e = std::fma(-a, y, 1.0);
    y        = std::fma(y, e, y);
    e        = std::fma(-a, y, 1.0);
    return std::fma(y, e, y);
}

static bool pow2_significand(float a) {
    uint32_t u;
    std::memcpy(&u, &a, 4);
    const bool normal = (u & 0x7f800000u) != 0;
    return normal ? (u & 0x007fffffu) == 0 : ((u & 0x007fffffu) & ((u & 0x007fffffu) - 1)) == 0;
}

static void check_rcp(float a, std::mt19937_64 & rng) {
    if (!shp::rcp_route_ok(a)) {
        return;
    }
    ++rcp_checked;
    const double exact = 1.0 / static_cast<double>(a);
    // a start about 2^-20 off, coarser than any hardware estimate
    const double y0 = exact * (1.0 + std::ldexp(static_cast<double>(static_cast<int64_t>(rng() % 2001) - 1000), -30));
    const double y  = newton2(static_cast<double>(a), y0);
    const bool   ok = pow2_significand(a) ? y == exact
                                          : (y == exact || y == std::nextafter(exact, HUGE_VAL) ||
                                             y == std::nextafter(exact, -HUGE_VAL));
    if (!ok && ++rcp_bad <= 10) {
        std::printf("reciprocal a=%a y=%a exact=%a\n", a, y, exact);
    }
}

static void check(float q, float a) {
    if (!shp::rcp_route_ok(a) || !std::isfinite(q)) {
        return;
    }
    const volatile float want = q / a;  // IEEE f32 division
    const double         y    = shp::rcp_d(static_cast<double>(a));
    // Power-of-two divisors get the exact reciprocal (check_rcp), so only the
    // others are also checked with a reciprocal one ulp off.
    const int    ny    = pow2_significand(a) ? 1 : 3;
    const double ys[3] = { y, std::nextafter(y, HUGE_VAL), std::nextafter(y, -HUGE_VAL) };
    for (int k = 0; k < ny; ++k) {
        const double yy = ys[k];
        ++checked;
        const float got = shp::div_by_rcp(q, yy);
        if (std::memcmp(&got, (const void *) &want, 4) != 0 && !(std::isnan(got) && std::isnan(want))) {
            if (++bad <= 10) {
                std::printf("mismatch q=%a a=%a got=%a want=%a\n", q, a, got, (float) want);
            }
        }
    }
}

int main() {
    std::mt19937_64 rng(20260728);
    std::uniform_int_distribution<uint32_t> bits(0, 0xffffffffu);
    std::uniform_real_distribution<double> u01(0.0, 1.0);
    for (int i = 0; i < 2000000; ++i) {
        check(from_bits(bits(rng)), from_bits(bits(rng)));
    }
    for (int i = 0; i < 2000000; ++i) {
        const float q = static_cast<float>(u01(rng));
        const float a = static_cast<float>(std::exp(std::log(1e-3) + u01(rng) * (std::log(1e3) - std::log(1e-3))));
        check(q, a);
        check(q * q, a);
    }
    for (int e = -149; e <= 127; ++e) {
        const float a = std::ldexp(1.0f, e);
        for (int i = 0; i < 2000; ++i) {
            const float q = from_bits(bits(rng) & 0x807fffffu);  // subnormal or zero
            check(q, a);
            check(from_bits(bits(rng)), a);
            check(from_bits(bits(rng)), -a);
        }
    }
    for (int i = 0; i < 200000; ++i) {
        check(from_bits(bits(rng) & 0x807fffffu), from_bits(bits(rng) & 0x807fffffu));
        check(from_bits(bits(rng)), from_bits(bits(rng) & 0x807fffffu));
    }
    for (int i = 0; i < 2000000; ++i) {
        check_rcp(from_bits(bits(rng)), rng);
    }
    for (int e = -149; e <= 127; ++e) {
        check_rcp(std::ldexp(1.0f, e), rng);
        check_rcp(-std::ldexp(1.0f, e), rng);
    }
    std::printf("%ld %ld %ld %ld\n", checked, bad, rcp_checked, rcp_bad);
    return bad == 0 && rcp_bad == 0 ? 0 : 1;
}
