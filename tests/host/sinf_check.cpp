// Host check of shp::sin_f32_fast (shp_sinf.hpp) against the correctly rounded
// sine, (float)sin((double)t): the largest error in f32 ulps (of the correctly
// rounded value) over random t in [-2^15, 2^15], t near multiples of pi/2
// (where the reduction cancels), and small and subnormal t. Also reports how
// far glibc's sinf -- what the CPU oracle calls -- is from the same reference.
// Prints "<tested> <max ulp> <share exact> <glibc max ulp>" and exits non-zero
// if the error exceeds 2 ulp.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

#include "shp_sinf.hpp"

static long   tested = 0, exact = 0;
static double worst = 0.0, worst_glibc = 0.0;

static double ulps(float got, float ref) {
    if (got == ref) {
        return 0.0;
    }
    const float up = std::nextafter(std::fabs(ref), INFINITY) - std::fabs(ref);
    return std::fabs(static_cast<double>(got) - static_cast<double>(ref)) / (ref == 0.0f ? 1.4e-45 : up);
}

static void check(float t) {
    if (!shp::sin_fast_ok(t)) {
        return;
    }
    ++tested;
    const float ref = static_cast<float>(std::sin(static_cast<double>(t)));
    const float got = shp::sin_f32_fast(t);
    const double u  = ulps(got, ref);
    exact += u == 0.0;
    if (u > worst) {
        worst = u;
        if (u > 2.0) {
            std::printf("t=%a got=%a ref=%a (%.2f ulp)\n", t, got, ref, u);
        }
    }
    const double ug = ulps(sinf(t), ref);
    worst_glibc     = ug > worst_glibc ? ug : worst_glibc;
}

int main() {
    std::mt19937_64                        rng(20260728);
    std::uniform_real_distribution<float>  wide(-32767.0f, 32767.0f);
    std::uniform_real_distribution<float>  snake(-60.0f, 60.0f);
    for (int i = 0; i < 4000000; ++i) {
        check(wide(rng));
        check(snake(rng));
    }
    for (int k = -20800; k <= 20800; ++k) {  // around every multiple of pi/2 in range
        const float c = static_cast<float>(k * 1.5707963267948966);
        float       t = c;
        for (int j = 0; j < 8; ++j) {
            check(t);
            t = std::nextafter(t, INFINITY);
        }
        t = c;
        for (int j = 0; j < 8; ++j) {
            t = std::nextafter(t, -INFINITY);
            check(t);
        }
    }
    for (int e = -149; e < 0; ++e) {
        check(std::ldexp(1.0f, e));
        check(-std::ldexp(1.3f, e));
    }
    std::printf("%ld %.3f %.4f %.3f\n", tested, worst, static_cast<double>(exact) / tested, worst_glibc);
    return worst <= 2.0 ? 0 : 1;
}
