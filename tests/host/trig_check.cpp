// Host check of shp::sincos_f32_rn against libm: for every tested f32 angle
// the f32 results must equal (float)sin((double)x) / (float)cos((double)x).
// Inputs: uniform random angles over the exact-reduction range, every angle
// near a multiple of pi/2 (the worst cancellations) and small/denormal angles.
// Prints "<tested> <mismatches> <out_of_range_handled>" and exits non-zero on any mismatch.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

#include "shp_trig.hpp"

static long tested = 0, bad = 0;

static void check(float x) {
    float s, c;
    if (!shp::sincos_f32_rn(x, s, c)) {
        return;
    }
    ++tested;
    const float rs = static_cast<float>(std::sin(static_cast<double>(x)));
    const float rc = static_cast<float>(std::cos(static_cast<double>(x)));
    if (std::memcmp(&s, &rs, 4) != 0 || std::memcmp(&c, &rc, 4) != 0) {
        if (++bad < 10) {
            std::printf("mismatch x=%.9g s=%.9g/%.9g c=%.9g/%.9g\n", x, s, rs, c, rc);
        }
    }
}

int main(int argc, char ** argv) {
    const long n = argc > 1 ? std::atol(argv[1]) : 2000000;
    std::mt19937_64 rng(20260728);
    std::uniform_real_distribution<double> wide(-823549.0, 823549.0), narrow(-8192.0, 8192.0);
    for (long i = 0; i < n; ++i) {
        check(static_cast<float>(wide(rng)));
        check(static_cast<float>(narrow(rng)));
    }
    const long double pio2 = 1.5707963267948966192313216916397514L;
    for (long k = -524288; k <= 524288; k += (k > -64 && k < 64) ? 1 : 97) {
        float x = static_cast<float>(k * pio2);
        for (int d = 0; d < 3; ++d) {
            check(x);
            check(std::nextafterf(x, INFINITY));
            check(std::nextafterf(x, -INFINITY));
            x = std::nextafterf(x, INFINITY);
        }
    }
    for (float x = 1e-30f; x < 1.0f; x *= 1.37f) {
        check(x);
        check(-x);
    }
    check(0.0f);
    check(-0.0f);
    check(1.4e-45f);
    float s = 0.0f, c = 0.0f;
    const bool big = shp::sincos_f32_rn(3.0e6f, s, c);
    std::printf("%ld %ld %d\n", tested, bad, big ? 0 : 1);
    return bad == 0 && !big ? 0 : 1;
}
