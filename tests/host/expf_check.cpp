// Host check of shp::exp_f32_rn (shp_expf.hpp) over every f32 input: against
// the double exp rounded once to f32 ((float)exp((double)x), libm's double exp
// being within an ulp of double), counting the inputs where the two differ
// and the largest difference in f32 ulps; glibc's expf (what the CPU restatement
// calls) is measured against the same reference. NaN inputs must return NaN.
// Prints "<inputs> <mismatches> <max ulp> <glibc expf mismatches>" and exits
// non-zero if any result is more than 1 ulp off, any NaN is lost, or more than
// 1 input in 10^6 differs.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "shp_expf.hpp"

namespace {

struct Tally {
    uint64_t inputs = 0, mismatches = 0, glibc = 0, nan_lost = 0;
    uint32_t max_ulp = 0;
};

uint32_t bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

void run(uint64_t lo, uint64_t hi, Tally & t) {
    for (uint64_t u = lo; u < hi; ++u) {
        float x;
        const uint32_t b = static_cast<uint32_t>(u);
        std::memcpy(&x, &b, 4);
        ++t.inputs;
        const float got = shp::exp_f32_rn_host(x);
        if (x != x) {
            t.nan_lost += got == got;
            continue;
        }
        const float ref = static_cast<float>(std::exp(static_cast<double>(x)));
        if (bits(got) != bits(ref)) {
            ++t.mismatches;
            const uint32_t d = bits(got) > bits(ref) ? bits(got) - bits(ref) : bits(ref) - bits(got);
            t.max_ulp        = d > t.max_ulp ? d : t.max_ulp;
        }
        t.glibc += bits(expf(x)) != bits(ref);
    }
}

}  // namespace

int main() {
    const unsigned        n = std::thread::hardware_concurrency() > 0 ? std::thread::hardware_concurrency() : 4;
    std::vector<Tally>    part(n);
    std::vector<std::thread> th;
    const uint64_t        total = uint64_t{ 1 } << 32;
    for (unsigned i = 0; i < n; ++i) {
        th.emplace_back(run, total * i / n, total * (i + 1) / n, std::ref(part[i]));
    }
    Tally t;
    for (unsigned i = 0; i < n; ++i) {
        th[i].join();
        t.inputs += part[i].inputs;
        t.mismatches += part[i].mismatches;
        t.glibc += part[i].glibc;
        t.nan_lost += part[i].nan_lost;
        t.max_ulp = part[i].max_ulp > t.max_ulp ? part[i].max_ulp : t.max_ulp;
    }
    std::printf("%llu %llu %u %llu\n", static_cast<unsigned long long>(t.inputs),
                static_cast<unsigned long long>(t.mismatches), t.max_ulp, static_cast<unsigned long long>(t.glibc));
    return (t.max_ulp <= 1 && t.nan_lost == 0 && t.mismatches * 1000000 <= t.inputs) ? 0 : 1;
}
