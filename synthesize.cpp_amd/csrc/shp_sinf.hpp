// Branch-free f32 sine for |t| < 2^15, used by the Snake kernel.
//
// Reduction (Cody-Waite, with FMA): k = rint(t * 2/pi); r = t - k*pi/2 with
// pi/2 split into three f32 parts HI + MID + LO. The first step is exact: k*HI
// is a multiple of 2^-23 (HI's ulp) and so is t for |t| >= 1, and their
// difference is below 1 in magnitude, so it fits in 24 bits. The next two
// steps each round once relative to r. The three parts are the f32 roundings
// of pi/2 and of its successive remainders, taken from a 60-digit pi (LO must
// not come from a double pi/2, which is itself 2^-54 off: k*LO would then be
// wrong by ~3%, tens of ulps for r near 0 at |k| ~ 2^14); what is left,
// |pi/2 - HI - MID - LO| ~ 1e-23, times |k| < 2^15 is far below r's ulp.
// Polynomials on |r| <= pi/4 (z = r^2): sin r = r + r^3 (s1 + z (s2 + z s3)),
// cos r = 1 + z (c1 + z (c2 + z (c3 + z c4))), coefficients fitted on
// z in [0, (pi/4)^2] by iteratively reweighted least squares (relative error of the exact
// polynomials: 1.4e-8 and 2.6e-10), then rounded to f32. The quadrant k mod 4
// picks +-sin r or +-cos r.
// tests/host/sinf_check.cpp measures the error against the correctly rounded
// sine (double sin rounded to f32) over the whole range: at most 1 ulp, the
// same bound glibc's sinf meets there.
#pragma once

#include <cmath>

#ifndef SHP_HD
#    if defined(__HIPCC__)
#        define SHP_HD __host__ __device__
#    else
#        define SHP_HD
#    endif
#endif

namespace shp {

constexpr float kSinFastLimit = 32768.0f;  // |t| below this takes sin_f32_fast

// True when sin_f32_fast covers t (finite and |t| < kSinFastLimit).
SHP_HD inline bool sin_fast_ok(float t) {
    return std::fabs(t) < kSinFastLimit;
}

// +-sin t: sin_f32_fast(t) up to its sign, without the quadrant's sign flip.
// For a caller that squares the sine (Snake's sin^2): (-v)*(-v) and v*v are
// the same f32 product, so the square is bit for bit sin_f32_fast(t)^2.
SHP_HD inline float sin_f32_fast_unsigned(float t) {
    const float k = std::rint(t * 0x1.45f306p-1f);  // t * 2/pi
    float       r = std::fma(-k, 0x1.921fb6p+0f, t);
    r             = std::fma(-k, -0x1.777a5cp-25f, r);
    r             = std::fma(-k, -0x1.ee59dap-50f, r);
    const float z = r * r;
    float       s = std::fma(z, -0x1.9ac6cep-13f, 0x1.110c22p-7f);
    s             = std::fma(z, s, -0x1.555552p-3f);
    s             = std::fma(r * z, s, r);
    float c       = std::fma(z, 0x1.9a6dp-16f, -0x1.6c0e02p-10f);
    c             = std::fma(z, c, 0x1.55554cp-5f);
    c             = std::fma(z, c, -0.5f);
    c             = std::fma(z, c, 1.0f);
    return (static_cast<int>(k) & 1) ? c : s;
}

SHP_HD inline float sin_f32_fast(float t) {
    const float v = sin_f32_fast_unsigned(t);
    return (static_cast<int>(std::rint(t * 0x1.45f306p-1f)) & 2) ? -v : v;  // the quadrant's sign
}

}  // namespace shp
