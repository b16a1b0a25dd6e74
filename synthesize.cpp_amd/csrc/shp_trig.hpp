// cos/sin of an f32 angle, evaluated in double and rounded once to f32.
//
// Rope needs cos/sin of angles up to the largest position (thousands of
// radians) to the last f32 bit. The reduction r = x - k*pi/2 uses pi/2 split
// into two 33-bit pieces and a 53-bit tail (Cody-Waite): for |k| <= 2^19 the
// products k*P1 and k*P2 are exact, so r carries ~100 bits of pi/2 and its
// absolute error is below 2^-78. sin and cos of r in [-pi/4, pi/4] are Taylor
// polynomials through r^19 / r^20 (truncation < 1e-18), evaluated in double
// with FMA. The f32 result equals the correctly rounded value except when the
// exact value lies within ~2^-50 relative of an f32 rounding midpoint.
//
// Compiles for host and device, so the host test suite checks it against
// libm's double sin/cos.
#pragma once

#include <cmath>

#if defined(__HIPCC__)
#    define SHP_HD __host__ __device__
#else
#    define SHP_HD
#endif

namespace shp {

// pi/2 = P1 + P2 + P3: P1, P2 hold 33 significant bits each, P3 is the rest.
constexpr double kPio2P1  = 1.5707963267341256;     // 0x3ff921fb54400000
constexpr double kPio2P2  = 6.077100506303966e-11;  // 0x3dd0b4611a600000
constexpr double kPio2P3  = 2.0222662487959506e-21; // 0x3ba3198a2e037073
constexpr double kInvPio2 = 0.6366197723675814;     // 2/pi
constexpr double kMaxK    = 524288.0;               // 2^19

// Returns false (outputs untouched) when |th| is beyond the exact-reduction range.
//
// Written for latency (one wave evaluates it once per rope position, on the
// launch's critical path): both polynomials by Estrin's scheme in z, z^2, z^4,
// z^8 (depth 4 instead of Horner's 9 and 10), the quadrant as an int32 (|k|
// <= 2^19), and the quadrant's swap and signs, and the signed zero, as
// selects rather than branches.
SHP_HD inline bool sincos_f32_rn(float th, float & s_out, float & c_out) {
    const double x = static_cast<double>(th);
    const double k = std::rint(x * kInvPio2);
    if (!(std::fabs(k) <= kMaxK)) {
        return false;
    }
    double r = std::fma(-k, kPio2P1, x);
    r        = std::fma(-k, kPio2P2, r);
    r        = std::fma(-k, kPio2P3, r);
    const double z  = r * r;
    const double z2 = z * z;
    const double z4 = z2 * z2;
    const double z8 = z4 * z4;
    // sin r = r + r z P(z), P(z) = s3 + s5 z + ... + s19 z^8 (Taylor)
    const double s01 = std::fma(0.008333333333333333, z, -0.16666666666666666);
    const double s23 = std::fma(2.7557319223985893e-06, z, -0.0001984126984126984);
    const double s45 = std::fma(1.6059043836821613e-10, z, -2.505210838544172e-08);
    const double s67 = std::fma(2.8114572543455206e-15, z, -7.647163731819816e-13);
    // cos r = 1 + z Q(z), Q(z) = -1/2 + c4 z + ... + c20 z^9 (Taylor)
    const double c01 = std::fma(0.041666666666666664, z, -0.5);
    const double c23 = std::fma(2.48015873015873e-05, z, -0.001388888888888889);
    const double c45 = std::fma(2.08767569878681e-09, z, -2.755731922398589e-07);
    const double c67 = std::fma(4.779477332387385e-14, z, -1.1470745597729725e-11);
    const double c89 = std::fma(4.110317623312165e-19, z, -1.5619206968586225e-16);
    const double s03 = std::fma(s23, z2, s01);
    const double s47 = std::fma(s67, z2, s45);
    const double c03 = std::fma(c23, z2, c01);
    const double c47 = std::fma(c67, z2, c45);
    const double ps  = std::fma(-8.22063524662433e-18, z8, std::fma(s47, z4, s03));
    const double pc  = std::fma(c89, z8, std::fma(c47, z4, c03));
    const double sr  = std::fma(r * z, ps, r);
    const double cr  = std::fma(z, pc, 1.0);
    // quadrant q = k mod 4: (sin, cos) = (sr, cr), (cr, -sr), (-sr, -cr), (-cr, sr)
    const int    q  = static_cast<int>(k) & 3;
    const double sa = (q & 1) != 0 ? cr : sr;
    const double ca = (q & 1) != 0 ? sr : cr;
    const float  sf = static_cast<float>((q & 2) != 0 ? -sa : sa);
    const float  cf = static_cast<float>(((q + 1) & 2) != 0 ? -ca : ca);
    s_out           = th == 0.0f ? th : sf;  // sin(-0) = -0
    c_out           = th == 0.0f ? 1.0f : cf;
    return true;
}

}  // namespace shp
